// Per-row top-k of |v| for gfx950: LDS radix-select + in-LDS sort.
//
// Semantics follow the reference's segmented-sort top-k
// (modules/topk_cuda/src/topk_cuda_utils.cuh:51-149, topk_cuda.cu:186-233):
// per row the k largest |v| with NaN ranked below every number, ordered by
// |v| descending, equal keys by ascending column (CUB's radix sort is stable),
// emitting the column and the signed value.  Instead of sorting every row,
// one workgroup per row finds the k-th largest composite key
//     K = key(|v|) << 16 | (0xFFFF - column)
// with MSB-first 8-bit radix passes over LDS histograms, keeps the k entries
// with K >= that threshold (K is unique per column, so exactly k) and sorts
// only those k entries in LDS.
//
// The row values are cached in LDS when they fit, so the row is read from
// HBM once; `v` can be computed on the fly as a - b or as a - dequant(NF4)
// so that the error-correction pass never materialises the error matrix.
#include "bsq_internal.hpp"
#include "nf4_codec.hpp"
#include "scalar_codecs.hpp"
#include "wave_ops.hpp"

#include <algorithm>
#include <cfloat>

namespace bsq {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kCacheMaxCols = 16384;  // 64 KiB of LDS row cache

// Marks the error section present.  During a compress the flags word holds
// 0 or kFlagError (cleared before the pass, set only here), so every row that
// finds an entry above FLT_EPSILON stores the same value: a relaxed store at
// workgroup scope, merged in each XCD's L2 and visible once the kernel ends.
// A device-scope atomicOr per row serialises at the memory side instead
// (about 10 ns apiece: 8192 rows added 78 us to a 21 us launch).
__device__ __forceinline__ void set_error_flag(uint32_t *flags) {
    __hip_atomic_store(flags, kFlagError, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ uint32_t order_key(float v) {
    // |v| as an ordered integer, NaN below +0 (build_sort_inputs_kernel maps
    // NaN to -inf, topk_cuda_utils.cuh:62-66).
    return __builtin_isnan(v) ? 0u : (__float_as_uint(fabsf(v)) + 1u);
}

template <TopkSource SRC>
__device__ __forceinline__ float load_value(const TopkArgs &a, const float *Ls, float dq, uint64_t e) {
    const float x = a.a[e];
    if constexpr (SRC == TopkSource::Dense) {
        return x;
    } else if constexpr (SRC == TopkSource::DenseMinusDense) {
        return x - a.b[e];
    } else {
        // decode of one element exactly as the NF4 / NF4_DQ decoder writes it
        // (quantization_cuda.cu:287-341), then the subtraction of
        // subtract_kernel (src/bitsqz_llm.cu:164-173).
        float s;
        if constexpr (SRC == TopkSource::DenseMinusNF4DQ) s = dq * e4m3_decode(a.scales_u8[e >> 6]);
        else s = a.scales_f32[e >> 6];
        if (s == 0.0f || !__builtin_isfinite(s)) s = 1.0f;
        const uint32_t byte = a.codes[e >> 1];
        const uint32_t code = (e & 1) ? (byte & 15u) : (byte >> 4);
        return x - s * Ls[code];
    }
}

// The values of the 4 consecutive elements e .. e + 3 (e % 4 == 0, the four
// in one row and one 64-element block, a 16-byte aligned): one 16-byte load
// of a (and of b), and for the NF4 sources one 2-byte code load and one block
// scale, decoded exactly as load_value does element by element.
template <TopkSource SRC>
__device__ __forceinline__ void load_quad(const TopkArgs &a, const float *Ls, float dq, uint64_t e, float (&v)[4]) {
    // a is streamed (read once here): a non-temporal load
    const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.a + e));
    if constexpr (SRC == TopkSource::Dense) {
        v[0] = x.x;
        v[1] = x.y;
        v[2] = x.z;
        v[3] = x.w;
    } else if constexpr (SRC == TopkSource::DenseMinusDense) {
        const float4 y = *reinterpret_cast<const float4 *>(a.b + e);
        v[0] = x.x - y.x;
        v[1] = x.y - y.y;
        v[2] = x.z - y.z;
        v[3] = x.w - y.w;
    } else {
        float s;
        if constexpr (SRC == TopkSource::DenseMinusNF4DQ) s = dq * e4m3_decode(a.scales_u8[e >> 6]);
        else s = a.scales_f32[e >> 6];
        if (s == 0.0f || !__builtin_isfinite(s)) s = 1.0f;
        const uint32_t h = *reinterpret_cast<const uint16_t *>(a.codes + (e >> 1));
        v[0] = x.x - s * Ls[(h >> 4) & 15u];
        v[1] = x.y - s * Ls[h & 15u];
        v[2] = x.z - s * Ls[(h >> 12) & 15u];
        v[3] = x.w - s * Ls[(h >> 8) & 15u];
    }
}

// Inclusive scan of one value per thread over the 256-thread workgroup.
__device__ __forceinline__ uint32_t block_inclusive_scan(uint32_t v, uint32_t *wsum) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(v, off);
        if (lane >= off) v += t;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    uint32_t add = 0;
    for (int w = 0; w < wave; ++w) add += wsum[w];
    __syncthreads();
    return v + add;
}

struct Shared {
    uint32_t hist[256];
    uint32_t wsum[kThreads / 64];
    uint32_t digit, above;  // chosen digit, count strictly above it
    uint32_t ncand;
    unsigned long long kt, kth;  // filter threshold, k-th largest composite key (fast path)
    float L[16];
    float wmax[kThreads / 64];  // per-wave maxima of the row's NF4_DQ block maxima
    float gwmax[kThreads / 64];  // per-wave maxima of the per-row maxima (fused NF4_DQ encode)
};

// Fast path (row cached, k <= 256): at most this many candidates are ranked
// directly; more fall back to the radix select.
constexpr uint32_t kFastCap = 512;

__device__ __forceinline__ unsigned long long composite_key(float v, uint32_t c) {
    return (static_cast<unsigned long long>(order_key(v)) << 16) | (0xFFFFu - c);
}

// Number of the n keys in `buf` (LDS, 16-byte aligned) greater than `mine`:
// 16-byte reads, several in flight, so the loop runs at LDS throughput
// rather than one read latency per key.
__device__ __forceinline__ uint32_t count_greater(const unsigned long long *buf, uint32_t n,
                                                  unsigned long long mine) {
    const ulonglong2 *b2 = reinterpret_cast<const ulonglong2 *>(buf);
    uint32_t c0 = 0, c1 = 0;
#pragma unroll 8
    for (uint32_t j = 0; j < n / 2; ++j) {
        const ulonglong2 t = b2[j];
        c0 += t.x > mine ? 1u : 0u;
        c1 += t.y > mine ? 1u : 0u;
    }
    if (n & 1u) c0 += buf[n - 1] > mine ? 1u : 0u;
    return c0 + c1;
}

// Magnitude form of a composite-key threshold K = key(|t|) << 16 | (0xFFFF - c)
// with key(|t|) >= 1 (a number): |v| reaches key(|t|) exactly when
// fabsf(v) >= mag (NaN never does), and the composite key of (v, col) is
// >= K exactly when fabsf(v) > mag, or fabsf(v) == mag and col <= c.
struct MagThreshold {
    float mag;
    uint32_t col;
    __device__ explicit MagThreshold(unsigned long long K)
        : mag(__uint_as_float(static_cast<uint32_t>(K >> 16) - 1u)), col(0xFFFFu - static_cast<uint32_t>(K & 0xFFFFu)) {}
    __device__ bool reaches_key(float v) const { return fabsf(v) >= mag; }
    __device__ bool reaches(float v, uint32_t c) const {
        const float x = fabsf(v);
        return x > mag || (x == mag && c <= col);
    }
};

// One radix pass: histogram of digit (K >> shift) & 255 over entries whose
// already-decided high part equals `prefix`, then choose the digit holding
// the rank-`remaining` largest entry.  Returns in sh.digit / sh.above.
__device__ __forceinline__ void choose_digit(Shared &sh, uint32_t remaining) {
    const uint32_t d = threadIdx.x;                 // thread d owns bin 255 - d
    const uint32_t h = sh.hist[255 - d];
    const uint32_t incl = block_inclusive_scan(h, sh.wsum);  // entries with digit >= 255 - d
    const uint32_t above = incl - h;
    if (above < remaining && remaining <= incl) {
        sh.digit = 255 - d;
        sh.above = above;
    }
    __syncthreads();
}

template <TopkSource SRC, bool CACHED>
__global__ __launch_bounds__(kThreads) void topk_select_kernel(TopkArgs a) {
    extern __shared__ unsigned char dyn[];
    __shared__ Shared sh;
    const uint32_t cols = a.cols, k = a.k;
    const uint32_t r = blockIdx.x;
    const uint64_t row0 = static_cast<uint64_t>(r) * cols;
    // dynamic LDS: [row cache: cols floats if CACHED][candidates: P u64][selected bitmap]
    float *cache = reinterpret_cast<float *>(dyn);
    const uint32_t cache_bytes = CACHED ? ((cols * 4 + 15) & ~15u) : 0u;
    uint32_t P = 1;
    while (P < k) P <<= 1;
    unsigned long long *cand = reinterpret_cast<unsigned long long *>(dyn + cache_bytes);
    uint32_t *selbits = reinterpret_cast<uint32_t *>(dyn + cache_bytes + P * 8);
    const uint32_t nwords = (cols + 31) / 32;

    if (threadIdx.x < 16) {
        constexpr float Lc[16] = BSQ_NF4_LEVELS;
        sh.L[threadIdx.x] = Lc[threadIdx.x];
    }
    for (uint32_t w = threadIdx.x; w < nwords; w += kThreads) selbits[w] = 0;
    if (threadIdx.x == 0) {
        sh.ncand = 0;
        sh.kt = 0;
        sh.kth = 0;
    }
    float dq = 1.0f;
    if constexpr (SRC == TopkSource::DenseMinusNF4DQ) {
        dq = *a.dq;
        if (dq == 0.0f || !__builtin_isfinite(dq)) dq = 1.0f;
    }
    __syncthreads();

    auto value_at = [&](uint32_t c) -> float {
        if constexpr (CACHED) return cache[c];
        else return load_value<SRC>(a, sh.L, dq, row0 + c);
    };

    // Phase 0: values of the row (into LDS when cached) and the any-nonzero
    // test of device_buffer_has_nonzero (src/bitsqz_llm.cu:175-184, 396-423).
    bool nonzero = false;
    unsigned long long tmax = 0;  // largest composite key among this thread's columns
    const bool vec4 = ((cols & 3u) == 0) && ((reinterpret_cast<uintptr_t>(a.a) & 15u) == 0) &&
                      (SRC != TopkSource::DenseMinusDense || (reinterpret_cast<uintptr_t>(a.b) & 15u) == 0) &&
                      ((SRC != TopkSource::DenseMinusNF4 && SRC != TopkSource::DenseMinusNF4DQ) ||
                       (reinterpret_cast<uintptr_t>(a.codes) & 1u) == 0);
    if constexpr (CACHED) {
        if (SRC == TopkSource::Dense && vec4) {
            // 16-byte loads, several in flight per lane: the row is read once
            const float4 *src4 = reinterpret_cast<const float4 *>(a.a + row0);
            float4 *cache4 = reinterpret_cast<float4 *>(cache);
#pragma unroll 8
            for (uint32_t c4 = threadIdx.x; c4 < cols / 4; c4 += kThreads) {
                const float4 v4 = src4[c4];
                cache4[c4] = v4;
                const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    nonzero |= fabsf(vv[u]) > FLT_EPSILON;
                    const unsigned long long K = composite_key(vv[u], 4 * c4 + u);
                    tmax = K > tmax ? K : tmax;
                }
            }
        } else if (vec4) {
            // the subtracting sources, 4 columns at a time (one 16-byte load
            // of a, and of b or of two code bytes and the block scale)
            float4 *cache4 = reinterpret_cast<float4 *>(cache);
#pragma unroll 4
            for (uint32_t c4 = threadIdx.x; c4 < cols / 4; c4 += kThreads) {
                float vv[4];
                load_quad<SRC>(a, sh.L, dq, row0 + 4 * c4, vv);
                cache4[c4] = float4{vv[0], vv[1], vv[2], vv[3]};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    nonzero |= fabsf(vv[u]) > FLT_EPSILON;
                    const unsigned long long K = composite_key(vv[u], 4 * c4 + u);
                    tmax = K > tmax ? K : tmax;
                }
            }
        } else {
#pragma unroll 4
            for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
                const float v = load_value<SRC>(a, sh.L, dq, row0 + c);
                cache[c] = v;
                nonzero |= fabsf(v) > FLT_EPSILON;
                const unsigned long long K = composite_key(v, c);
                tmax = K > tmax ? K : tmax;
            }
        }
    } else if (a.flags) {
        for (uint32_t c = threadIdx.x; c < cols; c += kThreads)
            nonzero |= fabsf(load_value<SRC>(a, sh.L, dq, row0 + c)) > FLT_EPSILON;
    }
    if (a.flags && __syncthreads_or(nonzero ? 1 : 0)) {
        if (threadIdx.x == 0) set_error_flag(a.flags);
    }
    __syncthreads();

    uint16_t *out_idx = a.indices + static_cast<uint64_t>(r) * k;
    float *out_val = a.values + static_cast<uint64_t>(r) * k;
    if constexpr (CACHED) {
        // the filter needs at least k non-empty lanes (lanes own 4 columns
        // each on the 16-byte path, 1 otherwise)
        const uint32_t groups = (SRC == TopkSource::Dense && vec4) ? cols / 4 : cols;
        if (k <= kThreads && k <= groups) {
            // Filter: the k-th largest of the lane (or lane-pair) maxima is a key
            // that at least k entries reach, and few more than k do for any
            // spread-out row.  Rank the entries at or above it directly (keys are
            // unique); fall back to the radix select when there are too many.
            unsigned long long *tm = reinterpret_cast<unsigned long long *>(dyn + cache_bytes);
            unsigned long long *buf = tm + kThreads;
            // pairs of lanes when k allows: half the maxima to rank against
            const uint32_t nonempty = min(kThreads, groups);
            const bool pairs = 2 * k <= nonempty + 1 && k <= kThreads / 2;
            if (pairs) {
                const unsigned long long other = static_cast<unsigned long long>(static_cast<uint32_t>(
                    __builtin_amdgcn_update_dpp(0, static_cast<int>(tmax & 0xffffffffu), 0xB1, 0xF, 0xF, false))) |
                    (static_cast<unsigned long long>(static_cast<uint32_t>(
                        __builtin_amdgcn_update_dpp(0, static_cast<int>(tmax >> 32), 0xB1, 0xF, 0xF, false))) << 32);
                if ((threadIdx.x & 1u) == 0) tm[threadIdx.x >> 1] = other > tmax ? other : tmax;
            } else {
                tm[threadIdx.x] = tmax;
            }
            const uint32_t ng = pairs ? kThreads / 2 : kThreads;
            __syncthreads();
            // group g's maximum is ranked by thread g alone (the first ng threads,
            // whole waves), so every maximum is compared against the others once
            if (threadIdx.x < ng) {
                const unsigned long long gmax = tm[threadIdx.x];
                // one group ranks k-1: the maxima of non-empty groups are distinct
                if (count_greater(tm, ng, gmax) == k - 1) sh.kt = gmax;
            }
            __syncthreads();
            const unsigned long long kt = sh.kt;
            // Candidates: the entries whose magnitude reaches the threshold's
            // (one float compare each): every entry with composite key >= kt,
            // plus equal magnitudes in later columns, which the exact ranking
            // below sorts out.  A NaN threshold (key 0) takes the radix path.
            const bool kt_number = (kt >> 16) != 0;
            const MagThreshold th(kt_number ? kt : (1ull << 16));
            // count with a bitmask of this lane's hits (<= 64 entries per lane)
            unsigned long long hits = 0;
            uint32_t cnt = 0;
            const bool quads = (cols & 3u) == 0;
            if (quads) {
                const float4 *cache4 = reinterpret_cast<const float4 *>(cache);
                uint32_t i = 0;
#pragma unroll 4
                for (uint32_t c4 = threadIdx.x; c4 < cols / 4; c4 += kThreads, ++i) {
                    const float4 q = cache4[c4];
                    const unsigned long long b0 = th.reaches_key(q.x), b1 = th.reaches_key(q.y),
                                             b2 = th.reaches_key(q.z), b3 = th.reaches_key(q.w);
                    hits |= (b0 | (b1 << 1) | (b2 << 2) | (b3 << 3)) << (4 * i);
                }
            } else {
                uint32_t i = 0;
                for (uint32_t c = threadIdx.x; c < cols; c += kThreads, ++i)
                    hits |= static_cast<unsigned long long>(th.reaches_key(cache[c])) << i;
            }
            cnt = static_cast<uint32_t>(__popcll(hits));
            const uint32_t incl = block_inclusive_scan(cnt, sh.wsum);
            if (threadIdx.x == kThreads - 1) sh.ncand = kt_number ? incl : kFastCap + 1;
            __syncthreads();
            const uint32_t total = sh.ncand;
            if (total <= kFastCap) {
                uint32_t pos = incl - cnt;
                while (hits) {
                    const uint32_t b = static_cast<uint32_t>(__ffsll(static_cast<long long>(hits)) - 1);
                    hits &= hits - 1;
                    const uint32_t c = quads ? 4 * (threadIdx.x + kThreads * (b >> 2)) + (b & 3u)
                                             : threadIdx.x + kThreads * b;
                    buf[pos++] = composite_key(cache[c], c);
                }
                __syncthreads();
                for (uint32_t i = threadIdx.x; i < total; i += kThreads) {
                    const unsigned long long mine = buf[i];
                    const uint32_t rank = count_greater(buf, total, mine);
                    if (rank < k) {
                        const uint32_t col = 0xFFFFu - static_cast<uint32_t>(mine & 0xFFFFu);
                        out_idx[rank] = static_cast<uint16_t>(col);
                        out_val[rank] = cache[col];
                        if (rank == k - 1) sh.kth = mine;
                    }
                }
                if (a.residual) {
                    __syncthreads();
                    // the k-th largest key is a number here (it reaches kt)
                    const MagThreshold kth(sh.kth);
                    float *res = a.residual + row0;
                    if ((cols & 3u) == 0 && (reinterpret_cast<uintptr_t>(a.residual) & 15u) == 0) {
                        const float4 *cache4 = reinterpret_cast<const float4 *>(cache);
#pragma unroll 4
                        for (uint32_t c4 = threadIdx.x; c4 < cols / 4; c4 += kThreads) {
                            float4 v = cache4[c4];
                            const uint32_t c = 4 * c4;
                            v.x = kth.reaches(v.x, c + 0) ? 0.0f : v.x;
                            v.y = kth.reaches(v.y, c + 1) ? 0.0f : v.y;
                            v.z = kth.reaches(v.z, c + 2) ? 0.0f : v.z;
                            v.w = kth.reaches(v.w, c + 3) ? 0.0f : v.w;
                            reinterpret_cast<float4 *>(res)[c4] = v;
                        }
                    } else {
                        for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
                            const float v = cache[c];
                            res[c] = kth.reaches(v, c) ? 0.0f : v;
                        }
                    }
                }
                return;  // uniform
            }
            __syncthreads();  // the radix path below reuses this LDS
            for (uint32_t w = threadIdx.x; w < nwords; w += kThreads) selbits[w] = 0;
            if (threadIdx.x == 0) sh.ncand = 0;
            __syncthreads();
        }
    }

    // Phase 1: radix select on the 32-bit key, then (if the threshold key is
    // shared by more entries than still needed) on the inverted column.
    uint32_t prefix = 0, mask = 0, remaining = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        sh.hist[threadIdx.x] = 0;
        __syncthreads();
        for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
            const uint32_t key = order_key(value_at(c));
            if ((key & mask) == prefix) atomicAdd(&sh.hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        choose_digit(sh, remaining);
        prefix |= sh.digit << shift;
        mask |= 255u << shift;
        remaining -= sh.above;
        __syncthreads();
    }
    const uint32_t tkey = prefix;
    // entries with key == tkey: `remaining` of them are still needed.  Count them.
    sh.hist[threadIdx.x] = 0;
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < cols; c += kThreads)
        if (order_key(value_at(c)) == tkey) atomicAdd(&sh.hist[0], 1u);
    __syncthreads();
    const uint32_t n_eq = sh.hist[0];
    uint32_t tinv = 0;  // threshold on (0xFFFF - column) among key == tkey
    if (n_eq > remaining) {
        uint32_t cpre = 0, cmask = 0;
        for (int shift = 8; shift >= 0; shift -= 8) {
            __syncthreads();
            sh.hist[threadIdx.x] = 0;
            __syncthreads();
            for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
                const uint32_t inv = 0xFFFFu - c;
                if (order_key(value_at(c)) == tkey && (inv & cmask) == cpre)
                    atomicAdd(&sh.hist[(inv >> shift) & 255u], 1u);
            }
            __syncthreads();
            choose_digit(sh, remaining);
            cpre |= sh.digit << shift;
            cmask |= 255u << shift;
            remaining -= sh.above;
            __syncthreads();
        }
        tinv = cpre;
    }
    __syncthreads();

    // Phase 2: collect the k entries with K >= (tkey, tinv).
    for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
        const uint32_t key = order_key(value_at(c));
        if (key > tkey || (key == tkey && (0xFFFFu - c) >= tinv)) {
            const uint32_t slot = atomicAdd(&sh.ncand, 1u);
            if (slot < P) cand[slot] = (static_cast<unsigned long long>(key) << 16) | (0xFFFFu - c);
            atomicOr(&selbits[c >> 5], 1u << (c & 31));
        }
    }
    __syncthreads();
    for (uint32_t i = k + threadIdx.x; i < P; i += kThreads) cand[i] = 0ull;  // pads sort last
    __syncthreads();

    // Phase 3: order the k entries by K descending.
    if (k <= kThreads) {
        // rank sort: each thread places one entry
        if (threadIdx.x < k) {
            const unsigned long long mine = cand[threadIdx.x];
            uint32_t rank = 0;
            for (uint32_t j = 0; j < k; ++j) rank += (cand[j] > mine) ? 1u : 0u;
            const uint32_t col = 0xFFFFu - static_cast<uint32_t>(mine & 0xFFFFu);
            out_idx[rank] = static_cast<uint16_t>(col);
            out_val[rank] = value_at(col);
        }
    } else {
        // bitonic sort, descending, over P entries
        for (uint32_t size = 2; size <= P; size <<= 1) {
            for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                for (uint32_t i = threadIdx.x; i < P / 2; i += kThreads) {
                    const uint32_t lo = 2 * i - (i & (stride - 1));
                    const uint32_t hi = lo + stride;
                    const bool desc = (lo & size) == 0;
                    const unsigned long long x = cand[lo], y = cand[hi];
                    if ((x < y) == desc) {
                        cand[lo] = y;
                        cand[hi] = x;
                    }
                }
                __syncthreads();
            }
        }
        for (uint32_t j = threadIdx.x; j < k; j += kThreads) {
            const uint32_t col = 0xFFFFu - static_cast<uint32_t>(cand[j] & 0xFFFFu);
            out_idx[j] = static_cast<uint16_t>(col);
            out_val[j] = value_at(col);
        }
    }

    // Phase 4: separation (topk_separation + zero_selected_entries_kernel,
    // topk_cuda.cu:194-201, topk_cuda_utils.cuh:95-111): the row with the
    // selected entries zeroed.  Every element is read by the thread that
    // writes it, so the residual may alias the input.
    if (a.residual) {
        __syncthreads();
        float *res = a.residual + row0;
        for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
            const bool sel = (selbits[c >> 5] >> (c & 31)) & 1u;
            const float v = sel ? 0.0f : value_at(c);
            res[c] = v;
        }
    }
}

// Register-resident variant for rows of up to 14336 columns with cols % 4 == 0
// and k <= 256: each lane keeps its NV4 column quads of the row in
// VGPRs (lane t owns columns 4 (t + 256 m) .. + 3), so LDS holds only the
// small selection arrays and many rows run per CU.  Selection as in the
// cached kernel's filter path (k-th largest lane maximum, then ranking of
// the entries at or above it), with the radix select over the registers as
// the fallback when the filter keeps more than kFastCap entries.
template <TopkSource SRC, int NV4>
__global__ __launch_bounds__(kThreads) void topk_reg_kernel(TopkArgs a) {
    constexpr bool ENC = SRC == TopkSource::EncodeNF4 || SRC == TopkSource::EncodeNF4DQ;
    __shared__ Shared sh;
    __shared__ Nf4LevelTable etab;  // encode sources: the NF4 code and level table (unused, and dropped, otherwise)
    __shared__ __attribute__((aligned(16))) unsigned long long bk[kFastCap];
    __shared__ float bv[kFastCap];
    // the row's selected columns, one bit each (separation: residual, bitmap)
    __shared__ uint32_t rowbits[NV4 * 32];
    // encode sources: each wave's block maxima and (scale, +-1 / scale) per
    // block, slot 4 m + (lane / 16) % 4 (unused, and dropped, otherwise)
    __shared__ float enc_bmax[kThreads / 64][4 * NV4];
    __shared__ float2 enc_scl[kThreads / 64][4 * NV4];
    const uint32_t cols = a.cols, k = a.k, q4 = cols / 4;
    const uint32_t r = blockIdx.x, tid = threadIdx.x;
    const uint64_t row0 = static_cast<uint64_t>(r) * cols;
    if (tid < 16) {
        constexpr float Lc[16] = BSQ_NF4_LEVELS;
        sh.L[tid] = Lc[tid];
    }
    if (tid == 0) {
        sh.kt = 0;
        sh.kth = 0;
        sh.ncand = 0;
        if (a.flags_reset && r == 0) *a.flags_reset = 0u;
    }
    const bool separate = a.residual || a.sel_bits;  // uniform
    if (separate)
        for (uint32_t w = tid; w < NV4 * 32; w += kThreads) rowbits[w] = 0u;
    float dq = 1.0f;
    if constexpr (SRC == TopkSource::DenseMinusNF4DQ) {
        dq = *a.dq;
        if (dq == 0.0f || !__builtin_isfinite(dq)) dq = 1.0f;
    }
    if constexpr (ENC) {
        nf4_level_table_build(etab);
        if constexpr (SRC == TopkSource::EncodeNF4DQ) {
            if (!a.enc_row_gmax) {  // uniform
                const float raw = dq_raw_from_gmax(*a.enc_gmax);
                dq = dq_effective(raw);
                if (r == 0 && tid == 0) *a.enc_dq_out = raw;
            }
        }
    }
    __syncthreads();

    // NF4_DQ's global scale from the separation's per-row maxima: this
    // workgroup reduces them itself (max is order-free, so every workgroup
    // gets the same bits), with the loads issued ahead of the row's so the
    // reduction overlaps the row's memory round trip; no launch in between
    constexpr int kGq = kInlineGmaxRows / (4 * kThreads);
    f32x4 gq[kGq];
    if constexpr (SRC == TopkSource::EncodeNF4DQ) {
        if (a.enc_row_gmax) {  // uniform
#pragma unroll
            for (int j = 0; j < kGq; ++j) {
                const uint32_t i4 = tid + kThreads * j;
                gq[j] = 4 * i4 < a.enc_gmax_rows ? reinterpret_cast<const f32x4 *>(a.enc_row_gmax)[i4]
                                                 : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    }

    const bool quad_ok = (SRC != TopkSource::DenseMinusNF4 && SRC != TopkSource::DenseMinusNF4DQ) ||
                         (reinterpret_cast<uintptr_t>(a.codes) & 1u) == 0;
    // the row: v[m][u] = column 4 (tid + 256 m) + u.  Absent columns (>= cols)
    // hold NaN: their composite keys are below every real entry's (NaN key 0,
    // and a smaller inverted column than any real NaN), so they never reach
    // the selection and need no bound checks.
    float v[NV4][4];
#pragma unroll
    for (int m = 0; m < NV4; ++m) {
        const uint32_t c4 = tid + kThreads * m;
        if (c4 < q4) {
            if constexpr (SRC == TopkSource::Dense || ENC) {
                // streamed: a non-temporal load, unless the caller reads the
                // input again soon (keep_input: kept in the caches)
                const f32x4 *src = reinterpret_cast<const f32x4 *>(a.a + row0) + c4;
                const f32x4 x = (SRC == TopkSource::Dense && a.keep_input) ? *src : __builtin_nontemporal_load(src);
                v[m][0] = x.x;
                v[m][1] = x.y;
                v[m][2] = x.z;
                v[m][3] = x.w;
            } else if (quad_ok) {
                load_quad<SRC>(a, sh.L, dq, row0 + 4 * c4, v[m]);
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) v[m][u] = load_value<SRC>(a, sh.L, dq, row0 + 4 * c4 + u);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) v[m][u] = __builtin_nanf("");
        }
    }
    if constexpr (SRC == TopkSource::EncodeNF4DQ) {
        if (a.enc_row_gmax) {  // uniform
            float gm = 0.0f;
#pragma unroll
            for (int j = 0; j < kGq; ++j) gm = fmaxf(gm, fmaxf(fmaxf(gq[j].x, gq[j].y), fmaxf(gq[j].z, gq[j].w)));
            for (int off = 32; off >= 1; off >>= 1) gm = fmaxf(gm, __shfl_xor(gm, off));
            if ((tid & 63) == 0) sh.gwmax[tid >> 6] = gm;
            __syncthreads();
            gm = fmaxf(fmaxf(sh.gwmax[0], sh.gwmax[1]), fmaxf(sh.gwmax[2], sh.gwmax[3]));
            const float raw = dq_raw_from_gmax(__float_as_uint(gm));
            dq = dq_effective(raw);
            if (r == 0 && tid == 0) *a.enc_dq_out = raw;
        }
    }
    if constexpr (ENC) {
        if (a.enc_sel) {  // uniform: entries a separation took out read as 0
            const uint32_t *srow = a.enc_sel + (row0 >> 5);
#pragma unroll
            for (int m = 0; m < NV4; ++m) {
                const uint32_t c4 = tid + kThreads * m;
                if (c4 < q4) {
                    const uint32_t nib = srow[c4 >> 3] >> (4u * (c4 & 7u));
#pragma unroll
                    for (int u = 0; u < 4; ++u) v[m][u] = ((nib >> u) & 1u) ? 0.0f : v[m][u];
                }
            }
        }
        // Encode, exactly as quant_encode_kernel does chunk by chunk: the
        // quads of the 16 lanes of one DPP row at one m are one 64-element
        // block (cols % 64 == 0); block absmax of the sanitised values,
        // scale (NF4: the absmax; NF4_DQ: dq * E4M3(absmax / dq)), codes of
        // v / scale.  Then v becomes the error a - scale * L[code] of the
        // raw value, as the DenseMinusNF4(DQ) sources compute it from the
        // stored encoding.  Padding rows (whole DPP rows past the row end)
        // store nothing and stay NaN.
        //
        // The scale of a block is the same in its 16 lanes, and its chain
        // (NF4_DQ: a division, the E4M3 encode and decode; then 1 / scale)
        // costs the same issue slots whether one lane needs it or 64.  So
        // the wave's 4 NV4 block maxima go to LDS (slot 4 m + block of the
        // DPP row), one lane per block runs the chain once for all of them,
        // and the quads read their block's scale back.
        const int g = static_cast<int>((tid >> 4) & 3u), wv = static_cast<int>(tid >> 6), wl = static_cast<int>(tid & 63u);
#pragma unroll
        for (int m = 0; m < NV4; ++m) {
            float lm = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) lm = fmaxf(lm, fabsf(sanitize(v[m][u])));
            const float bm = row16_max(lm);
            if ((tid & 15u) == 0) enc_bmax[wv][4 * m + g] = bm;
        }
        __syncthreads();
        if (wl < 4 * NV4) {
            const float bm = enc_bmax[wv][wl];
            const float absmax = (bm > 0.0f) ? bm : 1.0f;
            float scale;
            uint32_t scode = 0;
            if constexpr (SRC == TopkSource::EncodeNF4DQ) {
                scode = e4m3_encode(absmax / dq);
                scale = dq * e4m3_decode(scode);
                if (scale == 0.0f || !__builtin_isfinite(scale)) scale = 1.0f;
            } else {
                scale = absmax;
            }
            const float inv = 1.0f / scale;
            // |w| < 2 in the whole block unless its scale fell far below its
            // absmax (an NF4_DQ scale code of 0 replaced by 1); rounding is
            // monotone, so the block's largest |w| is exactly fl(bm * inv).
            // The flag rides in the sign of inv (> 0).
            enc_scl[wv][wl] = float2{scale, (bm * inv < 2.0f) ? inv : -inv};
            const uint32_t c4b = static_cast<uint32_t>(64 * wv + 16 * (wl & 3) + kThreads * (wl >> 2));
            if (c4b < q4) {
                const uint64_t blk = (row0 + 4ull * c4b) >> 6;
                if constexpr (SRC == TopkSource::EncodeNF4DQ) a.enc_scales_u8[blk] = static_cast<uint8_t>(scode);
                else a.enc_scales_f32[blk] = scale;
            }
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < NV4; ++m) {
            const uint32_t c4 = tid + kThreads * m;
            const bool inside = c4 < q4;
            const float2 sc = enc_scl[wv][4 * m + g];
            const float scale = sc.x, inv = fabsf(sc.y);
            const bool small = sc.y > 0.0f;  // the table for the whole block
            uint32_t packed = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float w = sanitize(v[m][u]) * inv;
                float lv;
                uint32_t c;
                if (small) {
                    c = nf4_code_level_small(etab, w, lv);
                } else {
                    c = (fabsf(w) < 2.0f) ? nf4_code_level_small(etab, w, lv) : nf4_code_scan_inline(sh.L, w);
                    lv = sh.L[c];
                }
                // element 2j in the high nibble: bytes (c0 c1) (c2 c3)
                packed |= c << (8 * (u >> 1) + 4 * (1 - (u & 1)));
                v[m][u] = inside ? v[m][u] - scale * lv : __builtin_nanf("");
                // the error is formed here: left to the compiler, the
                // subtraction sinks to the first later use and the levels
                // and scales of every quad stay live until then
                asm volatile("" : "+v"(v[m][u]));
            }
            if (inside) {
                const uint64_t e = row0 + 4ull * c4;
                *reinterpret_cast<uint16_t *>(a.enc_codes + (e >> 1)) = static_cast<uint16_t>(packed);
            }
        }
    }
    // keys are recomputed from the values in every phase (an opaque copy of
    // the lane index stops the compiler from keeping 2 * 4 * NV4 key registers
    // live across the phases)
    auto key_of = [&](uint32_t t, int m, int u) -> unsigned long long {
        return composite_key(v[m][u], 4 * (t + kThreads * m) + u);
    };
    auto lane_id = [&]() -> uint32_t {
        uint32_t t = threadIdx.x;
        asm volatile("" : "+v"(t));
        // the row values too: keys derived from them in one phase are
        // recomputed in the next instead of being kept live across it
#pragma unroll
        for (int m = 0; m < NV4; ++m)
#pragma unroll
            for (int u = 0; u < 4; ++u) asm volatile("" : "+v"(v[m][u]));
        return t;
    };
    // the lane's largest |v| (a compare-select skips NaN, which ranks lowest;
    // all-NaN lanes keep -1), i.e. its largest 32-bit order key
    float mx = -1.0f;
#pragma unroll
    for (int m = 0; m < NV4; ++m)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float f = fabsf(v[m][u]);
            mx = f > mx ? f : mx;
        }
    const uint32_t key32 = mx >= 0.0f ? __float_as_uint(mx) + 1u : 0u;
    const bool nonzero = mx > FLT_EPSILON;  // false for NaN-only and padding lanes
    if (a.flags && __syncthreads_or(nonzero ? 1 : 0)) {
        if (tid == 0) set_error_flag(a.flags);
    }
    // filter threshold: the top 16 bits of the k-th largest lane maximum's
    // order key, by two 8-bit radix passes over one key per lane (k lanes
    // hold a key >= it, so at least k entries pass; the candidates are then
    // ranked exactly, so any such lower bound gives the same result)
    uint32_t prefix = 0, remaining = k;
#pragma unroll
    for (int shift = 24; shift >= 16; shift -= 8) {
        sh.hist[tid] = 0;
        __syncthreads();
        const uint32_t hmask = shift == 24 ? 0u : 0xFF000000u;
        if ((key32 & hmask) == prefix) atomicAdd(&sh.hist[(key32 >> shift) & 255u], 1u);
        __syncthreads();
        choose_digit(sh, remaining);
        prefix |= sh.digit << shift;
        remaining -= sh.above;
    }
    unsigned long long kt = static_cast<unsigned long long>(prefix) << 16;
    uint32_t lt;
    // candidates by magnitude (a superset of the top k, ranked exactly
    // below); a threshold without a number takes the radix path
    const bool kt_number = (kt >> 16) != 0;
    const MagThreshold th(kt_number ? kt : (1ull << 16));
    uint32_t cnt = 0;
    lt = lane_id();
#pragma unroll
    for (int m = 0; m < NV4; ++m) {
#pragma unroll
        for (int u = 0; u < 4; ++u) cnt += th.reaches_key(v[m][u]) ? 1u : 0u;
        __builtin_amdgcn_sched_barrier(0);
    }
    uint32_t incl = block_inclusive_scan(cnt, sh.wsum);
    if (tid == kThreads - 1) sh.ncand = kt_number ? incl : kFastCap + 1;
    __syncthreads();
    uint32_t total = sh.ncand;
    bool exact = false;  // candidates are exactly the keys >= kt (radix path)
    if (total > kFastCap) {
        // fallback: exact threshold by radix select over the registers, on the
        // 32-bit key, then on the inverted column among equal keys
        // (each pass re-derives the keys from the laundered row values:
        // keys hoisted out of the pass loop would hold 4 NV4 more registers
        // for the whole kernel, and cost the fast path its occupancy)
        uint32_t prefix = 0, mask = 0, remaining = k;
        for (int shift = 24; shift >= 0; shift -= 8) {
            sh.hist[tid] = 0;
            (void)lane_id();
            __syncthreads();
#pragma unroll
            for (int m = 0; m < NV4; ++m)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t key = order_key(v[m][u]);
                    if ((key & mask) == prefix) atomicAdd(&sh.hist[(key >> shift) & 255u], 1u);
                    __builtin_amdgcn_sched_barrier(0);
                }
            __syncthreads();
            choose_digit(sh, remaining);
            prefix |= sh.digit << shift;
            mask |= 255u << shift;
            remaining -= sh.above;
            __syncthreads();
        }
        const uint32_t tkey = prefix;
        uint32_t cpre = 0, cmask = 0;
        for (int shift = 8; shift >= 0; shift -= 8) {
            sh.hist[tid] = 0;
            lt = lane_id();  // the inverted columns too: derived per pass, not held
            __syncthreads();
#pragma unroll
            for (int m = 0; m < NV4; ++m)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t inv = 0xFFFFu - (4 * (lt + kThreads * m) + u);
                    if (order_key(v[m][u]) == tkey && (inv & cmask) == cpre)
                        atomicAdd(&sh.hist[(inv >> shift) & 255u], 1u);
                    __builtin_amdgcn_sched_barrier(0);
                }
            __syncthreads();
            choose_digit(sh, remaining);
            cpre |= sh.digit << shift;
            cmask |= 255u << shift;
            remaining -= sh.above;
            __syncthreads();
        }
        kt = (static_cast<unsigned long long>(tkey) << 16) | cpre;  // exactly k keys are >= kt
        cnt = 0;
        lt = lane_id();
#pragma unroll
        for (int m = 0; m < NV4; ++m) {
#pragma unroll
            for (int u = 0; u < 4; ++u) cnt += (key_of(lt, m, u) >= kt) ? 1u : 0u;
            __builtin_amdgcn_sched_barrier(0);
        }
        incl = block_inclusive_scan(cnt, sh.wsum);
        total = k;
        exact = true;
    }
    // collect the candidates with their values, then rank them (on the
    // filter path the key is formed only for the few entries that pass)
    uint32_t pos = incl - cnt;
    lt = lane_id();
    if (!exact) {  // uniform
#pragma unroll
        for (int m = 0; m < NV4; ++m) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (th.reaches_key(v[m][u])) {
                    bk[pos] = key_of(lt, m, u);
                    bv[pos] = v[m][u];
                    ++pos;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
#pragma unroll
        for (int m = 0; m < NV4; ++m) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const unsigned long long K = key_of(lt, m, u);
                if (K >= kt) {
                    bk[pos] = K;
                    bv[pos] = v[m][u];
                    ++pos;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __syncthreads();
    uint16_t *out_idx = a.indices + static_cast<uint64_t>(r) * k;
    float *out_val = a.values + static_cast<uint64_t>(r) * k;
    for (uint32_t i = tid; i < total; i += kThreads) {
        const unsigned long long mine = bk[i];
        const uint32_t rank = count_greater(bk, total, mine);
        if (rank < k) {
            const uint32_t col = 0xFFFFu - static_cast<uint32_t>(mine & 0xFFFFu);
            out_idx[rank] = static_cast<uint16_t>(col);
            out_val[rank] = bv[i];
            if (separate) atomicOr(&rowbits[col >> 5], 1u << (col & 31u));
        }
    }
    if (separate) {
        // the selected entries from the row's bitmap in LDS (set by the
        // ranking above: one bit test per element instead of a key
        // comparison)
        __syncthreads();
        if (a.sel_bits)  // cols % 64 == 0: whole words
            for (uint32_t w = tid; w < cols / 32; w += kThreads) a.sel_bits[(row0 >> 5) + w] = rowbits[w];
        float4 *res4 = a.residual ? reinterpret_cast<float4 *>(a.residual + row0) : nullptr;
        lt = lane_id();
        // with row_gmax (cols % 64 == 0): a 64-element block is the quads of
        // 16 consecutive lanes (one DPP row) at one m, its absmax a 4-step
        // DPP max
        float gm = 0.0f;
        if (a.residual || a.row_gmax)  // uniform
#pragma unroll
        for (int m = 0; m < NV4; ++m) {
            const uint32_t c4 = lt + kThreads * m;
            // columns 4 c4 .. 4 c4 + 3: bits 4 (c4 % 8) .. + 3 of word c4 / 8
            const uint32_t nib = rowbits[min(c4 >> 3, static_cast<uint32_t>(NV4 * 32 - 1))] >> (4u * (c4 & 7u));
            float4 o;
            o.x = (nib & 1u) ? 0.0f : v[m][0];
            o.y = (nib & 2u) ? 0.0f : v[m][1];
            o.z = (nib & 4u) ? 0.0f : v[m][2];
            o.w = (nib & 8u) ? 0.0f : v[m][3];
            if (a.residual) {  // uniform
                if (c4 < q4) res4[c4] = o;
            }
            if (a.row_gmax) {  // uniform
                auto san = [](float x) { return __builtin_isfinite(x) ? fabsf(x) : 0.0f; };
                const float bm = row16_max(fmaxf(fmaxf(san(o.x), san(o.y)), fmaxf(san(o.z), san(o.w))));
                if (c4 < q4) gm = fmaxf(gm, bm > 0.0f ? bm : 1.0f);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (a.row_gmax) {
            for (int off = 32; off >= 1; off >>= 1) gm = fmaxf(gm, __shfl_xor(gm, off));
            __syncthreads();
            if ((tid & 63) == 0) sh.wmax[tid >> 6] = gm;
            __syncthreads();
            if (tid == 0) a.row_gmax[r] = fmaxf(fmaxf(sh.wmax[0], sh.wmax[1]), fmaxf(sh.wmax[2], sh.wmax[3]));
        }
    }
}

// The composite key of rank `rank` (0 = largest) of one row: MSB-first 8-bit
// radix select over the 48-bit composite keys (unique per column, so the
// result is exact).  Uniform across the workgroup.
template <class F>
__device__ unsigned long long radix_select48(Shared &sh, uint32_t cols, uint32_t rank, F &&value_at) {
    unsigned long long prefix = 0, mask = 0;
    uint32_t remaining = rank + 1;
    for (int shift = 40; shift >= 0; shift -= 8) {
        sh.hist[threadIdx.x] = 0;
        __syncthreads();
        for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
            const unsigned long long K = composite_key(value_at(c), c);
            if ((K & mask) == prefix) atomicAdd(&sh.hist[static_cast<uint32_t>(K >> shift) & 255u], 1u);
        }
        __syncthreads();
        choose_digit(sh, remaining);
        prefix |= static_cast<unsigned long long>(sh.digit) << shift;
        mask |= 255ull << shift;
        remaining -= sh.above;
        __syncthreads();
    }
    return prefix;
}

// Top-k with k above kTopkMaxK (up to every column of the row): workgroup
// (r, b) emits the ranks [b * kTopkMaxK, min(k, (b + 1) * kTopkMaxK)) of row
// r.  Its rank boundaries come from two radix selects; the band's entries
// (at most kTopkMaxK, keys unique) are collected and bitonic-sorted in LDS.
// The row is cached in LDS when it fits.  Separation, when asked for, is a
// second pass (topk_separate_kernel) over the emitted indices, since the
// bands of a row run in different workgroups.
template <TopkSource SRC, bool CACHED>
__global__ __launch_bounds__(kThreads) void topk_band_kernel(TopkArgs a) {
    extern __shared__ unsigned char dyn[];
    __shared__ Shared sh;
    const uint32_t cols = a.cols, k = a.k;
    const uint32_t r = blockIdx.x;
    const uint32_t lo = blockIdx.y * kTopkMaxK, hi = min(k, lo + kTopkMaxK);
    const uint64_t row0 = static_cast<uint64_t>(r) * cols;
    float *cache = reinterpret_cast<float *>(dyn);
    const uint32_t cache_bytes = CACHED ? ((cols * 4 + 15) & ~15u) : 0u;
    uint32_t P = 1;
    while (P < hi - lo) P <<= 1;
    unsigned long long *cand = reinterpret_cast<unsigned long long *>(dyn + cache_bytes);
    if (threadIdx.x < 16) {
        constexpr float Lc[16] = BSQ_NF4_LEVELS;
        sh.L[threadIdx.x] = Lc[threadIdx.x];
    }
    if (threadIdx.x == 0) sh.ncand = 0;
    float dq = 1.0f;
    if constexpr (SRC == TopkSource::DenseMinusNF4DQ) {
        dq = *a.dq;
        if (dq == 0.0f || !__builtin_isfinite(dq)) dq = 1.0f;
    }
    __syncthreads();
    bool nonzero = false;
    for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
        const float v = load_value<SRC>(a, sh.L, dq, row0 + c);
        if constexpr (CACHED) cache[c] = v;
        nonzero |= fabsf(v) > FLT_EPSILON;
    }
    if (a.flags && blockIdx.y == 0 && __syncthreads_or(nonzero ? 1 : 0)) {
        if (threadIdx.x == 0) set_error_flag(a.flags);
    }
    __syncthreads();
    auto value_at = [&](uint32_t c) -> float {
        if constexpr (CACHED) return cache[c];
        else return load_value<SRC>(a, sh.L, dq, row0 + c);
    };
    // band: lower <= K (rank hi - 1), and K < upper (rank lo - 1) unless lo == 0
    const unsigned long long lower = radix_select48(sh, cols, hi - 1, value_at);
    const unsigned long long upper = lo > 0 ? radix_select48(sh, cols, lo - 1, value_at) : ~0ull;
    for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
        const unsigned long long K = composite_key(value_at(c), c);
        if (K >= lower && (lo == 0 || K < upper)) {
            const uint32_t slot = atomicAdd(&sh.ncand, 1u);
            if (slot < P) cand[slot] = K;
        }
    }
    __syncthreads();
    for (uint32_t i = (hi - lo) + threadIdx.x; i < P; i += kThreads) cand[i] = 0ull;  // pads sort last
    __syncthreads();
    for (uint32_t size = 2; size <= P; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = threadIdx.x; i < P / 2; i += kThreads) {
                const uint32_t l = 2 * i - (i & (stride - 1));
                const uint32_t h = l + stride;
                const bool desc = (l & size) == 0;
                const unsigned long long x = cand[l], y = cand[h];
                if ((x < y) == desc) {
                    cand[l] = y;
                    cand[h] = x;
                }
            }
            __syncthreads();
        }
    }
    uint16_t *out_idx = a.indices + static_cast<uint64_t>(r) * k + lo;
    float *out_val = a.values + static_cast<uint64_t>(r) * k + lo;
    for (uint32_t j = threadIdx.x; j < hi - lo; j += kThreads) {
        const uint32_t col = 0xFFFFu - static_cast<uint32_t>(cand[j] & 0xFFFFu);
        out_idx[j] = static_cast<uint16_t>(col);
        out_val[j] = value_at(col);
    }
}

// residual = a with the k selected columns of every row zeroed
// (zero_selected_entries_kernel, topk_cuda_utils.cuh:95-111); the residual
// may alias the input.  One workgroup per row.
__global__ __launch_bounds__(kThreads) void topk_separate_kernel(const float *__restrict__ a, float *residual,
                                                                 uint32_t cols, uint32_t k,
                                                                 const uint16_t *__restrict__ idx) {
    const uint64_t row0 = static_cast<uint64_t>(blockIdx.x) * cols;
    if (residual != a)
        for (uint32_t c = threadIdx.x; c < cols; c += kThreads) residual[row0 + c] = a[row0 + c];
    __syncthreads();
    const uint16_t *ri = idx + static_cast<uint64_t>(blockIdx.x) * k;
    for (uint32_t j = threadIdx.x; j < k; j += kThreads) residual[row0 + ri[j]] = 0.0f;
}

template <TopkSource SRC>
void launch_band(const TopkArgs &a, hipStream_t stream) {
    const bool cached = a.cols <= kCacheMaxCols;
    const size_t cache_bytes = cached ? ((a.cols * 4u + 15u) & ~15u) : 0u;
    const size_t lds = cache_bytes + static_cast<size_t>(kTopkMaxK) * 8;
    BSQ_REQUIRE(lds + sizeof(Shared) <= 160u * 1024u, "top-k: band does not fit in LDS");
    const dim3 grid(a.rows, static_cast<unsigned>(ceil_div(a.k, kTopkMaxK)));
    auto run = [&](auto kern) {
        BSQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(lds)));
        kern<<<grid, kThreads, lds, stream>>>(a);
        BSQ_HIP(hipGetLastError());
    };
    if (cached) run(topk_band_kernel<SRC, true>);
    else run(topk_band_kernel<SRC, false>);
    if (a.residual) {
        BSQ_REQUIRE(SRC == TopkSource::Dense, "top-k: separation reads a dense source");
        topk_separate_kernel<<<a.rows, kThreads, 0, stream>>>(a.a, a.residual, a.cols, a.k, a.indices);
        BSQ_HIP(hipGetLastError());
    }
}

template <TopkSource SRC, int NV4>
void launch_reg(const TopkArgs &a, hipStream_t stream) {
    topk_reg_kernel<SRC, NV4><<<a.rows, kThreads, 0, stream>>>(a);
}

// Whether the register-resident kernel serves this shape: rows up to 11264
// columns (44 values per lane, about 120 VGPRs: four rows per CU, one more
// than the LDS-cached kernel fits), and up to 14336 columns with 56 values
// per lane (148 VGPRs, three rows per CU, where the LDS-cached kernel holds
// two: C5's 14336-column passes 535 -> 376 and 398 -> 238 us).
bool reg_eligible(const TopkArgs &a) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(a.a) | reinterpret_cast<uintptr_t>(a.residual) |
                         (a.source == TopkSource::DenseMinusDense ? reinterpret_cast<uintptr_t>(a.b) : 0);
    if (a.k > kTopkMaxK || (a.cols & 3u) != 0 || (al & 15u) != 0 || a.k > kThreads || a.k > a.cols / 4) return false;
    return ceil_div(a.cols / 4, kThreads) <= 14;
}

// True (and launched) when the register-resident kernel serves this shape.
template <TopkSource SRC>
bool try_launch_reg(const TopkArgs &a, hipStream_t stream) {
    if (!reg_eligible(a)) return false;
    const uint32_t nv4 = static_cast<uint32_t>(ceil_div(a.cols / 4, kThreads));
    if (nv4 <= 2) launch_reg<SRC, 2>(a, stream);
    else if (nv4 <= 4) launch_reg<SRC, 4>(a, stream);
    else if (nv4 <= 8) launch_reg<SRC, 8>(a, stream);
    else if (nv4 <= 11) launch_reg<SRC, 11>(a, stream);
    else if (nv4 <= 14) launch_reg<SRC, 14>(a, stream);
    else return false;
    return true;
}

__global__ __launch_bounds__(256) void topk_scatter_kernel(const uint16_t *__restrict__ idx0,
                                                           const float *__restrict__ val0, uint32_t k0,
                                                           const uint16_t *__restrict__ idx1,
                                                           const float *__restrict__ val1, uint32_t k1, uint32_t cols,
                                                           float *__restrict__ dense, bool accumulate,
                                                           const uint32_t *__restrict__ gate0) {
    const uint64_t r = blockIdx.x;
    const uint32_t t = threadIdx.x, nt = blockDim.x;
    float *row = dense + r * cols;
    // this thread's first entry of the second set, fetched before the first
    // set's updates so its latency overlaps them
    uint32_t c1 = 0xFFFFFFFFu;
    float v1 = 0.0f;
    if (t < k1) {
        c1 = idx1[r * k1 + t];
        v1 = val1[r * k1 + t];
    }
    if (gate0 && !(*gate0 & kFlagError)) k0 = 0;
    for (uint32_t j = t; j < k0; j += nt) {
        const uint32_t c = idx0[r * k0 + j];
        if (c < cols) {
            if (accumulate) row[c] += val0[r * k0 + j];
            else row[c] = val0[r * k0 + j];
        }
    }
    if (k1 == 0) return;
    __syncthreads();  // the first set lands before the second (same order as the reference)
    if (c1 < cols) row[c1] += v1;
    for (uint32_t j = t + nt; j < k1; j += nt) {
        const uint32_t c = idx1[r * k1 + j];
        if (c < cols) row[c] += val1[r * k1 + j];
    }
}

// One top-k set at flat positions, as the reference's scatter_add_topk_kernel
// writes it (topk_cuda_utils.cuh:132-149): dense[r * cols + idx] += v, so an
// index >= cols lands in a later row.  Used for loaded objects whose indices
// are not all below cols; positions past the end of the matrix (where the
// reference would write outside the buffer) are skipped.
__global__ __launch_bounds__(256) void topk_scatter_flat_kernel(const uint16_t *__restrict__ idx,
                                                                const float *__restrict__ val, uint32_t k,
                                                                uint64_t total, uint32_t cols, uint64_t n,
                                                                float *__restrict__ dense) {
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= total) return;
    const uint64_t p = (e / k) * cols + idx[e];
    if (p < n) dense[p] += val[e];
}

template <TopkSource SRC>
void launch_src(const TopkArgs &a, hipStream_t stream) {
    if (a.k > kTopkMaxK) {
        launch_band<SRC>(a, stream);
        return;
    }
    if (try_launch_reg<SRC>(a, stream)) return;
    uint32_t P = 1;
    while (P < a.k) P <<= 1;
    const bool cached = a.cols <= kCacheMaxCols;
    const size_t cache_bytes = cached ? ((a.cols * 4u + 15u) & ~15u) : 0u;
    size_t lds = cache_bytes + static_cast<size_t>(P) * 8 + ((a.cols + 31) / 32) * 4;
    if (cached && a.k <= kThreads) lds = std::max(lds, cache_bytes + static_cast<size_t>(kThreads + kFastCap) * 8);
    BSQ_REQUIRE(lds + sizeof(Shared) <= 160u * 1024u, "top-k: row too large for the LDS sort");
    if (cached) {
        auto kern = topk_select_kernel<SRC, true>;
        if (lds > 64u * 1024u)
            BSQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        kern<<<a.rows, kThreads, lds, stream>>>(a);
    } else {
        auto kern = topk_select_kernel<SRC, false>;
        if (lds > 64u * 1024u)
            BSQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        kern<<<a.rows, kThreads, lds, stream>>>(a);
    }
}

}  // namespace

bool topk_encode_supported(uint32_t rows, uint32_t cols, uint32_t k, const float *a, const uint8_t *codes) {
    TopkArgs t;
    t.a = a;
    t.rows = rows;
    t.cols = cols;
    t.k = k;
    return rows > 0 && rows <= 65535 && k >= 1 && cols % 64 == 0 && cols <= 65535 && reg_eligible(t) &&
           (reinterpret_cast<uintptr_t>(codes) & 1u) == 0;
}

bool topk_selbits_supported(uint32_t rows, uint32_t cols, uint32_t k, const float *a) {
    TopkArgs t;
    t.a = a;
    t.rows = rows;
    t.cols = cols;
    t.k = k;
    return rows > 0 && rows <= 65535 && k >= 1 && k <= kTopkMaxK && cols % 64 == 0 && cols <= 65535 &&
           reg_eligible(t);
}

bool launch_topk_select(const TopkArgs &args, hipStream_t stream) {
    TopkArgs a = args;
    const bool reg = a.k >= 1 && a.k <= kTopkMaxK && reg_eligible(a);
    const bool gmax =
        a.row_gmax && (a.residual || a.sel_bits) && a.source == TopkSource::Dense && a.cols % 64 == 0 && reg;
    if (!gmax) a.row_gmax = nullptr;
    BSQ_REQUIRE(!a.sel_bits || (topk_selbits_supported(a.rows, a.cols, a.k, a.a) && !a.residual &&
                                a.source == TopkSource::Dense),
                "top-k: the selection bitmap needs a dense source in the register kernel's shapes");
    BSQ_REQUIRE(a.rows > 0 && a.cols > 0 && a.cols <= 65535 && a.rows <= 65535, "top-k: bad shape");
    BSQ_REQUIRE(a.k >= 1 && a.k <= a.cols, "top-k: k must be in [1, cols]");
    BSQ_REQUIRE(a.a && a.indices && a.values, "top-k: null pointer");
    BSQ_REQUIRE(!(a.flags_reset && a.flags), "top-k: a pass that sets the flags word cannot also clear it");
    if (a.flags_reset && !reg) {
        BSQ_HIP(hipMemsetAsync(a.flags_reset, 0, sizeof(uint32_t), stream));
        a.flags_reset = nullptr;
    }
    switch (a.source) {
        case TopkSource::Dense: launch_src<TopkSource::Dense>(a, stream); break;
        case TopkSource::DenseMinusDense:
            BSQ_REQUIRE(a.b, "top-k: null subtrahend");
            launch_src<TopkSource::DenseMinusDense>(a, stream);
            break;
        case TopkSource::DenseMinusNF4:
            BSQ_REQUIRE(a.scales_f32 && a.codes, "top-k: null NF4 subtrahend");
            launch_src<TopkSource::DenseMinusNF4>(a, stream);
            break;
        case TopkSource::DenseMinusNF4DQ:
            BSQ_REQUIRE(a.scales_u8 && a.codes && a.dq, "top-k: null NF4_DQ subtrahend");
            launch_src<TopkSource::DenseMinusNF4DQ>(a, stream);
            break;
        case TopkSource::EncodeNF4:
        case TopkSource::EncodeNF4DQ: {
            const bool dq = a.source == TopkSource::EncodeNF4DQ;
            BSQ_REQUIRE(topk_encode_supported(a.rows, a.cols, a.k, a.a, a.enc_codes) && !a.residual,
                        "top-k: shape outside the fused encode pass");
            BSQ_REQUIRE(dq ? (a.enc_scales_u8 && (a.enc_gmax || a.enc_row_gmax) && a.enc_dq_out)
                           : (a.enc_scales_f32 != nullptr),
                        "top-k: null encode output");
            BSQ_REQUIRE(!a.enc_row_gmax || (dq && a.enc_gmax_rows > 0 && a.enc_gmax_rows % 4 == 0 &&
                                            a.enc_gmax_rows <= kInlineGmaxRows &&
                                            (reinterpret_cast<uintptr_t>(a.enc_row_gmax) & 15u) == 0),
                        "top-k: per-row maxima outside the fused reduction's limits");
            const bool ok = dq ? try_launch_reg<TopkSource::EncodeNF4DQ>(a, stream)
                               : try_launch_reg<TopkSource::EncodeNF4>(a, stream);
            BSQ_REQUIRE(ok, "top-k: fused encode pass not launched");
            break;
        }
    }
    BSQ_HIP(hipGetLastError());
    return gmax;
}

void launch_topk_scatter(const uint16_t *idx0, const float *val0, uint32_t k0, const uint16_t *idx1,
                         const float *val1, uint32_t k1, uint32_t rows, uint32_t cols, float *dense,
                         bool accumulate, hipStream_t stream, const uint32_t *gate0) {
    BSQ_REQUIRE(rows > 0 && cols > 0 && dense, "top-k scatter: bad arguments");
    if (!accumulate) BSQ_HIP(hipMemsetAsync(dense, 0, static_cast<size_t>(rows) * cols * sizeof(float), stream));
    if (k0 == 0 && k1 == 0) return;
    if (k0 == 0) {
        idx0 = idx1;
        val0 = val1;
        k0 = k1;
        k1 = 0;
        idx1 = nullptr;
        val1 = nullptr;
        gate0 = nullptr;
    }
    topk_scatter_kernel<<<rows, 256, 0, stream>>>(idx0, val0, k0, idx1, val1, k1, cols, dense, accumulate, gate0);
    BSQ_HIP(hipGetLastError());
}

void launch_topk_scatter_flat(const uint16_t *idx, const float *val, uint32_t k, uint32_t rows, uint32_t cols,
                              float *dense, hipStream_t stream) {
    BSQ_REQUIRE(rows > 0 && cols > 0 && dense, "top-k scatter: bad arguments");
    const uint64_t total = static_cast<uint64_t>(rows) * k;
    if (total == 0) return;
    BSQ_REQUIRE(idx && val, "top-k scatter: null list");
    topk_scatter_flat_kernel<<<static_cast<unsigned>(ceil_div(total, 256)), 256, 0, stream>>>(
        idx, val, k, total, cols, static_cast<uint64_t>(rows) * cols, dense);
    BSQ_HIP(hipGetLastError());
}

}  // namespace bsq
