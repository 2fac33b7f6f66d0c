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

#include <cfloat>

namespace bsq {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kCacheMaxCols = 16384;  // 64 KiB of LDS row cache

__device__ __forceinline__ uint32_t order_key(float v) {
    // |v| as an ordered integer, NaN below +0 (build_sort_inputs_kernel maps
    // NaN to -inf, topk_cuda_utils.cuh:62-66).
    return __builtin_isnan(v) ? 0u : (__float_as_uint(fabsf(v)) + 1u);
}

__device__ __forceinline__ float e4m3_decode(uint32_t v) {
    const uint32_t ef = (v >> 3) & 15u, mf = v & 7u;
    float r;
    if (ef == 0) r = (static_cast<float>(mf) / 8.0f) * 0.015625f;
    else r = (1.0f + static_cast<float>(mf) / 8.0f) * __builtin_ldexpf(1.0f, static_cast<int>(ef) - 7);
    return (v & 0x80u) ? -r : r;
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
    float L[16];
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
    if (threadIdx.x == 0) sh.ncand = 0;
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
    if constexpr (CACHED) {
        for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
            const float v = load_value<SRC>(a, sh.L, dq, row0 + c);
            cache[c] = v;
            nonzero |= fabsf(v) > FLT_EPSILON;
        }
    } else if (a.flags) {
        for (uint32_t c = threadIdx.x; c < cols; c += kThreads)
            nonzero |= fabsf(load_value<SRC>(a, sh.L, dq, row0 + c)) > FLT_EPSILON;
    }
    if (a.flags && __syncthreads_or(nonzero ? 1 : 0)) {
        if (threadIdx.x == 0) atomicOr(a.flags, kFlagError);
    }
    __syncthreads();

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
    uint16_t *out_idx = a.indices + static_cast<uint64_t>(r) * k;
    float *out_val = a.values + static_cast<uint64_t>(r) * k;
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

__global__ void topk_scatter_kernel(const uint16_t *__restrict__ idx0, const float *__restrict__ val0, uint32_t k0,
                                    const uint16_t *__restrict__ idx1, const float *__restrict__ val1, uint32_t k1,
                                    uint32_t cols, float *__restrict__ dense, bool accumulate,
                                    const uint32_t *__restrict__ gate0) {
    const uint64_t r = blockIdx.x;
    float *row = dense + r * cols;
    if (gate0 && !(*gate0 & kFlagError)) k0 = 0;
    for (uint32_t j = threadIdx.x; j < k0; j += blockDim.x) {
        const uint32_t c = idx0[r * k0 + j];
        if (c < cols) {
            if (accumulate) row[c] += val0[r * k0 + j];
            else row[c] = val0[r * k0 + j];
        }
    }
    if (k1 == 0) return;
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < k1; j += blockDim.x) {
        const uint32_t c = idx1[r * k1 + j];
        if (c < cols) row[c] += val1[r * k1 + j];
    }
}

template <TopkSource SRC>
void launch_src(const TopkArgs &a, hipStream_t stream) {
    uint32_t P = 1;
    while (P < a.k) P <<= 1;
    const bool cached = a.cols <= kCacheMaxCols;
    const size_t cache_bytes = cached ? ((a.cols * 4u + 15u) & ~15u) : 0u;
    const size_t lds = cache_bytes + static_cast<size_t>(P) * 8 + ((a.cols + 31) / 32) * 4;
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

void launch_topk_select(const TopkArgs &a, hipStream_t stream) {
    BSQ_REQUIRE(a.rows > 0 && a.cols > 0 && a.cols <= 65535 && a.rows <= 65535, "top-k: bad shape");
    BSQ_REQUIRE(a.k >= 1 && a.k <= a.cols, "top-k: k must be in [1, cols]");
    BSQ_REQUIRE(a.k <= kTopkMaxK, "top-k: k above the supported maximum (8192)");
    BSQ_REQUIRE(a.a && a.indices && a.values, "top-k: null pointer");
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
    }
    BSQ_HIP(hipGetLastError());
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
    topk_scatter_kernel<<<rows, 64, 0, stream>>>(idx0, val0, k0, idx1, val1, k1, cols, dense, accumulate, gate0);
    BSQ_HIP(hipGetLastError());
}

}  // namespace bsq
