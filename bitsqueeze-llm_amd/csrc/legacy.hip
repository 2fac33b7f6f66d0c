// The reference's legacy quantisation formats on gfx950.
//
// The reference implements these as OpenMP CPU codecs behind one dispatcher
// (legacy_modules/quantization/src/quantization.cpp:125-489): Q8_0, Q4_0,
// Q2_K, Q2_K_FAST, BF16, FP16, FP8, FP4, MXFP8, MXFP4, NVFP4, NF4, NF4_DQ.
// Here every format is a set of HBM-streaming kernels that write the
// format's serialised payload image (the format struct, then its arrays,
// byte-identical to the reference's apart from the pointer fields) straight
// into device memory, and decode from such an image:
//
//   * block formats (Q8_0, Q4_0, MXFP8, MXFP4): a lane owns 8 consecutive
//     elements, a 32-element block is an aligned quad of lanes, the block
//     absmax a 2-step xor shuffle;
//   * tensor-scale formats (FP8, FP4, NVFP4): a reduction pass of the finite
//     absmax (one atomic max per workgroup into a word of the image's pointer
//     field, which the host rewrites afterwards), then the encode pass; NVFP4
//     blocks of 16 are lane pairs;
//   * Q2_K / Q2_K_FAST: a lane owns one 16-element block, an aligned group of
//     16 lanes one 256-element super-block; the interleaved 2-bit code bytes
//     are OR-combined across the group by xor shuffles;
//   * BF16 / FP16: elementwise, 8 per lane;
//   * NF4 / NF4_DQ: the packed object's codec (quant.hip) on the legacy
//     layout.
//
// Every floating-point step is the reference's own, in its order, with the
// x86-64 semantics its build has (lrintf of NaN or of an out-of-range value
// is LONG_MIN; float to int8 goes through int32); this file is compiled with
// -ffp-contract=off.  The encode and decode results are bit-identical to the
// reference's single-threaded results (its FP4 encoder's element-parallel
// loop can race on a shared byte; this build writes each byte once).
#include "bsq_internal.hpp"
#include "scalar_codecs.hpp"

#include <bitsqz_llm_c.h>
#include <quantization.hpp>

#include <climits>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

namespace bsq {
namespace {

constexpr int kLT = 256;  // threads per workgroup

// ---------------------------------------------------------------------------
// payload layout (reference get_*_array_size, e.g. q8_0_impl.cpp:3-6)
// ---------------------------------------------------------------------------
struct Layout {
    uint64_t header = 0;        // format struct bytes
    uint64_t a_off = 0, a_len = 0;  // first array (scales / records / data)
    uint64_t b_off = 0, b_len = 0;  // second array (codes), if any
    uint64_t total = 0;
    uint64_t nb = 0, bs = 0;    // blocks, block size (0 where the struct has none)
    int scale_off = -1;         // f32 scale field of the struct, if any
    int scratch_off = -1;       // 8-byte pointer field used as reduction scratch
};

constexpr uint64_t kMaxElements = 1ull << 40;  // Q2_K counts super-blocks in 32 bits

bool method_known(int m) { return m >= Q8_0 && m <= Q2_K_FAST; }

Layout layout_of(int m, uint64_t n) {
    BSQ_REQUIRE(method_known(m), "legacy: unknown quantization method");
    BSQ_REQUIRE(n > 0 && n <= kMaxElements, "legacy: element count out of range");
    Layout L;
    const uint64_t half = (n + 1) / 2;
    auto blocks = [&](uint64_t bs) {
        L.bs = bs;
        L.nb = ceil_div(n, bs);
    };
    switch (m) {
        case Q8_0: blocks(32); L.header = 40; L.a_len = 4 * L.nb; L.b_len = n; break;
        case Q4_0: blocks(32); L.header = 40; L.a_len = 4 * L.nb; L.b_len = half; break;
        case MXFP8: blocks(32); L.header = 40; L.a_len = L.nb; L.b_len = n; break;
        case MXFP4: blocks(32); L.header = 40; L.a_len = L.nb; L.b_len = half; break;
        case NF4: blocks(64); L.header = 40; L.a_len = 4 * L.nb; L.b_len = half; break;
        case NVFP4: blocks(16); L.header = 48; L.a_len = L.nb; L.b_len = half; L.scale_off = 24; L.scratch_off = 32; break;
        case NF4_DQ: blocks(64); L.header = 48; L.a_len = L.nb; L.b_len = half; L.scale_off = 24; L.scratch_off = 32; break;
        case Q2_K:
        case Q2_K_FAST: L.header = 32; L.a_len = ceil_div(n, 256) * sizeof(super_block_q2_k); break;
        case BF16:
        case FP16: L.header = 16; L.a_len = 2 * n; break;
        case FP8: L.header = 24; L.a_len = n; L.scale_off = 8; L.scratch_off = 16; break;
        case FP4: L.header = 24; L.a_len = half; L.scale_off = 8; L.scratch_off = 16; break;
        default: fail("legacy: unknown quantization method");
    }
    L.a_off = L.header;
    L.b_off = L.a_off + L.a_len;
    L.total = L.b_off + L.b_len;
    return L;
}

// The format struct with zero pointers and zero scale (the scale fields are
// written by the encode kernels).
struct Header {
    uint32_t w[12];
};

Header header_of(int m, uint64_t n, const Layout &L) {
    Header h;
    std::memset(&h, 0, sizeof h);
    auto put64 = [&](int off, uint64_t v) { std::memcpy(reinterpret_cast<uint8_t *>(h.w) + off, &v, 8); };
    put64(0, n);
    if (m == Q2_K || m == Q2_K_FAST) {
        const uint64_t nsb = ceil_div(n, 256);
        put64(8, nsb * 256);
        const uint32_t c = static_cast<uint32_t>(nsb);
        std::memcpy(reinterpret_cast<uint8_t *>(h.w) + 16, &c, 4);
    } else if (L.bs) {
        put64(8, L.nb);
        put64(16, L.bs);
    }
    return h;
}

// ---------------------------------------------------------------------------
// scalar semantics
// ---------------------------------------------------------------------------

// lrintf as the x86-64 build computes it: round to nearest even; NaN and
// results outside the range of long give LONG_MIN.
__device__ __forceinline__ long long lrint_x86(float v) {
    const float r = __builtin_rintf(v);
    return (fabsf(r) < 9.223372036854775808e18f) ? static_cast<long long>(r) : LLONG_MIN;
}
// (int)lrintf(v): the low 32 bits of the long (0 for NaN and |v| >= 2^63).
// Branch-free: outside the int32 range r = m * 2^(e - 23) with e >= 31, whose
// low 32 bits are m << (e - 23) for e < 55 and 0 from there on.
__device__ __forceinline__ int lrint_int(float v) {
    const float r = __builtin_rintf(v);
    const uint32_t b = __float_as_uint(r);
    const int e = static_cast<int>((b >> 23) & 0xFFu) - 127;
    const uint32_t m = (b & 0x7FFFFFu) | 0x800000u;
    uint32_t lo = (e >= 31 && e < 55) ? (m << static_cast<uint32_t>(e - 23 < 0 ? 0 : e - 23)) : 0u;
    lo = (b >> 31) ? (0u - lo) : lo;
    return fabsf(r) < 2147483648.0f ? static_cast<int>(r) : static_cast<int>(lo);
}
// clamp(lrintf(v), -lim, lim) with the long result of the x86-64 build:
// NaN and |v| >= 2^63 give LONG_MIN, which clamps to -lim.
__device__ __forceinline__ int lrint_clamp(float v, float lim) {
    const float r = __builtin_rintf(v);
    if (!(fabsf(r) < 9.223372036854775808e18f)) return -static_cast<int>(lim);
    return static_cast<int>(r < -lim ? -lim : (r > lim ? lim : r));
}

// FP32 -> FP16, IEEE round to nearest even, NaN -> sign | 0x7E00
// (datatype/fp16/fp16.hpp:119-152 on an x86-64 build without F16C).
__device__ __forceinline__ uint32_t fp16_from_f32(float f) {
    const uint32_t u = __float_as_uint(f), sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u;
    if (a >= 0x477FF000u) return sign | 0x7C00u;
    if (a >= 0x38800000u) {
        const uint32_t m = a - 0x38000000u, keep = m >> 13, rem = m & 0x1FFFu;
        return sign | (keep + ((rem > 0x1000u || (rem == 0x1000u && (keep & 1u))) ? 1u : 0u));
    }
    if (a < 0x33000000u) return sign;
    const uint32_t shift = 126u - (a >> 23), mant = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t keep = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    return sign | (keep + ((rem > half || (rem == half && (keep & 1u))) ? 1u : 0u));
}

// FP16 -> FP32, exact; NaN payload moved up with the quiet bit set
// (fp16.hpp:73-95).
__device__ __forceinline__ float fp16_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1Fu) return __uint_as_float(sign | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0u));
    if (e != 0) return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
    return __uint_as_float(sign | __float_as_uint(static_cast<float>(m) * 0x1.0p-24f));
}

// FP32 -> BF16 (datatype/bf16.hpp:44-60).
__device__ __forceinline__ uint32_t bf16_from_f32(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0) return ((u >> 16) | 0x0040u) & 0xFFFFu;
    const uint32_t low = u & 0xFFFFu, odd = (u >> 16) & 1u;
    if (low > 0x8000u || (low == 0x8000u && odd)) u += 0x10000u;
    return u >> 16;
}

// E2M1 levels 0, 0.5, 1, 1.5, 2, 3, 4, 6 (fp4_impl.cpp:54-70).
__device__ __forceinline__ float e2m1_level(int i) {
    return i < 4 ? 0.5f * static_cast<float>(i) : (i < 6 ? static_cast<float>(i - 2) : (i == 6 ? 4.0f : 6.0f));
}

// E2M1 encode (fp4_impl.cpp:72-95): non-finite -> 6, nearest level by a
// linear scan with strict '<'.
__device__ __forceinline__ uint32_t e2m1_encode(float x) {
    const uint32_t sign = __builtin_signbit(x) ? 8u : 0u;
    float ax = fabsf(x);
    if (ax == 0.0f) return sign;
    if (!__builtin_isfinite(ax) || ax > 6.0f) ax = 6.0f;
    uint32_t best = 0;
    float be = fabsf(0.0f - ax);
#pragma unroll
    for (int i = 1; i < 8; ++i) {
        const float e = fabsf(e2m1_level(i) - ax);
        if (e < be) {
            be = e;
            best = static_cast<uint32_t>(i);
        }
    }
    return sign | best;
}

__device__ __forceinline__ float e2m1_decode(uint32_t c) {
    const float r = e2m1_level(static_cast<int>(c & 7u));
    return (c & 8u) ? -r : r;
}

// MX shared exponent (mxfp8_impl.cpp:121-127, mxfp4_impl.cpp:123-128):
// (int8)ceil(log2(absmax / max_norm)).  log2 of the FP32 quotient in FP64,
// rounded once to FP32: the ceiling matches the host's log2f on every
// positive float (checked exhaustively against the CPU checksum).
__device__ __forceinline__ int mx_scale_exp(float amax, float max_norm) {
    if (!(amax > 0.0f)) return 0;
    const float t = amax / max_norm;
    if (!(t > 0.0f)) return 0;
    const float l = static_cast<float>(log2(static_cast<double>(t)));
    return static_cast<int8_t>(static_cast<int32_t>(__builtin_ceilf(l)));
}

// ---------------------------------------------------------------------------
// memory helpers
// ---------------------------------------------------------------------------

// 8 consecutive inputs of chunk c (elements past n read 0).
__device__ __forceinline__ void load8(const float *__restrict__ x, uint64_t c, uint64_t n, bool vec, float v[8]) {
    const uint64_t e = 8 * c;
    if (vec && e + 8 <= n) {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(x + e), b = *reinterpret_cast<const f32x4 *>(x + e + 4);
        v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
        v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (e + i < n) ? x[e + i] : 0.0f;
    }
}

// 8 consecutive outputs of chunk c (elements past n not written).
__device__ __forceinline__ void store8(float *__restrict__ y, uint64_t c, uint64_t n, bool vec, const float v[8]) {
    const uint64_t e = 8 * c;
    if (vec && e + 8 <= n) {
        *reinterpret_cast<f32x4 *>(y + e) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4 *>(y + e + 4) = f32x4{v[4], v[5], v[6], v[7]};
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (e + i < n) y[e + i] = v[i];
    }
}

// `len` (<= 8) bytes b[0..len) to p: whole dwords when p is 4-byte aligned.
__device__ __forceinline__ void store_bytes(uint8_t *p, const uint32_t lo, const uint32_t hi, int len, bool al4) {
    if (al4 && len == 8) {
        reinterpret_cast<uint32_t *>(p)[0] = lo;
        reinterpret_cast<uint32_t *>(p)[1] = hi;
    } else if (al4 && len == 4) {
        *reinterpret_cast<uint32_t *>(p) = lo;
    } else {
        for (int i = 0; i < len; ++i) p[i] = static_cast<uint8_t>(((i < 4) ? lo >> (8 * i) : hi >> (8 * (i - 4))) & 0xFFu);
    }
}

__device__ __forceinline__ void load_bytes(const uint8_t *p, int len, bool al4, uint32_t &lo, uint32_t &hi) {
    if (al4 && len == 8) {
        lo = reinterpret_cast<const uint32_t *>(p)[0];
        hi = reinterpret_cast<const uint32_t *>(p)[1];
    } else if (al4 && len == 4) {
        lo = *reinterpret_cast<const uint32_t *>(p);
        hi = 0;
    } else {
        lo = hi = 0;
        for (int i = 0; i < len; ++i) {
            const uint32_t b = p[i];
            if (i < 4) lo |= b << (8 * i);
            else hi |= b << (8 * (i - 4));
        }
    }
}

// 8 byte codes (or 8 nibbles, element 2j in the high nibble) of one chunk.
template <bool NIBBLE>
__device__ __forceinline__ void pack_codes(const uint32_t q[8], uint32_t &lo, uint32_t &hi) {
    if constexpr (NIBBLE) {
        lo = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) lo |= (((q[2 * j] & 15u) << 4) | (q[2 * j + 1] & 15u)) << (8 * j);
        hi = 0;
    } else {
        lo = (q[0] & 255u) | ((q[1] & 255u) << 8) | ((q[2] & 255u) << 16) | ((q[3] & 255u) << 24);
        hi = (q[4] & 255u) | ((q[5] & 255u) << 8) | ((q[6] & 255u) << 16) | ((q[7] & 255u) << 24);
    }
}

template <bool NIBBLE>
__device__ __forceinline__ void unpack_codes(uint32_t lo, uint32_t hi, uint32_t q[8]) {
    if constexpr (NIBBLE) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t b = (lo >> (8 * j)) & 255u;
            q[2 * j] = b >> 4;
            q[2 * j + 1] = b & 15u;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            q[j] = (lo >> (8 * j)) & 255u;
            q[4 + j] = (hi >> (8 * j)) & 255u;
        }
    }
}

// Store the codes of chunk c (elements 8c .. 8c+7, those < n; the low nibble
// after an odd count's last element stays 0).
template <bool NIBBLE>
__device__ __forceinline__ void put_chunk_codes(uint8_t *codes, uint64_t c, uint64_t n, uint32_t q[8], bool al4) {
    const uint64_t e = 8 * c, valid = (n - e < 8) ? n - e : 8;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (static_cast<uint64_t>(i) >= valid) q[i] = 0;
    uint32_t lo, hi;
    pack_codes<NIBBLE>(q, lo, hi);
    const int len = NIBBLE ? static_cast<int>((valid + 1) / 2) : static_cast<int>(valid);
    store_bytes(codes + (NIBBLE ? 4 * c : 8 * c), lo, hi, len, al4);
}

template <bool NIBBLE>
__device__ __forceinline__ void get_chunk_codes(const uint8_t *codes, uint64_t c, uint64_t n, uint32_t q[8], bool al4) {
    const uint64_t e = 8 * c, valid = (n - e < 8) ? n - e : 8;
    const int len = NIBBLE ? static_cast<int>((valid + 1) / 2) : static_cast<int>(valid);
    uint32_t lo, hi;
    load_bytes(codes + (NIBBLE ? 4 * c : 8 * c), len, al4, lo, hi);
    unpack_codes<NIBBLE>(lo, hi, q);
}

__device__ __forceinline__ float max_if_greater(float a, float o) { return o > a ? o : a; }

__device__ __forceinline__ uint64_t gtid() { return static_cast<uint64_t>(blockIdx.x) * kLT + threadIdx.x; }
__device__ __forceinline__ uint64_t gstride() { return static_cast<uint64_t>(gridDim.x) * kLT; }

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------

__global__ void header_kernel(uint8_t *__restrict__ img, Header h, int words) {
    if (threadIdx.x < static_cast<unsigned>(words)) reinterpret_cast<uint32_t *>(img)[threadIdx.x] = h.w[threadIdx.x];
}

// Block-of-32 formats.  A quad of lanes is one block; the loop runs over
// whole quads so that every shuffle partner is active.
// Workgroup 0 writes the format struct (`hw` words of `h`) to `img`.
__device__ __forceinline__ void write_header(uint8_t *img, const Header &h, int hw) {
    if (blockIdx.x == 0 && threadIdx.x < static_cast<unsigned>(hw)) reinterpret_cast<uint32_t *>(img)[threadIdx.x] = h.w[threadIdx.x];
}

template <int M>
__global__ __launch_bounds__(kLT) void blk32_encode_kernel(const float *__restrict__ x, uint64_t n, bool vec,
                                                           uint8_t *__restrict__ scales, uint8_t *__restrict__ codes,
                                                           bool al4, uint8_t *__restrict__ img, Header h, int hw) {
    constexpr bool kNib = (M == Q4_0 || M == MXFP4);
    write_header(img, h, hw);
    const uint64_t chunks = ceil_div(n, 8), nb = ceil_div(n, 32), span = (chunks + 3) & ~3ull;
    for (uint64_t c = gtid(); c < span; c += gstride()) {
        float v[8];
        load8(x, c, n, vec, v);
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float f = v[i];
            if constexpr (M == MXFP8 || M == MXFP4) f = __builtin_isfinite(f) ? f : 0.0f;
            f = fabsf(f);
            if (f > a) a = f;
        }
        a = max_if_greater(a, __shfl_xor(a, 1));
        a = max_if_greater(a, __shfl_xor(a, 2));
        const uint64_t b = c >> 2;
        const bool writer = (c & 3) == 0 && b < nb;
        uint32_t q[8];
        if constexpr (M == Q8_0 || M == Q4_0) {
            // q8_0_impl.cpp:80-93, q4_0_impl.cpp:84-107
            constexpr float kDiv = (M == Q8_0) ? 127.0f : 7.0f;
            constexpr float kLim = (M == Q8_0) ? 127.0f : 7.0f;
            const float scale = (a > 0.0f) ? (a / kDiv) : 0.0f;
            const float inv = (scale > 0.0f) ? (1.0f / scale) : 0.0f;
            if (writer) reinterpret_cast<float *>(scales)[b] = scale;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                q[i] = static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(lrint_clamp(v[i] * inv, kLim))));
            }
        } else if constexpr (M == MXFP8) {
            // mxfp8_impl.cpp:144-157: elements divided by 2^e
            const int e = mx_scale_exp(a, 448.0f);
            if (writer) scales[b] = static_cast<uint8_t>(static_cast<int8_t>(e));
            const float scale = __builtin_ldexpf(1.0f, e);
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = e4m3_encode(v[i] / scale);
        } else {
            // mxfp4_impl.cpp:155-167: elements times 2^-e
            const int e = mx_scale_exp(a, 6.0f);
            if (writer) scales[b] = static_cast<uint8_t>(static_cast<int8_t>(e));
            const float inv = __builtin_ldexpf(1.0f, -e);
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = e2m1_encode(v[i] * inv);
        }
        if (c < chunks) put_chunk_codes<kNib>(codes, c, n, q, al4);
    }
}

template <int M>
__global__ __launch_bounds__(kLT) void blk32_decode_kernel(const uint8_t *__restrict__ scales,
                                                           const uint8_t *__restrict__ codes, uint64_t n, bool al4,
                                                           float *__restrict__ y, bool vec) {
    constexpr bool kNib = (M == Q4_0 || M == MXFP4);
    const uint64_t chunks = ceil_div(n, 8);
    for (uint64_t c = gtid(); c < chunks; c += gstride()) {
        const uint64_t b = c >> 2;
        uint32_t q[8];
        get_chunk_codes<kNib>(codes, c, n, q, al4);
        float v[8];
        if constexpr (M == Q8_0 || M == Q4_0) {
            const float s = reinterpret_cast<const float *>(scales)[b];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int iv = (M == Q8_0) ? static_cast<int>(static_cast<int8_t>(q[i]))
                                           : (static_cast<int>(static_cast<int8_t>(static_cast<uint8_t>(q[i] << 4))) >> 4);
                v[i] = s * static_cast<float>(iv);
            }
        } else {
            const float s = __builtin_ldexpf(1.0f, static_cast<int>(static_cast<int8_t>(scales[b])));
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = s * ((M == MXFP8) ? e4m3_decode(q[i]) : e2m1_decode(q[i]));
        }
        store8(y, c, n, vec, v);
    }
}

// Largest finite |x| (fp8_impl.cpp:103-114): one atomic max per workgroup on
// the bit pattern (non-negative floats order as their bits).  Launched with
// at most one workgroup per CU (device-scope atomics on one word serialise
// across the XCDs); each lane keeps 4 chunk loads in flight.
__global__ __launch_bounds__(kLT) void finite_absmax_kernel(const float *__restrict__ x, uint64_t n, bool vec,
                                                            uint32_t *__restrict__ word) {
    __shared__ float red[kLT / 64];
    constexpr int kU = 4;
    const uint64_t chunks = ceil_div(n, 8), stride = gstride();
    float a = 0.0f;
    for (uint64_t c0 = gtid(); c0 < chunks; c0 += kU * stride) {
        float v[kU][8];
#pragma unroll
        for (int u = 0; u < kU; ++u) load8(x, c0 + u * stride, n, vec, v[u]);
#pragma unroll
        for (int u = 0; u < kU; ++u)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float f = __builtin_isfinite(v[u][i]) ? fabsf(v[u][i]) : 0.0f;
                if (f > a) a = f;
            }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) a = max_if_greater(a, __shfl_xor(a, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = red[0];
        for (int w = 1; w < kLT / 64; ++w) m = max_if_greater(m, red[w]);
        if (m > 0.0f) atomicMax(word, __float_as_uint(m));
    }
}

// FP8 (fp8_impl.cpp:116-131) and FP4 (fp4_impl.cpp:127-153).
template <bool FP4>
__global__ __launch_bounds__(kLT) void gscale_encode_kernel(const float *__restrict__ x, uint64_t n, bool vec,
                                                            const uint32_t *__restrict__ word,
                                                            float *__restrict__ scale_field,
                                                            uint8_t *__restrict__ codes, bool al4) {
    const float amax = __uint_as_float(*word);
    float scale = (amax == 0.0f) ? 1.0f : amax / (FP4 ? 6.0f : 448.0f);
    if (scale == 0.0f) scale = 1.0f;
    const float inv = 1.0f / scale;
    if (gtid() == 0) *scale_field = scale;
    const uint64_t chunks = ceil_div(n, 8);
    for (uint64_t c = gtid(); c < chunks; c += gstride()) {
        float v[8];
        load8(x, c, n, vec, v);
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = FP4 ? e2m1_encode(v[i] * inv) : e4m3_encode(v[i] * inv);
        put_chunk_codes<FP4>(codes, c, n, q, al4);
    }
}

template <bool FP4>
__global__ __launch_bounds__(kLT) void gscale_decode_kernel(const float *__restrict__ scale_field,
                                                            const uint8_t *__restrict__ codes, uint64_t n, bool al4,
                                                            float *__restrict__ y, bool vec) {
    const float s = *scale_field;
    const uint64_t chunks = ceil_div(n, 8);
    for (uint64_t c = gtid(); c < chunks; c += gstride()) {
        uint32_t q[8];
        get_chunk_codes<FP4>(codes, c, n, q, al4);
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = s * (FP4 ? e2m1_decode(q[i]) : e4m3_decode(q[i]));
        store8(y, c, n, vec, v);
    }
}

// NVFP4 (nvfp4_impl.cpp:174-238): a lane pair is one block of 16.
__global__ __launch_bounds__(kLT) void nvfp4_encode_kernel(const float *__restrict__ x, uint64_t n, bool vec,
                                                           const uint32_t *__restrict__ word,
                                                           float *__restrict__ ts_field,
                                                           uint8_t *__restrict__ bscales,
                                                           uint8_t *__restrict__ codes, bool al4) {
    const float amax = __uint_as_float(*word);
    const float ts = (amax == 0.0f) ? 1.0f : amax / 6.0f;
    const float inv_ts = 1.0f / ts;
    if (gtid() == 0) *ts_field = ts;
    const uint64_t chunks = ceil_div(n, 8), nb = ceil_div(n, 16), span = (chunks + 1) & ~1ull;
    for (uint64_t c = gtid(); c < span; c += gstride()) {
        float v[8];
        load8(x, c, n, vec, v);
        float bm = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float t = v[i] / ts;
            if (!__builtin_isfinite(t)) t = 0.0f;
            t = fabsf(t);
            if (t > bm) bm = t;
        }
        bm = max_if_greater(bm, __shfl_xor(bm, 1));
        const float target = bm / 6.0f;
        const uint32_t code = e4m3_encode((target > 0.0f) ? target : 1.0f);
        const uint64_t b = c >> 1;
        if ((c & 1) == 0 && b < nb) bscales[b] = static_cast<uint8_t>(code);
        const float inv_bs = 1.0f / e4m3_decode(code);
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = e2m1_encode(v[i] * inv_ts * inv_bs);
        if (c < chunks) put_chunk_codes<true>(codes, c, n, q, al4);
    }
}

__global__ __launch_bounds__(kLT) void nvfp4_decode_kernel(const float *__restrict__ ts_field,
                                                           const uint8_t *__restrict__ bscales,
                                                           const uint8_t *__restrict__ codes, uint64_t n, bool al4,
                                                           float *__restrict__ y, bool vec) {
    const float ts = *ts_field;
    const uint64_t chunks = ceil_div(n, 8);
    for (uint64_t c = gtid(); c < chunks; c += gstride()) {
        const float s = ts * e4m3_decode(bscales[c >> 1]);
        uint32_t q[8];
        get_chunk_codes<true>(codes, c, n, q, al4);
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = s * e2m1_decode(q[i]);
        store8(y, c, n, vec, v);
    }
}

// clamp((int)lrintf(v), 0, 3).  With `small` (every |v| below 2^30, a bound
// the caller proves for the whole block) the int32 conversion is exact and
// NaN converts to 0 as on the host; otherwise the exact low-word rule.
__device__ __forceinline__ int code2(float v, bool small) {
    const int l = small ? static_cast<int>(__builtin_rintf(v)) : lrint_int(v);
    return l < 0 ? 0 : (l > 3 ? 3 : l);
}

// Weighted least-squares block fit of Q2_K (q2_k_impl.cpp:59-140).
__device__ __forceinline__ void q2k_fit(const float w[16], float &scale_out, float &min_out) {
    float mn = w[0], mx = w[0], sw = fabsf(w[0]), sx = sw * w[0];
    float lo = w[0];  // the block's own minimum (mn is clipped at 0 below and later replaced)
#pragma unroll
    for (int i = 1; i < 16; ++i) {
        const float aw = fabsf(w[i]);
        if (w[i] < mn) mn = w[i];
        if (w[i] > mx) mx = w[i];
        if (w[i] < lo) lo = w[i];
        sw += aw;
        sx += aw * w[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
        scale_out = 0.0f;
        min_out = mn;
        return;
    }
    float iscale = 3.0f / (mx - mn);
    float best_scale = 1.0f / iscale, best_err = 0.0f;
    // every non-NaN w lies in [lo, mx], so |iscale (w - mn)| <= |iscale| dev
    auto small_for = [&](float isc) {
        const float dev = fmaxf(fabsf(mx - mn), fabsf(lo - mn));
        return fabsf(isc) * dev < 1073741824.0f;
    };
    bool small = small_for(iscale);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int l = code2(iscale * (w[i] - mn), small);
        best_err += fabsf(w[i]) * fabsf(best_scale * static_cast<float>(l) + mn - w[i]);
    }
#pragma unroll 1
    for (int is = 0; is <= 15; ++is) {
        iscale = (-0.5f + 0.1f * static_cast<float>(is) + 3.0f) / (mx - mn);
        small = small_for(iscale);
        float sl = 0, sl2 = 0, sxl = 0;
        uint32_t la = 0;  // 16 two-bit codes
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int l = code2(iscale * (w[i] - mn), small);
            la |= static_cast<uint32_t>(l) << (2 * i);
            const float aw = fabsf(w[i]), fl = static_cast<float>(l);
            sl += aw * fl;
            sl2 += aw * fl * fl;
            sxl += aw * fl * w[i];
        }
        const float D = sw * sl2 - sl * sl;
        if (D > 0) {
            float ts = (sw * sxl - sx * sl) / D;
            float tm = (sl2 * sx - sl * sxl) / D;
            if (tm > 0) {
                tm = 0;
                ts = sxl / sl2;
            }
            float err = 0;
#pragma unroll
            for (int i = 0; i < 16; ++i)
                err += fabsf(w[i]) * fabsf(ts * static_cast<float>((la >> (2 * i)) & 3u) + tm - w[i]);
            if (err < best_err) {
                best_err = err;
                best_scale = ts;
                mn = tm;
            }
        }
    }
    scale_out = best_scale;
    min_out = mn;
}

// Range fit of Q2_K_FAST (q2_k_fast_impl.cpp:6-22).
__device__ __forceinline__ void q2k_fit_fast(const float w[16], float &scale_out, float &min_out) {
    float mn = INFINITY, mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (w[i] < mn) mn = w[i];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float s = w[i] - mn;
        if (s > mx) mx = s;
    }
    scale_out = mx / 3.0f;
    min_out = mn;
}

// Q2_K / Q2_K_FAST encode (q2_k_impl.cpp:142-236, q2_k_fast_impl.cpp:24-125).
// Lane j of an aligned 16-lane group owns block j of super-block s.  Record:
// dword 0 = super_scale | super_min << 16, bytes 4..19 block scale / min
// nibbles, bytes 20..83 the codes; code byte (h, l) holds elements l, l + 32,
// l + 64, l + 96 of half h, so lane j's 16 codes land at bytes
// 20 + 32 (j / 8) + 16 (j % 2) + i with shift 2 ((j % 8) / 2).
template <bool FAST>
__global__ __launch_bounds__(kLT) void q2k_encode_kernel(const float *__restrict__ x, uint64_t n, bool vec,
                                                         uint8_t *__restrict__ rec, uint8_t *__restrict__ img,
                                                         Header h, int hw) {
    write_header(img, h, hw);
    const uint64_t nsb = ceil_div(n, 256);
    const int j = static_cast<int>(threadIdx.x & 15);
    for (uint64_t t = gtid(); t < nsb * 16; t += gstride()) {
        const uint64_t s = t >> 4, e0 = 256 * s + 16 * static_cast<uint64_t>(j);
        float w[16];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float v[8];
            load8(x, e0 / 8 + h, n, vec, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) w[8 * h + i] = v[i];
        }
        float sc, mnv;
        if constexpr (FAST) q2k_fit_fast(w, sc, mnv);
        else q2k_fit(w, sc, mnv);
        // max over the group: max_scale (from -inf, NaN skipped) and max |min|
        float ms = (sc > -INFINITY) ? sc : -INFINITY, mm = (fabsf(mnv) > 0.0f) ? fabsf(mnv) : 0.0f;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            ms = max_if_greater(ms, __shfl_xor(ms, off));
            mm = max_if_greater(mm, __shfl_xor(mm, off));
        }
        uint32_t bsc = 0, ss, sm;
        if (ms > 0) {
            const float is = 15.0f / ms;
            bsc = static_cast<uint32_t>(lrint_int(is * sc)) & 0xFFu;
            ss = fp16_from_f32(ms / 15.0f);
        } else {
            ss = fp16_from_f32(0.0f);
        }
        if (mm > 0) {
            const float is = 7.0f / mm;
            int l = lrint_int(is * mnv);
            l = l < -8 ? -8 : (l > 7 ? 7 : l);
            bsc = (bsc | ((static_cast<uint32_t>(l) & 0xFu) << 4)) & 0xFFu;
            sm = fp16_from_f32(mm / 7.0f);
        } else {
            sm = fp16_from_f32(0.0f);
        }
        // codes of this block against the stored (FP16) super scales
        const float tsc = fp16_to_f32(ss) * static_cast<float>(bsc & 0xFu);
        const int mq = static_cast<int>(static_cast<int8_t>(static_cast<uint8_t>((bsc >> 4) << 4))) >> 4;
        const float tmn = fp16_to_f32(sm) * static_cast<float>(mq);
        const uint32_t shift = 2u * static_cast<uint32_t>((j & 7) >> 1);
        uint32_t cw[4] = {0u, 0u, 0u, 0u};
        // |(w - tmn) / tsc| <= dev / tsc for every non-NaN w of the block
        float blo = w[0], bhi = w[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) {
            blo = w[i] < blo ? w[i] : blo;
            bhi = w[i] > bhi ? w[i] : bhi;
        }
        const bool small = !(tsc > 0.0f) || fmaxf(fabsf(bhi - tmn), fabsf(blo - tmn)) < 1073741824.0f * tsc;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float v = (tsc > 0.0f) ? (w[i] - tmn) / tsc : 0.0f;
            const int l = code2(v, small);
            cw[i >> 2] |= (static_cast<uint32_t>(l) << shift) << (8 * (i & 3));
        }
        // OR the four contributions (lanes j, j ^ 2, j ^ 4, j ^ 6 share bytes)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            cw[k] |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(cw[k]), 2));
            cw[k] |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(cw[k]), 4));
        }
        uint8_t *r = rec + s * sizeof(super_block_q2_k);
        // lane j writes dword (j / 2) % 4 of its 16-byte run
        const int kk = (j >> 1) & 3;
        const uint32_t mine = kk == 0 ? cw[0] : (kk == 1 ? cw[1] : (kk == 2 ? cw[2] : cw[3]));
        reinterpret_cast<uint32_t *>(r + 20 + 32 * (j >> 3) + 16 * (j & 1))[kk] = mine;
        // block bytes: lanes 4a .. 4a + 3 form dword a of bytes 4..19
        uint32_t bw = bsc << (8 * (j & 3));
        bw |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(bw), 1));
        bw |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(bw), 2));
        if ((j & 3) == 0) reinterpret_cast<uint32_t *>(r + 4)[j >> 2] = bw;
        if (j == 0) reinterpret_cast<uint32_t *>(r)[0] = ss | (sm << 16);
    }
}

// Q2_K decode (q2_k_impl.cpp:348-422): min_j + scale_j * code.
__global__ __launch_bounds__(kLT) void q2k_decode_kernel(const uint8_t *__restrict__ rec, uint64_t n,
                                                         float *__restrict__ y, bool vec) {
    const uint64_t nsb = ceil_div(n, 256);
    for (uint64_t t = gtid(); t < nsb * 16; t += gstride()) {
        const uint64_t s = t >> 4;
        const int j = static_cast<int>(t & 15);
        const uint8_t *r = rec + s * sizeof(super_block_q2_k);
        const uint32_t d0 = *reinterpret_cast<const uint32_t *>(r);
        const uint32_t bsc = r[4 + j];
        const float sc = fp16_to_f32(d0 & 0xFFFFu) * static_cast<float>(bsc & 0xFu);
        const int mq = static_cast<int>(static_cast<int8_t>(static_cast<uint8_t>((bsc >> 4) << 4))) >> 4;
        const float mnv = fp16_to_f32(d0 >> 16) * static_cast<float>(mq);
        const uint32_t *cp = reinterpret_cast<const uint32_t *>(r + 20 + 32 * (j >> 3) + 16 * (j & 1));
        const uint32_t shift = 2u * static_cast<uint32_t>((j & 7) >> 1);
        float v[16];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t word = cp[k];
#pragma unroll
            for (int b = 0; b < 4; ++b)
                v[4 * k + b] = mnv + sc * static_cast<float>(((word >> (8 * b)) >> shift) & 3u);
        }
        const uint64_t c0 = (256 * s + 16 * static_cast<uint64_t>(j)) / 8;
        store8(y, c0, n, vec, v);
        store8(y, c0 + 1, n, vec, v + 8);
    }
}

template <bool FP16>
__global__ __launch_bounds__(kLT) void half_encode_kernel(const float *__restrict__ x, uint64_t n, bool vec,
                                                          uint16_t *__restrict__ q, uint8_t *__restrict__ img,
                                                          Header h, int hw) {
    write_header(img, h, hw);
    const uint64_t chunks = ceil_div(n, 8);
    for (uint64_t c = gtid(); c < chunks; c += gstride()) {
        float v[8];
        load8(x, c, n, vec, v);
        uint32_t h[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = FP16 ? fp16_from_f32(v[i]) : bf16_from_f32(v[i]);
        const uint64_t e = 8 * c;
        if (e + 8 <= n) {  // q is 16-byte aligned (payload + 16)
            uint4 o;
            o.x = h[0] | (h[1] << 16); o.y = h[2] | (h[3] << 16);
            o.z = h[4] | (h[5] << 16); o.w = h[6] | (h[7] << 16);
            *reinterpret_cast<uint4 *>(q + e) = o;
        } else {
            for (int i = 0; i < 8; ++i)
                if (e + i < n) q[e + i] = static_cast<uint16_t>(h[i]);
        }
    }
}

template <bool FP16>
__global__ __launch_bounds__(kLT) void half_decode_kernel(const uint16_t *__restrict__ q, uint64_t n,
                                                          float *__restrict__ y, bool vec) {
    const uint64_t chunks = ceil_div(n, 8);
    for (uint64_t c = gtid(); c < chunks; c += gstride()) {
        const uint64_t e = 8 * c;
        uint32_t h[8];
        if (e + 8 <= n) {
            const uint4 w = *reinterpret_cast<const uint4 *>(q + e);
            h[0] = w.x & 0xFFFFu; h[1] = w.x >> 16; h[2] = w.y & 0xFFFFu; h[3] = w.y >> 16;
            h[4] = w.z & 0xFFFFu; h[5] = w.z >> 16; h[6] = w.w & 0xFFFFu; h[7] = w.w >> 16;
        } else {
            for (int i = 0; i < 8; ++i) h[i] = (e + i < n) ? q[e + i] : 0u;
        }
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = FP16 ? fp16_to_f32(h[i]) : __uint_as_float(h[i] << 16);
        store8(y, c, n, vec, v);
    }
}

// Checksums over every float pattern in [lo, hi) of the device FP16 (0) and
// BF16 (1) conversions and MX exponents (2: max 448, 3: max 6).
__global__ __launch_bounds__(kLT) void legacy_sweep_kernel(int kind, uint64_t lo, uint64_t hi,
                                                           unsigned long long *__restrict__ out) {
    unsigned long long acc = 0;
    for (uint64_t p = lo + gtid(); p < hi; p += gstride()) {
        const float f = __uint_as_float(static_cast<uint32_t>(p));
        uint32_t r;
        if (kind == 0) r = fp16_from_f32(f);
        else if (kind == 1) r = bf16_from_f32(f);
        else r = static_cast<uint8_t>(static_cast<int8_t>(mx_scale_exp(f, kind == 2 ? 448.0f : 6.0f)));
        acc += (static_cast<unsigned long long>(r) + 1ull) * (p % 65521ull);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
    if ((threadIdx.x & 63) == 0) atomicAdd(out, acc);
}

unsigned grid_for_items(uint64_t items, uint64_t per_cu = 16) {
    const uint64_t want = ceil_div(items, kLT), cap = static_cast<uint64_t>(cu_count()) * per_cu;
    return static_cast<unsigned>(want < 1 ? 1 : (want < cap ? want : cap));
}

bool al(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

uint64_t legacy_payload_bytes(int method, uint64_t n) { return layout_of(method, n).total; }

// Writes the payload image of `x` (n floats, device) to `img` (device,
// 16-byte aligned, legacy_payload_bytes(method, n) bytes).  The image's
// pointer fields are left unspecified (the tensor-scale formats use one as
// reduction scratch).
void launch_legacy_encode(int method, const float *x, uint64_t n, uint8_t *img, hipStream_t st) {
    const Layout L = layout_of(method, n);
    BSQ_REQUIRE(x && img && al(img, 16), "legacy encode: null or misaligned buffer");
    const bool vec = al(x, 16);
    uint8_t *a = img + L.a_off, *b = img + L.b_off;
    const bool al4 = al(method == Q2_K || method == Q2_K_FAST || method == BF16 || method == FP16 ||
                                method == FP8 || method == FP4 ? a : b, 4);
    const Header h = header_of(method, n, L);
    const int hw = static_cast<int>(L.header / 4);
    // formats with a reduction pass (or the packed object's codec) write the
    // struct first: it also zeroes the scratch word
    const bool separate_header = method == FP8 || method == FP4 || method == NVFP4 || method == NF4 || method == NF4_DQ;
    if (separate_header) {
        header_kernel<<<1, 64, 0, st>>>(img, h, hw);
        BSQ_HIP(hipGetLastError());
    }
    const unsigned g8 = grid_for_items(ceil_div(n, 8) + 3), g1 = grid_for_items(ceil_div(n, 8), 1);
    uint32_t *word = L.scratch_off >= 0 ? reinterpret_cast<uint32_t *>(img + L.scratch_off) : nullptr;
    switch (method) {
        case Q8_0: blk32_encode_kernel<Q8_0><<<g8, kLT, 0, st>>>(x, n, vec, a, b, al4, img, h, hw); break;
        case Q4_0: blk32_encode_kernel<Q4_0><<<g8, kLT, 0, st>>>(x, n, vec, a, b, al4, img, h, hw); break;
        case MXFP8: blk32_encode_kernel<MXFP8><<<g8, kLT, 0, st>>>(x, n, vec, a, b, al4, img, h, hw); break;
        case MXFP4: blk32_encode_kernel<MXFP4><<<g8, kLT, 0, st>>>(x, n, vec, a, b, al4, img, h, hw); break;
        case FP8:
        case FP4:
            finite_absmax_kernel<<<g1, kLT, 0, st>>>(x, n, vec, word);
            BSQ_HIP(hipGetLastError());
            if (method == FP8)
                gscale_encode_kernel<false><<<g8, kLT, 0, st>>>(x, n, vec, word,
                                                                reinterpret_cast<float *>(img + L.scale_off), a, al4);
            else
                gscale_encode_kernel<true><<<g8, kLT, 0, st>>>(x, n, vec, word,
                                                               reinterpret_cast<float *>(img + L.scale_off), a, al4);
            break;
        case NVFP4:
            finite_absmax_kernel<<<g1, kLT, 0, st>>>(x, n, vec, word);
            BSQ_HIP(hipGetLastError());
            nvfp4_encode_kernel<<<g8, kLT, 0, st>>>(x, n, vec, word, reinterpret_cast<float *>(img + L.scale_off), a, b,
                                                    al(b, 4));
            break;
        case Q2_K:
        case Q2_K_FAST: {
            const unsigned g = grid_for_items(ceil_div(n, 256) * 16);
            if (method == Q2_K) q2k_encode_kernel<false><<<g, kLT, 0, st>>>(x, n, vec, a, img, h, hw);
            else q2k_encode_kernel<true><<<g, kLT, 0, st>>>(x, n, vec, a, img, h, hw);
            break;
        }
        case BF16:
            half_encode_kernel<false><<<g8, kLT, 0, st>>>(x, n, vec, reinterpret_cast<uint16_t *>(a), img, h, hw);
            break;
        case FP16:
            half_encode_kernel<true><<<g8, kLT, 0, st>>>(x, n, vec, reinterpret_cast<uint16_t *>(a), img, h, hw);
            break;
        case NF4:
            launch_quant_encode(x, n, kMethodNF4, reinterpret_cast<float *>(a), nullptr, nullptr, b, nullptr, st);
            break;
        case NF4_DQ:
            launch_quant_encode(x, n, kMethodNF4DQ, nullptr, a, reinterpret_cast<float *>(img + L.scale_off), b, word,
                                st);
            break;
        default: fail("legacy encode: unknown method");
    }
    BSQ_HIP(hipGetLastError());
}

// Decodes the payload image `img` (device, 16-byte aligned) of n elements to
// `y` (device).
void launch_legacy_decode(int method, const uint8_t *img, uint64_t n, float *y, hipStream_t st) {
    const Layout L = layout_of(method, n);
    BSQ_REQUIRE(y && img && al(img, 16), "legacy decode: null or misaligned buffer");
    const bool vec = al(y, 16);
    const uint8_t *a = img + L.a_off, *b = img + L.b_off;
    const bool al4 = al(method == FP8 || method == FP4 ? a : b, 4);
    const unsigned g8 = grid_for_items(ceil_div(n, 8));
    const float *sf = L.scale_off >= 0 ? reinterpret_cast<const float *>(img + L.scale_off) : nullptr;
    switch (method) {
        case Q8_0: blk32_decode_kernel<Q8_0><<<g8, kLT, 0, st>>>(a, b, n, al4, y, vec); break;
        case Q4_0: blk32_decode_kernel<Q4_0><<<g8, kLT, 0, st>>>(a, b, n, al4, y, vec); break;
        case MXFP8: blk32_decode_kernel<MXFP8><<<g8, kLT, 0, st>>>(a, b, n, al4, y, vec); break;
        case MXFP4: blk32_decode_kernel<MXFP4><<<g8, kLT, 0, st>>>(a, b, n, al4, y, vec); break;
        case FP8: gscale_decode_kernel<false><<<g8, kLT, 0, st>>>(sf, a, n, al4, y, vec); break;
        case FP4: gscale_decode_kernel<true><<<g8, kLT, 0, st>>>(sf, a, n, al4, y, vec); break;
        case NVFP4: nvfp4_decode_kernel<<<g8, kLT, 0, st>>>(sf, a, b, n, al4, y, vec); break;
        case Q2_K:
        case Q2_K_FAST: q2k_decode_kernel<<<grid_for_items(ceil_div(n, 256) * 16), kLT, 0, st>>>(a, n, y, vec); break;
        case BF16: half_decode_kernel<false><<<g8, kLT, 0, st>>>(reinterpret_cast<const uint16_t *>(a), n, y, vec); break;
        case FP16: half_decode_kernel<true><<<g8, kLT, 0, st>>>(reinterpret_cast<const uint16_t *>(a), n, y, vec); break;
        case NF4:
            launch_quant_decode(n, kMethodNF4, reinterpret_cast<const float *>(a), nullptr, nullptr, b, y, st);
            break;
        case NF4_DQ: launch_quant_decode(n, kMethodNF4DQ, nullptr, a, sf, b, y, st); break;
        default: fail("legacy decode: unknown method");
    }
    BSQ_HIP(hipGetLastError());
}

void launch_legacy_sweep(int kind, uint64_t lo, uint64_t hi, unsigned long long *out, hipStream_t st) {
    BSQ_REQUIRE(kind >= 0 && kind <= 3 && lo <= hi && hi <= (1ull << 32), "legacy sweep: bad arguments");
    legacy_sweep_kernel<<<static_cast<unsigned>(cu_count()) * 8, kLT, 0, st>>>(kind, lo, hi, out);
    BSQ_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// host dispatcher (reference quantization.cpp:125-489)
// ---------------------------------------------------------------------------
namespace {

// Device staging per GPU, grown on demand and kept until the process ends.
struct Staging {
    int device = -1;
    hipStream_t stream = nullptr;
    void *buf = nullptr;
    uint64_t cap = 0;
};
std::mutex g_mu;
std::vector<Staging> g_staging;

Staging &staging_for_current(uint64_t need) {
    int dev = 0;
    BSQ_HIP(hipGetDevice(&dev));
    Staging *s = nullptr;
    for (auto &e : g_staging)
        if (e.device == dev) s = &e;
    if (!s) {
        g_staging.push_back(Staging{});
        s = &g_staging.back();
        s->device = dev;
        BSQ_HIP(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    }
    if (s->cap < need) {
        if (s->buf) BSQ_HIP(hipFree(s->buf));
        s->buf = nullptr;
        s->cap = 0;
        BSQ_HIP(hipMalloc(&s->buf, need));
        s->cap = need;
    }
    return *s;
}

uint64_t round256(uint64_t v) { return (v + 255) & ~255ull; }

// Payload size the format struct at `p` implies, or 0 for an unknown method
// or sizes that wrap (the reference's get_*_array_size functions).
uint64_t implied_payload(int method, const uint8_t *p) {
    uint64_t n, nb;
    std::memcpy(&n, p, 8);
    auto mul_ok = [](uint64_t a, uint64_t b, uint64_t &r) { return !__builtin_mul_overflow(a, b, &r); };
    auto add_ok = [](uint64_t a, uint64_t b, uint64_t &r) { return !__builtin_add_overflow(a, b, &r); };
    uint64_t t1 = 0, t2 = 0, r = 0;
    const uint64_t half = n / 2 + (n & 1);
    switch (method) {
        case Q8_0:
        case Q4_0:
        case NF4:
            std::memcpy(&nb, p + 8, 8);
            if (!mul_ok(nb, 4, t1)) return 0;
            t2 = method == Q8_0 ? n : half;
            if (!add_ok(t1, t2, r) || !add_ok(r, 40, r)) return 0;
            return r;
        case MXFP8:
        case MXFP4:
            std::memcpy(&nb, p + 8, 8);
            t2 = method == MXFP8 ? n : half;
            if (!add_ok(nb, t2, r) || !add_ok(r, 40, r)) return 0;
            return r;
        case NVFP4:
        case NF4_DQ:
            std::memcpy(&nb, p + 8, 8);
            if (!add_ok(nb, half, r) || !add_ok(r, 48, r)) return 0;
            return r;
        case Q2_K:
        case Q2_K_FAST: {
            uint32_t nsb;
            std::memcpy(&nsb, p + 16, 4);
            return 32 + static_cast<uint64_t>(nsb) * sizeof(super_block_q2_k);
        }
        case BF16:
        case FP16:
            if (!mul_ok(n, 2, t1) || !add_ok(t1, 16, r)) return 0;
            return r;
        case FP8:
            if (!add_ok(n, 24, r)) return 0;
            return r;
        case FP4:
            if (!add_ok(half, 24, r)) return 0;
            return r;
        default: return 0;
    }
}

uint64_t header_bytes(int method) {
    switch (method) {
        case Q8_0: case Q4_0: case MXFP8: case MXFP4: case NF4: return 40;
        case NVFP4: case NF4_DQ: return 48;
        case Q2_K: case Q2_K_FAST: return 32;
        case BF16: case FP16: return 16;
        case FP8: case FP4: return 24;
        default: return 0;
    }
}

// Re-bases the array pointers of the format struct at `p` (its arrays follow
// it) (quantization.cpp:14-90).
void fixup_pointers(int method, uint8_t *p) {
    uint64_t nb = 0;
    std::memcpy(&nb, p + 8, 8);
    auto put = [&](int off, const void *v) { std::memcpy(p + off, &v, sizeof(void *)); };
    switch (method) {
        case Q8_0: case Q4_0: case NF4: put(24, p + 40); put(32, p + 40 + 4 * nb); break;
        case MXFP8: case MXFP4: put(24, p + 40); put(32, p + 40 + nb); break;
        case NVFP4: case NF4_DQ: put(32, p + 48); put(40, p + 48 + nb); break;
        case Q2_K: case Q2_K_FAST: put(24, p + 32); break;
        case BF16: case FP16: put(8, p + 16); break;
        case FP8: case FP4: put(16, p + 24); break;
        default: break;
    }
}

constexpr uint64_t kOuter = sizeof(quantization_buffer_t);
static_assert(sizeof(quantization_buffer_t) == 24, "quantization_buffer_t layout");
static_assert(sizeof(q8_0_array_t) == 40 && sizeof(nvfp4_array_t) == 48 && sizeof(q2_k_array_t) == 32 &&
                  sizeof(fp8_array_t) == 24 && sizeof(bf16_array_t) == 16 && sizeof(super_block_q2_k) == 84 &&
                  sizeof(nf4_dq_array_t) == 48,
              "legacy struct layouts");

template <typename F>
int legacy_guarded(F &&f) {
    try {
        const int rc = f();
        if (rc == 0) set_last_error("");
        return rc;
    } catch (const std::exception &e) {
        set_last_error(e.what());
        return 1;
    } catch (...) {
        set_last_error("unknown error");
        return 1;
    }
}

// The checks the decoders rely on: the header's counts are the ones the
// format's compress writes for its element count.
bool decodable(int method, const uint8_t *p, uint64_t n) {
    if (n == 0 || n > kMaxElements) return false;
    const Layout L = layout_of(method, n);
    uint64_t f1 = 0, f2 = 0;
    std::memcpy(&f1, p + 8, 8);
    std::memcpy(&f2, p + 16, 8);
    if (method == Q2_K || method == Q2_K_FAST) {
        uint32_t nsb;
        std::memcpy(&nsb, p + 16, 4);
        return nsb == ceil_div(n, 256);
    }
    if (L.bs) return f1 == L.nb && f2 == L.bs;
    return true;
}

}  // namespace
}  // namespace bsq

using namespace bsq;

int quantization_compress(const float *src, unsigned long long num_elements, quantization_method_t method,
                          quantization_buffer_t **out) {
    if (!src || num_elements == 0 || !out || *out) return 1;
    if (!method_known(method)) return 1;
    return legacy_guarded([&]() -> int {
        const Layout L = layout_of(method, num_elements);
        auto *buf = static_cast<quantization_buffer_t *>(std::calloc(1, kOuter + L.total));
        if (!buf) return 1;
        try {
            std::lock_guard<std::mutex> lk(g_mu);
            const uint64_t src_bytes = round256(4 * num_elements);
            Staging &s = staging_for_current(src_bytes + round256(L.total));
            float *d_src = static_cast<float *>(s.buf);
            uint8_t *d_img = static_cast<uint8_t *>(s.buf) + src_bytes;
            BSQ_HIP(hipMemcpyAsync(d_src, src, 4 * num_elements, hipMemcpyHostToDevice, s.stream));
            launch_legacy_encode(method, d_src, num_elements, d_img, s.stream);
            uint8_t *payload = reinterpret_cast<uint8_t *>(buf) + kOuter;
            BSQ_HIP(hipMemcpyAsync(payload, d_img, L.total, hipMemcpyDeviceToHost, s.stream));
            BSQ_HIP(hipStreamSynchronize(s.stream));
            // the struct as the reference writes it: counts, the device's
            // scale, zero padding, then pointers into this block
            uint8_t scale[4] = {0, 0, 0, 0};
            if (L.scale_off >= 0) std::memcpy(scale, payload + L.scale_off, 4);
            std::memcpy(payload, header_of(method, num_elements, L).w, L.header);
            if (L.scale_off >= 0) std::memcpy(payload + L.scale_off, scale, 4);
            fixup_pointers(method, payload);
        } catch (...) {
            std::free(buf);
            throw;
        }
        buf->method = method;
        buf->shape.num_elements = num_elements;
        buf->payload = reinterpret_cast<uint8_t *>(buf) + kOuter;
        *out = buf;
        return 0;
    });
}

int quantization_decompress(const quantization_buffer_t *buf, float *dst, unsigned long long dst_num_elements) {
    if (!buf || !dst || !buf->payload) return 1;
    const int method = buf->method;
    if (!method_known(method)) return 1;
    const uint8_t *p = static_cast<const uint8_t *>(buf->payload);
    uint64_t n = 0;
    std::memcpy(&n, p, 8);
    if (dst_num_elements < n) return 1;
    if (method == Q2_K || method == Q2_K_FAST) {
        uint32_t nsb;
        std::memcpy(&nsb, p + 16, 4);
        if (nsb == 0) return 1;  // q2_k_impl.cpp:349-351
    }
    if (n == 0) return 0;  // nothing to write (the reference's loops run zero times)
    return legacy_guarded([&]() -> int {
        if (!decodable(method, p, n)) {
            set_last_error("legacy decompress: header counts do not match the element count");
            return 1;
        }
        const Layout L = layout_of(method, n);
        std::lock_guard<std::mutex> lk(g_mu);
        const uint64_t img_bytes = round256(L.total);
        Staging &s = staging_for_current(img_bytes + round256(4 * n));
        uint8_t *d_img = static_cast<uint8_t *>(s.buf);
        float *d_dst = reinterpret_cast<float *>(static_cast<uint8_t *>(s.buf) + img_bytes);
        BSQ_HIP(hipMemcpyAsync(d_img, p, L.total, hipMemcpyHostToDevice, s.stream));
        launch_legacy_decode(method, d_img, n, d_dst, s.stream);
        BSQ_HIP(hipMemcpyAsync(dst, d_dst, 4 * n, hipMemcpyDeviceToHost, s.stream));
        BSQ_HIP(hipStreamSynchronize(s.stream));
        return 0;
    });
}

long long quantization_get_packed_size(const quantization_buffer_t *buf) {
    if (!buf || !buf->payload) return 0;
    const uint64_t pl = implied_payload(buf->method, static_cast<const uint8_t *>(buf->payload));
    if (pl == 0 || pl > static_cast<uint64_t>(LLONG_MAX) - kOuter) return 0;
    return static_cast<long long>(kOuter + pl);
}

quantization_buffer_t *load_quantization_from_buffer(const void *buffer, long long buffer_size) {
    if (!buffer || buffer_size < static_cast<long long>(kOuter)) return nullptr;
    int method;
    std::memcpy(&method, buffer, 4);
    // the format struct must be inside the buffer before its fields are read
    const uint64_t hb = header_bytes(method);
    if (hb == 0 || static_cast<uint64_t>(buffer_size) < kOuter + hb) return nullptr;
    auto *buf = static_cast<quantization_buffer_t *>(std::calloc(1, static_cast<size_t>(buffer_size)));
    if (!buf) return nullptr;
    std::memcpy(buf, buffer, static_cast<size_t>(buffer_size));
    buf->payload = reinterpret_cast<uint8_t *>(buf) + kOuter;
    const long long expected = quantization_get_packed_size(buf);
    if (expected == 0 || buffer_size < expected) {
        std::free(buf);
        return nullptr;
    }
    fixup_pointers(method, static_cast<uint8_t *>(buf->payload));
    return buf;
}

void quantization_free(quantization_buffer_t *buf) { std::free(buf); }

// ---------------------------------------------------------------------------
// extern "C" entry points (include/bitsqz_llm_c.h)
// ---------------------------------------------------------------------------
extern "C" {

BSQ_API int bsq_legacy_compress(int method, const float *src, uint64_t n, void **out) {
    return quantization_compress(src, n, static_cast<quantization_method_t>(method),
                                 reinterpret_cast<quantization_buffer_t **>(out));
}

BSQ_API int bsq_legacy_decompress(const void *buf, float *dst, uint64_t n) {
    return quantization_decompress(static_cast<const quantization_buffer_t *>(buf), dst, n);
}

BSQ_API long long bsq_legacy_packed_size(const void *buf) {
    return quantization_get_packed_size(static_cast<const quantization_buffer_t *>(buf));
}

BSQ_API void *bsq_legacy_load(const void *buffer, long long size) { return load_quantization_from_buffer(buffer, size); }

BSQ_API void bsq_legacy_free(void *buf) { quantization_free(static_cast<quantization_buffer_t *>(buf)); }

BSQ_API long long bsq_legacy_payload_bytes(int method, uint64_t n) {
    if (!method_known(method) || n == 0 || n > kMaxElements) return -1;
    return static_cast<long long>(legacy_payload_bytes(method, n));
}

BSQ_API int bsq_legacy_encode_device(int method, const float *d_src, uint64_t n, void *d_payload, void *stream) {
    return legacy_guarded([&]() -> int {
        launch_legacy_encode(method, d_src, n, static_cast<uint8_t *>(d_payload), static_cast<hipStream_t>(stream));
        return 0;
    });
}

BSQ_API int bsq_legacy_decode_device(int method, const void *d_payload, uint64_t n, float *d_dst, void *stream) {
    return legacy_guarded([&]() -> int {
        launch_legacy_decode(method, static_cast<const uint8_t *>(d_payload), n, d_dst,
                             static_cast<hipStream_t>(stream));
        return 0;
    });
}

BSQ_API int bsq_legacy_sweep(int kind, uint64_t lo, uint64_t hi, unsigned long long *d_checksum, void *stream) {
    return legacy_guarded([&]() -> int {
        launch_legacy_sweep(kind, lo, hi, d_checksum, static_cast<hipStream_t>(stream));
        return 0;
    });
}

}  // extern "C"
