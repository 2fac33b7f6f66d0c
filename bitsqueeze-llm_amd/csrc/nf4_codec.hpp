// NF4 / NF4_DQ element encoding shared by the quantiser (quant.hip) and the
// fused encode + error top-k pass (topk.hip): the reference's nearest-level
// rule (quantization_cuda.cu:43-58) with its tie behaviour, and the NF4_DQ
// global scale (quantization_cuda.cu:222-249).
#pragma once

#include "bsq_internal.hpp"

namespace bsq {
namespace {

__device__ __forceinline__ float sanitize(float x) { return __builtin_isfinite(x) ? x : 0.0f; }

// The reference's linear scan: first index minimising |fl(v - L[i])|
// (quantization_cuda.cu:43-58).  Used only where |v| >= 2 or v is not finite.
__device__ __noinline__ uint32_t nf4_code_scan(float v) {
    constexpr float L[16] = BSQ_NF4_LEVELS;
    if (!__builtin_isfinite(v)) v = 0.0f;
    uint32_t best = 0;
    float best_err = fabsf(v - L[0]);
#pragma unroll
    for (int i = 1; i < 16; ++i) {
        const float err = fabsf(v - L[i]);
        if (err < best_err) {
            best_err = err;
            best = i;
        }
    }
    return best;
}

// The same scan over the levels held in `L` (LDS), inline and not unrolled:
// a call to the out-of-line scan from a kernel that holds many values in
// registers makes the compiler park them in callee-saved registers around
// the call, which spreads them over far more registers than they need.
__device__ __forceinline__ uint32_t nf4_code_scan_inline(const float *L, float v) {
    if (!__builtin_isfinite(v)) v = 0.0f;
    uint32_t best = 0;
    float best_err = fabsf(v - L[0]);
#pragma unroll 1
    for (int i = 1; i < 16; ++i) {
        const float err = fabsf(v - L[i]);
        if (err < best_err) {
            best_err = err;
            best = static_cast<uint32_t>(i);
        }
    }
    return best;
}

// Nearest NF4 code with the reference's tie rule: for |v| < 2 the scan's
// answer is the number of exact decision thresholds at or below v, found
// here with one table lookup and one comparison.  [-1, 1] is
// cut into 256 bins of width 1/128; bin b holds code_lo = #{T_i <= -1 + b/128}
// and the threshold lying inside the bin, if any (no bin holds two: the
// closest thresholds are 0.085 apart).  Every threshold is at least 2.3e-4
// from a bin edge, while the bin index floor((v + 1) * 128) computed in FP32
// is off by one only for v within 1.2e-7 of an edge, where the count is the
// same on both sides; v in [1, 2) and (-2, -1] clamp to the end bins (codes
// 15 and 0).  |v| >= 2 and non-finite v take the scan.  Exhaustively
// checked against the scan over all 2^32 floats by the GPU test suite.
struct Nf4Table {
    uint2 ent[256];  // (bits of the threshold inside bin b, code_lo): one 8-byte read
};

__device__ __forceinline__ void nf4_table_build(Nf4Table &t) {
    constexpr float T[15] = BSQ_NF4_THRESHOLDS;
    for (int b = threadIdx.x; b < 256; b += blockDim.x) {
        const float e0 = -1.0f + static_cast<float>(b) / 128.0f, e1 = -1.0f + static_cast<float>(b + 1) / 128.0f;
        uint32_t lo = 0;
        float thr = __builtin_inff();
#pragma unroll
        for (int i = 0; i < 15; ++i) {
            lo += (T[i] <= e0) ? 1u : 0u;
            if (T[i] > e0 && T[i] < e1) thr = T[i];
        }
        t.ent[b] = uint2{__float_as_uint(thr), lo};
    }
}

// the table path alone: |v| < 2
__device__ __forceinline__ uint32_t nf4_code_small(const Nf4Table &t, float v) {
    const int b = min(max(static_cast<int>((v + 1.0f) * 128.0f), 0), 255);
    const uint2 e = t.ent[b];
    return e.y + ((v >= __uint_as_float(e.x)) ? 1u : 0u);
}

// The same bins with the two candidate levels of each: (bits of the
// threshold, code_lo, L[code_lo], L[code_lo + 1]) in one 16-byte entry, so an
// encoder that also needs the level of the code (the fused encode + error
// pass) reads both with one lookup.
struct Nf4LevelTable {
    uint4 ent[256];
};

__device__ __forceinline__ void nf4_level_table_build(Nf4LevelTable &t) {
    constexpr float T[15] = BSQ_NF4_THRESHOLDS;
    constexpr float L[16] = BSQ_NF4_LEVELS;
    for (int b = threadIdx.x; b < 256; b += blockDim.x) {
        const float e0 = -1.0f + static_cast<float>(b) / 128.0f, e1 = -1.0f + static_cast<float>(b + 1) / 128.0f;
        uint32_t lo = 0;
        float thr = __builtin_inff();
#pragma unroll
        for (int i = 0; i < 15; ++i) {
            lo += (T[i] <= e0) ? 1u : 0u;
            if (T[i] > e0 && T[i] < e1) thr = T[i];
        }
        // a bin whose code_lo is 15 holds no threshold (thr = inf): its upper
        // level is never taken
        t.ent[b] = uint4{__float_as_uint(thr), lo, __float_as_uint(L[lo]), __float_as_uint(L[lo < 15 ? lo + 1 : 15])};
    }
}

// code of v (|v| < 2, as nf4_code_small) and its level L[code]
__device__ __forceinline__ uint32_t nf4_code_level_small(const Nf4LevelTable &t, float v, float &level) {
    const int b = min(max(static_cast<int>((v + 1.0f) * 128.0f), 0), 255);
    const uint4 e = t.ent[b];
    const bool up = v >= __uint_as_float(e.x);
    level = __uint_as_float(up ? e.w : e.z);
    return e.y + (up ? 1u : 0u);
}

__device__ __forceinline__ uint32_t nf4_code(const Nf4Table &t, float v) {
    if (fabsf(v) < 2.0f) return nf4_code_small(t, v);
    return nf4_code_scan(v);
}

__device__ __forceinline__ float dq_raw_from_gmax(uint32_t gbits) {
    // store_dq_scale_kernel (quantization_cuda.cu:222-233)
    const float g = __uint_as_float(gbits);
    if (g == 0.0f || !__builtin_isfinite(g)) return 1.0f;
    return g / kE4M3Max;
}

__device__ __forceinline__ float dq_effective(float dq) {
    // nf4_dq_compress_kernel / nf4_dq_decompress_kernel (quantization_cuda.cu:246-249, 324-327)
    return (dq == 0.0f || !__builtin_isfinite(dq)) ? 1.0f : dq;
}

}  // namespace
}  // namespace bsq
