// Scalar FP8 E4M3 codec shared by the NF4_DQ block scales (quant.hip) and the
// legacy FP8 / MXFP8 / NVFP4 formats (legacy.hip).  The reference writes the
// same encoder in quantization_cuda.cu:64-109 and, identically, in
// legacy_modules/quantization/src/impl/fp8_impl.cpp:51-82,
// mxfp8_impl.cpp:56-87 and nvfp4_impl.cpp:62-93 (saturation at 448, frexp
// split, round-to-nearest-even mantissa, subnormal mantissa clamped at 7);
// the decoder has no NaN code (0x7F decodes to 480).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "bsq_internal.hpp"

namespace bsq {

// FP8 E4M3 encode exactly as quantization_cuda.cu:64-109 writes it.
__device__ __forceinline__ uint32_t e4m3_encode(float value) {
    if (!__builtin_isfinite(value)) value = (value < 0.0f) ? -kE4M3Max : kE4M3Max;
    const uint32_t sign = __builtin_signbit(value) ? 1u : 0u;
    float a = fabsf(value);
    if (a == 0.0f) return sign << 7;
    if (a > kE4M3Max) a = kE4M3Max;
    int e2 = 0;
    const float mant = frexpf(a, &e2);
    int ef = e2 - 1 + 7;
    if (ef <= 0) {
        int mf = static_cast<int>(rintf(a * 512.0f));
        if (mf > 7) mf = 7;
        return (sign << 7) | static_cast<uint32_t>(mf & 7);
    }
    int mf = static_cast<int>(rintf(((mant * 2.0f) - 1.0f) * 8.0f));
    if (mf > 7) {
        mf = 0;
        ef += 1;
    }
    if (ef >= 16) {
        ef = 15;
        mf = 7;
    }
    return (sign << 7) | (static_cast<uint32_t>(ef & 15) << 3) | static_cast<uint32_t>(mf & 7);
}

// FP8 E4M3 decode (quantization_cuda.cu:111-128); 0x7F decodes to 480.
__device__ __forceinline__ float e4m3_decode(uint32_t v) {
    const uint32_t ef = (v >> 3) & 15u, mf = v & 7u;
    float r;
    if (ef == 0) r = (static_cast<float>(mf) / 8.0f) * 0.015625f;  // 2^(1-7)
    else r = (1.0f + static_cast<float>(mf) / 8.0f) * __builtin_ldexpf(1.0f, static_cast<int>(ef) - 7);
    return (v & 0x80u) ? -r : r;
}

}  // namespace bsq
