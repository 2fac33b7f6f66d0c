// Cross-lane reductions for one 64-lane wave through DPP lane moves (VALU
// operations; no LDS round trip, unlike __shfl_*).
#pragma once

#include <hip/hip_runtime.h>

namespace bsq {

// v of the lane selected by the DPP control CTRL; lanes of rows outside
// ROW_MASK (and lanes whose source is out of range) read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_read(double v) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(u & 0xffffffffu), CTRL, ROW_MASK, 0xF, false));
    const unsigned hi = static_cast<unsigned>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), CTRL, ROW_MASK, 0xF, false));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// v of the lane selected by CTRL, for controls whose source lane always
// exists (quad permutations, row mirrors): no old value to initialise
template <int CTRL>
__device__ __forceinline__ double dpp_perm(double v) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_mov_dpp(static_cast<int>(u & 0xffffffffu), CTRL, 0xF, 0xF, false));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_mov_dpp(static_cast<int>(u >> 32), CTRL, 0xF, 0xF, false));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// sum over each aligned group of 4 lanes, in every lane of the group
__device__ __forceinline__ double quad_sum(double v) {
    v += dpp_perm<0xB1>(v);  // quad_perm [1, 0, 3, 2]
    v += dpp_perm<0x4E>(v);  // quad_perm [2, 3, 0, 1]
    return v;
}

// sum over all 64 lanes (every lane must be active), returned to every lane
__device__ __forceinline__ double wave_sum_dpp(double v) {
    v = quad_sum(v);
    v += dpp_perm<0x141>(v);       // row_half_mirror: 8-lane sums
    v += dpp_perm<0x140>(v);       // row_mirror: 16-lane row sums
    v += dpp_read<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
    v += dpp_read<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3: lane 63 holds the total
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffu), 63));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), 63));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// float v of the lane selected by the DPP control CTRL (all rows, all banks).
template <int CTRL>
__device__ __forceinline__ float dpp_read_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// fmaxf over each aligned group of 16 lanes (one DPP row), in every lane of
// the group; all 16 lanes must be active.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_read_f32<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, dpp_read_f32<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, dpp_read_f32<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_read_f32<0x140>(v));  // row_mirror
    return v;
}

}  // namespace bsq
