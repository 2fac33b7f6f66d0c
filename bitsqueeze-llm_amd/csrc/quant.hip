// NF4 / NF4_DQ block-64 quantisation for gfx950.
//
// Behaviour follows the reference codec bit for bit:
//   modules/quantization_cuda/src/quantization_cuda.cu:20-341 (CUDA kernels)
//   legacy_modules/quantization/src/impl/nf4_impl.cpp:73-164,
//   legacy_modules/quantization/src/impl/nf4_dq_impl.cpp:83-275 (CPU codec that the
//   reference's own test requires to equal the CUDA codec exactly,
//   tests/quantization_cuda/test_nf4_cuda.cu:109-114).
//
// Layout of the work: one thread owns 8 consecutive elements (two 16-byte
// loads, one 4-byte store of packed nibbles), so one 64-element block is an
// aligned group of 8 lanes and its absmax is a 3-step DPP reduction.  Kernels
// are persistent grid-stride loops sized to the CU count.
//
// This file is compiled with -ffp-contract=off: every multiply and subtract
// below must round on its own, as in the reference.
#include "bsq_internal.hpp"

#include <cfloat>

namespace bsq {
namespace {

constexpr int kThreads = 256;

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

// Nearest NF4 code with the reference's tie rule.  For |v| < 2 the scan's
// answer is the number of exact decision thresholds at or below v.
__device__ __forceinline__ uint32_t nf4_code(float v) {
    constexpr float T[15] = BSQ_NF4_THRESHOLDS;
    if (fabsf(v) < 2.0f) {
        uint32_t c = 0;
#pragma unroll
        for (int i = 0; i < 15; ++i) c += (v >= T[i]) ? 1u : 0u;
        return c;
    }
    return nf4_code_scan(v);
}

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

// max over the aligned group of 8 lanes (quad xor-1, quad xor-2, half-row
// mirror), all lanes of the group active.
__device__ __forceinline__ float group8_max(float v) {
    int x = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false)));
    x = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false)));
    x = __float_as_int(v);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false)));
    return v;
}

// Loads the 8 elements of `chunk` (zeros past n).
__device__ __forceinline__ void load8(const float *__restrict__ x, uint64_t n, uint64_t chunk,
                                      bool vec_ok, float (&v)[8]) {
    const uint64_t e0 = chunk * 8;
    if (vec_ok && e0 + 8 <= n) {
        const float4 a = *reinterpret_cast<const float4 *>(x + e0);
        const float4 b = *(reinterpret_cast<const float4 *>(x + e0) + 1);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (e0 + i < n) ? x[e0 + i] : 0.0f;
    }
}

// Stores the packed nibbles of `chunk`: byte j = code(2j) << 4 | code(2j + 1).
__device__ __forceinline__ void store_codes(uint8_t *__restrict__ codes, uint64_t n, uint64_t chunk,
                                            bool vec_ok, const uint32_t (&c)[8]) {
    const uint64_t e0 = chunk * 8;
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) word |= ((c[2 * j] << 4) | c[2 * j + 1]) << (8 * j);
    if (vec_ok && e0 + 8 <= n) {
        *reinterpret_cast<uint32_t *>(codes + chunk * 4) = word;
    } else {
        const uint64_t nbytes = (n - e0 + 1) / 2;  // e0 < n here
        for (uint64_t j = 0; j < 4 && j < nbytes; ++j)
            codes[chunk * 4 + j] = static_cast<uint8_t>(word >> (8 * j));
    }
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

// Pass 1 of NF4_DQ: max over blocks of the block scale (absmax, or 1 for an
// all-zero block), accumulated as float bits (all values >= 0) with one
// atomicMax per workgroup.  Replaces compute_block_absmax_kernel +
// cub::DeviceReduce::Max (quantization_cuda.cu:186-220, 594-602).
__global__ __launch_bounds__(kThreads) void dq_gmax_kernel(const float *__restrict__ x, uint64_t n,
                                                            bool vec_ok, uint32_t *__restrict__ gmax) {
    const uint64_t nchunks = ceil_div(n, 8), nblocks = ceil_div(n, kQuantBlock);
    float local = 0.0f;
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads; base < nchunks;
         base += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint64_t chunk = base + threadIdx.x;
        float v[8];
        if (chunk < nchunks) load8(x, n, chunk, vec_ok, v);
        else
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(sanitize(v[i])));
        m = group8_max(m);
        if (chunk / 8 < nblocks) local = fmaxf(local, m > 0.0f ? m : 1.0f);
    }
    // workgroup max
    for (int off = 32; off >= 1; off >>= 1) local = fmaxf(local, __shfl_xor(local, off));
    __shared__ float wmax[kThreads / 64];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = local;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = wmax[0];
        for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, wmax[w]);
        atomicMax(gmax, __float_as_uint(m));
    }
}

template <bool DQ>
__global__ __launch_bounds__(kThreads) void quant_encode_kernel(
    const float *__restrict__ x, uint64_t n, bool vec_ok, float *__restrict__ scales_f32,
    uint8_t *__restrict__ scales_u8, const uint32_t *__restrict__ gmax, float *__restrict__ dq_out,
    uint8_t *__restrict__ codes) {
    const uint64_t nchunks = ceil_div(n, 8);
    float dq = 1.0f;
    if constexpr (DQ) {
        const float raw = dq_raw_from_gmax(*gmax);
        dq = dq_effective(raw);
        if (blockIdx.x == 0 && threadIdx.x == 0) *dq_out = raw;
    }
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads; base < nchunks;
         base += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint64_t chunk = base + threadIdx.x;
        const bool valid = chunk < nchunks;
        float v[8];
        if (valid) load8(x, n, chunk, vec_ok, v);
        else
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = sanitize(v[i]);
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
        m = group8_max(m);
        const float absmax = (m > 0.0f) ? m : 1.0f;
        float scale;
        uint32_t scode = 0;
        if constexpr (DQ) {
            scode = e4m3_encode(absmax / dq);
            scale = dq * e4m3_decode(scode);
            if (scale == 0.0f || !__builtin_isfinite(scale)) scale = 1.0f;
        } else {
            scale = absmax;
        }
        const float inv = 1.0f / scale;
        if (valid && (threadIdx.x & 7) == 0) {
            if constexpr (DQ) scales_u8[chunk / 8] = static_cast<uint8_t>(scode);
            else scales_f32[chunk / 8] = scale;
        }
        if (valid) {
            uint32_t c[8];
            const uint64_t e0 = chunk * 8;
#pragma unroll
            for (int i = 0; i < 8; ++i) c[i] = (e0 + i < n) ? nf4_code(v[i] * inv) : 0u;  // odd tail: low nibble 0
            store_codes(codes, n, chunk, vec_ok, c);
        }
    }
}

template <bool DQ>
__global__ __launch_bounds__(kThreads) void quant_decode_kernel(
    uint64_t n, bool vec_ok, const float *__restrict__ scales_f32, const uint8_t *__restrict__ scales_u8,
    const float *__restrict__ dq_ptr, const uint8_t *__restrict__ codes, float *__restrict__ out) {
    constexpr float Lc[16] = BSQ_NF4_LEVELS;
    __shared__ float L[16];
    if (threadIdx.x < 16) L[threadIdx.x] = Lc[threadIdx.x];
    __syncthreads();
    const uint64_t nchunks = ceil_div(n, 8);
    float dq = 1.0f;
    if constexpr (DQ) dq = dq_effective(*dq_ptr);
    for (uint64_t chunk = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; chunk < nchunks;
         chunk += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint64_t e0 = chunk * 8, b = chunk / 8;
        float s;
        if constexpr (DQ) s = dq * e4m3_decode(scales_u8[b]);
        else s = scales_f32[b];
        if (s == 0.0f || !__builtin_isfinite(s)) s = 1.0f;
        const bool full = vec_ok && e0 + 8 <= n;
        uint32_t word = 0;
        if (full) {
            word = *reinterpret_cast<const uint32_t *>(codes + chunk * 4);
        } else {
            const uint64_t nbytes = (n - e0 + 1) / 2;
            for (uint64_t j = 0; j < 4 && j < nbytes; ++j)
                word |= static_cast<uint32_t>(codes[chunk * 4 + j]) << (8 * j);
        }
        float o[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t byte = (word >> (8 * j)) & 0xFFu;
            o[2 * j] = s * L[byte >> 4];
            o[2 * j + 1] = s * L[byte & 15u];
        }
        if (full) {
            f32x4 *dst = reinterpret_cast<f32x4 *>(out + e0);
            const f32x4 lo = {o[0], o[1], o[2], o[3]}, hi = {o[4], o[5], o[6], o[7]};
            __builtin_nontemporal_store(lo, dst);
            __builtin_nontemporal_store(hi, dst + 1);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (e0 + i < n) out[e0 + i] = o[i];
        }
    }
}

__global__ void nf4_code_batch_kernel(const float *__restrict__ v, uint64_t n, uint8_t *__restrict__ c) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        c[i] = static_cast<uint8_t>(nf4_code(v[i]));
}

__global__ void e4m3_encode_batch_kernel(const float *__restrict__ v, uint64_t n, uint8_t *__restrict__ c) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        c[i] = static_cast<uint8_t>(e4m3_encode(v[i]));
}

__global__ void e4m3_decode_batch_kernel(const uint8_t *__restrict__ c, uint64_t n, float *__restrict__ v) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        v[i] = e4m3_decode(c[i]);
}

__global__ __launch_bounds__(kThreads) void nf4_code_sweep_kernel(uint64_t lo, uint64_t hi,
                                                                  unsigned long long *__restrict__ hist,
                                                                  unsigned long long *__restrict__ checksum) {
    __shared__ unsigned int h[16];
    if (threadIdx.x < 16) h[threadIdx.x] = 0;
    __syncthreads();
    unsigned long long cs = 0;
    unsigned int hl[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) hl[i] = 0;
    for (uint64_t p = lo + static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; p < hi;
         p += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint32_t bits = static_cast<uint32_t>(p);
        const uint32_t c = nf4_code(__uint_as_float(bits));
#pragma unroll
        for (int i = 0; i < 16; ++i) hl[i] += (c == static_cast<uint32_t>(i)) ? 1u : 0u;
        cs += static_cast<unsigned long long>(c) * (bits % 65521u);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) atomicAdd(&h[i], hl[i]);
    __syncthreads();
    if (threadIdx.x < 16) atomicAdd(&hist[threadIdx.x], static_cast<unsigned long long>(h[threadIdx.x]));
    atomicAdd(checksum, cs);
}

unsigned grid_for(uint64_t work_items, unsigned per_cu = 8) {
    const uint64_t want = ceil_div(work_items, kThreads);
    const uint64_t cap = static_cast<uint64_t>(cu_count()) * per_cu;
    return static_cast<unsigned>(want < 1 ? 1 : (want < cap ? want : cap));
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

void launch_quant_encode(const float *x, uint64_t n, int method, float *scales_f32, uint8_t *scales_u8,
                         float *dq_out, uint8_t *codes, uint32_t *gmax_scratch, hipStream_t stream) {
    BSQ_REQUIRE(n > 0, "quant encode: empty input");
    const bool vec_ok = aligned16(x) && ((reinterpret_cast<uintptr_t>(codes) & 3u) == 0);
    const uint64_t nchunks = ceil_div(n, 8);
    const unsigned grid = grid_for(nchunks);
    if (method == kMethodNF4) {
        BSQ_REQUIRE(scales_f32 && codes, "quant encode: null NF4 output");
        quant_encode_kernel<false><<<grid, kThreads, 0, stream>>>(x, n, vec_ok, scales_f32, nullptr, nullptr,
                                                                  nullptr, codes);
    } else if (method == kMethodNF4DQ) {
        BSQ_REQUIRE(scales_u8 && codes && dq_out && gmax_scratch, "quant encode: null NF4_DQ output");
        BSQ_HIP(hipMemsetAsync(gmax_scratch, 0, sizeof(uint32_t), stream));
        dq_gmax_kernel<<<grid, kThreads, 0, stream>>>(x, n, vec_ok, gmax_scratch);
        quant_encode_kernel<true><<<grid, kThreads, 0, stream>>>(x, n, vec_ok, nullptr, scales_u8, gmax_scratch,
                                                                 dq_out, codes);
    } else {
        fail("quant encode: unsupported method");
    }
    BSQ_HIP(hipGetLastError());
}

void launch_quant_decode(uint64_t n, int method, const float *scales_f32, const uint8_t *scales_u8,
                         const float *dq, const uint8_t *codes, float *out, hipStream_t stream) {
    BSQ_REQUIRE(n > 0, "quant decode: empty output");
    const bool vec_ok = aligned16(out) && ((reinterpret_cast<uintptr_t>(codes) & 3u) == 0);
    const unsigned grid = grid_for(ceil_div(n, 8));
    if (method == kMethodNF4) {
        BSQ_REQUIRE(scales_f32 && codes, "quant decode: null NF4 input");
        quant_decode_kernel<false><<<grid, kThreads, 0, stream>>>(n, vec_ok, scales_f32, nullptr, nullptr, codes,
                                                                  out);
    } else if (method == kMethodNF4DQ) {
        BSQ_REQUIRE(scales_u8 && codes && dq, "quant decode: null NF4_DQ input");
        quant_decode_kernel<true><<<grid, kThreads, 0, stream>>>(n, vec_ok, nullptr, scales_u8, dq, codes, out);
    } else {
        fail("quant decode: unsupported method");
    }
    BSQ_HIP(hipGetLastError());
}

void launch_nf4_code_batch(const float *v, uint64_t n, uint8_t *codes, hipStream_t stream) {
    if (n == 0) return;
    nf4_code_batch_kernel<<<grid_for(n), kThreads, 0, stream>>>(v, n, codes);
    BSQ_HIP(hipGetLastError());
}

void launch_e4m3_encode_batch(const float *v, uint64_t n, uint8_t *codes, hipStream_t stream) {
    if (n == 0) return;
    e4m3_encode_batch_kernel<<<grid_for(n), kThreads, 0, stream>>>(v, n, codes);
    BSQ_HIP(hipGetLastError());
}

void launch_e4m3_decode_batch(const uint8_t *c, uint64_t n, float *v, hipStream_t stream) {
    if (n == 0) return;
    e4m3_decode_batch_kernel<<<grid_for(n), kThreads, 0, stream>>>(c, n, v);
    BSQ_HIP(hipGetLastError());
}

void launch_nf4_code_sweep(uint64_t lo, uint64_t hi, unsigned long long *hist16, unsigned long long *checksum,
                           hipStream_t stream) {
    BSQ_REQUIRE(lo <= hi && hi <= (1ull << 32), "nf4 sweep: bad range");
    BSQ_HIP(hipMemsetAsync(hist16, 0, 16 * sizeof(unsigned long long), stream));
    BSQ_HIP(hipMemsetAsync(checksum, 0, sizeof(unsigned long long), stream));
    if (hi == lo) return;
    nf4_code_sweep_kernel<<<grid_for(hi - lo, 16), kThreads, 0, stream>>>(lo, hi, hist16, checksum);
    BSQ_HIP(hipGetLastError());
}

}  // namespace bsq
