// NF4 / NF4_DQ block-64 quantisation for gfx950.
//
// Behaviour follows the reference codec bit for bit:
//   modules/quantization_cuda/src/quantization_cuda.cu:20-341 (CUDA kernels)
//   legacy_modules/quantization/src/impl/nf4_impl.cpp:73-164,
//   legacy_modules/quantization/src/impl/nf4_dq_impl.cpp:83-275 (CPU codec that the
//   reference's own test requires to equal the CUDA codec exactly,
//   tests/quantization_cuda/test_nf4_cuda.cu:109-114).
//
// Layout of the work: the encoders give a lane 8 consecutive elements (a
// 64-element block is an aligned group of 8 lanes, its absmax a 3-step DPP
// reduction); the decoder stages 4096-element tiles through LDS so that its
// stores are contiguous per instruction.  Kernels are persistent grid-stride
// loops sized to the CU count.
//
// This file is compiled with -ffp-contract=off: every multiply and subtract
// below must round on its own, as in the reference.
#include "bsq_internal.hpp"
#include "nf4_codec.hpp"
#include "scalar_codecs.hpp"

#include <cfloat>

namespace bsq {
namespace {

constexpr int kThreads = 256;

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

// Loads the 8 elements of `chunk` (zeros past n).  The input is streamed:
// non-temporal loads, which do not allocate in the caches (measured with the
// caches holding other dirty data, as the pipeline leaves them: 53 us instead
// of 77 us for the NF4 encode of 4096 x 11008, 93 instead of 125 us for the
// two NF4_DQ passes).
__device__ __forceinline__ void load8(const float *__restrict__ x, uint64_t n, uint64_t chunk,
                                      bool vec_ok, float (&v)[8]) {
    const uint64_t e0 = chunk * 8;
    if (vec_ok && e0 + 8 <= n) {
        const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(x + e0));
        const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(x + e0) + 1);
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


// Encode side: one thread owns chunks of 8 consecutive elements (two 16-byte
// loads, one 4-byte store of packed nibbles), so a 64-element block is an
// aligned group of 8 lanes and the per-block scale work is shared by 8 lanes.
// Each thread takes kUnroll chunks per loop iteration, their loads issued
// together before any is used (one chunk per iteration left these kernels
// latency-bound); the encoder also issues the next iteration's loads before
// encoding the current one (two chunks per iteration measured best with
// that: four take 144 VGPRs, three waves per SIMD).
constexpr int kUnroll = 2;

// Pass 1 of NF4_DQ: max over blocks of the block scale (absmax, or 1 for an
// all-zero block), as float bits (all values >= 0): each workgroup writes
// its maximum to out[blockIdx.x] (PARTIAL; rows_gmax_kernel reduces those)
// or takes it into out[0] with atomicMax.  Replaces
// compute_block_absmax_kernel + cub::DeviceReduce::Max
// (quantization_cuda.cu:186-220, 594-602).
template <bool PARTIAL>
__global__ __launch_bounds__(kThreads) void dq_gmax_kernel(const float *__restrict__ x, uint64_t n,
                                                            bool vec_ok, uint32_t *__restrict__ out) {
    const uint64_t nchunks = ceil_div(n, 8), nblocks = ceil_div(n, kQuantBlock);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    float local = 0.0f;
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads; base < nchunks; base += kUnroll * stride) {
        float v[kUnroll][8];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t chunk = base + u * stride + threadIdx.x;
            if (chunk < nchunks) load8(x, n, chunk, vec_ok, v[u]);
            else
#pragma unroll
                for (int i = 0; i < 8; ++i) v[u][i] = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t chunk = base + u * stride + threadIdx.x;
            float m = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(sanitize(v[u][i])));
            m = group8_max(m);
            if (chunk / 8 < nblocks) local = fmaxf(local, m > 0.0f ? m : 1.0f);
        }
    }
    // workgroup max
    for (int off = 32; off >= 1; off >>= 1) local = fmaxf(local, __shfl_xor(local, off));
    __shared__ float wmax[kThreads / 64];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = local;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = wmax[0];
        for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, wmax[w]);
        if constexpr (PARTIAL) out[blockIdx.x] = __float_as_uint(m);
        else atomicMax(out, __float_as_uint(m));
    }
}

// SEL: sel[chunk] flags the chunk's elements that a separation took out
// (bit i = element 8 chunk + i); they are encoded as 0, as the residual
// holds them.
// NF4_DQ: the global scale comes from *gmax, or, when row_gmax is given,
// from the largest of row_gmax[0 .. gmax_rows) (a separation's per-row
// maxima; gmax_rows a multiple of 4 up to kInlineGmaxRows), which every
// workgroup reduces itself.
template <bool DQ, bool SEL>
__global__ __launch_bounds__(kThreads) void quant_encode_kernel(
    const float *__restrict__ x, uint64_t n, bool vec_ok, float *__restrict__ scales_f32,
    uint8_t *__restrict__ scales_u8, const uint32_t *__restrict__ gmax, const float *__restrict__ row_gmax,
    uint32_t gmax_rows, float *__restrict__ dq_out, uint8_t *__restrict__ codes,
    uint32_t *__restrict__ flags_reset, const uint8_t *__restrict__ sel) {
    __shared__ Nf4Table tab;
    __shared__ float gwmax[kThreads / 64];
    // the pipeline's flags word, cleared here when no earlier kernel of the
    // compress does it (saves a fill launch); nothing reads it before this
    // kernel ends
    if (flags_reset && blockIdx.x == 0 && threadIdx.x == 0) *flags_reset = 0u;
    const uint64_t nchunks = ceil_div(n, 8);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    float dq = 1.0f;  // NF4_DQ: set below, before the first encode
    // chunks of one iteration: loaded one iteration ahead (two register
    // sets), so the loads of iteration i + 1 are in flight while iteration i
    // is encoded
    auto load_it = [&](uint64_t base, float (&v)[kUnroll][8], uint32_t (&sb)[kUnroll]) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t chunk = base + u * stride + threadIdx.x;
            if (chunk < nchunks) {
                load8(x, n, chunk, vec_ok, v[u]);
                if constexpr (SEL) sb[u] = sel[chunk];
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[u][i] = 0.0f;
                if constexpr (SEL) sb[u] = 0u;
            }
        }
    };
    auto encode_it = [&](uint64_t base, float (&v)[kUnroll][8], const uint32_t (&sb)[kUnroll]) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t chunk = base + u * stride + threadIdx.x;
            const bool valid = chunk < nchunks;
            // sanitised values (a selected entry reads as 0) and this lane's
            // largest |value|
            if constexpr (SEL) {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[u][i] = ((sb[u] >> i) & 1u) ? 0.0f : v[u][i];
            }
            float lm = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[u][i] = sanitize(v[u][i]);
                lm = fmaxf(lm, fabsf(v[u][i]));
            }
            const float m = group8_max(lm);
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
                // |v inv| < 2 (the table) unless a block scale fell far below
                // the block's absmax (an NF4_DQ scale code of 0 replaced by 1).
                // Rounding is monotone, so the chunk's largest |v inv| is
                // exactly fl(lm inv): one test per chunk; the per-element end
                // test and the scan only for a chunk that needs them.
                uint32_t c[8];
                const uint64_t e0 = chunk * 8;
                if (lm * inv < 2.0f && e0 + 8 <= n) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) c[i] = nf4_code_small(tab, v[u][i] * inv);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) c[i] = (e0 + i < n) ? nf4_code(tab, v[u][i] * inv) : 0u;  // odd tail: low nibble 0
                }
                store_codes(codes, n, chunk, vec_ok, c);
            }
        }
    };
    const uint64_t step = static_cast<uint64_t>(kUnroll) * stride;
    float va[kUnroll][8], vb[kUnroll][8];
    uint32_t sa[kUnroll] = {}, sbb[kUnroll] = {};
    uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads;
    // the first two iterations' loads go out before the code table is built
    // and the global scale read (neither feeds an address), so the table
    // work and the barrier overlap the first memory round trip
    if (base < nchunks) load_it(base, va, sa);
    if (base + step < nchunks) load_it(base + step, vb, sbb);
    if constexpr (DQ) {
        if (row_gmax) {  // uniform: wave maxima of the per-row maxima to LDS
            constexpr int kGq = kInlineGmaxRows / (4 * kThreads);
            float gm = 0.0f;
#pragma unroll
            for (int j = 0; j < kGq; ++j) {
                const uint32_t i4 = threadIdx.x + kThreads * j;
                if (4 * i4 < gmax_rows) {
                    const f32x4 g = reinterpret_cast<const f32x4 *>(row_gmax)[i4];
                    gm = fmaxf(gm, fmaxf(fmaxf(g.x, g.y), fmaxf(g.z, g.w)));
                }
            }
            for (int off = 32; off >= 1; off >>= 1) gm = fmaxf(gm, __shfl_xor(gm, off));
            if ((threadIdx.x & 63) == 0) gwmax[threadIdx.x >> 6] = gm;
        }
    }
    nf4_table_build(tab);
    __syncthreads();
    if constexpr (DQ) {
        // max is order-free: every workgroup gets the same bits
        const uint32_t gbits =
            row_gmax ? __float_as_uint(fmaxf(fmaxf(gwmax[0], gwmax[1]), fmaxf(gwmax[2], gwmax[3]))) : *gmax;
        const float raw = dq_raw_from_gmax(gbits);
        dq = dq_effective(raw);
        if (blockIdx.x == 0 && threadIdx.x == 0) *dq_out = raw;
    }
    for (bool first = true; base < nchunks; base += 2 * step, first = false) {  // uniform
        if (!first && base + step < nchunks) load_it(base + step, vb, sbb);
        encode_it(base, va, sa);
        if (base + step >= nchunks) break;
        if (base + 2 * step < nchunks) load_it(base + 2 * step, va, sa);
        encode_it(base + step, vb, sbb);
    }
}

// Decode: a workgroup decodes tiles of 4096 elements.  Lane t reads the
// 8 code bytes and the block scale of elements 16 t .. 16 t + 15 of the tile
// (one 8-byte load; the 16 elements lie in one 64-element block), writes the
// 16 values to an LDS tile, and the tile leaves as 16-byte stores in which
// consecutive lanes write consecutive addresses (each store instruction of
// the workgroup covers 4 KB contiguously).  Two LDS tiles alternate, so one
// barrier per tile suffices.  The ragged end of the section (n not a
// multiple of 4096) is decoded element by element.
constexpr int kDecTile = kThreads * 16;

template <bool DQ>
__global__ __launch_bounds__(kThreads) void quant_decode_kernel(
    uint64_t n, bool vec_ok, const float *__restrict__ scales_f32, const uint8_t *__restrict__ scales_u8,
    const float *__restrict__ dq_ptr, const uint8_t *__restrict__ codes, float *__restrict__ out) {
    constexpr float Lc[16] = BSQ_NF4_LEVELS;
    __shared__ float L[16];
    __shared__ __attribute__((aligned(16))) float tile[2][kDecTile];
    if (threadIdx.x < 16) L[threadIdx.x] = Lc[threadIdx.x];
    __syncthreads();
    float dq = 1.0f;
    if constexpr (DQ) dq = dq_effective(*dq_ptr);
    auto scale_of = [&](uint64_t b) {
        float s;
        if constexpr (DQ) s = dq * e4m3_decode(scales_u8[b]);
        else s = scales_f32[b];
        return (s == 0.0f || !__builtin_isfinite(s)) ? 1.0f : s;
    };
    const uint64_t ntiles = vec_ok ? n / kDecTile : 0;
    int buf = 0;
    for (uint64_t t = blockIdx.x; t < ntiles; t += gridDim.x, buf ^= 1) {
        const uint64_t e0 = t * kDecTile + 16ull * threadIdx.x;
        const uint2 w = *reinterpret_cast<const uint2 *>(codes + e0 / 2);
        const float s = scale_of(e0 / kQuantBlock);
        float *dst = tile[buf] + 16 * threadIdx.x;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t word = h ? w.y : w.x;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint32_t b0 = (word >> (16 * q)) & 0xFFu, b1 = (word >> (16 * q + 8)) & 0xFFu;
                *reinterpret_cast<float4 *>(dst + 8 * h + 4 * q) =
                    float4{s * L[b0 >> 4], s * L[b0 & 15u], s * L[b1 >> 4], s * L[b1 & 15u]};
            }
        }
        __syncthreads();
        float4 *o = reinterpret_cast<float4 *>(out + t * kDecTile);
        const float4 *src = reinterpret_cast<const float4 *>(tile[buf]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // non-temporal: the output is not read again here
            const float4 v = src[threadIdx.x + kThreads * j];
            __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4 *>(o + threadIdx.x + kThreads * j));
        }
        // the next tile writes the other buffer; this one is reused two
        // tiles later, after the barrier of the next tile
    }
    // tail (and unaligned sections): element by element
    const uint64_t done = ntiles * kDecTile;
    for (uint64_t e = done + static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; e < n;
         e += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint8_t byte = codes[e >> 1];
        const uint32_t code = (e & 1) ? (byte & 15u) : (byte >> 4);
        out[e] = scale_of(e / kQuantBlock) * L[code];
    }
}

// Decode of a direct section fused with the top-k scatter of the decompress
// (quantization_cuda.cu:287-341, then topk_cuda_utils.cuh:132-149 for the
// error set and the outlier set, src/bitsqz_llm.cu:1373-1387): one
// workgroup per row decodes the row into LDS, adds the error set (when the
// gate word has the error flag) and then the outlier set there (indices >=
// cols skipped, as the separate scatter does), and stores the row once.
// Each element gets fl(fl(decoded + error) + outlier), as from decode +
// scatter, without the scatter's read-modify-write pass over the matrix.
// The row's top-k entries are requested before the codes are decoded.
constexpr int kRowThreads = 512;  // eight waves per row: the LDS row limits workgroups per CU

template <bool DQ>
__global__ __launch_bounds__(kRowThreads) void quant_decode_rows_kernel(
    uint32_t cols, bool vec_ok, const float *__restrict__ scales_f32, const uint8_t *__restrict__ scales_u8,
    const float *__restrict__ dq_ptr, const uint8_t *__restrict__ codes, const uint16_t *__restrict__ idx0,
    const float *__restrict__ val0, uint32_t k0, const uint32_t *__restrict__ gate0,
    const uint16_t *__restrict__ idx1, const float *__restrict__ val1, uint32_t k1, float *__restrict__ out) {
    constexpr float Lc[16] = BSQ_NF4_LEVELS;
    __shared__ float L[16];
    extern __shared__ __attribute__((aligned(16))) float row[];
    const uint32_t t = threadIdx.x;
    const uint64_t r = blockIdx.x, e0 = r * cols;
    if (t < 16) L[t] = Lc[t];
    // first entries of both sets (the common case k <= 512: all of them)
    if (gate0 && !(*gate0 & kFlagError)) k0 = 0;
    uint32_t c0 = 0xFFFFFFFFu, c1 = 0xFFFFFFFFu;
    float v0 = 0.0f, v1 = 0.0f;
    if (t < k0) {
        c0 = idx0[r * k0 + t];
        v0 = val0[r * k0 + t];
    }
    if (t < k1) {
        c1 = idx1[r * k1 + t];
        v1 = val1[r * k1 + t];
    }
    float dq = 1.0f;
    if constexpr (DQ) dq = dq_effective(*dq_ptr);
    auto scale_of = [&](uint64_t b) {
        float s;
        if constexpr (DQ) s = dq * e4m3_decode(scales_u8[b]);
        else s = scales_f32[b];
        return (s == 0.0f || !__builtin_isfinite(s)) ? 1.0f : s;
    };
    __syncthreads();  // L
    if (vec_ok) {
        // 16 elements (8 code bytes, one block scale) per lane per step
        for (uint32_t i = 16 * t; i < cols; i += 16 * kRowThreads) {
            const uint64_t e = e0 + i;
            const uint2 w = *reinterpret_cast<const uint2 *>(codes + e / 2);
            const float s = scale_of(e / kQuantBlock);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t word = h ? w.y : w.x;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const uint32_t b0 = (word >> (16 * q)) & 0xFFu, b1 = (word >> (16 * q + 8)) & 0xFFu;
                    *reinterpret_cast<float4 *>(row + i + 8 * h + 4 * q) =
                        float4{s * L[b0 >> 4], s * L[b0 & 15u], s * L[b1 >> 4], s * L[b1 & 15u]};
                }
            }
        }
    } else {
        for (uint32_t i = t; i < cols; i += kRowThreads) {
            const uint64_t e = e0 + i;
            const uint8_t byte = codes[e >> 1];
            const uint32_t code = (e & 1) ? (byte & 15u) : (byte >> 4);
            row[i] = scale_of(e / kQuantBlock) * L[code];
        }
    }
    __syncthreads();
    if (c0 < cols) row[c0] += v0;
    for (uint32_t j = t + kRowThreads; j < k0; j += kRowThreads) {
        const uint32_t c = idx0[r * k0 + j];
        if (c < cols) row[c] += val0[r * k0 + j];
    }
    __syncthreads();  // the error set lands before the outlier set
    if (c1 < cols) row[c1] += v1;
    for (uint32_t j = t + kRowThreads; j < k1; j += kRowThreads) {
        const uint32_t c = idx1[r * k1 + j];
        if (c < cols) row[c] += val1[r * k1 + j];
    }
    __syncthreads();
    if (vec_ok) {
        f32x4 *o = reinterpret_cast<f32x4 *>(out + e0);
        const f32x4 *src = reinterpret_cast<const f32x4 *>(row);
        // non-temporal: the decoded matrix is not read again here
        for (uint32_t i = t; i < cols / 4; i += kRowThreads) __builtin_nontemporal_store(src[i], o + i);
    } else {
        for (uint32_t i = t; i < cols; i += kRowThreads) out[e0 + i] = row[i];
    }
}

__global__ void nf4_code_batch_kernel(const float *__restrict__ v, uint64_t n, uint8_t *__restrict__ c) {
    __shared__ Nf4Table tab;
    nf4_table_build(tab);
    __syncthreads();
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        c[i] = static_cast<uint8_t>(nf4_code(tab, v[i]));
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
    __shared__ Nf4Table tab;
    nf4_table_build(tab);
    if (threadIdx.x < 16) h[threadIdx.x] = 0;
    __syncthreads();
    unsigned long long cs = 0;
    unsigned int hl[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) hl[i] = 0;
    for (uint64_t p = lo + static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; p < hi;
         p += static_cast<uint64_t>(gridDim.x) * kThreads) {
        const uint32_t bits = static_cast<uint32_t>(p);
        const uint32_t c = nf4_code(tab, __uint_as_float(bits));
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

// *gmax = bits of max_r row_gmax[r] (one workgroup; max is order-free).
__global__ __launch_bounds__(kThreads) void rows_gmax_kernel(const float *__restrict__ row_gmax, uint32_t rows,
                                                             uint32_t *__restrict__ gmax) {
    __shared__ float red[kThreads / 64];
    float m = 0.0f;
    for (uint32_t i = threadIdx.x; i < rows; i += kThreads) m = fmaxf(m, row_gmax[i]);
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) *gmax = __float_as_uint(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
}

unsigned grid_for(uint64_t work_items, unsigned per_cu = 8) {
    const uint64_t want = ceil_div(work_items, kThreads);
    const uint64_t cap = static_cast<uint64_t>(cu_count()) * per_cu;
    return static_cast<unsigned>(want < 1 ? 1 : (want < cap ? want : cap));
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }


}  // namespace

void launch_nf4dq_gmax(const float *x, uint64_t n, uint8_t *codes, uint32_t *gmax, hipStream_t stream) {
    BSQ_REQUIRE(n > 0 && x && codes && gmax, "NF4_DQ global scale: bad arguments");
    const bool vec_ok = aligned16(x) && ((reinterpret_cast<uintptr_t>(codes) & 3u) == 0);
    const unsigned grid = grid_for(ceil_div(n, 8));
    // the workgroup maxima go to the start of the code buffer, which the
    // encode overwrites afterwards (ceil(n / 2) bytes hold 4 bytes for each
    // of the at most n / 2048 workgroups), and one workgroup reduces them: no
    // allocation, and no device-scope atomics on one word (those serialise
    // across the XCDs, which held this pass to one workgroup per CU and
    // ~4 TB/s)
    uint32_t *partial = reinterpret_cast<uint32_t *>(codes);
    if ((reinterpret_cast<uintptr_t>(codes) & 3u) == 0 && 4ull * grid <= ceil_div(n, 2)) {
        dq_gmax_kernel<true><<<grid, kThreads, 0, stream>>>(x, n, vec_ok, partial);
        rows_gmax_kernel<<<1, kThreads, 0, stream>>>(reinterpret_cast<const float *>(partial), grid, gmax);
    } else {  // a code buffer that cannot hold aligned words: one workgroup per CU, atomics
        BSQ_HIP(hipMemsetAsync(gmax, 0, sizeof(uint32_t), stream));
        dq_gmax_kernel<false><<<grid_for(ceil_div(n, 8), 1), kThreads, 0, stream>>>(x, n, vec_ok, gmax);
    }
    BSQ_HIP(hipGetLastError());
}

void launch_rows_gmax(const float *row_gmax, uint32_t rows, uint32_t *gmax, hipStream_t stream) {
    BSQ_REQUIRE(row_gmax && rows > 0 && gmax, "NF4_DQ global scale: bad arguments");
    rows_gmax_kernel<<<1, kThreads, 0, stream>>>(row_gmax, rows, gmax);
    BSQ_HIP(hipGetLastError());
}

namespace {
// one chunk per thread until the grid reaches its cap (small sections keep
// every CU busy); the unrolled loop then covers the rest.  The cap is the
// variant's occupancy in workgroups per CU (five or six: 80 to 90
// registers), so every workgroup is resident from the start: eight per CU
// ran as a round of five and a round of three (supplement encode 54.5 ->
// 50.5 us).
template <bool DQ, bool SEL>
unsigned encode_grid(uint64_t n) {
    static const unsigned per_cu = [] {
        int b = 0;
        BSQ_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &b, reinterpret_cast<const void *>(quant_encode_kernel<DQ, SEL>), kThreads, 0));
        return static_cast<unsigned>(b > 0 ? b : 1);
    }();
    return grid_for(ceil_div(n, 8), per_cu);
}

template <bool DQ>
void encode_pass(const float *x, uint64_t n, float *scales_f32, uint8_t *scales_u8, const uint32_t *gmax,
                 float *dq_out, uint8_t *codes, uint32_t *flags_reset, const uint8_t *sel, hipStream_t stream,
                 const float *row_gmax = nullptr, uint32_t gmax_rows = 0) {
    const bool vec_ok = aligned16(x) && ((reinterpret_cast<uintptr_t>(codes) & 3u) == 0);
    const unsigned grid = sel ? encode_grid<DQ, true>(n) : encode_grid<DQ, false>(n);
    BSQ_REQUIRE(!sel || n % kQuantBlock == 0, "quant encode: a selection bitmap needs whole blocks");
    BSQ_REQUIRE(!row_gmax || (DQ && gmax_rows > 0 && gmax_rows % 4 == 0 && gmax_rows <= kInlineGmaxRows &&
                              aligned16(row_gmax)),
                "quant encode: per-row maxima outside the in-kernel reduction's limits");
    if (sel)
        quant_encode_kernel<DQ, true><<<grid, kThreads, 0, stream>>>(x, n, vec_ok, scales_f32, scales_u8, gmax,
                                                                     row_gmax, gmax_rows, dq_out, codes,
                                                                     flags_reset, sel);
    else
        quant_encode_kernel<DQ, false><<<grid, kThreads, 0, stream>>>(x, n, vec_ok, scales_f32, scales_u8, gmax,
                                                                      row_gmax, gmax_rows, dq_out, codes,
                                                                      flags_reset, nullptr);
    BSQ_HIP(hipGetLastError());
}
}  // namespace

void launch_quant_encode(const float *x, uint64_t n, int method, float *scales_f32, uint8_t *scales_u8,
                         float *dq_out, uint8_t *codes, uint32_t *gmax_scratch, hipStream_t stream,
                         uint32_t *flags_reset, const uint8_t *sel) {
    BSQ_REQUIRE(n > 0, "quant encode: empty input");
    if (method == kMethodNF4) {
        BSQ_REQUIRE(scales_f32 && codes, "quant encode: null NF4 output");
        encode_pass<false>(x, n, scales_f32, nullptr, nullptr, nullptr, codes, flags_reset, sel, stream);
    } else if (method == kMethodNF4DQ) {
        BSQ_REQUIRE(scales_u8 && codes && dq_out && gmax_scratch, "quant encode: null NF4_DQ output");
        // the global scale pass reads x itself: the selected entries would count
        BSQ_REQUIRE(!sel, "quant encode: NF4_DQ with a selection bitmap takes the per-row maxima");
        launch_nf4dq_gmax(x, n, codes, gmax_scratch, stream);
        encode_pass<true>(x, n, nullptr, scales_u8, gmax_scratch, dq_out, codes, flags_reset, nullptr, stream);
    } else {
        fail("quant encode: unsupported method");
    }
    BSQ_HIP(hipGetLastError());
}


void launch_quant_encode_dq_rows(const float *x, uint64_t n, const float *row_gmax, uint32_t rows,
                                 uint8_t *scales_u8, float *dq_out, uint8_t *codes, uint32_t *gmax_scratch,
                                 hipStream_t stream, const uint8_t *sel) {
    BSQ_REQUIRE(n > 0 && rows > 0 && row_gmax && scales_u8 && codes && dq_out && gmax_scratch,
                "quant encode: bad NF4_DQ arguments");
    if (rows <= kInlineGmaxRows && rows % 4 == 0 && aligned16(row_gmax)) {
        // few enough maxima: the encode's workgroups reduce them, no launch
        encode_pass<true>(x, n, nullptr, scales_u8, nullptr, dq_out, codes, nullptr, sel, stream, row_gmax, rows);
        return;
    }
    rows_gmax_kernel<<<1, kThreads, 0, stream>>>(row_gmax, rows, gmax_scratch);
    BSQ_HIP(hipGetLastError());
    encode_pass<true>(x, n, nullptr, scales_u8, gmax_scratch, dq_out, codes, nullptr, sel, stream);
}

void launch_quant_decode(uint64_t n, int method, const float *scales_f32, const uint8_t *scales_u8,
                         const float *dq, const uint8_t *codes, float *out, hipStream_t stream) {
    BSQ_REQUIRE(n > 0, "quant decode: empty output");
    const bool vec_ok = aligned16(out) && ((reinterpret_cast<uintptr_t>(codes) & 7u) == 0);
    const unsigned grid = grid_for(ceil_div(n, 16), 16);  // 16 per CU: more loads in flight than 8 gave
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

bool quant_decode_rows_supported(uint32_t rows, uint32_t cols) {
    return rows > 0 && cols > 0 && cols <= kDecodeRowsMaxCols;
}

void launch_quant_decode_rows(uint32_t rows, uint32_t cols, int method, const float *scales_f32,
                              const uint8_t *scales_u8, const float *dq, const uint8_t *codes,
                              const uint16_t *idx0, const float *val0, uint32_t k0, const uint32_t *gate0,
                              const uint16_t *idx1, const float *val1, uint32_t k1, float *out,
                              hipStream_t stream) {
    BSQ_REQUIRE(quant_decode_rows_supported(rows, cols) && codes && out, "row decode: bad arguments");
    BSQ_REQUIRE((k0 == 0 || (idx0 && val0)) && (k1 == 0 || (idx1 && val1)), "row decode: null top-k list");
    // 16-element steps: rows start on 16 elements, 8-byte code and 16-byte
    // output alignment
    const bool vec_ok = cols % 16 == 0 && ((reinterpret_cast<uintptr_t>(codes) & 7u) == 0) && aligned16(out);
    const size_t lds = static_cast<size_t>(cols) * sizeof(float);
    auto go = [&](auto kern) {
        BSQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(lds)));
        kern<<<rows, kRowThreads, lds, stream>>>(cols, vec_ok, scales_f32, scales_u8, dq, codes, idx0, val0, k0, gate0,
                                              idx1, val1, k1, out);
    };
    if (method == kMethodNF4) {
        BSQ_REQUIRE(scales_f32, "row decode: null NF4 scales");
        go(quant_decode_rows_kernel<false>);
    } else if (method == kMethodNF4DQ) {
        BSQ_REQUIRE(scales_u8 && dq, "row decode: null NF4_DQ scales");
        go(quant_decode_rows_kernel<true>);
    } else {
        fail("row decode: unsupported method");
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
