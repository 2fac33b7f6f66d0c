// Reconstruction from NF4 / NF4_DQ factors on the gfx950 matrix cores
// (reference modules/reconstruct_lowrank_cuda/src/reconstruct_lowrank_cuda.cu:
// 21-62 with the decode of modules/quantization_cuda/src/
// quantization_cuda.cu:287-341 inline): out = U diag(S) V^T from the packed
// U (m x q) and V (n x q), the decompress side's reconstruction.
//
// U and V stay in their packed form: one workgroup per 128 x 128 output tile
// copies the nibbles of its 128 rows of U and of V (and their block scales)
// into LDS once, and every slice of the K loop decodes its MFMA operand
// fragments from there (two codes per 256-entry level-pair lookup), so the
// main loop reads no global memory and needs no barrier.  Each value is
// decoded exactly as the standalone decoder writes it (scale * L[code], the
// scale guarded as there), then scaled by S[k], and the lane / k order of the
// MFMA products is that of the FP32 reconstruction GEMM, so the output is
// bit-identical to decoding U and V and reconstructing.  The top-k sets are
// scatter-added afterwards by topk_scatter_kernel, error set first.
#include "bsq_internal.hpp"
#include "tile_map.hpp"

namespace bsq {
namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int TT = 128, BK = 16, KS = 4;

struct QFactor {
    const uint8_t *codes = nullptr;       // rows x K nibbles, two per byte, element 2j in the high nibble
    const float *scales_f32 = nullptr;    // NF4: one per 64 elements
    const uint8_t *scales_u8 = nullptr;   // NF4_DQ: E4M3 code per 64 elements
    const float *dq = nullptr;            // NF4_DQ: the section's global scale
};

struct ReconQArgs {
    QFactor u, v;
    const float *s = nullptr;           // S (K), FP32
    float *out = nullptr;               // M x N row-major
    int M = 0, N = 0, K = 0;
};

__device__ __forceinline__ float e4m3_value(uint32_t v) {
    // quantization_cuda.cu:111-128 (nf4_dq_impl.cpp:104-129)
    const uint32_t ef = (v >> 3) & 15u, mf = v & 7u;
    float r;
    if (ef == 0) r = (static_cast<float>(mf) / 8.0f) * 0.015625f;
    else r = (1.0f + static_cast<float>(mf) / 8.0f) * __builtin_ldexpf(1.0f, static_cast<int>(ef) - 7);
    return (v & 0x80u) ? -r : r;
}

// Block scale b of a factor, as the decoder computes it (quantization_cuda.cu:
// 300-305, 322-332): NF4 the stored scale, NF4_DQ dq * E4M3(code); 0 or a
// non-finite value becomes 1.  `dq` is already guarded the same way.
template <bool DQ>
__device__ __forceinline__ float block_scale(const QFactor &f, uint64_t b, float dq) {
    float s;
    if constexpr (DQ) s = dq * e4m3_value(f.scales_u8[b]);
    else s = f.scales_f32[b];
    return (s == 0.0f || !__builtin_isfinite(s)) ? 1.0f : s;
}

__device__ __forceinline__ float guarded_dq(const float *p) {
    const float dq = *p;
    return (dq == 0.0f || !__builtin_isfinite(dq)) ? 1.0f : dq;
}

// LDS layout of one workgroup (bytes): codes of the tile's U rows and V rows
// (row pitch K/2 + 16: 16-byte aligned rows that start four banks apart),
// their block scales as floats, S, and the table of level pairs
// L2[b] = (L[b >> 4], L[b & 15]).  The epilogue's staging of the output
// (32 x 64 floats per wave) reuses the start of the block.
struct Layout {
    int pitch, cA, cB, sA, sB, sv, l2, bytes;
    __host__ __device__ explicit Layout(int K) {
        pitch = K / 2 + 16;
        cA = 0;
        cB = cA + TT * pitch;
        sA = cB + TT * pitch;
        sB = sA + TT * (K / 64) * 4;
        sv = sB + TT * (K / 64) * 4;
        l2 = sv + K * 4;
        bytes = l2 + 256 * 8;
        if (bytes < 4 * 32 * 64 * 4) bytes = 4 * 32 * 64 * 4;
    }
};

// Codes (uint4 chunks, row by row) and block scales of rows r0 .. r0 + rows - 1
// of a factor into LDS; rows past the factor are left alone (their products
// only reach output rows or columns that are never stored).
template <bool DQ>
__device__ __forceinline__ void stage_factor(const QFactor &f, int r0, int rows, int K, unsigned char *smem,
                                             int c_off, int s_off, int pitch, float dq) {
    const int chunks = K / 32;  // 16-byte chunks per row
    const uint4 *src = reinterpret_cast<const uint4 *>(f.codes + static_cast<uint64_t>(r0) * (K / 2));
    for (int i = threadIdx.x; i < rows * chunks; i += kThreads) {
        const int r = i / chunks, c = i - r * chunks;
        *reinterpret_cast<uint4 *>(smem + c_off + r * pitch + 16 * c) = src[static_cast<uint64_t>(r) * chunks + c];
    }
    const int nb = K / 64;
    float *sc = reinterpret_cast<float *>(smem + s_off);
    const uint64_t b0 = static_cast<uint64_t>(r0) * nb;
    for (int i = threadIdx.x; i < rows * nb; i += kThreads) sc[i] = block_scale<DQ>(f, b0 + i, dq);
}

// Four consecutive elements k .. k + 3 (k % 4 == 0) of row `row`, decoded:
// one 2-byte code read, two level-pair lookups, the block scale.
__device__ __forceinline__ void decode4(const unsigned char *smem, int c_off, int s_off, int pitch, int K, int row,
                                        int k, const float2 *L2, float (&o)[KS]) {
    const uint32_t h = *reinterpret_cast<const uint16_t *>(smem + c_off + row * pitch + (k >> 1));
    const float sc = reinterpret_cast<const float *>(smem + s_off)[row * (K / 64) + (k >> 6)];
    const float2 l01 = L2[h & 0xFFu], l23 = L2[h >> 8];
    o[0] = sc * l01.x;
    o[1] = sc * l01.y;
    o[2] = sc * l23.x;
    o[3] = sc * l23.y;
}

template <bool DQ>
__global__ __launch_bounds__(kThreads) void recon_q_kernel(ReconQArgs g) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int K = g.K;
    const Layout lay(K);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * 64, wn0 = (wave & 1) * 64;
    int tile_m, tile_n, z;
    const int ny = static_cast<int>(ceil_div(g.M, TT)), nx = static_cast<int>(ceil_div(g.N, TT));
    xcd_tile(ny, nx, 1, tile_m, tile_n, z);
    const int m0 = tile_m * TT, n0 = tile_n * TT;

    float dqa = 1.0f, dqb = 1.0f;
    if constexpr (DQ) {
        dqa = guarded_dq(g.u.dq);
        dqb = guarded_dq(g.v.dq);
    }
    stage_factor<DQ>(g.u, m0, min(TT, g.M - m0), K, smem, lay.cA, lay.sA, lay.pitch, dqa);
    stage_factor<DQ>(g.v, n0, min(TT, g.N - n0), K, smem, lay.cB, lay.sB, lay.pitch, dqb);
    float *Sv = reinterpret_cast<float *>(smem + lay.sv);
    for (int k = tid; k < K; k += kThreads) Sv[k] = g.s[k];
    float2 *L2 = reinterpret_cast<float2 *>(smem + lay.l2);
    {
        constexpr float Lc[16] = BSQ_NF4_LEVELS;
        L2[tid] = float2{Lc[tid >> 4], Lc[tid & 15]};  // 256 threads, 256 pairs
    }
    __syncthreads();

    f32x4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

    const int kk = lane >> 4, cc = lane & 15;
    for (int j = 0; j < K / BK; ++j) {
        const int kb = j * BK + KS * kk;  // this lane's four k values
        const float4 s4 = *reinterpret_cast<const float4 *>(Sv + kb);
        float a[4][KS], b[4][KS];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            decode4(smem, lay.cA, lay.sA, lay.pitch, K, wm0 + i * 16 + cc, kb, L2, a[i]);
            a[i][0] *= s4.x;
            a[i][1] *= s4.y;
            a[i][2] *= s4.z;
            a[i][3] *= s4.w;
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) decode4(smem, lay.cB, lay.sB, lay.pitch, K, wn0 + jj * 16 + cc, kb, L2, b[jj]);
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][s2], b[jj][s2], acc[i][jj], 0, 0, 0);
    }

    // epilogue: every wave leaves with its own 64 x 64 block through its own
    // 8 KB of LDS in two 32-row passes (16-byte stores; columns XOR-swizzled
    // by 16 on alternate groups of four rows), after one barrier (the codes
    // are consumed)
    const bool vec_out = ((g.N & 3) == 0) && ((reinterpret_cast<uintptr_t>(g.out) & 15u) == 0);
    __syncthreads();
    float *Cw = reinterpret_cast<float *>(smem) + wave * (32 * 64);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rl = 16 * ii + 4 * (lane >> 4) + r, col = 16 * jj + (lane & 15);
                    Cw[rl * 64 + (col ^ (16 * ((rl >> 2) & 1)))] = acc[2 * h + ii][jj][r];
                }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int rl = 4 * q + (lane >> 4), c4 = 4 * (lane & 15);
            const int gi = m0 + wm0 + 32 * h + rl, gj = n0 + wn0 + c4;
            if (gi >= g.M) continue;
            const float4 v = *reinterpret_cast<const float4 *>(&Cw[rl * 64 + (c4 ^ (16 * ((rl >> 2) & 1)))]);
            const uint64_t e = static_cast<uint64_t>(gi) * g.N + gj;
            if (vec_out && gj + 4 <= g.N) {
                *reinterpret_cast<float4 *>(g.out + e) = v;
            } else {
                const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (gj + u < g.N) g.out[e + u] = vv[u];
            }
        }
    }
}

template <bool DQ>
void launch_q(const ReconQArgs &g, size_t lds, hipStream_t stream) {
    auto kern = recon_q_kernel<DQ>;
    BSQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(lds)));
    const unsigned grid = static_cast<unsigned>(ceil_div(g.M, TT) * ceil_div(g.N, TT));
    kern<<<grid, kThreads, lds, stream>>>(g);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool recon_q_supported(int m, int n, int k, const uint8_t *u_codes, const uint8_t *v_codes) {
    return m > 0 && n > 0 && k >= 64 && k <= kReconQMaxK && k % 64 == 0 && aligned16(u_codes) &&
           aligned16(v_codes);
}

void launch_recon_q(int method, const uint8_t *u_codes, const float *u_scales_f32, const uint8_t *u_scales_u8,
                    const float *u_dq, const uint8_t *v_codes, const float *v_scales_f32, const uint8_t *v_scales_u8,
                    const float *v_dq, const float *S, int m, int n, int k, float *out, hipStream_t stream) {
    BSQ_REQUIRE(recon_q_supported(m, n, k, u_codes, v_codes) && S && out, "packed reconstruct: bad arguments");
    BSQ_REQUIRE(method == kMethodNF4 || method == kMethodNF4DQ, "packed reconstruct: factors are not NF4 / NF4_DQ");
    const bool dq = method == kMethodNF4DQ;
    BSQ_REQUIRE(dq ? (u_scales_u8 && v_scales_u8 && u_dq && v_dq) : (u_scales_f32 && v_scales_f32),
                "packed reconstruct: missing block scales");
    ReconQArgs g;
    g.u = QFactor{u_codes, u_scales_f32, u_scales_u8, u_dq};
    g.v = QFactor{v_codes, v_scales_f32, v_scales_u8, v_dq};
    g.s = S;
    g.out = out;
    g.M = m;
    g.N = n;
    g.K = k;
    const size_t lds = static_cast<size_t>(Layout(k).bytes);
    if (dq) launch_q<true>(g, lds, stream);
    else launch_q<false>(g, lds, stream);
    BSQ_HIP(hipGetLastError());
}

}  // namespace bsq
