// FP32 GEMM on the gfx950 matrix cores (v_mfma_f32_16x16x4_f32).
//
//   C[M x N] = op(A)[M x K] * op(B)[K x N]   (row-major storage everywhere)
//     op(A) = A          (TA = false, A is M x K, lda >= K)
//           = A^T        (TA = true,  A is K x M, lda >= M)
//     op(B) = B          (TB = false, B is K x N, ldb >= N)
//           = B^T        (TB = true,  B is N x K, ldb >= K)
//
// Used for the randomised range finder (X = op(A) R, Y = op(A)^T X with the
// big activation matrix read row-major in place, so no transposed copy is
// ever made), the small basis rotations (X * W) and the low-rank
// reconstruction U diag(S) V^T, which scales the A fragments by S (fetched a
// slice ahead with the operand tiles) and can subtract from a minuend in the
// epilogue (error = residual - U S V^T).
//
// Tiling: 256 threads = 4 waves in a 2 x 2 grid; workgroup tile 128 x 128,
// BK = 16; each wave owns 64 x 64 as 4 x 4 MFMA 16x16 blocks (64 AGPRs).
// Three main loops share that tiling:
//   gemm_dma_kernel     operand tiles go global -> LDS directly
//                       (global_load_lds_dwordx4) through a ring of four
//                       slices, three in flight while one is multiplied;
//   gemm_streamk_kernel the same ring in a persistent grid that splits
//                       tiles x K slices evenly over two workgroups per CU;
//   gemm_mfma_kernel    the fallback for shapes the DMA layout does not take
//                       (K not a multiple of 16, unaligned operands): tiles
//                       move global -> registers -> LDS one slice ahead.
// All use the same k order per lane, so for the same K partition their
// results are identical.  Skinny shapes are split along K so the grid fills
// the 256 CUs several times over (stream-K on the DMA path when the split
// grid is not a whole number of rounds); partial products go to a workspace
// summed in a fixed order, so results are deterministic.
#include "bsq_internal.hpp"
#include "tile_map.hpp"

namespace bsq {
namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 16;
constexpr int KS = BK / 4;  // k-values per lane per slice

struct GemmArgs {
    const float *A;
    const float *B;
    float *C;                 // output (or split-K workspace base)
    const float *a_colscale;  // optional: op(A)[:, kk] *= a_colscale[kk]
    const float *minuend;     // optional: C = minuend - acc (ldc layout)
    int M, N, K;
    int lda, ldb, ldc;
    int k_per_split;          // K range of one split (multiple of BK)
    int splits;               // K ranges, i.e. work items per output tile
    uint64_t split_stride;    // elements between split-K partial outputs
    bool vec_a, vec_b;        // 16-byte loads allowed (alignment of base and leading dim)
};

// LDS tile layouts.  The 16x16x4 MFMA takes, in lane l = 16 kk + i, the
// operand element (row / column i, k), and the k order inside a BK slice is
// free as long as both operands use the same one.  Lane kk takes
// k = KS kk + s at MFMA step s (s = 0..KS-1, KS = BK / 4 = 4), so:
//   k-contiguous tiles (A with TA = false, B with TB = true) are kept as
//   [row][k] (pitch 20 floats): a lane's KS k-values of a fragment are one
//   16-byte read, and the rows of 16 lanes start 20 banks apart; the global
//   tile is stored as loaded (16-byte LDS writes);
//   k-major tiles (A with TA = true, B with TB = false) are kept as [k][col]
//   (pitch R + 4): one 4-byte read per step, 16-byte LDS writes.
constexpr int PK = BK + 4;

// k-contiguous operand tile: R rows x BK k-values.  256 threads: thread t
// covers row (t % R) + R * pass, k quad (t / R) (BK / 4 quads per row).
template <int R>
struct KContig {
    static constexpr int N4 = R * BK / 4 / kThreads;  // float4 per thread
    using Tile = float[R][PK];
    float4 v[N4];
    __device__ __forceinline__ void load(const float *__restrict__ P, int ld, int r0, int rows, int k0, int kend,
                                         bool vec, const float *__restrict__ colscale) {
        const int t = threadIdx.x;
#pragma unroll
        for (int q = 0; q < N4; ++q) {
            const int lin = t + q * kThreads;  // 0 .. R * BK / 4 - 1
            const int r = lin % R, kq = lin / R;
            const int gr = r0 + r, gk = k0 + kq * 4;
            float4 x;
            if (vec && gr < rows && gk + 4 <= kend) {
                x = *reinterpret_cast<const float4 *>(P + static_cast<uint64_t>(gr) * ld + gk);
            } else {
                const float *row = P + static_cast<uint64_t>(gr) * ld;
                x.x = (gr < rows && gk + 0 < kend) ? row[gk + 0] : 0.0f;
                x.y = (gr < rows && gk + 1 < kend) ? row[gk + 1] : 0.0f;
                x.z = (gr < rows && gk + 2 < kend) ? row[gk + 2] : 0.0f;
                x.w = (gr < rows && gk + 3 < kend) ? row[gk + 3] : 0.0f;
            }
            if (colscale) {
                x.x *= (gk + 0 < kend) ? colscale[gk + 0] : 0.0f;
                x.y *= (gk + 1 < kend) ? colscale[gk + 1] : 0.0f;
                x.z *= (gk + 2 < kend) ? colscale[gk + 2] : 0.0f;
                x.w *= (gk + 3 < kend) ? colscale[gk + 3] : 0.0f;
            }
            v[q] = x;
        }
    }
    __device__ __forceinline__ void store(Tile &S) const {
        const int t = threadIdx.x;
#pragma unroll
        for (int q = 0; q < N4; ++q) {
            const int lin = t + q * kThreads;
            *reinterpret_cast<float4 *>(&S[lin % R][(lin / R) * 4]) = v[q];
        }
    }
    // the KS k-values (k = KS kk + s) of row `row` for this lane
    __device__ __forceinline__ static void frag(const Tile &S, int row, int kk, float (&o)[KS]) {
        const float4 lo = *reinterpret_cast<const float4 *>(&S[row][4 * kk]);
        o[0] = lo.x;
        o[1] = lo.y;
        o[2] = lo.z;
        o[3] = lo.w;
    }
};

// k-major operand tile: BK k-rows x Cn contiguous values.
template <int Cn>
struct KMajor {
    static constexpr int N4 = Cn * BK / 4 / kThreads;
    using Tile = float[BK][Cn + 4];
    float4 v[N4];
    __device__ __forceinline__ void load(const float *__restrict__ P, int ld, int c0, int cols, int k0, int kend,
                                         bool vec, const float *__restrict__ rowscale) {
        const int t = threadIdx.x;
        constexpr int C4 = Cn / 4;
#pragma unroll
        for (int q = 0; q < N4; ++q) {
            const int lin = t + q * kThreads;
            const int c = (lin % C4) * 4, kk = lin / C4;
            const int gc = c0 + c, gk = k0 + kk;
            float4 x;
            const float *row = P + static_cast<uint64_t>(gk) * ld;
            if (vec && gk < kend && gc + 4 <= cols) {
                x = *reinterpret_cast<const float4 *>(row + gc);
            } else {
                x.x = (gk < kend && gc + 0 < cols) ? row[gc + 0] : 0.0f;
                x.y = (gk < kend && gc + 1 < cols) ? row[gc + 1] : 0.0f;
                x.z = (gk < kend && gc + 2 < cols) ? row[gc + 2] : 0.0f;
                x.w = (gk < kend && gc + 3 < cols) ? row[gc + 3] : 0.0f;
            }
            if (rowscale) {
                const float sc = (gk < kend) ? rowscale[gk] : 0.0f;
                x.x *= sc;
                x.y *= sc;
                x.z *= sc;
                x.w *= sc;
            }
            v[q] = x;
        }
    }
    __device__ __forceinline__ void store(Tile &S) const {
        const int t = threadIdx.x;
        constexpr int C4 = Cn / 4;
#pragma unroll
        for (int q = 0; q < N4; ++q) {
            const int lin = t + q * kThreads;
            *reinterpret_cast<float4 *>(&S[lin / C4][(lin % C4) * 4]) = v[q];
        }
    }
    __device__ __forceinline__ static void frag(const Tile &S, int col, int kk, float (&o)[KS]) {
#pragma unroll
        for (int s = 0; s < KS; ++s) o[s] = S[KS * kk + s][col];
    }
};


// RECON: the low-rank reconstruction form (column scale on op(A), optional
// minuend), instantiated separately so the power-iteration GEMMs carry no
// epilogue branches and profiles tell the two apart.
template <bool TA, bool TB, bool RECON>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(GemmArgs g) {
    constexpr int WM = BM / 2, WN = BN / 2;  // wave tile
    constexpr int FM = WM / 16, FN = WN / 16;
    using TileA = typename std::conditional<TA, KMajor<BM>, KContig<BM>>::type;
    using TileB = typename std::conditional<TB, KContig<BN>, KMajor<BN>>::type;
    // one LDS block: the double-buffered operand tiles, reused by the
    // reconstruction epilogue to stage the output tile
    constexpr size_t kABytes = 2 * sizeof(typename TileA::Tile), kBBytes = 2 * sizeof(typename TileB::Tile);
    constexpr size_t kCBytes = RECON ? sizeof(float) * (BM / 2) * (BN + 4) : 0;
    constexpr size_t kSmem = (kABytes + kBBytes > kCBytes) ? kABytes + kBBytes : kCBytes;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kSmem];
    typename TileA::Tile *As = reinterpret_cast<typename TileA::Tile *>(smem);
    typename TileB::Tile *Bs = reinterpret_cast<typename TileB::Tile *>(smem + kABytes);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    int tile_m, tile_n, zs;
    xcd_tile(ceil_div(g.M, BM), ceil_div(g.N, BN), g.splits, tile_m, tile_n, zs);
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int kbeg = zs * g.k_per_split;
    const int kend = min(g.K, kbeg + g.k_per_split);

    f32x4v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

    TileA ta;
    TileB tb;
    auto load = [&](int k0) {
        ta.load(g.A, g.lda, m0, g.M, k0, kend, g.vec_a, nullptr);
        tb.load(g.B, g.ldb, n0, g.N, k0, kend, g.vec_b, nullptr);
    };

    int buf = 0;
    const int kk = lane >> 4, cc = lane & 15;
    // RECON: op(A)[:, k] *= colscale[k] on this lane's KS k-values
    // (k = k0 + KS kk + s), fetched one slice ahead with the operand tiles
    float sc[KS];
    auto load_scale = [&](int k0) {
        if constexpr (RECON) {
#pragma unroll
            for (int st = 0; st < KS; ++st) {
                const int kx = k0 + KS * kk + st;
                sc[st] = (g.a_colscale && kx < kend) ? g.a_colscale[kx] : 1.0f;
            }
        }
    };
    if (kbeg < kend) {
        load(kbeg);
        load_scale(kbeg);
        ta.store(As[0]);
        tb.store(Bs[0]);
    }
    __syncthreads();
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
        const bool more = k0 + BK < kend;
        float a[FM][KS], b[FN][KS];
#pragma unroll
        for (int i = 0; i < FM; ++i) TileA::frag(As[buf], wm0 + i * 16 + cc, kk, a[i]);
        if constexpr (RECON) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int st = 0; st < KS; ++st) a[i][st] *= sc[st];
        }
        if (more) {
            load(k0 + BK);
            load_scale(k0 + BK);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) TileB::frag(Bs[buf], wn0 + j * 16 + cc, kk, b[j]);
#pragma unroll
        for (int st = 0; st < KS; ++st)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][st], b[j][st], acc[i][j], 0, 0, 0);
        if (more) {
            ta.store(As[buf ^ 1]);
            tb.store(Bs[buf ^ 1]);
        }
        __syncthreads();
        buf ^= 1;
    }

    // epilogue: fragment (i, j) register r holds row 4*(lane/16) + r, column lane % 16
    float *C = g.C + static_cast<uint64_t>(zs) * g.split_stride;
    if constexpr (RECON) {
        // the reconstruction writes (and may subtract from) a full m x n matrix:
        // stage the tile through LDS (the operand buffers are free now) in two
        // 64-row halves so that rows leave as 16-byte stores and the minuend
        // arrives as 16-byte loads, issued before the staging
        constexpr int CP = BN + 4, HM = BM / 2;
        float(*Cs)[CP] = reinterpret_cast<float(*)[CP]>(smem);
        constexpr int Q = HM * BN / 4 / kThreads;  // float4 per thread per half
        const bool vec_c = ((g.ldc & 3) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15u) == 0) &&
                           (!g.minuend || (reinterpret_cast<uintptr_t>(g.minuend) & 15u) == 0);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float4 mv[Q];
            if (g.minuend && vec_c) {
#pragma unroll
                for (int q = 0; q < Q; ++q) {
                    const int lin = tid + q * kThreads, rr = h * HM + lin / (BN / 4), c4 = lin % (BN / 4);
                    const int gi = m0 + rr, gj = n0 + 4 * c4;
                    mv[q] = (gi < g.M && gj + 4 <= g.N)
                                ? *reinterpret_cast<const float4 *>(g.minuend + static_cast<uint64_t>(gi) * g.ldc + gj)
                                : float4{0.f, 0.f, 0.f, 0.f};
                }
            }
            __syncthreads();  // the operand tiles (h = 0) or the previous half (h = 1) are consumed
            if (wm0 == h * HM) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            Cs[i * 16 + 4 * (lane >> 4) + r][wn0 + j * 16 + (lane & 15)] = acc[i][j][r];
            }
            __syncthreads();
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const int lin = tid + q * kThreads, rl = lin / (BN / 4), c4 = lin % (BN / 4);
                const int gi = m0 + h * HM + rl, gj = n0 + 4 * c4;
                if (gi >= g.M) continue;
                float4 v = *reinterpret_cast<const float4 *>(&Cs[rl][4 * c4]);
                const uint64_t e = static_cast<uint64_t>(gi) * g.ldc + gj;
                if (vec_c && gj + 4 <= g.N) {
                    if (g.minuend) v = float4{mv[q].x - v.x, mv[q].y - v.y, mv[q].z - v.z, mv[q].w - v.w};
                    *reinterpret_cast<float4 *>(C + e) = v;
                } else {
                    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (gj + u < g.N) C[e + u] = g.minuend ? g.minuend[e + u] - vv[u] : vv[u];
                }
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gi = m0 + wm0 + i * 16 + 4 * (lane >> 4) + r;
                const int gj = n0 + wn0 + j * 16 + (lane & 15);
                if (gi < g.M && gj < g.N) C[static_cast<uint64_t>(gi) * g.ldc + gj] = acc[i][j][r];
            }
}

// ---------------------------------------------------------------------------
// Pipelined variant: operand tiles go global -> LDS directly
// (global_load_lds_dwordx4, 16 bytes per lane, no VGPR staging) through a
// ring of kStages slices, so kStages - 1 slices are in flight while one is
// multiplied.  Each wave-instruction fills one 1 KB LDS chunk, lane l at byte
// 16 l, so the tile layouts are unpadded and XOR-swizzled at 16-byte
// granularity to keep the fragment reads free of bank conflicts:
//   k-contiguous tile (rows x 16 k): float index r*16 + 4*(q ^ f(r)) + e for
//     k = 4q + e, f(r) = (r >> 1) & 3;
//   k-major tile (16 k x 128 cols): float index kr*128 + (c ^ 16*((kr >> 2) & 1)).
// Requires K % BK == 0, 16-byte aligned bases and leading dimensions, and
// the k-major extents (M for TA, N for !TB) a multiple of 4 (rows beyond the
// matrix are clamped to its last row or quad: their outputs are discarded).
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;
constexpr int kStages = 4;
constexpr int kDmaReconMaxK = 1024;  // RECON column scales staged in LDS

__device__ __forceinline__ void dma16(const float *g, const float *l) {
    __builtin_amdgcn_global_load_lds((glb_void_t *)(g), (lds_void_t *)(reinterpret_cast<size_t>(l)), 16, 0, 0);
}
// wave-level LDS barrier that does not drain the DMA queue: waits for this
// wave's DMAs down to `pending` outstanding, then the workgroup barrier; the
// asm statements keep the compiler from moving LDS accesses across it
template <int PENDING>
__device__ __forceinline__ void dma_barrier() {
    static_assert(PENDING >= 0 && PENDING < 64, "vmcnt has six bits");
    asm volatile("" ::: "memory");
    // vmcnt(PENDING) (bits 3:0 and 15:14), expcnt/lgkmcnt untouched
    __builtin_amdgcn_s_waitcnt(0xF70 | (PENDING & 15) | ((PENDING >> 4) << 14));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// one 1 KB chunk c (0 .. T/16 - 1) of a T x 16 operand tile (T = 128 or 64)
//   k-contiguous operand [row][k]: 16 rows per chunk, 16-byte quads of a row
//     XOR-swizzled by bits 1..2 of the row;
//   k-major operand [k][col]: 1024 / (4 T) k-rows per chunk, quads of a k-row
//     XOR-swizzled so that the four k-rows one fragment read touches fall in
//     different banks.
template <bool KMAJOR, int T>
__device__ __forceinline__ int kmajor_swizzle(int kr) {  // column XOR of k-row kr
    if constexpr (T == 128) return 16 * ((kr >> 2) & 1);
    else return 16 * ((kr >> 2) & 3);
}
template <bool KMAJOR, int T>
__device__ __forceinline__ void dma_chunk(const float *__restrict__ P, int ld, int r0, int extent, int k0, int c,
                                          const float *lds_tile) {
    const int l = threadIdx.x & 63;
    if constexpr (!KMAJOR) {  // P row-major [row][k]
        const int r = 16 * c + (l >> 2);
        const int q = (l & 3) ^ ((r >> 1) & 3);
        const int gr = min(r0 + r, extent - 1);
        dma16(P + static_cast<uint64_t>(gr) * ld + k0 + 4 * q, lds_tile + c * 256);
    } else {  // P row-major [k][col]
        constexpr int QPR = T / 4;  // quads per k-row
        const int kr = (64 / QPR) * c + l / QPR;
        const int cq = (l % QPR) ^ (kmajor_swizzle<KMAJOR, T>(kr) / 4);
        const int gc = min(r0 + 4 * cq, extent - 4);
        dma16(P + static_cast<uint64_t>(k0 + kr) * ld + gc, lds_tile + c * 256);
    }
}

template <bool KMAJOR, int T>
__device__ __forceinline__ void dma_frag(const float *S, int row, int kk, float (&o)[KS]) {
    if constexpr (!KMAJOR) {
        const float4 v = *reinterpret_cast<const float4 *>(&S[row * 16 + 4 * (kk ^ ((row >> 1) & 3))]);
        o[0] = v.x;
        o[1] = v.y;
        o[2] = v.z;
        o[3] = v.w;
    } else {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int kr = 4 * kk + s;
            o[s] = S[kr * T + (row ^ kmajor_swizzle<KMAJOR, T>(kr))];
        }
    }
}

// T x T output tile (T = 128, or 64 for grids that 128-wide tiles would
// leave short of the CU count); four waves of T/2 x T/2.
template <bool TA, bool TB, bool RECON, int T>
__global__ __launch_bounds__(kThreads) void gemm_dma_kernel(GemmArgs g) {
    static_assert(T == 128 || (T == 64 && !RECON), "gemm: tile size");
    constexpr int BM = T, BN = T;
    constexpr int kTileF = T * BK;     // floats per operand tile
    constexpr int kStageF = 2 * kTileF;  // A + B
    constexpr int kChunks = T / 16;    // 1 KB DMA chunks per operand tile
    constexpr int kCpw = kChunks / 4;  // chunks per wave per operand
    constexpr int kDmaPerSlice = 2 * kCpw;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 16, FN = WN / 16;
    // one LDS object per stage: the compiler's wait insertion then sees that a
    // DMA into one stage cannot alias the fragment reads of another
    __shared__ __attribute__((aligned(1024))) float st0[kStageF];
    __shared__ __attribute__((aligned(1024))) float st1[kStageF];
    __shared__ __attribute__((aligned(1024))) float st2[kStageF];
    __shared__ __attribute__((aligned(1024))) float st3[kStageF];
    __shared__ float scs[RECON ? kDmaReconMaxK : 1];  // RECON: the column scales of op(A)

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    int tile_m, tile_n, zs;
    xcd_tile(ceil_div(g.M, BM), ceil_div(g.N, BN), g.splits, tile_m, tile_n, zs);
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int kbeg = zs * g.k_per_split;
    const int kend = min(g.K, kbeg + g.k_per_split);
    const int nk = (kend - kbeg) / BK;

    f32x4v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

    if constexpr (RECON) {
        for (int t = tid; t < kend - kbeg; t += kThreads) scs[t] = g.a_colscale ? g.a_colscale[kbeg + t] : 1.0f;
        // visible after the first barrier of the loop
    }
    // each wave issues chunks kCpw w .. kCpw w + kCpw - 1 of A and of B
    auto issue = [&](const float *st, int j) {
        const int k0 = kbeg + j * BK;
#pragma unroll
        for (int h = 0; h < kCpw; ++h) {
            const int c = kCpw * wave + h;
            dma_chunk<TA, T>(g.A, g.lda, m0, g.M, k0, c, st);
            dma_chunk<!TB, T>(g.B, g.ldb, n0, g.N, k0, c, st + kTileF);
        }
    };
    const int kk = lane >> 4, cc = lane & 15;
    // RECON: the minuend of this wave's 64 x 64 output block (16 float4 per
    // lane, in the layout the epilogue stores) is requested right after the
    // last operand slice, so it arrives while the last slices are multiplied.
    // Every lane issues all kMv loads (addresses clamped into the matrix), so
    // the waits below can count them.
    constexpr int kMv = RECON ? WM * WN / 4 / 64 : 0;
    float4 mvall[RECON ? kMv : 1];
    const bool vec_c = RECON && ((g.ldc & 3) == 0) &&
                       ((reinterpret_cast<uintptr_t>(g.C + static_cast<uint64_t>(zs) * g.split_stride) & 15u) == 0) &&
                       (!g.minuend || (reinterpret_cast<uintptr_t>(g.minuend) & 15u) == 0);
    const bool mv_on = RECON && g.minuend && vec_c && g.N >= 4;
    auto issue_minuend = [&]() {
        asm volatile("" ::: "memory");  // stays behind the last slice's DMA
#pragma unroll
        for (int q = 0; q < kMv; ++q) {
            const int gi = min(m0 + wm0 + 4 * q + (lane >> 4), g.M - 1), gj = min(n0 + wn0 + 4 * (lane & 15), g.N - 4);
            mvall[q] = *reinterpret_cast<const float4 *>(g.minuend + static_cast<uint64_t>(gi) * g.ldc + gj);
        }
        asm volatile("" ::: "memory");
    };
    // slice j sits in stage j % 4: cur holds it, nxt (= stage (j + 3) % 4, read
    // in iteration j - 1) receives slice j + 3
    auto body = [&](const float *cur, const float *nxt, int j) {
        const int ahead = min(kStages - 2, nk - 1 - j);  // slices issued after j
        if (mv_on && j + kStages - 1 >= nk) {  // the minuend loads follow the last slice
            if (ahead >= 2) dma_barrier<2 * kDmaPerSlice + kMv>();
            else if (ahead == 1) dma_barrier<kDmaPerSlice + kMv>();
            else dma_barrier<kMv>();
        } else {
            if (ahead >= 2) dma_barrier<2 * kDmaPerSlice>();
            else if (ahead == 1) dma_barrier<kDmaPerSlice>();
            else dma_barrier<0>();
        }
        if (j + kStages - 1 < nk) {
            issue(nxt, j + kStages - 1);
            if (mv_on && j + kStages - 1 == nk - 1) issue_minuend();
        }
        float a[FM][KS], b[FN][KS];
#pragma unroll
        for (int i = 0; i < FM; ++i) dma_frag<TA, T>(cur, wm0 + i * 16 + cc, kk, a[i]);
        if constexpr (RECON) {
#pragma unroll
            for (int s2 = 0; s2 < KS; ++s2) {
                const float sc = scs[j * BK + KS * kk + s2];
#pragma unroll
                for (int i = 0; i < FM; ++i) a[i][s2] *= sc;
            }
        }
#pragma unroll
        for (int jj = 0; jj < FN; ++jj) dma_frag<!TB, T>(cur + kTileF, wn0 + jj * 16 + cc, kk, b[jj]);
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int jj = 0; jj < FN; ++jj)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][s2], b[jj][s2], acc[i][jj], 0, 0, 0);
    };
    if (0 < nk) issue(st0, 0);
    if (1 < nk) issue(st1, 1);
    if (2 < nk) issue(st2, 2);
    if (mv_on && nk <= kStages - 1) issue_minuend();
    for (int j = 0; j < nk; j += kStages) {
        body(st0, st3, j);
        if (j + 1 < nk) body(st1, st0, j + 1);
        if (j + 2 < nk) body(st2, st1, j + 2);
        if (j + 3 < nk) body(st3, st2, j + 3);
    }

    float *C = g.C + static_cast<uint64_t>(zs) * g.split_stride;
    // fragment (i, j) register r holds row 4*(lane/16) + r, column lane % 16
    if constexpr (RECON) {
        // every wave leaves with its own 64 x 64 block through its own 16 KB
        // of the ring, after one barrier (the ring is consumed): rows go out
        // as 16-byte stores, the minuend comes in as 16-byte loads; columns
        // are XOR-swizzled by 16 on alternate groups of four rows (the
        // fragment writes of rows r and r + 4 then hit disjoint banks)
        __syncthreads();
        float *Cw = wave == 0 ? st0 : (wave == 1 ? st1 : (wave == 2 ? st2 : st3));
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rl = 16 * i + 4 * (lane >> 4) + r, col = 16 * j + (lane & 15);
                    Cw[rl * WN + (col ^ (16 * ((rl >> 2) & 1)))] = acc[i][j][r];
                }
#pragma unroll
        for (int q = 0; q < kMv; ++q) {
            const int rl = 4 * q + (lane >> 4), c4 = 4 * (lane & 15);
            const int gi = m0 + wm0 + rl, gj = n0 + wn0 + c4;
            if (gi >= g.M) continue;
            float4 v = *reinterpret_cast<const float4 *>(&Cw[rl * WN + (c4 ^ (16 * ((rl >> 2) & 1)))]);
            const uint64_t e = static_cast<uint64_t>(gi) * g.ldc + gj;
            if (vec_c && gj + 4 <= g.N) {
                if (mv_on) v = float4{mvall[q].x - v.x, mvall[q].y - v.y, mvall[q].z - v.z, mvall[q].w - v.w};
                *reinterpret_cast<float4 *>(C + e) = v;
            } else {
                const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (gj + u < g.N) C[e + u] = g.minuend ? g.minuend[e + u] - vv[u] : vv[u];
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gi = m0 + wm0 + i * 16 + 4 * (lane >> 4) + r;
                const int gj = n0 + wn0 + j * 16 + (lane & 15);
                if (gi < g.M && gj < g.N) C[static_cast<uint64_t>(gi) * g.ldc + gj] = acc[i][j][r];
            }
}

// ---------------------------------------------------------------------------
// Stream-K form of the DMA-pipelined kernel for the long-K, few-tile products
// of the range finder (n x q outputs, K = m or n).  A persistent grid of G
// workgroups (two per CU) splits the flattened space of tiles x K slices, in
// pairs of slices, into G equal contiguous ranges, so every CU does the same
// work whatever the tile count, and each workgroup fills its DMA ring once:
// the ring runs on across tile boundaries, and the partial tile that ends at
// a boundary is written out while the next tile's slices are already in
// flight.  Logical workgroup L (pair ranges [L P / G, (L + 1) P / G), P =
// tiles x slices / 2) is placed so that each XCD runs a contiguous eighth of
// the space (a few A panels).  Each workgroup writes the partial tile of every
// tile it touches to slot (tile, L - first owner) and streamk_reduce_kernel
// sums each tile's slots in that fixed order, so results are deterministic.
// Needs an even number of slices per tile (tile boundaries then fall between
// pairs, after the second or fourth slice of an unrolled group of four).
struct StreamK {
    float *ws;     // partial tiles [tile][part][128][128]
    int tiles_n;   // output tiles per row of tiles
    int nk;        // K slices per tile (even)
    int pairs;     // tiles x nk / 2
    int maxparts;  // workspace slots per tile
};

// logical workgroup whose range holds slice pair `pr`
__host__ __device__ __forceinline__ int sk_owner(int64_t pr, int64_t pairs, int G) {
    return static_cast<int>(((pr + 1) * G - 1) / pairs);
}

// (two waves per SIMD requested explicitly: left to itself the register
// allocator splits the accumulators between AGPRs and VGPRs around the
// partial-tile writes and needs more than half the register file)
template <bool TA, bool TB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_streamk_kernel(
    GemmArgs g, StreamK sk) {
    constexpr int T = 128, BM = T, BN = T;
    constexpr int kTileF = T * BK;
    constexpr int kStageF = 2 * kTileF;
    constexpr int kChunks = T / 16;
    constexpr int kCpw = kChunks / 4;
    constexpr int kDmaPerSlice = 2 * kCpw;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 16, FN = WN / 16;
    __shared__ __attribute__((aligned(1024))) float st0[kStageF];
    __shared__ __attribute__((aligned(1024))) float st1[kStageF];
    __shared__ __attribute__((aligned(1024))) float st2[kStageF];
    __shared__ __attribute__((aligned(1024))) float st3[kStageF];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    const int G = static_cast<int>(gridDim.x);
    const int bid = static_cast<int>(blockIdx.x), xcd = bid % kXcds, loc = bid / kXcds;
    const int L = xcd * (G / kXcds) + min(xcd, G % kXcds) + loc;
    const int64_t pairs = sk.pairs;
    const int p0 = static_cast<int>(static_cast<int64_t>(L) * pairs / G);
    const int n = 2 * (static_cast<int>(static_cast<int64_t>(L + 1) * pairs / G) - p0);  // slices
    const int it0 = 2 * p0;

    f32x4v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

    // the next slice to issue, as running (tile row, tile column, slice)
    const int tile0 = it0 / sk.nk;
    int i_ks = it0 - tile0 * sk.nk;
    int i_tm = tile0 / sk.tiles_n, i_tn = tile0 - i_tm * sk.tiles_n;
    auto issue = [&](const float *st) {
        const int m0 = i_tm * BM, n0 = i_tn * BN, k0 = i_ks * BK;
#pragma unroll
        for (int h = 0; h < kCpw; ++h) {
            const int c = kCpw * wave + h;
            dma_chunk<TA, T>(g.A, g.lda, m0, g.M, k0, c, st);
            dma_chunk<!TB, T>(g.B, g.ldb, n0, g.N, k0, c, st + kTileF);
        }
        // advanced by selects: a branch here would split the MFMA chains
        // across blocks and their accumulators across register classes
        const bool wrap = i_ks + 1 == sk.nk;
        i_ks = wrap ? 0 : i_ks + 1;
        const int tn1 = i_tn + (wrap ? 1 : 0);
        const bool wrap2 = tn1 == sk.tiles_n;
        i_tn = wrap2 ? 0 : tn1;
        i_tm += wrap2 ? 1 : 0;
    };
    const int kk = lane >> 4, cc = lane & 15;
    // the tile being accumulated and its slices done so far
    int c_tile = tile0, c_ks = it0 - tile0 * sk.nk;
    // after the pair ending with local slice jl: at a tile's end or the range's
    // end, the partial tile goes to its slot and the accumulators restart
    auto pair_done = [&](int jl) {
        c_ks += 2;
        const bool tile_end = c_ks == sk.nk;
        if (tile_end || jl + 1 == n) {  // uniform
            const int first = sk_owner(static_cast<int64_t>(c_tile) * (sk.nk / 2), pairs, G);
            float *W = sk.ws + (static_cast<uint64_t>(c_tile) * sk.maxparts + (L - first)) * (T * T);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        W[(wm0 + i * 16 + 4 * (lane >> 4) + r) * T + wn0 + j * 16 + (lane & 15)] = acc[i][j][r];
                    acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
                }
        }
        c_ks = tile_end ? 0 : c_ks;
        c_tile += tile_end ? 1 : 0;
    };
    // local slice j sits in stage j % 4: cur holds it, nxt (= stage (j + 3) % 4,
    // read in iteration j - 1) receives local slice j + 3
    auto body = [&](const float *cur, const float *nxt, int j) {
        const int ahead = min(kStages - 2, n - 1 - j);
        if (ahead >= 2) dma_barrier<2 * kDmaPerSlice>();
        else if (ahead == 1) dma_barrier<kDmaPerSlice>();
        else dma_barrier<0>();
        if (j + kStages - 1 < n) issue(nxt);
        float a[FM][KS], b[FN][KS];
#pragma unroll
        for (int i = 0; i < FM; ++i) dma_frag<TA, T>(cur, wm0 + i * 16 + cc, kk, a[i]);
#pragma unroll
        for (int jj = 0; jj < FN; ++jj) dma_frag<!TB, T>(cur + kTileF, wn0 + jj * 16 + cc, kk, b[jj]);
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int jj = 0; jj < FN; ++jj)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][s2], b[jj][s2], acc[i][jj], 0, 0, 0);
    };
    // steady state: every slice of the group has two slices issued behind
    // the next one and issues its own successor three ahead
    auto steady = [&](const float *cur, const float *nxt) {
        dma_barrier<2 * kDmaPerSlice>();
        issue(nxt);
        float a[FM][KS], b[FN][KS];
#pragma unroll
        for (int i = 0; i < FM; ++i) dma_frag<TA, T>(cur, wm0 + i * 16 + cc, kk, a[i]);
#pragma unroll
        for (int jj = 0; jj < FN; ++jj) dma_frag<!TB, T>(cur + kTileF, wn0 + jj * 16 + cc, kk, b[jj]);
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int jj = 0; jj < FN; ++jj)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][s2], b[jj][s2], acc[i][jj], 0, 0, 0);
    };
    if (0 < n) issue(st0);
    if (1 < n) issue(st1);
    if (2 < n) issue(st2);
    int j = 0;
    for (; j + 2 * kStages <= n; j += kStages) {
        steady(st0, st3);
        steady(st1, st0);
        pair_done(j + 1);
        steady(st2, st1);
        steady(st3, st2);
        pair_done(j + 3);
    }
    for (; j < n; j += kStages) {  // the last two to six slices (n is even)
        body(st0, st3, j);
        body(st1, st0, j + 1);
        pair_done(j + 1);
        if (j + 2 < n) {
            body(st2, st1, j + 2);
            body(st3, st2, j + 3);
            pair_done(j + 3);
        }
    }
}

// C = the sum of each tile's partial tiles in slot order.  One workgroup per
// 16 rows of a tile, 16-byte accesses.
__global__ __launch_bounds__(256) void streamk_reduce_kernel(StreamK sk, int G, int M, int N, int ldc,
                                                             float *__restrict__ C) {
    constexpr int T = 128;
    const int tile = static_cast<int>(blockIdx.x) / (T / 16), rb = (static_cast<int>(blockIdx.x) % (T / 16)) * 16;
    const int64_t pb = static_cast<int64_t>(tile) * (sk.nk / 2);
    const int parts = sk_owner(pb + sk.nk / 2 - 1, sk.pairs, G) - sk_owner(pb, sk.pairs, G) + 1;
    const int tm = tile / sk.tiles_n, tn = tile - tm * sk.tiles_n;
    const bool vec = (ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(C) & 15u) == 0);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int lin = threadIdx.x + 256 * q, r = rb + lin / (T / 4), c4 = (lin % (T / 4)) * 4;
        const float *W = sk.ws + static_cast<uint64_t>(tile) * sk.maxparts * (T * T) + r * T + c4;
        float4 s = *reinterpret_cast<const float4 *>(W);
        for (int p = 1; p < parts; ++p) {
            const float4 v = *reinterpret_cast<const float4 *>(W + static_cast<uint64_t>(p) * (T * T));
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
        const int gi = tm * T + r, gj = tn * T + c4;
        if (gi >= M) continue;
        float *out = C + static_cast<uint64_t>(gi) * ldc + gj;
        if (vec && gj + 4 <= N) {
            *reinterpret_cast<float4 *>(out) = s;
        } else {
            const float sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (gj + u < N) out[u] = sv[u];
        }
    }
}

// C[i, j] = sum_z W[z][i, j] in a fixed order.
__global__ void splitk_reduce_kernel(const float *__restrict__ W, int splits, uint64_t stride, int M, int N,
                                     int ldc, float *__restrict__ C) {
    // rows by grid-stride, columns by lane: no 64-bit division per element
    for (int i = blockIdx.y; i < M; i += gridDim.y)
        for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < N; j += gridDim.x * blockDim.x) {
            const uint64_t t = static_cast<uint64_t>(i) * N + j;
            // the partials' loads are issued eight at a time, summed in split order
            float s = W[t];
            int z = 1;
            for (; z + 8 <= splits; z += 8) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = W[(z + u) * stride + t];
#pragma unroll
                for (int u = 0; u < 8; ++u) s += v[u];
            }
            for (; z < splits; ++z) s += W[z * stride + t];
            C[static_cast<uint64_t>(i) * ldc + j] = s;
        }
}

// Split count minimising the modelled time.  Measured on gfx950, a CU works
// through ~1 slice of one 128 x 128 x 16 tile per 1.1 us when it holds two
// or more workgroups (1.2 us with one), so the time is the busiest CU's share:
// ceil(workgroups / CUs) x slices per workgroup x 1.1 us, plus, with splits,
// the fixed-order reduce (~5 us of launch and latency plus its bytes at
// ~5 TB/s).  Fits the power-iteration shapes to within ~7 %.
int choose_splits(int M, int N, int K) {
    const uint64_t tiles = ceil_div(M, BM) * ceil_div(N, BN);
    const uint64_t cus = static_cast<uint64_t>(cu_count());
    const uint64_t ksteps = ceil_div(K, BK);
    double best = 0.0;
    int best_s = 1;
    for (int s = 1; s <= 32; ++s) {
        if (s > 1 && ksteps / s < 16) break;  // keep >= 16 slices per split (short K: no split)
        const uint64_t per_cu = ceil_div(tiles * s, cus);
        const double step_us = per_cu >= 2 ? 1.1 : 1.2;  // one workgroup alone hides less latency
        const double t = static_cast<double>(per_cu) * ceil_div(ksteps, s) * step_us +
                         (s > 1 ? 5.0 + (s + 1.0) * M * N * 4.0 / 5e6 : 0.0);
        if (s == 1 || t < best) {
            best = t;
            best_s = s;
        }
    }
    return best_s;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Stream-K layout of a product that split-K would split (K a whole number of
// slice pairs): G = two workgroups per CU, and the most owners any tile has.
struct SkPlan {
    bool on = false;
    int G = 0;
    StreamK sk{};
    uint64_t bytes = 0;
};
SkPlan streamk_plan(int M, int N, int K) {
    SkPlan p;
    const int splits = choose_splits(M, N, K);
    if (K % (2 * BK) != 0 || splits <= 1) return p;
    const int tiles_n = static_cast<int>(ceil_div(N, 128));
    const int tiles = static_cast<int>(ceil_div(M, 128)) * tiles_n;
    // a split-K grid of whole rounds (two workgroups on every CU) is already
    // balanced, and its fixed-order sum is the same; stream-K is for the rest
    if ((static_cast<int64_t>(tiles) * splits) % (2 * static_cast<int64_t>(cu_count())) == 0) return p;
    const int nk = K / BK;
    const int64_t pairs = static_cast<int64_t>(tiles) * (nk / 2);
    const int G = static_cast<int>(std::min<int64_t>(2 * static_cast<int64_t>(cu_count()), pairs));
    int maxparts = 1;
    for (int t = 0; t < tiles; ++t) {
        const int64_t b = static_cast<int64_t>(t) * (nk / 2);
        maxparts = std::max(maxparts, sk_owner(b + nk / 2 - 1, pairs, G) - sk_owner(b, pairs, G) + 1);
    }
    p.on = true;
    p.G = G;
    p.sk.tiles_n = tiles_n;
    p.sk.nk = nk;
    p.sk.pairs = static_cast<int>(pairs);
    p.sk.maxparts = maxparts;
    p.bytes = static_cast<uint64_t>(tiles) * maxparts * 128 * 128 * sizeof(float);
    return p;
}

}  // namespace

// Workspace bytes needed by launch_gemm for the given shape (split-K partials
// on the register-staged path, stream-K partial tiles on the DMA path).
uint64_t gemm_workspace_bytes(int M, int N, int K) {
    const int splits = choose_splits(M, N, K);
    const uint64_t split_bytes = splits > 1 ? static_cast<uint64_t>(splits) * M * N * sizeof(float) : 0;
    return std::max(split_bytes, streamk_plan(M, N, K).bytes);
}

void launch_gemm(bool ta, bool tb, int M, int N, int K, const float *A, int lda, const float *B, int ldb, float *C,
                 int ldc, const float *a_colscale, const float *minuend, float *workspace, uint64_t workspace_bytes,
                 hipStream_t stream) {
    BSQ_REQUIRE(M > 0 && N > 0 && K > 0 && A && B && C, "gemm: bad arguments");
    int splits = (minuend || a_colscale) ? 1 : choose_splits(M, N, K);
    if (splits > 1 && (!workspace || static_cast<uint64_t>(splits) * M * N * sizeof(float) > workspace_bytes))
        splits = 1;
    GemmArgs g{};
    g.A = A;
    g.B = B;
    g.a_colscale = a_colscale;
    g.minuend = minuend;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = lda;
    g.ldb = ldb;
    g.vec_a = aligned16(A) && (lda % 4 == 0);
    g.vec_b = aligned16(B) && (ldb % 4 == 0);
    g.k_per_split = static_cast<int>(ceil_div(ceil_div(K, splits), BK) * BK);
    if (splits > 1) {
        g.C = workspace;
        g.ldc = N;
        g.split_stride = static_cast<uint64_t>(M) * N;
    } else {
        g.C = C;
        g.ldc = ldc;
        g.split_stride = 0;
    }
    g.splits = splits;
    dim3 grid(static_cast<unsigned>(ceil_div(N, BN) * ceil_div(M, BM) * splits));
    const bool recon = a_colscale || minuend;
    // the DMA-pipelined kernel wherever its layout constraints hold, else the
    // register-staged one
    const bool dma = g.vec_a && g.vec_b && (K % BK == 0) && (!ta || M % 4 == 0) &&
                     (tb || N % 4 == 0) && (!recon || K <= kDmaReconMaxK);
    // the long-K products in stream-K form
    if (dma && !recon && splits > 1) {
        SkPlan pl = streamk_plan(M, N, K);
        if (pl.on && pl.bytes <= workspace_bytes) {
            pl.sk.ws = workspace;
            g.C = C;
            g.ldc = ldc;
            g.split_stride = 0;
            g.splits = 1;
            g.k_per_split = K;
            const dim3 sgrid(static_cast<unsigned>(pl.G));
            if (!ta && !tb) gemm_streamk_kernel<false, false><<<sgrid, kThreads, 0, stream>>>(g, pl.sk);
            else if (ta && !tb) gemm_streamk_kernel<true, false><<<sgrid, kThreads, 0, stream>>>(g, pl.sk);
            else if (!ta && tb) gemm_streamk_kernel<false, true><<<sgrid, kThreads, 0, stream>>>(g, pl.sk);
            else gemm_streamk_kernel<true, true><<<sgrid, kThreads, 0, stream>>>(g, pl.sk);
            BSQ_HIP(hipGetLastError());
            const int tiles = static_cast<int>(ceil_div(M, 128) * ceil_div(N, 128));
            streamk_reduce_kernel<<<static_cast<unsigned>(tiles * 8), 256, 0, stream>>>(pl.sk, pl.G, M, N, ldc, C);
            BSQ_HIP(hipGetLastError());
            return;
        }
    }
    // 64 x 64 tiles when 128 x 128 ones (unsplit) would not give every CU two
    // workgroups: the short-K products of the orthonormalisation
    const bool t64 = dma && !recon && splits == 1 &&
                     ceil_div(M, BM) * ceil_div(N, BN) < 2 * static_cast<uint64_t>(cu_count());
    if (t64) {
        grid.x = static_cast<unsigned>(ceil_div(N, 64) * ceil_div(M, 64));  // unsplit
        if (!ta && !tb) gemm_dma_kernel<false, false, false, 64><<<grid, kThreads, 0, stream>>>(g);
        else if (ta && !tb) gemm_dma_kernel<true, false, false, 64><<<grid, kThreads, 0, stream>>>(g);
        else if (!ta && tb) gemm_dma_kernel<false, true, false, 64><<<grid, kThreads, 0, stream>>>(g);
        else gemm_dma_kernel<true, true, false, 64><<<grid, kThreads, 0, stream>>>(g);
    } else if (dma) {
        if (recon) {
            BSQ_REQUIRE(!ta && tb, "gemm: column scale / minuend only in the A * B^T form");
            gemm_dma_kernel<false, true, true, 128><<<grid, kThreads, 0, stream>>>(g);
        } else if (!ta && !tb) gemm_dma_kernel<false, false, false, 128><<<grid, kThreads, 0, stream>>>(g);
        else if (ta && !tb) gemm_dma_kernel<true, false, false, 128><<<grid, kThreads, 0, stream>>>(g);
        else if (!ta && tb) gemm_dma_kernel<false, true, false, 128><<<grid, kThreads, 0, stream>>>(g);
        else gemm_dma_kernel<true, true, false, 128><<<grid, kThreads, 0, stream>>>(g);
    } else if (recon) {
        BSQ_REQUIRE(!ta && tb, "gemm: column scale / minuend only in the A * B^T form");
        gemm_mfma_kernel<false, true, true><<<grid, kThreads, 0, stream>>>(g);
    } else if (!ta && !tb) gemm_mfma_kernel<false, false, false><<<grid, kThreads, 0, stream>>>(g);
    else if (ta && !tb) gemm_mfma_kernel<true, false, false><<<grid, kThreads, 0, stream>>>(g);
    else if (!ta && tb) gemm_mfma_kernel<false, true, false><<<grid, kThreads, 0, stream>>>(g);
    else gemm_mfma_kernel<true, true, false><<<grid, kThreads, 0, stream>>>(g);
    BSQ_HIP(hipGetLastError());
    if (splits > 1) {
        const dim3 rgrid(static_cast<unsigned>(ceil_div(N, 256)),
                         static_cast<unsigned>(std::min<uint64_t>(M, static_cast<uint64_t>(cu_count()) * 8)));
        splitk_reduce_kernel<<<rgrid, 256, 0, stream>>>(workspace, splits, g.split_stride, M, N, ldc, C);
        BSQ_HIP(hipGetLastError());
    }
}

}  // namespace bsq
