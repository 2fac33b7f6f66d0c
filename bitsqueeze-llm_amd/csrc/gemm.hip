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
// reconstruction U diag(S) V^T, which folds diag(S) into the A-tile load and
// can subtract from a minuend in the epilogue (error = residual - U S V^T).
//
// Tiling: 256 threads = 4 waves in a 2 x 2 grid; workgroup tile BM x BN with
// BK = 16; each wave owns (BM/2) x (BN/2) as 16x16 MFMA blocks.  Tiles are
// staged global -> registers -> LDS (k-major, padded) with one LDS buffer
// in flight while the next K-step is fetched.  Split-K writes partial
// products to a workspace that a fixed-order reduction sums, so results are
// deterministic.
#include "bsq_internal.hpp"

namespace bsq {
namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int BK = 16;

struct GemmArgs {
    const float *A;
    const float *B;
    float *C;          // output (or split-K workspace base)
    const float *a_colscale;  // optional: op(A)[:, kk] *= a_colscale[kk]
    const float *minuend;     // optional: C = minuend - acc (ldc layout)
    int M, N, K;
    int lda, ldb, ldc;
    int k_per_split;   // K range of one blockIdx.z
    uint64_t split_stride;  // elements between split-K partial outputs
};

template <bool TA, bool TB, int BM, int BN>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(GemmArgs g) {
    constexpr int PAD = 4;
    constexpr int WM = BM / 2, WN = BN / 2;       // wave tile
    constexpr int FM = WM / 16, FN = WN / 16;     // 16x16 fragments per wave
    constexpr int A_ELEMS = BM * BK / kThreads;   // per thread per K-step
    constexpr int B_ELEMS = BN * BK / kThreads;
    __shared__ float As[2][BK][BM + PAD];
    __shared__ float Bs[2][BK][BN + PAD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kbeg = blockIdx.z * g.k_per_split;
    const int kend = min(g.K, kbeg + g.k_per_split);

    f32x4v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};

    float ra[A_ELEMS], rb[B_ELEMS];

    // global -> registers for the K-step starting at k0
    auto load_tiles = [&](int k0) {
        if constexpr (!TA) {
            // A row-major M x K: thread covers row (tid / (BK / A_ELEMS)), A_ELEMS consecutive k
            constexpr int TPR = BK / A_ELEMS;
            const int r = tid / TPR, kk = (tid % TPR) * A_ELEMS;
            const int gi = m0 + r;
#pragma unroll
            for (int e = 0; e < A_ELEMS; ++e) {
                const int gk = k0 + kk + e;
                float v = (gi < g.M && gk < kend) ? g.A[static_cast<uint64_t>(gi) * g.lda + gk] : 0.0f;
                if (g.a_colscale && gk < kend) v *= g.a_colscale[gk];
                ra[e] = v;
            }
        } else {
            // A stored K x M: thread covers k row (tid / (BM / A_ELEMS)), A_ELEMS consecutive m
            constexpr int TPR = BM / A_ELEMS;
            const int kk = tid / TPR, c = (tid % TPR) * A_ELEMS;
            const int gk = k0 + kk;
#pragma unroll
            for (int e = 0; e < A_ELEMS; ++e) {
                const int gi = m0 + c + e;
                float v = (gi < g.M && gk < kend) ? g.A[static_cast<uint64_t>(gk) * g.lda + gi] : 0.0f;
                if (g.a_colscale && gk < kend) v *= g.a_colscale[gk];
                ra[e] = v;
            }
        }
        if constexpr (!TB) {
            constexpr int TPR = BN / B_ELEMS;
            const int kk = tid / TPR, c = (tid % TPR) * B_ELEMS;
            const int gk = k0 + kk;
#pragma unroll
            for (int e = 0; e < B_ELEMS; ++e) {
                const int gj = n0 + c + e;
                rb[e] = (gj < g.N && gk < kend) ? g.B[static_cast<uint64_t>(gk) * g.ldb + gj] : 0.0f;
            }
        } else {
            constexpr int TPR = BK / B_ELEMS;
            const int r = tid / TPR, kk = (tid % TPR) * B_ELEMS;
            const int gj = n0 + r;
#pragma unroll
            for (int e = 0; e < B_ELEMS; ++e) {
                const int gk = k0 + kk + e;
                rb[e] = (gj < g.N && gk < kend) ? g.B[static_cast<uint64_t>(gj) * g.ldb + gk] : 0.0f;
            }
        }
    };
    auto store_tiles = [&](int buf) {
        if constexpr (!TA) {
            constexpr int TPR = BK / A_ELEMS;
            const int r = tid / TPR, kk = (tid % TPR) * A_ELEMS;
#pragma unroll
            for (int e = 0; e < A_ELEMS; ++e) As[buf][kk + e][r] = ra[e];
        } else {
            constexpr int TPR = BM / A_ELEMS;
            const int kk = tid / TPR, c = (tid % TPR) * A_ELEMS;
#pragma unroll
            for (int e = 0; e < A_ELEMS; ++e) As[buf][kk][c + e] = ra[e];
        }
        if constexpr (!TB) {
            constexpr int TPR = BN / B_ELEMS;
            const int kk = tid / TPR, c = (tid % TPR) * B_ELEMS;
#pragma unroll
            for (int e = 0; e < B_ELEMS; ++e) Bs[buf][kk][c + e] = rb[e];
        } else {
            constexpr int TPR = BK / B_ELEMS;
            const int r = tid / TPR, kk = (tid % TPR) * B_ELEMS;
#pragma unroll
            for (int e = 0; e < B_ELEMS; ++e) Bs[buf][kk + e][r] = rb[e];
        }
    };

    int buf = 0;
    if (kbeg < kend) {
        load_tiles(kbeg);
        store_tiles(0);
    }
    __syncthreads();
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
        const bool more = k0 + BK < kend;
        if (more) load_tiles(k0 + BK);
#pragma unroll
        for (int k4 = 0; k4 < BK; k4 += 4) {
            const int kr = k4 + (lane >> 4), cc = lane & 15;
            float a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) a[i] = As[buf][kr][wm0 + i * 16 + cc];
#pragma unroll
            for (int j = 0; j < FN; ++j) b[j] = Bs[buf][kr][wn0 + j * 16 + cc];
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more) store_tiles(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    // epilogue: fragment (i, j) register r holds row 4*(lane/16) + r, column lane % 16
    float *C = g.C + static_cast<uint64_t>(blockIdx.z) * g.split_stride;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gi = m0 + wm0 + i * 16 + 4 * (lane >> 4) + r;
                const int gj = n0 + wn0 + j * 16 + (lane & 15);
                if (gi < g.M && gj < g.N) {
                    const uint64_t e = static_cast<uint64_t>(gi) * g.ldc + gj;
                    const float v = acc[i][j][r];
                    C[e] = g.minuend ? g.minuend[e] - v : v;
                }
            }
}

// C[i, j] = sum_z W[z][i, j] in a fixed order.
__global__ void splitk_reduce_kernel(const float *__restrict__ W, int splits, uint64_t stride, int M, int N,
                                     int ldc, float *__restrict__ C) {
    const uint64_t total = static_cast<uint64_t>(M) * N;
    for (uint64_t t = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t i = t / N, j = t % N;
        const uint64_t e = i * ldc + j;
        float s = W[e];
        for (int z = 1; z < splits; ++z) s += W[z * stride + e];
        C[e] = s;
    }
}

template <bool TA, bool TB>
void launch_tiled(const GemmArgs &g, int splits, hipStream_t stream) {
    constexpr int BM = 128, BN = 128;
    dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM, splits);
    gemm_mfma_kernel<TA, TB, BM, BN><<<grid, kThreads, 0, stream>>>(g);
}

}  // namespace

// Workspace bytes needed by launch_gemm for the given shape (split-K partials).
uint64_t gemm_workspace_bytes(int M, int N, int K) {
    const uint64_t tiles = ceil_div(M, 128) * ceil_div(N, 128);
    const int cus = cu_count();
    int splits = 1;
    while (tiles * splits < static_cast<uint64_t>(cus) && splits < 16 && K / (splits * 2) >= 256) splits *= 2;
    return splits > 1 ? static_cast<uint64_t>(splits) * M * N * sizeof(float) : 0;
}

void launch_gemm(bool ta, bool tb, int M, int N, int K, const float *A, int lda, const float *B, int ldb, float *C,
                 int ldc, const float *a_colscale, const float *minuend, float *workspace, uint64_t workspace_bytes,
                 hipStream_t stream) {
    BSQ_REQUIRE(M > 0 && N > 0 && K > 0 && A && B && C, "gemm: bad arguments");
    const uint64_t tiles = ceil_div(M, 128) * ceil_div(N, 128);
    int splits = 1;
    if (!minuend) {
        const int cus = cu_count();
        while (tiles * splits < static_cast<uint64_t>(cus) && splits < 16 && K / (splits * 2) >= 256) splits *= 2;
        if (static_cast<uint64_t>(splits) * M * N * sizeof(float) > workspace_bytes || !workspace) splits = 1;
    }
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
    const int kps = static_cast<int>(ceil_div(ceil_div(K, splits), BK) * BK);
    g.k_per_split = kps;
    if (splits > 1) {
        g.C = workspace;
        g.ldc = N;
        g.split_stride = static_cast<uint64_t>(M) * N;
    } else {
        g.C = C;
        g.ldc = ldc;
        g.split_stride = 0;
    }
    if (!ta && !tb) launch_tiled<false, false>(g, splits, stream);
    else if (ta && !tb) launch_tiled<true, false>(g, splits, stream);
    else if (!ta && tb) launch_tiled<false, true>(g, splits, stream);
    else launch_tiled<true, true>(g, splits, stream);
    BSQ_HIP(hipGetLastError());
    if (splits > 1) {
        BSQ_REQUIRE(ldc == N, "gemm: split-K output must be dense");
        const uint64_t total = static_cast<uint64_t>(M) * N;
        uint64_t grid = ceil_div(total, 256);
        const uint64_t cap = static_cast<uint64_t>(cu_count()) * 8;
        if (grid > cap) grid = cap;
        splitk_reduce_kernel<<<static_cast<unsigned>(grid), 256, 0, stream>>>(workspace, splits, g.split_stride, M,
                                                                             N, ldc, C);
        BSQ_HIP(hipGetLastError());
    }
}

}  // namespace bsq
