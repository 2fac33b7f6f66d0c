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
// Tiling: 256 threads = 4 waves in a 2 x 2 grid; workgroup tile 128 x 128,
// BK = 32; each wave owns 64 x 64 as 4 x 4 MFMA 16x16 blocks (64 AGPRs).
// Tiles move global -> registers (16-byte loads where the layout allows)
// -> LDS (k-major, padded, so every MFMA operand read is 16 consecutive
// floats) while the previous tile is multiplied.  Skinny shapes are split
// along K so the grid fills the 256 CUs several times over; partial products
// go to a workspace summed in a fixed order, so results are deterministic.
#include "bsq_internal.hpp"

namespace bsq {
namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 32;
constexpr int PAD = 16;  // row stride = 16 mod 64 banks: MFMA operand reads conflict-free

struct GemmArgs {
    const float *A;
    const float *B;
    float *C;                 // output (or split-K workspace base)
    const float *a_colscale;  // optional: op(A)[:, kk] *= a_colscale[kk]
    const float *minuend;     // optional: C = minuend - acc (ldc layout)
    int M, N, K;
    int lda, ldb, ldc;
    int k_per_split;          // K range of one blockIdx.z (multiple of BK)
    uint64_t split_stride;    // elements between split-K partial outputs
    bool vec_a, vec_b;        // 16-byte loads allowed (alignment of base and leading dim)
};

// A "row-contiguous" operand tile: R rows x 32 k-values, k contiguous in
// memory (A for TA = false, B for TB = true).  Written to LDS transposed as
// S[k][row].  256 threads: thread t covers row (t % 128) + 128 * pass, k
// quad (t / 128) * 4 + 8 * q.
template <int R>
struct KContig {
    static constexpr int N4 = R * BK / 4 / kThreads;  // float4 per thread
    float4 v[N4];
    __device__ __forceinline__ void load(const float *__restrict__ P, int ld, int r0, int rows, int k0, int kend,
                                         bool vec, const float *__restrict__ colscale) {
        const int t = threadIdx.x;
#pragma unroll
        for (int q = 0; q < N4; ++q) {
            const int lin = t + q * kThreads;       // 0 .. R*8-1
            const int r = lin % R, kq = lin / R;    // kq in 0..7
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
    template <int LDW>
    __device__ __forceinline__ void store(float (*S)[LDW]) const {
        const int t = threadIdx.x;
#pragma unroll
        for (int q = 0; q < N4; ++q) {
            const int lin = t + q * kThreads;
            const int r = lin % R, kq = lin / R;
            S[kq * 4 + 0][r] = v[q].x;
            S[kq * 4 + 1][r] = v[q].y;
            S[kq * 4 + 2][r] = v[q].z;
            S[kq * 4 + 3][r] = v[q].w;
        }
    }
};

// A "k-major" operand tile: 32 k-rows x C contiguous values (A for TA = true,
// B for TB = false).  Written to LDS as S[k][c].
template <int Cn>
struct KMajor {
    static constexpr int N4 = Cn * BK / 4 / kThreads;
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
                const float s = (gk < kend) ? rowscale[gk] : 0.0f;
                x.x *= s;
                x.y *= s;
                x.z *= s;
                x.w *= s;
            }
            v[q] = x;
        }
    }
    template <int LDW>
    __device__ __forceinline__ void store(float (*S)[LDW]) const {
        const int t = threadIdx.x;
        constexpr int C4 = Cn / 4;
#pragma unroll
        for (int q = 0; q < N4; ++q) {
            const int lin = t + q * kThreads;
            const int c = (lin % C4) * 4, kk = lin / C4;
            *reinterpret_cast<float4 *>(&S[kk][c]) = v[q];
        }
    }
};

// RECON: the low-rank reconstruction form (column scale on op(A), optional
// minuend), instantiated separately so the power-iteration GEMMs carry no
// epilogue branches and profiles tell the two apart.
template <bool TA, bool TB, bool RECON>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(GemmArgs g) {
    constexpr int WM = BM / 2, WN = BN / 2;  // wave tile
    constexpr int FM = WM / 16, FN = WN / 16;
    __shared__ __attribute__((aligned(16))) float As[2][BK][BM + PAD];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK][BN + PAD];

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

    typename std::conditional<TA, KMajor<BM>, KContig<BM>>::type ta;
    typename std::conditional<TB, KContig<BN>, KMajor<BN>>::type tb;

    auto load = [&](int k0) {
        ta.load(g.A, g.lda, m0, g.M, k0, kend, g.vec_a, RECON ? g.a_colscale : nullptr);
        tb.load(g.B, g.ldb, n0, g.N, k0, kend, g.vec_b, nullptr);
    };

    int buf = 0;
    if (kbeg < kend) {
        load(kbeg);
        ta.store(As[0]);
        tb.store(Bs[0]);
    }
    __syncthreads();
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
        const bool more = k0 + BK < kend;
        if (more) load(k0 + BK);
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
        if (more) {
            ta.store(As[buf ^ 1]);
            tb.store(Bs[buf ^ 1]);
        }
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
                    C[e] = (RECON && g.minuend) ? g.minuend[e] - v : v;
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
        float s = W[t];
        for (int z = 1; z < splits; ++z) s += W[z * stride + t];
        C[i * ldc + j] = s;
    }
}

// Split count minimising the modelled time: rounds of resident workgroups
// (two 128x128 tiles fit one CU's LDS) times the K slice each one walks,
// plus the traffic of summing the partials.
int choose_splits(int M, int N, int K) {
    const uint64_t tiles = ceil_div(M, BM) * ceil_div(N, BN);
    const uint64_t slots = static_cast<uint64_t>(cu_count()) * 2;
    const uint64_t ksteps = ceil_div(K, BK);
    double best = 0.0;
    int best_s = 1;
    for (int s = 1; s <= 32; ++s) {
        if (s > 1 && ksteps / s < 8) break;  // keep >= 8 K steps per split
        const uint64_t rounds = ceil_div(tiles * s, slots);
        // one K step of a 128x128x32 tile ~ 2 * 128 * 128 * 32 / (256 flop/clk) cycles;
        // the reduce moves (s + 1) * M * N * 4 bytes at ~ 2 KB / clk chip-wide.
        const double t = static_cast<double>(rounds) * ceil_div(ksteps, s) * 4096.0 +
                         (s > 1 ? (s + 1.0) * M * N * 4.0 / 2048.0 : 0.0);
        if (s == 1 || t < best) {
            best = t;
            best_s = s;
        }
    }
    return best_s;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// Workspace bytes needed by launch_gemm for the given shape (split-K partials).
uint64_t gemm_workspace_bytes(int M, int N, int K) {
    const int splits = choose_splits(M, N, K);
    return splits > 1 ? static_cast<uint64_t>(splits) * M * N * sizeof(float) : 0;
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
    dim3 grid(static_cast<unsigned>(ceil_div(N, BN)), static_cast<unsigned>(ceil_div(M, BM)), splits);
    const bool recon = a_colscale || minuend;
    if (recon) {
        BSQ_REQUIRE(!ta && tb, "gemm: column scale / minuend only in the A * B^T form");
        gemm_mfma_kernel<false, true, true><<<grid, kThreads, 0, stream>>>(g);
    } else if (!ta && !tb) gemm_mfma_kernel<false, false, false><<<grid, kThreads, 0, stream>>>(g);
    else if (ta && !tb) gemm_mfma_kernel<true, false, false><<<grid, kThreads, 0, stream>>>(g);
    else if (!ta && tb) gemm_mfma_kernel<false, true, false><<<grid, kThreads, 0, stream>>>(g);
    else gemm_mfma_kernel<true, true, false><<<grid, kThreads, 0, stream>>>(g);
    BSQ_HIP(hipGetLastError());
    if (splits > 1) {
        const uint64_t total = static_cast<uint64_t>(M) * N;
        uint64_t rgrid = ceil_div(total, 256);
        const uint64_t cap = static_cast<uint64_t>(cu_count()) * 8;
        if (rgrid > cap) rgrid = cap;
        splitk_reduce_kernel<<<static_cast<unsigned>(rgrid), 256, 0, stream>>>(workspace, splits, g.split_stride, M,
                                                                              N, ldc, C);
        BSQ_HIP(hipGetLastError());
    }
}

}  // namespace bsq
