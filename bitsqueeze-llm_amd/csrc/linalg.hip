// Small dense FP64 linear algebra for the randomised SVD (k x k, k = rank).
//
//   gram      G = X^T X (FP32 X, FP64 products and sums), split over rows
//   chol_inv  G = L L^T (FP64, shifted retry on breakdown) and L^{-1} as FP32
//             (CholeskyQR: Q = X L^{-T}); unblocked, for ranks above 256 (the
//             blocked kernels for k <= 256 are in chol.hip)
//   syev      G = U diag(lambda) U^T (FP64): Householder tridiagonalisation,
//             bisection with Sturm counts, inverse iteration (clusters
//             re-orthogonalised), back-transformation
//
// The reference orthonormalises with Householder QR and finishes with a
// Jacobi SVD from cuSOLVER (modules/svd_lowrank_cuda/src/svd_lowrank_cuda.cu:
// 250-282, 390-408); both are replaced here by Gram-based factorisations whose
// Gram matrices are formed exactly in FP64 from the FP32 factors.
#include "bsq_internal.hpp"
#include "wave_ops.hpp"

#include <algorithm>
#include <cfloat>

namespace bsq {
namespace {

constexpr int kGramTile = 64;

// ---------------------------------------------------------------------------
// Gram: partial G over a row chunk for one lower 64x64 tile, on the FP64
// matrix cores (v_mfma_f64_16x16x4f64):
// 256 lanes = 4 waves, each a 32 x 32 quarter of the 64 x 64 tile as 2 x 2
// MFMA blocks.  Rows are staged 32 at a time through LDS (16-byte loads,
// the next chunk fetched while the current one is multiplied); the FP32
// inputs are widened to FP64 exactly, so every product and sum is FP64.
// MFMA operand lanes: A[i][k] and B[k][j] in lane 16 k + (i or j);
// accumulator register r of lane l holds D[4 r + l / 16][l % 16].
typedef double f64x4 __attribute__((ext_vector_type(4)));
constexpr int kGramRows = 32, kGramPitch = kGramTile + 16;  // pitch: 16-bank offset between k rows

template <bool VEC>
__global__ __launch_bounds__(256) void gram_mfma_kernel(const float *__restrict__ X, int M, int k, int ld,
                                                         int rows_per_split, double *__restrict__ P) {
    __shared__ __attribute__((aligned(16))) float xi[2][kGramRows][kGramPitch];
    __shared__ __attribute__((aligned(16))) float xj[2][kGramRows][kGramPitch];
    int t = blockIdx.x, ti = 0;
    while (t > ti) {
        t -= ti + 1;
        ++ti;
    }
    const int tj = t;
    const int r0 = blockIdx.y * rows_per_split, r1 = min(M, r0 + rows_per_split);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wi = (wave >> 1) * 32, wj = (wave & 1) * 32;
    // staging: 32 rows x 64 columns = 512 float4, two per lane per operand.
    // A chunk's loads are issued three chunks ahead of its multiply (a ring
    // of four register sets): one chunk's MFMAs take a fraction of a memory
    // latency, so a single chunk of lookahead would leave the MFMAs waiting.
    struct Stage {
        float4 i[2], j[2];
    };
    // branch-free loads (row and column clamped into X); the values outside
    // X are masked to zero only when the chunk goes to LDS, so nothing
    // consumes a load early and the three chunks of lookahead stay in flight
    auto load4 = [&](const float *row, int c) -> float4 {
        if constexpr (VEC) {  // k % 4 == 0: a quad is inside or wholly outside
            return *reinterpret_cast<const float4 *>(row + min(c, k - 4));
        } else {
            return float4{row[min(c, k - 1)], row[min(c + 1, k - 1)], row[min(c + 2, k - 1)], row[min(c + 3, k - 1)]};
        }
    };
    auto mask4 = [&](float4 v, bool rin, int c) -> float4 {
        v.x = (rin && c < k) ? v.x : 0.0f;
        v.y = (rin && c + 1 < k) ? v.y : 0.0f;
        v.z = (rin && c + 2 < k) ? v.z : 0.0f;
        v.w = (rin && c + 3 < k) ? v.w : 0.0f;
        return v;
    };
    auto fetch = [&](int rb, Stage &st) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int lin = tid + 256 * q, rr = lin >> 4, c4 = (lin & 15) * 4;
            const int r = rb + rr, ci = ti * kGramTile + c4, cj = tj * kGramTile + c4;
            const float *row = X + static_cast<uint64_t>(min(r, r1 - 1)) * ld;
            st.i[q] = load4(row, ci);
            st.j[q] = load4(row, cj);  // the same columns on diagonal tiles
        }
    };
    auto put = [&](int b, int rb, const Stage &st) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int lin = tid + 256 * q, rr = lin >> 4, c4 = (lin & 15) * 4;
            const bool rin = rb + rr < r1;
            *reinterpret_cast<float4 *>(&xi[b][rr][c4]) = mask4(st.i[q], rin, ti * kGramTile + c4);
            *reinterpret_cast<float4 *>(&xj[b][rr][c4]) = mask4(st.j[q], rin, tj * kGramTile + c4);
        }
    };
    f64x4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = f64x4{0.0, 0.0, 0.0, 0.0};
    const int kk = lane >> 4, cc = lane & 15;
    auto multiply = [&](int b) {
        const float(*BI)[kGramPitch] = xi[b];
        const float(*BJ)[kGramPitch] = xj[b];
#pragma unroll
        for (int st = 0; st < kGramRows / 4; ++st) {
            const int rr = 4 * st + kk;
            double av[2], bv[2];
#pragma unroll
            for (int a = 0; a < 2; ++a) av[a] = static_cast<double>(BI[rr][wi + 16 * a + cc]);
#pragma unroll
            for (int b2 = 0; b2 < 2; ++b2) bv[b2] = static_cast<double>(BJ[rr][wj + 16 * b2 + cc]);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b2 = 0; b2 < 2; ++b2)
                    acc[a][b2] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[a], bv[b2], acc[a][b2], 0, 0, 0);
        }
    };
    const int nch = r0 < r1 ? static_cast<int>(ceil_div(r1 - r0, kGramRows)) : 0;
    // Every step issues the same four loads (chunks past the end read the
    // clamped last row and are never multiplied), so the compiler's wait
    // counting sees a fixed ring and waits only for the chunk it stores.
    Stage s0, s1, s2, s3;
    if (nch > 0) {  // uniform
        fetch(r0, s0);
        fetch(r0 + kGramRows, s1);
        fetch(r0 + 2 * kGramRows, s2);
        put(0, r0, s0);
    }
    __syncthreads();
    // chunk c sits in register set c % 4 until it is put into LDS buffer c % 2
    auto step = [&](int c, Stage &ahead, const Stage &next) {
        fetch(r0 + (c + 3) * kGramRows, ahead);
        multiply(c & 1);
        put((c + 1) & 1, r0 + (c + 1) * kGramRows, next);
        __syncthreads();
    };
    int c = 0;
    for (; c + 4 <= nch; c += 4) {
        step(c, s3, s1);
        step(c + 1, s0, s2);
        step(c + 2, s1, s3);
        step(c + 3, s2, s0);
    }
    if (c < nch) step(c, s3, s1);
    if (c + 1 < nch) step(c + 1, s0, s2);
    if (c + 2 < nch) step(c + 2, s1, s3);
    double *out = P + static_cast<uint64_t>(blockIdx.y) * k * k;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = ti * kGramTile + wi + 16 * a + 4 * r + kk, j = tj * kGramTile + wj + 16 * b + cc;
                if (i < k && j < k && j <= i) out[static_cast<uint64_t>(i) * k + j] = acc[a][b][r];
            }
}

// G[i][j] = G[j][i] = sum_s P[s][i][j] (lower entries), fixed order.
// One row per workgroup (grid-stride), columns by lane.  With rowsq,
// rowsq[i] = sum over row i of the full symmetric G of (G - I)^2 (the
// squared Frobenius distance from I, split by rows, summed in a fixed order).
__global__ __launch_bounds__(256) void gram_reduce_kernel(const double *__restrict__ P, int splits, int k,
                                                          double *__restrict__ G, double *__restrict__ rowsq) {
    __shared__ double red[4];
    const uint64_t kk = static_cast<uint64_t>(k) * k;
    for (int i = blockIdx.x; i < k; i += gridDim.x) {  // uniform per workgroup
        double sq = 0.0;
        for (int j = threadIdx.x; j <= i; j += blockDim.x) {
            const uint64_t t = static_cast<uint64_t>(i) * k + j;
            // the partials' loads are issued eight at a time, summed in split order
            double s = 0.0;
            int z = 0;
            for (; z + 8 <= splits; z += 8) {
                double v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = P[(z + u) * kk + t];
#pragma unroll
                for (int u = 0; u < 8; ++u) s += v[u];
            }
            for (; z < splits; ++z) s += P[z * kk + t];
            G[t] = s;
            G[static_cast<uint64_t>(j) * k + i] = s;
            // row i of the full matrix: the lower entries here, the upper ones
            // mirrored from the rows below, so off-diagonal squares count twice
            sq += (j == i) ? (s - 1.0) * (s - 1.0) : 2.0 * s * s;
        }
        if (rowsq) {
            for (int off = 32; off >= 1; off >>= 1) sq += __shfl_xor(sq, off);
            if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
            __syncthreads();
            if (threadIdx.x == 0) rowsq[i] = (red[0] + red[1]) + (red[2] + red[3]);
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// block helpers (1024 threads)
// ---------------------------------------------------------------------------
constexpr int kBig = 1024;

__device__ double block_sum(double v, double *red) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double s = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += red[w];
    return s;
}

__device__ double block_max(double v, double *red) {
    for (int off = 32; off >= 1; off >>= 1) v = fmax(v, __shfl_xor(v, off));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double s = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) s = fmax(s, red[w]);
    return s;
}

// ---------------------------------------------------------------------------
// Cholesky + triangular inverse, one workgroup, FP64 workspace W (k x k).
// Output Linv (k x k FP32 row-major, zero above the diagonal) with
// L^{-1} (G + shift I) L^{-T} = I.  status[0] = number of shifted retries.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBig) void chol_inv_kernel(const double *__restrict__ G, int k,
                                                         double *__restrict__ W, float *__restrict__ Linv,
                                                         int *__restrict__ status, double *__restrict__ col_ext) {
    extern __shared__ double col_lds[];  // k doubles, or col_ext (global) when they do not fit
    double *col = col_ext ? col_ext : col_lds;
    __shared__ double red[kBig / 64];
    __shared__ int broke;
    const int tid = threadIdx.x;
    double dmax = 0.0;
    for (int i = tid; i < k; i += kBig) dmax = fmax(dmax, fabs(G[static_cast<uint64_t>(i) * k + i]));
    dmax = block_max(dmax, red);
    double shift = 0.0;
    int attempt = 0;
    for (;; ++attempt) {
        // W = lower(G) + shift I
        for (uint64_t t = tid; t < static_cast<uint64_t>(k) * k; t += kBig) {
            const int i = static_cast<int>(t / k), j = static_cast<int>(t % k);
            W[t] = (j <= i) ? G[t] + (i == j ? shift : 0.0) : 0.0;
        }
        if (tid == 0) broke = 0;
        __syncthreads();
        const double tiny = (dmax > 0.0 ? dmax : 1.0) * 1e-15;
        for (int j = 0; j < k; ++j) {
            const double d = W[static_cast<uint64_t>(j) * k + j];
            if (!(d > tiny)) {  // not positive definite at working precision (also NaN)
                if (tid == 0) broke = 1;
                __syncthreads();
                break;
            }
            const double dj = sqrt(d);
            for (int i = j + 1 + tid; i < k; i += kBig) {
                const double v = W[static_cast<uint64_t>(i) * k + j] / dj;
                W[static_cast<uint64_t>(i) * k + j] = v;
                col[i] = v;
            }
            __syncthreads();
            if (tid == 0) W[static_cast<uint64_t>(j) * k + j] = dj;
            const int n = k - j - 1;  // trailing lower triangle, rows/cols j+1..k-1
            for (int i2 = tid >> 5; i2 < n; i2 += kBig / 32) {
                const int i = j + 1 + i2;
                const double li = col[i];
                double *row = W + static_cast<uint64_t>(i) * k;
                for (int c2 = tid & 31; c2 <= i2; c2 += 32) {
                    const int c = j + 1 + c2;
                    row[c] -= li * col[c];
                }
            }
            __syncthreads();
        }
        if (!broke) break;
        if (attempt >= 6 || dmax == 0.0) {
            // zero or hopeless matrix: L = I
            for (uint64_t t = tid; t < static_cast<uint64_t>(k) * k; t += kBig) {
                const int i = static_cast<int>(t / k), j = static_cast<int>(t % k);
                W[t] = (i == j) ? 1.0 : 0.0;
            }
            __syncthreads();
            break;
        }
        shift = (shift == 0.0) ? dmax * 1e-12 * static_cast<double>(k) : shift * 100.0;
        __syncthreads();
    }
    // in-place inverse of the lower-triangular W (column j from the bottom up):
    // Linv[j][j] = 1 / L[j][j];  Linv[j+1:, j] = -Linv[j][j] * Linv[j+1:, j+1:] L[j+1:, j]
    for (int j = k - 1; j >= 0; --j) {
        const double ljj = 1.0 / W[static_cast<uint64_t>(j) * k + j];  // read before thread 0 overwrites it
        for (int i = j + 1 + tid; i < k; i += kBig) col[i] = W[static_cast<uint64_t>(i) * k + j];
        __syncthreads();
        for (int i = j + 1 + tid; i < k; i += kBig) {
            const double *row = W + static_cast<uint64_t>(i) * k;
            double s = 0.0;
            for (int m = j + 1; m <= i; ++m) s = fma(row[m], col[m], s);
            W[static_cast<uint64_t>(i) * k + j] = -ljj * s;
        }
        if (tid == 0) W[static_cast<uint64_t>(j) * k + j] = ljj;
        __syncthreads();
    }
    for (uint64_t t = tid; t < static_cast<uint64_t>(k) * k; t += kBig) {
        const int i = static_cast<int>(t / k), j = static_cast<int>(t % k);
        Linv[t] = (j <= i) ? static_cast<float>(W[t]) : 0.0f;
    }
    if (tid == 0 && status) status[0] = attempt;
}

// ---------------------------------------------------------------------------
// Householder tridiagonalisation of the symmetric W (full storage, in place):
// d[0..k), e[0..k-1), reflector j stored in W[j+1.., j] (first entry 1),
// tau[j].  One workgroup.
// ---------------------------------------------------------------------------
constexpr int kSytrdSegs = 8;  // matvec segments (rows of at most kBig / kSytrdSegs lanes each)
__global__ __launch_bounds__(kBig) void sytrd_kernel(double *__restrict__ W, int k, double *__restrict__ d,
                                                      double *__restrict__ e, double *__restrict__ tau,
                                                      double *__restrict__ vp_ext) {
    extern __shared__ double sm_lds[];  // v[k], p[k], or vp_ext (global) when they do not fit
    double *sm = vp_ext ? vp_ext : sm_lds;
    double *v = sm, *p = sm + k;
    __shared__ double part[kBig];  // the matvec's segment partial sums (segments x padded rows <= kBig)
    __shared__ double red[kBig / 64];
    const int tid = threadIdx.x;
    for (int j = 0; j + 2 < k; ++j) {
        const int n = k - j - 1;  // length of the reflector, rows j+1..k-1
        double sig = 0.0;
        for (int i = 1 + tid; i < n; i += kBig) {
            const double x = W[static_cast<uint64_t>(j + 1 + i) * k + j];
            sig = fma(x, x, sig);
        }
        sig = block_sum(sig, red);
        const double alpha = W[static_cast<uint64_t>(j + 1) * k + j];
        double t = 0.0, beta = alpha;
        if (sig > 0.0) {
            const double nrm = sqrt(fma(alpha, alpha, sig));
            beta = (alpha >= 0.0) ? -nrm : nrm;
            t = (beta - alpha) / beta;
            const double scal = 1.0 / (alpha - beta);
            for (int i = tid; i < n; i += kBig)
                v[i] = (i == 0) ? 1.0 : W[static_cast<uint64_t>(j + 1 + i) * k + j] * scal;
        } else {
            for (int i = tid; i < n; i += kBig) v[i] = (i == 0) ? 1.0 : 0.0;
        }
        __syncthreads();
        if (tid == 0) {
            d[j] = W[static_cast<uint64_t>(j) * k + j];
            e[j] = beta;
            tau[j] = t;
        }
        // store the reflector in column j below the diagonal
        for (int i = tid; i < n; i += kBig) W[static_cast<uint64_t>(j + 1 + i) * k + j] = v[i];
        if (t != 0.0) {
            // p = t * A' v  (A' = trailing block, full symmetric storage):
            // lanes take consecutive rows i (coalesced reads of row c of A',
            // which equals column c by symmetry); while the rows fit in the
            // workgroup, its lanes also split the sum over c into `segs`
            // contiguous segments (shorter dependent chains), combined through
            // LDS
            const int rows_pad = (n + 63) & ~63;  // whole waves per segment
            if (rows_pad <= kBig) {
                const int segs = min(kSytrdSegs, kBig / rows_pad);
                const int seg = tid / rows_pad, i = tid - seg * rows_pad;
                if (seg < segs && i < n) {
                    // eight loads in flight per lane (the operand comes from L2)
                    const int c0 = (n * seg) / segs, c1 = (n * (seg + 1)) / segs;
                    const double *col = W + static_cast<uint64_t>(j + 1) * k + (j + 1 + i);
                    double acc[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
                    int c = c0;
                    for (; c + 8 <= c1; c += 8) {
                        double a[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) a[u] = col[static_cast<uint64_t>(c + u) * k];
#pragma unroll
                        for (int u = 0; u < 8; ++u) acc[u] = fma(a[u], v[c + u], acc[u]);
                    }
                    for (; c < c1; ++c) acc[0] = fma(col[static_cast<uint64_t>(c) * k], v[c], acc[0]);
                    part[seg * rows_pad + i] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) +
                                               ((acc[4] + acc[5]) + (acc[6] + acc[7]));
                }
                __syncthreads();
                for (int i2 = tid; i2 < n; i2 += kBig) {
                    double s = 0.0;
                    for (int g = 0; g < segs; ++g) s += part[g * rows_pad + i2];
                    p[i2] = t * s;
                }
            } else {
                for (int i = tid; i < n; i += kBig) {
                    double s = 0.0;
                    for (int c = 0; c < n; ++c) s = fma(W[static_cast<uint64_t>(j + 1 + c) * k + (j + 1 + i)], v[c], s);
                    p[i] = t * s;
                }
            }
            __syncthreads();
            double pv = 0.0;
            for (int i = tid; i < n; i += kBig) pv = fma(p[i], v[i], pv);
            pv = block_sum(pv, red);
            const double half = 0.5 * t * pv;
            for (int i = tid; i < n; i += kBig) p[i] -= half * v[i];  // p <- w
            __syncthreads();
            // A' -= v w^T + w v^T: wave w takes rows r = w (mod 16), its lanes
            // consecutive columns
            // (eight 512-byte row pieces loaded before any is updated, so a
            // wave keeps eight L2 round trips in flight instead of one)
            const int lane = tid & 63, wave = tid >> 6;
            for (int r = wave; r < n; r += kBig / 64) {
                const double vr = v[r], pr = p[r];
                double *arow = W + static_cast<uint64_t>(j + 1 + r) * k + (j + 1);
                for (int c0 = lane; c0 < n; c0 += 64 * 8) {
                    double a[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) a[u] = (c0 + 64 * u < n) ? arow[c0 + 64 * u] : 0.0;
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int c = c0 + 64 * u;
                        if (c < n) arow[c] = a[u] - (vr * p[c] + pr * v[c]);
                    }
                }
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        if (k >= 2) {
            d[k - 2] = W[static_cast<uint64_t>(k - 2) * k + (k - 2)];
            e[k - 2] = W[static_cast<uint64_t>(k - 1) * k + (k - 2)];
            tau[k - 2] = 0.0;
        }
        d[k - 1] = W[static_cast<uint64_t>(k - 1) * k + (k - 1)];
        if (k >= 1) tau[k - 1] = 0.0;
    }
}

// ---------------------------------------------------------------------------
// Householder tridiagonalisation for 256 < k <= 512, the same reduction
// (LAPACK dsytd2 order: reflector j from column j, p = A v, w = tau p -
// (tau^2 / 2)(p.v) v, A -= v w^T + w v^T) spread over two kernels per column
// on a global-memory working copy A (full symmetric storage):
//   trd_step_kernel (one launch per column, many CUs): every workgroup
//     forms w_{j-1} from p_{j-1}, row j of A with update j-1 applied (its
//     column by symmetry) and reflector j; workgroup 0 writes d[j], e[j],
//     tau[j] and row j of H (zero up to column j); then one wave per row of
//     the trailing block applies update j-1 and forms p_j = A v_j in the
//     same pass;
//   trd_col_kernel (one workgroup) finishes the last column: w_{k-3},
//     d[k-2], e[k-2] and d[k-1].
// Every column thus costs one launch and one read and write of the
// trailing block on all CUs, instead of two reads and a write on one CU.
// ---------------------------------------------------------------------------
constexpr int kTrdColThreads = 512;  // one index per lane (k <= 512)

__global__ __launch_bounds__(kTrdColThreads) void trd_col_kernel(
    const double *__restrict__ A, int k, int j, const double *__restrict__ vprev, const double *__restrict__ p,
    double *__restrict__ w, double *__restrict__ vcur, double *__restrict__ d, double *__restrict__ e,
    double *__restrict__ tau, double *__restrict__ H) {
    __shared__ double red[kTrdColThreads / 64];
    __shared__ double s_wj, s_alpha;
    const int i = threadIdx.x;
    const bool in = i < k;
    // w_{j-1} on indices >= j (zero below): p_{j-1} = A_{j-1} v_{j-1}
    double wi = 0.0, vpi = 0.0;
    if (j > 0) {
        const double tp = tau[j - 1];
        const double pi = (in && i >= j) ? p[i] : 0.0;
        vpi = (in && i >= j) ? vprev[i] : 0.0;
        const double pv = block_sum(pi * vpi, red);
        wi = tp * pi - (0.5 * tp * tp * pv) * vpi;
        if (in) w[i] = wi;
        if (i == j) s_wj = wi;
        __syncthreads();
    }
    // row j with update j-1 applied (v_{j-1}[j] = 1), as trd_step_kernel
    // forms it
    double x = 0.0;
    if (in && i >= j) {
        x = A[static_cast<uint64_t>(j) * k + i];
        if (j > 0) x -= (vprev[j] * wi + s_wj * vpi);
    }
    if (i == j) d[j] = x;
    if (i == j + 1) s_alpha = x;
    const double sig = block_sum((in && i >= j + 2) ? x * x : 0.0, red);
    const double alpha = s_alpha;  // written before block_sum's barriers
    double t = 0.0, beta = alpha, scal = 0.0;
    if (sig > 0.0) {
        const double nrm = sqrt(fma(alpha, alpha, sig));
        beta = (alpha >= 0.0) ? -nrm : nrm;
        t = (beta - alpha) / beta;
        scal = 1.0 / (alpha - beta);
    }
    if (in) {
        const double v = (i == j + 1) ? 1.0 : ((i > j + 1) ? x * scal : 0.0);
        vcur[i] = v;
        H[static_cast<uint64_t>(j) * k + i] = v;
    }
    if (i == 0) {
        e[j] = beta;
        tau[j] = t;
    }
    if (j == k - 2) {  // the last call: d[k-1] with update k-3, H's last row zero
        if (i == k - 1) {
            d[k - 1] = A[static_cast<uint64_t>(k - 1) * k + (k - 1)] - (vpi * wi + wi * vpi);
            tau[k - 1] = 0.0;
        }
        if (in) H[static_cast<uint64_t>(k - 1) * k + i] = 0.0;
    }
}

// One column step j = 0 .. k-3 in one launch: every workgroup forms w_{j-1}
// and reflector j itself from the same data in the same order (so they all
// hold the same bits; workgroup 0 writes d[j], e[j], tau[j] and row j of H),
// then its waves take one trailing row each: update j-1 applied, p_j = A v_j.
// p is double-buffered: this launch reads p_{j-1} in every workgroup while
// others already write p_j.
constexpr int kTrdStepThreads = 512;  // one index per lane (k <= 512), 8 rows per workgroup
__global__ __launch_bounds__(kTrdStepThreads) void trd_step_kernel(
    double *__restrict__ A, int k, int j, const double *__restrict__ pprev, double *__restrict__ pout,
    double *__restrict__ d, double *__restrict__ e, double *__restrict__ tau, double *__restrict__ H) {
    __shared__ double red[kTrdStepThreads / 64];
    __shared__ double s_wj, s_alpha;
    __shared__ double sw[kTrdStepThreads], svp[kTrdStepThreads], sv[kTrdStepThreads];
    const int i = threadIdx.x;
    const bool in = i < k;
    const bool lead = blockIdx.x == 0;
    // this wave's trailing row, requested first: its loads do not depend on
    // the reflector, so their latency overlaps the two reductions below
    const int lane = i & 63;
    const int r = j + 1 + static_cast<int>(blockIdx.x) * (kTrdStepThreads / 64) + (i >> 6);
    constexpr int kMaxIt = kTrdStepThreads / 64;  // k <= 512: at most 8 columns per lane
    double *row = A + static_cast<uint64_t>(r < k ? r : j) * k;
    double a[kMaxIt];
#pragma unroll
    for (int u = 0; u < kMaxIt; ++u) {
        const int c = j + 1 + lane + 64 * u;
        a[u] = (r < k && c < k) ? row[c] : 0.0;
    }
    // w_{j-1} on indices >= j (zero below); v_{j-1} is row j-1 of H
    double wi = 0.0, vpi = 0.0;
    if (j > 0) {
        const double tp = tau[j - 1];
        const double pi = (in && i >= j) ? pprev[i] : 0.0;
        vpi = (in && i >= j) ? H[static_cast<uint64_t>(j - 1) * k + i] : 0.0;
        const double pv = block_sum(pi * vpi, red);
        wi = tp * pi - (0.5 * tp * tp * pv) * vpi;
        if (i == j) s_wj = wi;
        __syncthreads();
    }
    sw[i] = wi;
    svp[i] = vpi;
    // row j with update j-1 applied (v_{j-1}[j] = 1)
    double x = 0.0;
    if (in && i >= j) {
        x = A[static_cast<uint64_t>(j) * k + i];
        if (j > 0) x -= (H[static_cast<uint64_t>(j - 1) * k + j] * wi + s_wj * vpi);
    }
    if (lead && i == j) d[j] = x;
    if (i == j + 1) s_alpha = x;
    const double sig = block_sum((in && i >= j + 2) ? x * x : 0.0, red);
    const double alpha = s_alpha;
    double t = 0.0, beta = alpha, scal = 0.0;
    if (sig > 0.0) {
        const double nrm = sqrt(fma(alpha, alpha, sig));
        beta = (alpha >= 0.0) ? -nrm : nrm;
        t = (beta - alpha) / beta;
        scal = 1.0 / (alpha - beta);
    }
    const double v = (in && i == j + 1) ? 1.0 : ((in && i > j + 1) ? x * scal : 0.0);
    sv[i] = v;
    if (lead) {
        if (in) H[static_cast<uint64_t>(j) * k + i] = v;
        if (i == 0) {
            e[j] = beta;
            tau[j] = t;
        }
    }
    __syncthreads();
    // trailing rows: update j-1, then p_j = A v_j
    if (r >= k) return;  // whole waves, after the last barrier
    const bool upd = j > 0;
    const double vr = svp[r], wr = sw[r];
    double acc = 0.0;
#pragma unroll
    for (int u = 0; u < kMaxIt; ++u) {
        const int c = j + 1 + lane + 64 * u;
        if (c < k) {
            if (upd) {
                a[u] -= (vr * sw[c] + wr * svp[c]);
                row[c] = a[u];
            }
            acc = fma(a[u], sv[c], acc);
        }
    }
    acc = wave_sum_dpp(acc);
    if (lane == 0) pout[r] = acc;
}

// Number of eigenvalues of the tridiagonal (d, e) strictly below x.
__device__ int sturm_count(const double *d, const double *e2, int k, double x, double pivmin) {
    int cnt = 0;
    double q = d[0] - x;
    if (fabs(q) < pivmin) q = -pivmin;
    cnt += (q < 0.0);
    for (int i = 1; i < k; ++i) {
        // hardware reciprocal + one Newton step (~46 bits) instead of an IEEE
        // division: only the sign of q is used, and only near an eigenvalue
        double r = __builtin_amdgcn_rcp(q);
        r = fma(r, fma(-q, r, 1.0), r);
        q = fma(-e2[i - 1], r, d[i] - x);
        if (fabs(q) < pivmin) q = -pivmin;
        cnt += (q < 0.0);
    }
    return cnt;
}

__device__ void trid_factor(const double *d, const double *e, int k, double lam, double tiny, double *u0,
                            double *u1, double *u2, double *ml, int *piv, int st) {
    double dcur = d[0] - lam, ecur = (k > 1) ? e[0] : 0.0;
    for (int i = 0; i < k - 1; ++i) {
        const double sub = e[i];                        // T[i+1][i]
        const double dn = d[i + 1] - lam;               // T[i+1][i+1]
        const double en = (i + 2 < k) ? e[i + 1] : 0.0;  // T[i+1][i+2]
        if (fabs(dcur) >= fabs(sub)) {
            piv[i * st] = 0;
            const double p = (dcur == 0.0) ? tiny : dcur;
            const double m = sub / p;
            ml[i * st] = m;
            u0[i * st] = p;
            u1[i * st] = ecur;
            u2[i * st] = 0.0;
            dcur = dn - m * ecur;
            ecur = en;
        } else {
            piv[i * st] = 1;
            const double m = dcur / sub;
            ml[i * st] = m;
            u0[i * st] = sub;
            u1[i * st] = dn;
            u2[i * st] = en;
            dcur = ecur - m * dn;
            ecur = -m * en;
        }
    }
    u0[(k - 1) * st] = (fabs(dcur) < tiny) ? (dcur < 0.0 ? -tiny : tiny) : dcur;
}

__device__ void trid_apply(int k, double tiny, const double *__restrict__ u0, const double *__restrict__ u1,
                           const double *__restrict__ u2, const double *__restrict__ ml,
                           const int *__restrict__ piv, int st, double *__restrict__ b, int bst) {
    // forward: the running pair (cur = b[i], nxt = b[i + 1]) stays in registers
    double cur = b[0];
    for (int i = 0; i < k - 1; ++i) {
        double nxt = b[(i + 1) * bst];
        if (piv[i * st]) {
            const double t = cur;
            cur = nxt;
            nxt = t;
        }
        nxt -= ml[i * st] * cur;
        b[i * bst] = cur;
        cur = nxt;
    }
    b[(k - 1) * bst] = cur;
    // backward: x[i] needs x[i + 1], x[i + 2] (registers)
    double x1 = 0.0, x2 = 0.0;
    for (int i = k - 1; i >= 0; --i) {
        double s = b[i * bst];
        if (i + 1 < k) s -= u1[i * st] * x1;
        if (i + 2 < k) s -= u2[i * st] * x2;
        double p = u0[i * st];
        if (fabs(p) < tiny) p = (p < 0.0) ? -tiny : tiny;
        const double x = s / p;
        b[i * bst] = x;
        x2 = x1;
        x1 = x;
    }
}

__device__ __forceinline__ double start_entry(int t, int i) {
    // deterministic pseudo-random start vector
    uint32_t h = static_cast<uint32_t>(t) * 0x9E3779B9u ^ (static_cast<uint32_t>(i) + 0x7F4A7C15u) * 0x85EBCA6Bu;
    h ^= h >> 13;
    h *= 0xC2B2AE35u;
    h ^= h >> 16;
    return 0.5 + static_cast<double>(h & 0xFFFF) / 65536.0;
}

// Inverse iteration, one thread per eigenvalue: Z[t][0..k) = eigenvector of
// the tridiagonal for lambda[t].  Scratch is interleaved across threads
// (element i of thread t at i * k + t): 5 k doubles + k ints per thread.
__global__ void invit_kernel(const double *__restrict__ d, const double *__restrict__ e, int k,
                             const double *__restrict__ lambda, const double *__restrict__ tnorm_p,
                             double *__restrict__ Z, double *__restrict__ scratch, int *__restrict__ iscratch) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= k) return;
    const double tnorm = fmax(tnorm_p[0], DBL_MIN);
    const double tiny = tnorm * DBL_EPSILON;
    const uint64_t kk = static_cast<uint64_t>(k) * k;
    double *u0 = scratch + t, *u1 = u0 + kk, *u2 = u1 + kk, *ml = u2 + kk, *b = ml + kk;
    int *piv = iscratch + t;
    trid_factor(d, e, k, lambda[t], tiny, u0, u1, u2, ml, piv, k);
    for (int i = 0; i < k; ++i) b[static_cast<uint64_t>(i) * k] = start_entry(t, i);
    for (int it = 0; it < 3; ++it) {
        trid_apply(k, tiny, u0, u1, u2, ml, piv, k, b, k);
        double nrm = 0.0;
        for (int i = 0; i < k; ++i) nrm = fma(b[static_cast<uint64_t>(i) * k], b[static_cast<uint64_t>(i) * k], nrm);
        const double inv = nrm > 0.0 ? 1.0 / sqrt(nrm) : 0.0;
        for (int i = 0; i < k; ++i) b[static_cast<uint64_t>(i) * k] *= inv;
    }
    double *z = Z + static_cast<uint64_t>(t) * k;
    for (int i = 0; i < k; ++i) z[i] = b[static_cast<uint64_t>(i) * k];
}

// LDS variant of trid_factor / trid_apply for invit_lds_kernel.  Each
// recurrence runs one eigenvalue per lane, so its operands are staged in
// registers one chunk of kInvChunk steps ahead: the LDS round trips of a
// chunk overlap the arithmetic of the one before (a load issued at the step
// that needs it would put an LDS round trip on every step).  The pivots are
// stored as reciprocals so the backward pass has no division.
constexpr int kInvChunk = 8;
constexpr int kInvPad = 2 * kInvChunk;  // zero entries after d and e

// one elimination step of P (T - lam I) = L U; returns the new dcur.  The
// multiplier is the quotient num / p from the hardware reciprocal with one
// correction step (m0 + r0 (num - p m0)).  The pivot itself is stored
// (zero replaced by tiny): its reciprocal is refined afterwards by all lanes.
__device__ __forceinline__ double tridl_step(double dcur, double &ecur, double sub, double dn, double en,
                                             double tiny, double *__restrict__ pv, double *__restrict__ u1,
                                             double *__restrict__ u2, double *__restrict__ ml,
                                             int *__restrict__ piv, int at) {
    const bool keep = fabs(dcur) >= fabs(sub);
    const double p = keep ? ((dcur == 0.0) ? tiny : dcur) : sub;
    const double num = keep ? sub : dcur;
    const double r0 = __builtin_amdgcn_rcp(p);
    const double m0 = num * r0;
    const double m = fma(r0, fma(-p, m0, num), m0);
    piv[at] = keep ? 0 : 1;
    ml[at] = m;
    pv[at] = p;
    u1[at] = keep ? ecur : dn;
    u2[at] = keep ? 0.0 : en;
    const double ndcur = fma(-m, keep ? ecur : dn, keep ? dn : ecur);
    ecur = keep ? en : -m * en;
    return ndcur;
}

// 1 / p as the back substitution uses it: the hardware reciprocal and two
// Newton steps, pivots below tiny replaced by +-tiny
__device__ __forceinline__ double tridl_pivot_inverse(double p, double tiny, double inv_tiny) {
    double rp = __builtin_amdgcn_rcp(p);
    rp = fma(rp, fma(-p, rp, 1.0), rp);
    rp = fma(rp, fma(-p, rp, 1.0), rp);
    return (fabs(p) < tiny) ? (p < 0.0 ? -inv_tiny : inv_tiny) : rp;
}

// d, e: the tridiagonal in LDS, e[k - 1 ..] and d[k ..] zero (kInvPad
// entries); per-eigenvalue arrays with stride ST
template <int ST>
__device__ void tridl_factor(const double *__restrict__ d, const double *__restrict__ e, int k, double lam,
                             double tiny, double *__restrict__ u0inv, double *__restrict__ pv,
                             double *__restrict__ u1, double *__restrict__ u2, double *__restrict__ ml,
                             int *__restrict__ piv) {
    constexpr int C = kInvChunk;
    double dcur = d[0] - lam, ecur = e[0];
    double dq[C], eq[C + 1];  // step i0 + s: d[i0 + 1 + s], e[i0 + s], e[i0 + 1 + s]
#pragma unroll
    for (int s = 0; s < C; ++s) dq[s] = d[1 + s];
#pragma unroll
    for (int s = 0; s <= C; ++s) eq[s] = e[s];
    int i0 = 0;
    for (; i0 + C <= k - 1; i0 += C) {
        double dx[C], ex[C + 1];
#pragma unroll
        for (int s = 0; s < C; ++s) dx[s] = d[i0 + C + 1 + s];
#pragma unroll
        for (int s = 0; s <= C; ++s) ex[s] = e[i0 + C + s];
#pragma unroll
        for (int s = 0; s < C; ++s)
            dcur = tridl_step(dcur, ecur, eq[s], dq[s] - lam, eq[s + 1], tiny, pv, u1, u2, ml, piv, (i0 + s) * ST);
#pragma unroll
        for (int s = 0; s < C; ++s) dq[s] = dx[s];
#pragma unroll
        for (int s = 0; s <= C; ++s) eq[s] = ex[s];
    }
#pragma unroll
    for (int s = 0; s < C; ++s)  // fewer than C steps left, operands already staged
        if (i0 + s < k - 1)
            dcur = tridl_step(dcur, ecur, eq[s], dq[s] - lam, eq[s + 1], tiny, pv, u1, u2, ml, piv, (i0 + s) * ST);
    u0inv[(k - 1) * ST] = 1.0 / ((fabs(dcur) < tiny) ? (dcur < 0.0 ? -tiny : tiny) : dcur);
}

// Right-hand side of a solve: the iterate b (stride ST) scaled by `scale` as
// it is read.
template <int ST>
struct InvRhs {
    const double *b;
    double scale;
    __device__ __forceinline__ double operator()(int i) const { return b[i * ST] * scale; }
};

// (T - lam I) x = rhs from the factors; x (stride st) may be the array rhs
// reads.  u1 / u2 must be zero in row k - 1 and u2 in row k - 2.  Returns
// sum x_i^2.
template <int st, class Rhs>
__device__ double tridl_solve(int k, const double *__restrict__ u0inv, const double *__restrict__ u1,
                              const double *__restrict__ u2, const double *__restrict__ ml,
                              const int *__restrict__ piv, const Rhs &rhs, double *__restrict__ y, double *x) {
    constexpr int C = kInvChunk;
    // forward elimination rhs -> y (step i: rhs(i + 1), piv[i], ml[i])
    double cur = rhs(0);
    {
        double nb[C], mq[C];
        int pq[C];
        const int full = (k - 1) / C * C;
        if (full > 0) {
#pragma unroll
            for (int s = 0; s < C; ++s) {
                nb[s] = rhs(1 + s);
                mq[s] = ml[s * st];
                pq[s] = piv[s * st];
            }
        }
        for (int i0 = 0; i0 < full; i0 += C) {
            double nbx[C], mx[C];
            int px[C];
            if (i0 + C < full) {
#pragma unroll
                for (int s = 0; s < C; ++s) {
                    nbx[s] = rhs(i0 + C + 1 + s);
                    mx[s] = ml[(i0 + C + s) * st];
                    px[s] = piv[(i0 + C + s) * st];
                }
            }
#pragma unroll
            for (int s = 0; s < C; ++s) {
                const bool sw = pq[s] != 0;
                double nxt = sw ? cur : nb[s];
                cur = sw ? nb[s] : cur;
                nxt = fma(-mq[s], cur, nxt);
                y[(i0 + s) * st] = cur;
                cur = nxt;
            }
#pragma unroll
            for (int s = 0; s < C; ++s) {
                nb[s] = nbx[s];
                mq[s] = mx[s];
                pq[s] = px[s];
            }
        }
        for (int i = full; i < k - 1; ++i) {
            const double v = rhs(i + 1);
            const bool sw = piv[i * st] != 0;
            double nxt = sw ? cur : v;
            cur = sw ? v : cur;
            nxt = fma(-ml[i * st], cur, nxt);
            y[i * st] = cur;
            cur = nxt;
        }
        y[(k - 1) * st] = cur;
    }
    // back substitution y -> x; the term of the older unknown is added first
    double x1 = 0.0, x2 = 0.0, n0 = 0.0, n1 = 0.0;
    {
        double yq[C], aq[C], bq[C], rq[C];  // step i = top - s
        const int rem = k % C;  // the top rem rows first, then full chunks
        int top = k - 1;
        for (; top >= k - rem; --top) {
            const double s1 = fma(-u2[top * st], x2, y[top * st]);
            const double xi = fma(-u1[top * st], x1, s1) * u0inv[top * st];
            x[top * st] = xi;
            n0 = fma(xi, xi, n0);
            x2 = x1;
            x1 = xi;
        }
        if (top >= 0) {
#pragma unroll
            for (int s = 0; s < C; ++s) {
                const int i = top - s;
                yq[s] = y[i * st];
                aq[s] = u1[i * st];
                bq[s] = u2[i * st];
                rq[s] = u0inv[i * st];
            }
        }
        for (; top >= 0; top -= C) {
            double yx[C], ax[C], bx[C], rx[C];
            if (top - C >= 0) {
#pragma unroll
                for (int s = 0; s < C; ++s) {
                    const int i = top - C - s;
                    yx[s] = y[i * st];
                    ax[s] = u1[i * st];
                    bx[s] = u2[i * st];
                    rx[s] = u0inv[i * st];
                }
            }
#pragma unroll
            for (int s = 0; s < C; ++s) {
                const double s1 = fma(-bq[s], x2, yq[s]);
                const double xi = fma(-aq[s], x1, s1) * rq[s];
                x[(top - s) * st] = xi;
                if (s & 1) n1 = fma(xi, xi, n1);
                else n0 = fma(xi, xi, n0);
                x2 = x1;
                x1 = xi;
            }
#pragma unroll
            for (int s = 0; s < C; ++s) {
                yq[s] = yx[s];
                aq[s] = ax[s];
                bq[s] = bx[s];
                rq[s] = rx[s];
            }
        }
    }
    return n0 + n1;
}

// The same inverse iteration with every per-eigenvalue array in LDS: lane j
// (< P) of a one-wave workgroup runs the recurrences of eigenvalue
// blockIdx.x * P + j, its element i at i * P + j (P a compile-time stride, so
// the chunked loads and stores take immediate offsets).  The work off those
// chains (start vectors, refined pivot reciprocals, the scaled output) is
// spread over all 64 lanes.
template <int P>
__global__ __launch_bounds__(64) void invit_lds_kernel(const double *__restrict__ d, const double *__restrict__ e,
                                                       int k, const double *__restrict__ lambda,
                                                       const double *__restrict__ tnorm_p, double *__restrict__ Z) {
    extern __shared__ double sm[];
    __shared__ double nrm_inv[P];
    const uint64_t kp = static_cast<uint64_t>(k) * P;
    double *u0 = sm, *u1 = u0 + kp, *u2 = u1 + kp, *ml = u2 + kp, *b = ml + kp, *yv = b + kp, *ds = yv + kp,
           *es = ds + k + kInvPad;
    int *piv = reinterpret_cast<int *>(es + k + kInvPad);
    const int lane = threadIdx.x, t0 = blockIdx.x * P;
    const double tnorm = fmax(tnorm_p[0], DBL_MIN);
    const double tiny = tnorm * DBL_EPSILON, inv_tiny = 1.0 / tiny;
    for (int i = lane; i < k + kInvPad; i += 64) {
        ds[i] = (i < k) ? d[i] : 0.0;
        es[i] = (i + 1 < k) ? e[i] : 0.0;
    }
    // start vectors; the rows of u1 / u2 the factorisation leaves unwritten but
    // the back substitution reads (times a zero unknown)
    for (int q = lane; q < k * P; q += 64) b[q] = start_entry(t0 + q % P, q / P);
    if (lane < P) {
        u1[(k - 1) * P + lane] = 0.0;
        u2[(k - 1) * P + lane] = 0.0;
        if (k >= 2) u2[(k - 2) * P + lane] = 0.0;
    }
    __syncthreads();
    const int j = lane, t = t0 + j;
    const bool mine = j < P && t < k;
    if (mine) tridl_factor<P>(ds, es, k, lambda[t], tiny, u0 + j, yv + j, u1 + j, u2 + j, ml + j, piv + j);
    __syncthreads();
    for (int q = lane; q < (k - 1) * P; q += 64) u0[q] = tridl_pivot_inverse(yv[q], tiny, inv_tiny);
    __syncthreads();
    if (mine) {
        // two solves: lambda is within k * eps * ||T|| of the eigenvalue, so one
        // solve already grows the wanted component by ~1 / (k eps) over components
        // separated by more than the clustering tolerance (closer ones are redone
        // by cluster_kernel); the second leaves the iterate at working accuracy.
        // The first iterate's normalisation is applied as the second solve reads it.
        const double n1 = tridl_solve<P>(k, u0 + j, u1 + j, u2 + j, ml + j, piv + j, InvRhs<P>{b + j, 1.0},
                                         yv + j, b + j);
        const double n2 = tridl_solve<P>(k, u0 + j, u1 + j, u2 + j, ml + j, piv + j,
                                         InvRhs<P>{b + j, n1 > 0.0 ? 1.0 / sqrt(n1) : 0.0}, yv + j, b + j);
        nrm_inv[j] = n2 > 0.0 ? 1.0 / sqrt(n2) : 0.0;
    }
    __syncthreads();
    const int np = min(P, k - t0);
    for (int q = lane; q < np * k; q += 64) {
        const int jj = q / k, i = q - jj * k;
        Z[static_cast<uint64_t>(t0 + jj) * k + i] = b[i * P + jj] * nrm_inv[jj];
    }
}

// Re-runs inverse iteration for eigenvalue clusters (gap below
// 1e-9 * ||T||), one workgroup per cluster, orthogonalising each member
// against the earlier members after every solve.
__global__ void cluster_kernel(const double *__restrict__ d, const double *__restrict__ e, int k,
                               const double *__restrict__ lambda, const double *__restrict__ tnorm_p,
                               double *__restrict__ Z, double *__restrict__ scratch, int *__restrict__ iscratch) {
    __shared__ double red[16];
    __shared__ double bcast;
    const int c0 = blockIdx.x;
    const double tnorm = fmax(tnorm_p[0], DBL_MIN);
    const double tol = 1e-9 * tnorm;
    auto close = [&](int a) { return fabs(lambda[a] - lambda[a + 1]) <= tol; };
    if (c0 + 1 >= k || !close(c0)) return;
    if (c0 > 0 && close(c0 - 1)) return;  // not the first member
    int c1 = c0 + 1;
    while (c1 + 1 < k && close(c1)) ++c1;
    const double tiny = tnorm * DBL_EPSILON;
    // private region: the cluster's first index owns rows c0 of the
    // interleaved scratch planes, used here with stride 1 over a k block
    double *sc = scratch + 5ull * k * k + static_cast<uint64_t>(c0) * 4 * k;
    int *piv = iscratch + static_cast<uint64_t>(k) * k + static_cast<uint64_t>(c0) * k;
    for (int t = c0; t <= c1; ++t) {
        double *b = Z + static_cast<uint64_t>(t) * k;
        for (int i = threadIdx.x; i < k; i += blockDim.x) b[i] = start_entry(t + 977, i) - 0.5;
        if (threadIdx.x == 0) trid_factor(d, e, k, lambda[t], tiny, sc, sc + k, sc + 2 * k, sc + 3 * k, piv, 1);
        __syncthreads();
        for (int it = 0; it < 3; ++it) {
            if (threadIdx.x == 0) trid_apply(k, tiny, sc, sc + k, sc + 2 * k, sc + 3 * k, piv, 1, b, 1);
            __syncthreads();
            for (int pass = 0; pass < 2; ++pass) {
                for (int s = c0; s < t; ++s) {
                    const double *z = Z + static_cast<uint64_t>(s) * k;
                    double dot = 0.0;
                    for (int i = threadIdx.x; i < k; i += blockDim.x) dot = fma(z[i], b[i], dot);
                    dot = block_sum(dot, red);
                    for (int i = threadIdx.x; i < k; i += blockDim.x) b[i] -= dot * z[i];
                    __syncthreads();
                }
            }
            double nrm = 0.0;
            for (int i = threadIdx.x; i < k; i += blockDim.x) nrm = fma(b[i], b[i], nrm);
            nrm = block_sum(nrm, red);
            if (threadIdx.x == 0) bcast = nrm > 0.0 ? 1.0 / sqrt(nrm) : 0.0;
            __syncthreads();
            const double inv = bcast;
            for (int i = threadIdx.x; i < k; i += blockDim.x) b[i] *= inv;
            __syncthreads();
        }
    }
}

// Back-transformation: u_t = H_0 H_1 ... H_{k-3} z_t, one wave per
// eigenvector; writes Uh[i][t] (FP32, row-major k x k).  Lane l owns the
// rows i = l + 64 m for every reflector (entries above the reflector's first
// row are masked), so each lane only ever reads back its own stores of z.
__global__ void backtransform_kernel(const double *__restrict__ W, const double *__restrict__ tau, int k,
                                     double *__restrict__ Z, float *__restrict__ Uh) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (t >= k) return;
    double *z = Z + static_cast<uint64_t>(t) * k;
    for (int j = k - 3; j >= 0; --j) {
        const double tj = tau[j];
        if (tj == 0.0) continue;
        // v has v[0] = 1 at row j+1, then W[j+2.., j]
        const int i0 = (j + 1) & ~63;  // first 64-row group touching rows >= j+1
        double s = 0.0;
        for (int i = i0 + lane; i < k; i += 64) {
            if (i <= j) continue;
            const double vi = (i == j + 1) ? 1.0 : W[static_cast<uint64_t>(i) * k + j];
            s = fma(vi, z[i], s);
        }
        for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
        s *= tj;
        for (int i = i0 + lane; i < k; i += 64) {
            if (i <= j) continue;
            const double vi = (i == j + 1) ? 1.0 : W[static_cast<uint64_t>(i) * k + j];
            z[i] -= s * vi;
        }
    }
    for (int i = lane; i < k; i += 64) Uh[static_cast<uint64_t>(i) * k + t] = static_cast<float>(z[i]);
}

// Bisection by multisection: one workgroup of kMsThreads lanes per
// eigenvalue, kMsThreads - 1 interior points per pass (8 bits of the
// interval per pass with 256 lanes).  Each Sturm count is a sequential
// recurrence, so a pass costs one count's latency however many lanes share
// it, and more lanes mean fewer passes.  lambda[t] = t-th largest eigenvalue.
constexpr int kMsThreads = 256;
// e2[i] = e[i]^2 (i < k - 1), 0 for i = k - 1: the squared off-diagonal read
// from global memory by multisect_kernel when d and e2 do not fit in LDS.
__global__ void square_offdiag_kernel(const double *__restrict__ e, int k, double *__restrict__ e2) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < k) e2[i] = (i + 1 < k) ? e[i] * e[i] : 0.0;
}

template <bool GLOBAL>
__global__ __launch_bounds__(kMsThreads) void multisect_kernel(const double *__restrict__ d,
                                                               const double *__restrict__ e, int k,
                                                               double *__restrict__ lambda,
                                                               double *__restrict__ tnorm_out,
                                                               const double *__restrict__ e2g) {
    extern __shared__ double sm[];  // d[k], e2[k] (LDS variant)
    double *sd = GLOBAL ? const_cast<double *>(d) : sm;
    double *se2 = GLOBAL ? const_cast<double *>(e2g) : sm + k;
    constexpr int W = kMsThreads / 64;
    __shared__ double red[3][W];
    __shared__ unsigned long long masks[W];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double lo = 1e300, hi = -1e300, emax = 0.0;
    for (int i = tid; i < k; i += kMsThreads) {
        const double ei = (i + 1 < k) ? e[i] : 0.0;
        if (!GLOBAL) {
            sd[i] = d[i];
            se2[i] = ei * ei;
        }
        const double r = (i > 0 ? fabs(e[i - 1]) : 0.0) + fabs(ei);
        lo = fmin(lo, d[i] - r);
        hi = fmax(hi, d[i] + r);
        emax = fmax(emax, ei * ei);
    }
    for (int off = 32; off >= 1; off >>= 1) {
        lo = fmin(lo, __shfl_xor(lo, off));
        hi = fmax(hi, __shfl_xor(hi, off));
        emax = fmax(emax, __shfl_xor(emax, off));
    }
    if (lane == 0) {
        red[0][wave] = lo;
        red[1][wave] = hi;
        red[2][wave] = emax;
    }
    __syncthreads();
    lo = red[0][0];
    hi = red[1][0];
    emax = red[2][0];
    for (int w = 1; w < W; ++w) {
        lo = fmin(lo, red[0][w]);
        hi = fmax(hi, red[1][w]);
        emax = fmax(emax, red[2][w]);
    }
    const double tnorm = fmax(fabs(lo), fabs(hi));
    const double pivmin = DBL_MIN * fmax(1.0, emax) * 4.0;
    lo -= 2.0 * tnorm * DBL_EPSILON * k + pivmin;
    hi += 2.0 * tnorm * DBL_EPSILON * k + pivmin;
    const int t = blockIdx.x;
    const int target = k - 1 - t;  // ascending index of the wanted eigenvalue
    double a = lo, b = hi;
    // absolute tolerance k * eps * ||T|| (a backward-stable eigenvalue is not more
    // accurate than that)
    const double abstol = static_cast<double>(k) * DBL_EPSILON * tnorm + pivmin;
    for (int pass = 0; pass < 40; ++pass) {  // a, b and the exits are uniform
        if (b - a <= 2.0 * DBL_EPSILON * fmax(fabs(a), fabs(b)) + abstol) break;
        const double h = (b - a) / static_cast<double>(kMsThreads);
        const double x = a + h * (tid + 1);  // lanes 0..kMsThreads-2 interior, the last = b
        const int cnt = (tid < kMsThreads - 1) ? sturm_count(sd, se2, k, x, pivmin) : k + 1;
        // smallest point whose count exceeds target bounds the eigenvalue from above
        const unsigned long long above = __ballot(cnt > target);
        __syncthreads();  // the previous pass's masks are read
        if (lane == 0) masks[wave] = above;
        __syncthreads();
        int first = kMsThreads - 1;  // always found (the last lane)
        for (int w = W - 1; w >= 0; --w)
            if (masks[w]) first = w * 64 + __ffsll(masks[w]) - 1;
        const double nb = a + h * (first + 1);
        const double na = (first == 0) ? a : a + h * first;
        if (!(nb < b) && !(na > a)) break;
        a = na;
        b = fmin(nb, b);
    }
    if (tid == 0) {
        lambda[t] = 0.5 * (a + b);
        if (t == 0 && tnorm_out) tnorm_out[0] = tnorm;
    }
}

// Back-transformation with row-wise reflectors H[j][*]: u_t = H_0 ... H_{k-3} z_t.
// One wave per eigenvector with z in registers (KPL >= ceil(k / 64) values
// per lane); reflector rows are staged through LDS RB at a time and shared
// by the 4 waves of the workgroup; the dot products reduce through DPP.
template <int KPL, int RB = 32>
__global__ __launch_bounds__(256) void backtransform_rows_kernel(const double *__restrict__ H,
                                                                 const double *__restrict__ tau, int k,
                                                                 const double *__restrict__ Z,
                                                                 float *__restrict__ Uh) {
    // RB reflector rows per stage (two stages of RB * KPL * 64 doubles in LDS)
    static_assert(RB % 2 == 0 && (RB * KPL * 64) % 256 == 0, "stage shape");
    constexpr int NQ = RB * KPL * 64 / 256;  // staged doubles per lane
    __shared__ double hs[2][RB][KPL * 64];
    __shared__ double ts[2][RB];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * (blockDim.x >> 6) + wave;
    double z[KPL];
#pragma unroll
    for (int m = 0; m < KPL; ++m) {
        const int i = lane + 64 * m;
        z[m] = (t < k && i < k) ? Z[static_cast<uint64_t>(t) * k + i] : 0.0;
    }
    // stage s covers reflectors j0 = k - 3 - RB s down to max(0, j0 - RB + 1);
    // the next stage is fetched into registers while this one is applied
    double pre[NQ];
    double pt = 0.0;
    auto fetch = [&](int j0) {
        const int jl = max(0, j0 - RB + 1);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int lin = threadIdx.x + 256 * q, rr = lin / (KPL * 64), i = lin % (KPL * 64);
            const int j = j0 - rr;
            pre[q] = (j >= jl && i < k) ? H[static_cast<uint64_t>(j) * k + i] : 0.0;
        }
        pt = (threadIdx.x < RB && j0 - static_cast<int>(threadIdx.x) >= jl) ? tau[j0 - threadIdx.x] : 0.0;
    };
    auto put = [&](int bsel) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int lin = threadIdx.x + 256 * q;
            hs[bsel][lin / (KPL * 64)][lin % (KPL * 64)] = pre[q];
        }
        if (threadIdx.x < RB) ts[bsel][threadIdx.x] = pt;
    };
    int cur = 0;
    if (k - 3 >= 0) {
        fetch(k - 3);
        put(0);
    }
    __syncthreads();
    for (int j0 = k - 3; j0 >= 0; j0 -= RB) {
        const int jl = max(0, j0 - RB + 1);
        const bool more = j0 - RB >= 0;
        if (more) fetch(j0 - RB);
        // reflectors in pairs: a = H_j (applied first) and b = H_{j-1} need
        // v_a.z, v_b.z and v_b.v_a, three independent reductions that overlap,
        // then z -= s_a v_a + s_b v_b with s_b = tau_b (v_b.z - s_a v_b.v_a).
        // Rows past the stage are zero with tau zero and change nothing, so
        // every stage runs all RB rows.
#pragma unroll 2
        for (int rp = 0; rp < RB; rp += 2) {
            const double ta = ts[cur][rp], tb = ts[cur][rp + 1];
            double va[KPL], vb[KPL];
#pragma unroll
            for (int m = 0; m < KPL; ++m) {
                va[m] = hs[cur][rp][lane + 64 * m];
                vb[m] = hs[cur][rp + 1][lane + 64 * m];
            }
            double a = 0.0, b = 0.0, c = 0.0;
#pragma unroll
            for (int m = 0; m < KPL; ++m) {
                a = fma(va[m], z[m], a);
                b = fma(vb[m], z[m], b);
                c = fma(vb[m], va[m], c);
            }
            a = wave_sum_dpp(a);
            b = wave_sum_dpp(b);
            c = wave_sum_dpp(c);
            const double sa = ta * a, sb = tb * fma(-sa, c, b);
#pragma unroll
            for (int m = 0; m < KPL; ++m) z[m] = fma(-sb, vb[m], fma(-sa, va[m], z[m]));
        }
        if (more) put(cur ^ 1);
        __syncthreads();
        cur ^= 1;
    }
    if (t < k) {
#pragma unroll
        for (int m = 0; m < KPL; ++m) {
            const int i = lane + 64 * m;
            if (i < k) Uh[static_cast<uint64_t>(i) * k + t] = static_cast<float>(z[m]);
        }
    }
}

}  // namespace

bool sytrd_blocked_supported(int k);
void launch_sytrd_blocked(const double *G, int k, double *d, double *e, double *tau, double *H, hipStream_t stream);

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
// Row splits of the Gram: at most one workgroup per CU over all lower tiles
// (rounded down: one CU holding two workgroups would double the kernel's
// time), at least 128 rows each (fewer partial matrices to sum).
int gram_splits(int M, int k) {
    const int nt = static_cast<int>(ceil_div(k, kGramTile));
    const int tiles = nt * (nt + 1) / 2;
    const int splits = cu_count() / tiles;
    return std::max(1, std::min(splits, static_cast<int>(ceil_div(M, 128))));
}

uint64_t gram_workspace_bytes(int M, int k) {
    return static_cast<uint64_t>(gram_splits(M, k)) * k * k * sizeof(double);
}

void launch_gram(const float *X, int M, int k, int ld, double *G, double *workspace, hipStream_t stream,
                 double *rowsq) {
    const int nt = static_cast<int>(ceil_div(k, kGramTile));
    const int tiles = nt * (nt + 1) / 2;
    int splits = gram_splits(M, k);
    const int rows_per = static_cast<int>(ceil_div(ceil_div(M, splits), kGramRows) * kGramRows);
    splits = static_cast<int>(ceil_div(M, rows_per));
    const bool vec = (ld % 4 == 0) && (k % 4 == 0) && ((reinterpret_cast<uintptr_t>(X) & 15u) == 0);
    if (vec) gram_mfma_kernel<true><<<dim3(tiles, splits), 256, 0, stream>>>(X, M, k, ld, rows_per, workspace);
    else gram_mfma_kernel<false><<<dim3(tiles, splits), 256, 0, stream>>>(X, M, k, ld, rows_per, workspace);
    BSQ_HIP(hipGetLastError());
    gram_reduce_kernel<<<static_cast<unsigned>(k), 256, 0, stream>>>(workspace, splits, k, G, rowsq);
    BSQ_HIP(hipGetLastError());
}

// Unblocked fallback for ranks above the blocked kernel's range (k > 256).
// Dynamic LDS for `bytes` of per-launch vectors: the byte count when it fits
// beside the kernel's static LDS (raising the launch limit above 64 KiB),
// else 0 and the caller passes a global buffer instead.
size_t dyn_lds_or_zero(const void *kernel, size_t bytes) {
    constexpr size_t kLdsCap = 160 * 1024 - 2048;  // static LDS of these kernels stays below 2 KiB
    if (bytes > kLdsCap) return 0;
    if (bytes > 64 * 1024)
        BSQ_HIP(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
    return bytes;
}

void launch_chol_inv(const double *G, int k, double *W, float *Linv, int *status, double *ext, hipStream_t stream) {
    const size_t lds = dyn_lds_or_zero(reinterpret_cast<const void *>(chol_inv_kernel),
                                       static_cast<size_t>(k) * sizeof(double));
    chol_inv_kernel<<<1, kBig, lds, stream>>>(G, k, W, Linv, status, lds ? nullptr : ext);
    BSQ_HIP(hipGetLastError());
}

// Eigen-decomposition of the symmetric G (k x k FP64): lambda descending,
// Uh[i][t] = component i of eigenvector t (FP32).  `W` k*k doubles, `Z`
// k*k doubles, `small` >= 4k + 8 doubles, `scratch` 9*k*k + 2k doubles,
// `iscratch` 2*k*k ints.
void launch_syev(const double *G, int k, double *W, double *Z, double *small, double *scratch, int *iscratch,
                 double *lambda, float *Uh, hipStream_t stream) {
    BSQ_REQUIRE(k >= 1, "syev: empty matrix");
    double *d = small, *e = small + k, *tau = small + 2 * k, *tn = small + 3 * k;
    // global stand-ins for LDS vectors that do not fit (ranks above ~10000):
    // the last 2k doubles of the scratch, which the inverse-iteration kernels
    // below leave alone (they use 5k^2 + 4k^2 of its 9k^2 + 2k doubles)
    double *ext = scratch + 9ull * k * k;
    const size_t kb = static_cast<size_t>(k) * sizeof(double);
    // reflectors row-wise in W (H[j][i]) from the register kernel (k <= 256)
    // and the per-column kernels (k <= 512), column-wise otherwise
    bool reg = true;
    if (sytrd_blocked_supported(k)) {
        launch_sytrd_blocked(G, k, d, e, tau, W, stream);
    } else if (k > 256 && k <= kTrdColThreads) {
        // working copy and vectors in the scratch, which the eigenvector
        // kernels below only use afterwards
        double *A = scratch, *p0 = scratch + static_cast<size_t>(k) * k, *p1 = p0 + k, *w = p1 + k, *vl = w + k;
        BSQ_HIP(hipMemcpyAsync(A, G, static_cast<size_t>(k) * k * sizeof(double), hipMemcpyDeviceToDevice, stream));
        // one launch per reflector j = 0 .. k-3, then the last column
        for (int j = 0; j + 3 <= k; ++j) {
            const unsigned rows = static_cast<unsigned>(k - j - 1);
            trd_step_kernel<<<static_cast<unsigned>(ceil_div(rows, kTrdStepThreads / 64)), kTrdStepThreads, 0,
                              stream>>>(A, k, j, (j & 1) ? p0 : p1, (j & 1) ? p1 : p0, d, e, tau, W);
        }
        const int jl = k - 2;  // p_{k-3} was written by step k-3 into ((k-3) & 1) ? p1 : p0
        trd_col_kernel<<<1, kTrdColThreads, 0, stream>>>(A, k, jl, W + static_cast<size_t>(jl - 1) * k,
                                                         ((jl - 1) & 1) ? p1 : p0, w, vl, d, e, tau, W);
    } else {
        reg = false;
        BSQ_HIP(hipMemcpyAsync(W, G, static_cast<size_t>(k) * k * sizeof(double), hipMemcpyDeviceToDevice, stream));
        const size_t lds = dyn_lds_or_zero(reinterpret_cast<const void *>(sytrd_kernel), 2 * kb);
        sytrd_kernel<<<1, kBig, lds, stream>>>(W, k, d, e, tau, lds ? nullptr : ext);
    }
    BSQ_HIP(hipGetLastError());
    const size_t ms_lds = dyn_lds_or_zero(reinterpret_cast<const void *>(multisect_kernel<false>), 2 * kb);
    if (ms_lds) {
        multisect_kernel<false><<<k, kMsThreads, ms_lds, stream>>>(d, e, k, lambda, tn, nullptr);
    } else {
        square_offdiag_kernel<<<static_cast<unsigned>(ceil_div(k, 256)), 256, 0, stream>>>(e, k, ext);
        BSQ_HIP(hipGetLastError());
        multisect_kernel<true><<<k, kMsThreads, 0, stream>>>(d, e, k, lambda, tn, ext);
    }
    BSQ_HIP(hipGetLastError());
    // eigenvalues per workgroup whose LDS arrays fit: (6kP + 2(k + pad)) doubles + kP ints
    const int64_t lds_cap = 160 * 1024;
    const int64_t pad_bytes = 16 * (static_cast<int64_t>(k) + kInvPad);
    const int P = static_cast<int>(std::min<int64_t>(8, (lds_cap - pad_bytes) / (52 * static_cast<int64_t>(k))));
    if (P >= 1) {
        const size_t lds = (6 * static_cast<size_t>(k) * P + 2 * (k + kInvPad)) * sizeof(double) +
                           static_cast<size_t>(k) * P * sizeof(int);
        auto launch = [&](auto kernel) {
            BSQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
            kernel<<<static_cast<unsigned>(ceil_div(k, P)), 64, lds, stream>>>(d, e, k, lambda, tn, Z);
        };
        switch (P) {
            case 1: launch(invit_lds_kernel<1>); break;
            case 2: launch(invit_lds_kernel<2>); break;
            case 3: launch(invit_lds_kernel<3>); break;
            case 4: launch(invit_lds_kernel<4>); break;
            case 5: launch(invit_lds_kernel<5>); break;
            case 6: launch(invit_lds_kernel<6>); break;
            case 7: launch(invit_lds_kernel<7>); break;
            default: launch(invit_lds_kernel<8>); break;
        }
    } else {
        invit_kernel<<<static_cast<unsigned>(ceil_div(k, 64)), 64, 0, stream>>>(d, e, k, lambda, tn, Z, scratch,
                                                                               iscratch);
    }
    BSQ_HIP(hipGetLastError());
    cluster_kernel<<<k, 256, 0, stream>>>(d, e, k, lambda, tn, Z, scratch, iscratch);
    BSQ_HIP(hipGetLastError());
    if (reg) {
        // 4 eigenvectors per workgroup: k / 4 CUs share the reflector stream
        const unsigned g = static_cast<unsigned>(ceil_div(k, 4));
        if (k <= 64) backtransform_rows_kernel<1><<<g, 256, 0, stream>>>(W, tau, k, Z, Uh);
        else if (k <= 128) backtransform_rows_kernel<2><<<g, 256, 0, stream>>>(W, tau, k, Z, Uh);
        else if (k <= 192) backtransform_rows_kernel<3><<<g, 256, 0, stream>>>(W, tau, k, Z, Uh);
        else if (k <= 256) backtransform_rows_kernel<4><<<g, 256, 0, stream>>>(W, tau, k, Z, Uh);
        else backtransform_rows_kernel<8, 16><<<g, 256, 0, stream>>>(W, tau, k, Z, Uh);
    } else
        backtransform_kernel<<<static_cast<unsigned>(ceil_div(k, 4)), 256, 0, stream>>>(W, tau, k, Z, Uh);
    BSQ_HIP(hipGetLastError());
}

}  // namespace bsq
