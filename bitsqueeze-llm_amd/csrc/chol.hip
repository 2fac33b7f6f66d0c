// Blocked Cholesky factorisation and triangular inverse for CholeskyQR
// (k x k FP64 Gram matrices, k <= 256).
//
//   chol_blocked_kernel   one workgroup of 1024 lanes; the lower triangle of
//                         the padded KP x KP matrix (KP = 32 * NB) lives in
//                         registers, lane (ty, tx) holding element
//                         (32a + ty, 32b + tx) of every lower 32 x 32 block.
//                         Right-looking by 32-column panels: one wave
//                         factors and inverts the diagonal block, all lanes
//                         form the panel L_ij = A_ij L_jj^{-T} and apply the
//                         rank-32 trailing update from an LDS copy of the
//                         panel.  8 panel steps replace 256 column steps, so
//                         the workgroup synchronises ~50 times instead of
//                         ~1500.  Breakdown (pivot <= 1e-15 max|G_ii|) restarts
//                         with a diagonal shift, as the unblocked version does.
//   trinv_kernel          L^{-1} by blocked forward substitution on the FP64
//                         matrix cores, 16 columns per workgroup, so the
//                         inverse is spread over k / 16 CUs.  Writes B = L^{-T} in
//                         FP32 row-major (B[r][c] = L^{-1}[c][r]) so that the
//                         orthonormal basis is the plain product Q = X B.
//
//   ns_refine_kernel      the final basis's second pass: one Newton-Schulz
//                         step instead of a second Cholesky when the basis is
//                         already orthonormal to working accuracy (below).
//
// The reference orthonormalises with Householder QR (cuSOLVER geqrf/orgqr,
// modules/svd_lowrank_cuda/src/svd_lowrank_cuda.cu:250-282); any basis of the
// same column space serves the range finder.
#include "bsq_internal.hpp"

namespace bsq {
namespace {

constexpr int kCholThreads = 1024;

__device__ __forceinline__ constexpr int tri(int a, int b) { return a * (a + 1) / 2 + b; }

// value of `v` in lane `src` (src wave-uniform), via two scalar reads
__device__ __forceinline__ double lane_value(double v, int src) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffu), src));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), src));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// v if bit == 1, +0.0 if bit == 0 (bit is 0 or 1), by masking the bit pattern:
// lane-dependent selects would materialise one lane mask per call site and
// the fully unrolled loops below would keep dozens of them live.
__device__ __forceinline__ double keep_if(double v, unsigned bit) {
    const unsigned long long m = 0ull - static_cast<unsigned long long>(bit);
    return __longlong_as_double(static_cast<long long>(static_cast<unsigned long long>(__double_as_longlong(v)) & m));
}

// Opaque copy: the compiler must assume the value changed, so lane-dependent
// index and mask arithmetic derived from it stays inside the loop body that
// uses it instead of being hoisted (and kept live across the whole
// factorisation, which spills).
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// value of `v` in lane `src` (src may differ per lane), via the LDS crossbar
__device__ __forceinline__ double lane_fetch(double v, int src) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(src << 2, static_cast<int>(u & 0xffffffffu)));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(src << 2, static_cast<int>(u >> 32)));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// Orders one wave's LDS accesses: wait for its outstanding LDS operations and
// keep the compiler from moving memory accesses across.
__device__ __forceinline__ void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ double wg_max(double v, double *red) {
    for (int off = 32; off >= 1; off >>= 1) v = fmax(v, __shfl_xor(v, off));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double s = red[0];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) s = fmax(s, red[w]);
    return s;
}

// Lout: KP x KP row-major (lower blocks written: L; diagonal blocks with
// zeros above the diagonal).  LIout: NB blocks of 32 x 32, the inverses of
// the diagonal blocks of L (zeros above the diagonal).  status[0]: number of
// shifted restarts (7 = gave up, L = I).
template <int NB>
__global__ __launch_bounds__(kCholThreads) void chol_blocked_kernel(const double *__restrict__ G, int k,
                                                                     double *__restrict__ Lout,
                                                                     double *__restrict__ LIout,
                                                                     int *__restrict__ status,
                                                                     const int *__restrict__ run) {
    if (run && run[0] == 0) return;  // uniform: the refinement step replaced this pass
    constexpr int KP = NB * 32, NE = NB * (NB + 1) / 2, PR = (NB > 1) ? (NB - 1) * 32 : 1;
    __shared__ double Dg[32][33];                          // diagonal block (row-major)
    __shared__ __attribute__((aligned(16))) double LI[32][34];  // L_jj^{-1}, row-major
    __shared__ __attribute__((aligned(16))) double P[PR][34];   // panel rows below the diagonal block
    __shared__ double stash[NE][64];                       // wave 0's registers during its solo phase
    __shared__ double red[kCholThreads / 64];
    __shared__ int broke;

    double dmax = 0.0;
    for (int i = threadIdx.x; i < k; i += kCholThreads) dmax = fmax(dmax, fabs(G[static_cast<uint64_t>(i) * k + i]));
    dmax = wg_max(dmax, red);
    const double tiny = (dmax > 0.0 ? dmax : 1.0) * 1e-15;
    double shift = 0.0;
    int attempt = 0;
    bool identity = false;
    double r[NE];
    for (;; ++attempt) {
        int tid = opaque(static_cast<int>(threadIdx.x));
        int tx = tid & 31, ty = tid >> 5;
#pragma unroll
        for (int a = 0; a < NB; ++a)
#pragma unroll
            for (int b = 0; b <= a; ++b) {
                // branch-free: G (+ shift on the diagonal) inside, identity in the padding
                const int i = a * 32 + ty, c = b * 32 + tx;
                const unsigned inside = (static_cast<unsigned>(i - k) >> 31) & (static_cast<unsigned>(c - k) >> 31);
                const unsigned diag = 1u - min(1u, static_cast<unsigned>(i ^ c));
                const double g = G[inside ? static_cast<uint64_t>(i) * k + c : 0];
                r[tri(a, b)] = keep_if(g, inside) +
                               static_cast<double>(diag) * (inside ? shift : 1.0);
            }
        if (tid == 0) broke = 0;
        bool failed = false;
#pragma unroll
        for (int jb = 0; jb < NB; ++jb) {
            if (failed) break;
            tid = opaque(static_cast<int>(threadIdx.x));
            tx = tid & 31;
            ty = tid >> 5;
            const int lane = tid & 63, wave = tid >> 6;
            __syncthreads();  // readers of Dg / P from the previous step are done
            Dg[ty][tx] = r[tri(jb, jb)];
#pragma unroll
            for (int a = jb + 1; a < NB; ++a) P[(a - jb - 1) * 32 + ty][tx] = r[tri(a, jb)];
            __syncthreads();
            if (wave == 0) {
                // free wave 0's registers for the 32 x 32 factorisation
#pragma unroll
                for (int e = 0; e < NE; ++e) stash[e][lane] = r[e];
                // the compiler may not forward the stash into the reload below (that
                // would keep r live through the factorisation)
                asm volatile("" ::: "memory");
                // 8 x 8 lane grid, lane (lr, lc) holding the 4 x 4 sub-blocks
                // a = A[4lr.., 4lc..] and x = X[4lr.., 4lc..] of the diagonal
                // block and of its inverse (X starts as I).  Step t: scale column
                // t of A and row t of X by 1/sqrt(pivot), fetch the four column-t
                // values of this lane's rows and columns and the four row-t values
                // of X with lane permutes, then rank-1 update A's trailing columns
                // and X's trailing rows (Gauss-Jordan on [L | I] fused into the
                // factorisation).
                const int lr = lane >> 3, lc = lane & 7;
                double a[4][4], x[4][4];
                const double on_diag = static_cast<double>(1u - min(1u, static_cast<unsigned>(lr ^ lc)));
#pragma unroll
                for (int p = 0; p < 4; ++p)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        a[p][q] = Dg[4 * lr + p][4 * lc + q];
                        x[p][q] = (p == q) ? on_diag : 0.0;
                    }
                bool bad = false;
#pragma unroll
                for (int t = 0; t < 32; ++t) {
                    const int tb = t >> 2, tq = t & 3;
                    const double dtt = lane_value(a[tq][tq], tb * 9);
                    bad = bad || !(dtt > tiny);
                    const double inv = rsqrt(dtt);
                    const double fc = (lc == tb) ? inv : 1.0, fr = (lr == tb) ? inv : 1.0;
#pragma unroll
                    for (int p = 0; p < 4; ++p) a[p][tq] *= fc;  // column t of L (row t: sqrt(pivot))
#pragma unroll
                    for (int q = 0; q < 4; ++q) x[tq][q] *= fr;  // row t of L^{-1}
                    double lrow[4], lcol[4], xrow[4];
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        lrow[p] = lane_fetch(a[p][tq], lr * 8 + tb);  // L[4lr + p][t]
                        lcol[p] = lane_fetch(a[p][tq], lc * 8 + tb);  // L[4lc + p][t]
                        xrow[p] = lane_fetch(x[tq][p], tb * 8 + lc);  // X[t][4lc + p]
                    }
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        // only columns c > t of A and rows i > t of X change
                        const double cb = keep_if(lcol[p], static_cast<unsigned>(t - (4 * lc + p)) >> 31);
                        const double rb = keep_if(lrow[p], static_cast<unsigned>(t - (4 * lr + p)) >> 31);
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            a[q][p] = fma(-lrow[q], cb, a[q][p]);
                            x[p][q] = fma(-rb, xrow[q], x[p][q]);
                        }
                    }
                }
                if (bad && lane == 0) broke = 1;
#pragma unroll
                for (int p = 0; p < 4; ++p)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        LI[4 * lr + p][4 * lc + q] = x[p][q];  // exactly zero above the diagonal
                        LIout[static_cast<uint64_t>(jb) * 1024 + (4 * lr + p) * 32 + 4 * lc + q] = x[p][q];
                    }
                asm volatile("" ::: "memory");
#pragma unroll
                for (int e = 0; e < NE; ++e) r[e] = stash[e][lane];
            }
            __syncthreads();
            if (broke) {
                failed = true;
                break;
            }

            // panel: L_ij = A_ij L_jj^{-T}, element (32a + ty, 32 jb + tx)
            double acc[NB];
#pragma unroll
            for (int a = 0; a < NB; ++a) acc[a] = 0.0;
#pragma unroll 1
            for (int t = 0; t < 32; t += 2) {
                const double2 li = *reinterpret_cast<const double2 *>(&LI[tx][t]);
#pragma unroll
                for (int a = jb + 1; a < NB; ++a) {
                    const double2 pa = *reinterpret_cast<const double2 *>(&P[(a - jb - 1) * 32 + ty][t]);
                    acc[a] = fma(pa.x, li.x, fma(pa.y, li.y, acc[a]));
                }
            }
            __syncthreads();  // every lane has read the A panel
#pragma unroll
            for (int a = jb + 1; a < NB; ++a) {
                r[tri(a, jb)] = acc[a];
                P[(a - jb - 1) * 32 + ty][tx] = acc[a];
                Lout[static_cast<uint64_t>(a * 32 + ty) * KP + jb * 32 + tx] = acc[a];
            }
            __syncthreads();
            // trailing update A_ab -= L_aj L_bj^T for jb < b <= a
            if (jb + 1 < NB) {
#pragma unroll 1
                for (int t = 0; t < 32; t += 2) {  // two panel columns per pass: 16-byte LDS reads
                    double2 rv[NB];
#pragma unroll
                    for (int a = jb + 1; a < NB; ++a)
                        rv[a] = *reinterpret_cast<const double2 *>(&P[(a - jb - 1) * 32 + ty][t]);
#pragma unroll
                    for (int b = jb + 1; b < NB; ++b) {
                        const double2 cv = *reinterpret_cast<const double2 *>(&P[(b - jb - 1) * 32 + tx][t]);
#pragma unroll
                        for (int a = b; a < NB; ++a)
                            r[tri(a, b)] = fma(-rv[a].y, cv.y, fma(-rv[a].x, cv.x, r[tri(a, b)]));
                    }
                }
            }
        }
        if (!failed) break;
        if (attempt >= 6 || dmax == 0.0) {
            identity = true;
            break;
        }
        shift = (shift == 0.0) ? dmax * 1e-12 * static_cast<double>(k) : shift * 100.0;
        __syncthreads();
    }
    const int tid = threadIdx.x;
    if (identity) {
        __syncthreads();
        for (int t = tid; t < KP * KP; t += kCholThreads) {
            const int i = t / KP, c = t % KP;
            if (c <= i) Lout[t] = (i == c) ? 1.0 : 0.0;
        }
        for (int t = tid; t < NB * 1024; t += kCholThreads) {
            const int i = (t & 1023) >> 5, c = t & 31;
            LIout[t] = (i == c) ? 1.0 : 0.0;
        }
    }
    if (tid == 0 && status) status[0] = attempt;
}

// Columns c0 .. c0+15 of L^{-1}, block row by block row, on the FP64 matrix
// cores (v_mfma_f64_16x16x4f64):
//   X_cb = LI_cb[:, cols];  X_i = -LI_i * S_i,  S_i = sum_{t=cb}^{i-1} L_it X_t
// L and LI were written by a kernel on another XCD, so every piece of them
// this workgroup needs is loaded at the start, all in flight at once (1024
// lanes hold the widest strip in ~80 registers each: one memory latency
// instead of one per block row).  Block row i's panel L[i rows][cb * 32 ..
// i * 32) and LI_i then go from registers to LDS, and S_i (32 x 16, K =
// 32 (i - cb)) is formed by 16 waves (rh, kh): rows rh * 16 .. +16 over the
// k-steps s = kh (mod 8), the eight partial sums added through LDS; waves 0
// and 1 apply the lower-triangular LI_i.
// MFMA operand lanes: A[r][q] and B[q][c] in lane 16 q + (r or c);
// accumulator register u of lane l holds D[4 u + l / 16][l % 16].
// Output B = L^{-T} (k x k FP32 row-major): B[c][r] = L^{-1}[r][c].
typedef double f64x4 __attribute__((ext_vector_type(4)));
constexpr int kTrinvThreads = 1024;

template <int NB>
__global__ __launch_bounds__(kTrinvThreads) void trinv_kernel(const double *__restrict__ Lin,
                                                              const double *__restrict__ LIin, int k,
                                                              float *__restrict__ B, const int *__restrict__ run) {
    if (run && run[0] == 0) return;  // uniform
    constexpr int KP = NB * 32;
    constexpr int PP = (NB > 1 ? 32 * (NB - 1) : 32) + 4;  // panel pitch (doubles): 2-way banks for the A reads
    constexpr int XP = 17, LP = 36;
    // panel d (1 .. NB - 1): row lr, 16-byte pieces lp + 32 u, u < (d + 1) / 2
    constexpr int kPanelPieces = (NB * NB) / 4 + 1;  // >= sum_d (d + 1) / 2 for d < NB
    constexpr int kLiPieces = (NB > 1) ? ((NB - 1) * 512 + kTrinvThreads - 1) / kTrinvThreads : 1;
    __shared__ __attribute__((aligned(16))) double P[32][PP];
    __shared__ __attribute__((aligned(16))) double LIs[32][LP];
    __shared__ double X[KP][XP];
    __shared__ double SP[8][32][XP];
    __shared__ double S[32][XP];
    const int c0 = blockIdx.x * 16, cb = c0 >> 5, co = c0 & 31;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kq = lane >> 4, cc = lane & 15;
    const int rh = wave & 1, kh = wave >> 1;
    const int lr = tid >> 5, lp = tid & 31;
    const int nsteps = NB - 1 - cb;

    double pv[2 * kPanelPieces], lv[2 * kLiPieces];
    if (nsteps >= 1) {  // uniform (the last column block has no panels)
        int at = 0;
#pragma unroll
        for (int d = 1; d < NB; ++d) {
            const int dd = d <= nsteps ? d : 1;  // panels past the strip re-read panel 1 (not stored)
            const double2 *prow =
                reinterpret_cast<const double2 *>(Lin + static_cast<uint64_t>((cb + dd) * 32 + lr) * KP + cb * 32);
#pragma unroll
            for (int u = 0; u < (d + 1) / 2; ++u) {
                const double2 v = prow[min(lp + 32 * u, 16 * dd - 1)];
                pv[2 * at] = v.x;
                pv[2 * at + 1] = v.y;
                ++at;
            }
        }
#pragma unroll
        for (int v = 0; v < kLiPieces; ++v) {
            const int q = min(tid + kTrinvThreads * v, 512 * nsteps - 1);  // piece of blocks cb+1 ..
            const double2 w = reinterpret_cast<const double2 *>(LIin + static_cast<uint64_t>(cb + 1) * 1024)[q];
            lv[2 * v] = w.x;
            lv[2 * v + 1] = w.y;
        }
    }
    for (int t = tid; t < 32 * 16; t += kTrinvThreads) {
        const int r = t >> 4, j = t & 15;
        X[cb * 32 + r][j] = LIin[static_cast<uint64_t>(cb) * 1024 + r * 32 + co + j];
    }
    int at0 = 0;  // first panel piece of step d
#pragma unroll
    for (int d = 1; d < NB; ++d) {
        if (d <= nsteps) {  // uniform
            // panel d and LI_{cb+d} into LDS (the previous step's readers are done)
#pragma unroll
            for (int u = 0; u < (d + 1) / 2; ++u)
                if (lp + 32 * u < 16 * d)
                    *reinterpret_cast<double2 *>(&P[lr][2 * (lp + 32 * u)]) =
                        double2{pv[2 * (at0 + u)], pv[2 * (at0 + u) + 1]};
#pragma unroll
            for (int v = 0; v < kLiPieces; ++v) {
                const int q = tid + kTrinvThreads * v;
                if ((q >> 9) == d - 1) *reinterpret_cast<double2 *>(&LIs[(q >> 4) & 31][2 * (q & 15)]) =
                    double2{lv[2 * v], lv[2 * v + 1]};
            }
            __syncthreads();
            // S partials: wave (rh, kh) over k-steps s = kh + 8 j, j < d
            f64x4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int j = 0; j < d; ++j) {
                const int s = kh + 8 * j;
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(P[rh * 16 + cc][4 * s + kq], X[cb * 32 + 4 * s + kq][cc],
                                                           acc, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) SP[kh][rh * 16 + 4 * u + kq][cc] = acc[u];
            __syncthreads();
            if (tid < 512) {
                const int r = tid >> 4, c = tid & 15;
                double t = SP[0][r][c];
#pragma unroll
                for (int h = 1; h < 8; ++h) t += SP[h][r][c];
                S[r][c] = t;
            }
            __syncthreads();
            if (wave < 2) {  // wave-uniform; LI_i lower triangular: rows 0..15 need only k < 16
                f64x4 t = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
                for (int s = 0; s < 8; ++s)
                    if (rh == 1 || s < 4)
                        t = __builtin_amdgcn_mfma_f64_16x16x4f64(LIs[rh * 16 + cc][4 * s + kq], S[4 * s + kq][cc], t,
                                                                 0, 0, 0);
#pragma unroll
                for (int u = 0; u < 4; ++u) X[(cb + d) * 32 + rh * 16 + 4 * u + kq][cc] = -t[u];
            }
            __syncthreads();
        }
        at0 += (d + 1) / 2;
    }
    for (int jj = 0; jj < 16 && c0 + jj < k; ++jj) {
        float *brow = B + static_cast<uint64_t>(c0 + jj) * k;
        for (int r = tid; r < k; r += kTrinvThreads)
            brow[r] = (r >= cb * 32) ? static_cast<float>(X[r][jj]) : 0.0f;
    }
}

template <int NB>
void chol_blocked(const double *G, int k, double *Lbuf, float *B, int *status, const int *run, hipStream_t stream) {
    double *L = Lbuf, *LI = Lbuf + static_cast<uint64_t>(NB) * 32 * NB * 32;
    chol_blocked_kernel<NB><<<1, kCholThreads, 0, stream>>>(G, k, L, LI, status, run);
    BSQ_HIP(hipGetLastError());
    trinv_kernel<NB><<<static_cast<unsigned>(ceil_div(k, 16)), kTrinvThreads, 0, stream>>>(L, LI, k, B, run);
    BSQ_HIP(hipGetLastError());
}

// Second pass over an almost orthonormal basis Q with G = Q^T Q = I + E.
// When ||E||_F < kNsTol, B = 1.5 I - 0.5 G and Q B has orthogonality error
// O(||E||^2) (one Newton-Schulz step towards the polar factor; the column
// space is unchanged, B being nonsingular), which is what a second CholeskyQR
// pass achieves at the cost of a one-CU factorisation.  run[0] = 0 then, and
// the Cholesky kernels launched behind this one return at once; otherwise
// run[0] = 1, B is left alone and they compute B = L^{-T} as usual.
constexpr double kNsTol = 1e-3;
// One workgroup per row of B.  rowsq[r] is row r's share of ||E||_F^2
// (written by the Gram reduction); every workgroup sums the k shares in the
// same order, so all of them reach the same decision.
__global__ __launch_bounds__(256) void ns_refine_kernel(const double *__restrict__ G,
                                                        const double *__restrict__ rowsq, int k,
                                                        float *__restrict__ B, int *__restrict__ run) {
    __shared__ double red[4];
    const int tid = threadIdx.x, i = blockIdx.x;
    double s = (tid < k) ? rowsq[tid] : 0.0;  // k <= 256
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    const bool refine = tot < kNsTol * kNsTol;  // false for NaN
    if (i == 0 && tid == 0) run[0] = refine ? 0 : 1;
    if (!refine) return;
    for (int j = tid; j < k; j += 256) {
        const uint64_t t = static_cast<uint64_t>(i) * k + j;
        B[t] = static_cast<float>((i == j ? 1.5 : 0.0) - 0.5 * G[t]);
    }
}

}  // namespace

// FP64 doubles needed by launch_chol_blocked's L buffer for rank k.
uint64_t chol_blocked_buffer_doubles(int k) {
    const uint64_t nb = ceil_div(k, 32);
    return nb * 32 * nb * 32 + nb * 1024;
}

bool chol_blocked_supported(int k) { return k >= 1 && k <= 256; }

// G = L L^T (with shifted restarts on breakdown) and B = L^{-T} (FP32,
// k x k row-major), so that X B has orthonormal columns when G = X^T X.
void launch_chol_blocked(const double *G, int k, double *Lbuf, float *B, int *status, hipStream_t stream,
                         const int *run) {
    BSQ_REQUIRE(chol_blocked_supported(k), "chol: rank outside the blocked kernel's range");
    switch (ceil_div(k, 32)) {
        case 1: chol_blocked<1>(G, k, Lbuf, B, status, run, stream); break;
        case 2: chol_blocked<2>(G, k, Lbuf, B, status, run, stream); break;
        case 3: chol_blocked<3>(G, k, Lbuf, B, status, run, stream); break;
        case 4: chol_blocked<4>(G, k, Lbuf, B, status, run, stream); break;
        case 5: chol_blocked<5>(G, k, Lbuf, B, status, run, stream); break;
        case 6: chol_blocked<6>(G, k, Lbuf, B, status, run, stream); break;
        case 7: chol_blocked<7>(G, k, Lbuf, B, status, run, stream); break;
        default: chol_blocked<8>(G, k, Lbuf, B, status, run, stream); break;
    }
}

// B such that Q B is orthonormal for the almost orthonormal Q with Gram G
// (and row shares rowsq of ||G - I||_F^2): the Newton-Schulz step when it
// suffices, else B = L^{-T} from a Cholesky factorisation (decided on the
// device; run is one int of scratch).
void launch_orth_refine(const double *G, const double *rowsq, int k, double *Lbuf, float *B, int *status, int *run,
                        hipStream_t stream) {
    BSQ_REQUIRE(k >= 1 && k <= 256, "orth refine: rank outside the blocked kernels' range");
    ns_refine_kernel<<<static_cast<unsigned>(k), 256, 0, stream>>>(G, rowsq, k, B, run);
    BSQ_HIP(hipGetLastError());
    launch_chol_blocked(G, k, Lbuf, B, status, stream, run);
}

}  // namespace bsq
