// Blocked Cholesky factorisation and triangular inverse for CholeskyQR
// (k x k FP64 Gram matrices, k <= 256).
//
//   chol_blocked_kernel   one workgroup of 1024 lanes.  The 12 waves that do
//                         not share wave 0's SIMD hold the lower 16 x 16
//                         tiles of the padded KP x KP matrix (KP = 32 * NB)
//                         in MFMA accumulator layout; wave 0 factors and
//                         inverts the 32 x 32 diagonal blocks.
//                         Right-looking by 32-column panels with look-ahead:
//                         the panel solve L_ij = A_ij L_jj^{-T} and the rank-32
//                         trailing update run on the FP64 matrix cores, and
//                         wave 0 factors block j + 1 while the other waves
//                         finish the trailing update of step j.  Breakdown
//                         (pivot <= 1e-15 max|G_ii|) restarts with a diagonal
//                         shift, as the unblocked version does.
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

#include <algorithm>
#include <type_traits>

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

// Workgroup barrier for data exchanged through LDS only: waits for this wave's
// LDS operations but not for its global loads and stores, so loads into
// registers stay in flight across it (their first use waits for them) and the
// stores of L drain behind the next steps.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

typedef double f64x4 __attribute__((ext_vector_type(4)));

// Lower 16 x 16 tile number idx of an NT x NT tile grid, tiles ordered by
// column, then row: column J starts at J NT - J (J - 1) / 2.
template <int NT>
__device__ __forceinline__ void tile_coords(int idx, int &I, int &J) {
    int j = 0;
#pragma unroll
    for (int t = 1; t < NT; ++t) j = (idx >= t * NT - t * (t - 1) / 2) ? t : j;
    J = j;
    I = j + idx - (j * NT - j * (j - 1) / 2);
}

// 1 / d for a positive normal d: the hardware reciprocal estimate refined by
// two Newton steps, each of which doubles the number of correct bits.
__device__ __forceinline__ double recip_nr(double d) {
    double r = __builtin_amdgcn_rcp(d);
    r = fma(r, fma(-d, r, 1.0), r);
    return fma(r, fma(-d, r, 1.0), r);
}

// value of `v` in lane l - 1 (within each row of 16 lanes)
__device__ __forceinline__ double lane_below(double v) {
    const unsigned long long u = static_cast<unsigned long long>(__double_as_longlong(v));
    const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_mov_dpp(static_cast<int>(u & 0xffffffffu), 0x111, 0xF, 0xF, true));
    const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_mov_dpp(static_cast<int>(u >> 32), 0x111, 0xF, 0xF, true));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// Inverse Cholesky factor of the 16 x 16 block S[0..16)[0..16) (lower
// triangle used) on one wave: 8 x 8 lane grid, lane (lr, lc) holding the 2 x 2
// sub-blocks a[p][q] = A[2lr + p][2lc + q] of the block and x[p][q] =
// X[2lc + p][2lr + q] of the unscaled inverse (X starts as I; held transposed,
// so that row t + 1 of X sits in the lanes of column t + 1 of A).  Step t
// (pivot d = A[t][t]) is the rank-1 update A[i][c] -= A[i][t] A[c][t] / d for
// columns c > t and X[i] -= (A[i][t] / d) X[t] for rows i > t (Gauss-Jordan on
// [L | I] fused into the factorisation, the square roots deferred: with
// L[i][t] = A[i][t] / sqrt(d), row t of L^{-1} is X[t] / sqrt(d)).  It runs
// with look-ahead: column t + 1 of A and row t + 1 of X go first (their
// column-t inputs are in the same lane or one lane down, and A[t + 1][t] is one
// scalar read), so the next pivot and its reciprocal follow at once; the
// update of the columns and rows beyond t + 1 reads its inputs through lane
// permutes issued one step ahead.  Only the inverse is needed, so L itself is
// never formed: the pivots stay on A's diagonal and scale X's rows at the end.
// Writes L^{-1} (zeros above the diagonal) to LIo; returns true when a pivot
// is <= tiny (or NaN).
template <int PITCH>
__device__ __forceinline__ bool gj_factor16(const double (*S)[PITCH], double (*LIo)[PITCH], double tiny, int lane) {
    const int lr = lane >> 3, lc = lane & 7;
    double a[2][2], x[2][2];
    const double on_diag = static_cast<double>(1u - min(1u, static_cast<unsigned>(lr ^ lc)));
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            a[p][q] = S[2 * lr + p][2 * lc + q];
            x[p][q] = (p == q) ? on_diag : 0.0;
        }
    const double d0 = lane_value(a[0][0], 0);
    bool bad = !(d0 > tiny);
    double rd = recip_nr(d0);
    // step-t inputs of the trailing update: A[2lr + p][t], A[2lc + p][t], X[t][2lr + q]
    double lrow[2], lcol[2], xrow[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        lrow[p] = lane_fetch(a[p][0], lr * 8);
        lcol[p] = lane_fetch(a[p][0], lc * 8);
        xrow[p] = lane_fetch(x[0][p], lr * 8);
    }
#pragma unroll
    for (int t = 0; t < 15; ++t) {
        const int tb = t >> 1, tq = t & 1, tb1 = (t + 1) >> 1, tq1 = (t + 1) & 1;
        // column t + 1 of A and row t + 1 of X (lanes lc == tb1); their column-t
        // and row-t inputs: this lane (t even) or the lane below (t odd)
        const double at = lane_value(a[tq1][tq], tb1 * 8 + tb);  // A[t + 1][t]
        const double sv = keep_if(at * rd, lc == tb1 ? 1u : 0u);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const double colt = tq ? lane_below(a[p][1]) : a[p][0];  // A[2lr + p][t]
            a[p][tq1] = fma(-colt, sv, a[p][tq1]);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const double rowt = tq ? lane_below(x[1][q]) : x[0][q];  // X[t][2lr + q]
            x[tq1][q] = fma(-sv, rowt, x[tq1][q]);
        }
        const double dn = lane_value(a[tq1][tq1], tb1 * 9);
        bad = bad || !(dn > tiny);
        const double rdn = recip_nr(dn);
        double nrow[2], ncol[2], nxrow[2];
        if (t + 2 < 16) {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                nrow[p] = lane_fetch(a[p][tq1], lr * 8 + tb1);
                ncol[p] = lane_fetch(a[p][tq1], lc * 8 + tb1);
                nxrow[p] = lane_fetch(x[tq1][p], lr * 8 + tb1);
            }
            // columns c > t + 1 of A and rows i > t + 1 of X (the same index
            // 2lc + p): column t + 1 keeps its pivot, and A's lower triangle is
            // all that feeds X
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const double cb = keep_if(lcol[p] * rd, static_cast<unsigned>(t + 1 - (2 * lc + p)) >> 31);
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    a[q][p] = fma(-lrow[q], cb, a[q][p]);
                    x[p][q] = fma(-cb, xrow[q], x[p][q]);
                }
            }
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                lrow[p] = nrow[p];
                lcol[p] = ncol[p];
                xrow[p] = nxrow[p];
            }
        }
        rd = rdn;
    }
    // row i of L^{-1} = X[i] / sqrt(pivot i); pivot 2lc + p sits in lane (lc, lc)
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const double inv = rsqrt(lane_fetch(a[p][p], lc * 9));
#pragma unroll
        for (int q = 0; q < 2; ++q) LIo[2 * lc + p][2 * lr + q] = x[p][q] * inv;
    }
    return bad;
}

// Factors the 32 x 32 diagonal block in Dg (lower triangle used) on one wave
// and writes its inverse to LI (zeros above the diagonal), by
// 2 x 2 blocks of 16:
//   L11, L11^{-1} = gj_factor16(A11);   L21 = A21 L11^{-T};
//   L22, L22^{-1} = gj_factor16(A22 - L21 L21^T);
//   (L^{-1})21 = -L22^{-1} (L21 L11^{-1}).
// The four 16 x 16 products run on the matrix cores (four dependent
// 16 x 16 x 4 steps each); Dg's upper right quarter (unused by the lower
// triangle) and, once factored, its upper left quarter stage the transposes.
// MFMA operand lanes: A[r][q] and B[q][c] in lane 16 q + (r or c);
// accumulator register u of lane l holds D[4 u + l / 16][l % 16].
// Returns true when a pivot is <= tiny (or NaN).
template <int PITCH>
__device__ __forceinline__ bool factor_diag_block(double (*Dg)[PITCH], double (*LI)[PITCH], double tiny, int lane) {
    const int kq = lane >> 4, cc = lane & 15;
    bool bad = gj_factor16<PITCH>(Dg, LI, tiny, lane);
#pragma unroll
    for (int u = 0; u < 4; ++u) LI[4 * u + kq][16 + cc] = 0.0;
    wave_lds_fence();
    // L21 = A21 L11^{-T}: A = Dg[16 + r][k], B[k][c] = LI[c][k]  -> Dg[r][16 + c]
    f64x4 t = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int s = 0; s < 4; ++s)
        t = __builtin_amdgcn_mfma_f64_16x16x4f64(Dg[16 + cc][4 * s + kq], LI[cc][4 * s + kq], t, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) Dg[4 * u + kq][16 + cc] = t[u];
    wave_lds_fence();
    // A22 -= L21 L21^T: A[r][k] = -L21[r][k], B[k][c] = L21[c][k]
#pragma unroll
    for (int u = 0; u < 4; ++u) t[u] = Dg[16 + 4 * u + kq][16 + cc];
#pragma unroll
    for (int s = 0; s < 4; ++s)
        t = __builtin_amdgcn_mfma_f64_16x16x4f64(-Dg[cc][16 + 4 * s + kq], Dg[cc][16 + 4 * s + kq], t, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) Dg[16 + 4 * u + kq][16 + cc] = t[u];
    wave_lds_fence();
    // T = L21 L11^{-1} (A[r][k] = L21[r][k], B[k][c] = LI[k][c]) -> Dg[r][c]
    // (A11 is no longer needed)
    t = f64x4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int s = 0; s < 4; ++s)
        t = __builtin_amdgcn_mfma_f64_16x16x4f64(Dg[cc][16 + 4 * s + kq], LI[4 * s + kq][cc], t, 0, 0, 0);
    bad = gj_factor16<PITCH>(reinterpret_cast<const double (*)[PITCH]>(&Dg[16][16]),
                             reinterpret_cast<double (*)[PITCH]>(&LI[16][16]), tiny, lane) || bad;
#pragma unroll
    for (int u = 0; u < 4; ++u) Dg[4 * u + kq][cc] = t[u];
    wave_lds_fence();
    // (L^{-1})21 = -L22^{-1} T: A[r][k] = -LI[16 + r][16 + k], B[k][c] = T[k][c]
    t = f64x4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int s = 0; s < 4; ++s)
        t = __builtin_amdgcn_mfma_f64_16x16x4f64(-LI[16 + cc][16 + 4 * s + kq], Dg[4 * s + kq][cc], t, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) LI[16 + 4 * u + kq][cc] = t[u];
    return bad;
}

// Tile (I, J) of G in the MFMA accumulator layout (register u of lane l holds
// element (16 I + 4 u + l / 16, 16 J + l % 16)): G plus `shift` on the
// diagonal inside, the identity in the padding.  Off-diagonal tiles inside G
// (the common case) are plain loads from a wave-uniform base; the others clamp
// their loads into G and mask them, so no lane branches.
__device__ __forceinline__ f64x4 load_tile(const double *__restrict__ G, int k, int I, int J, double shift, int kq,
                                           int cc) {
    f64x4 t;
    if (I != J && 16 * I + 16 <= k && 16 * J + 16 <= k) {  // uniform
        const double *__restrict__ g0 = G + static_cast<size_t>(16 * I) * k + 16 * J;
#pragma unroll
        for (int u = 0; u < 4; ++u) t[u] = g0[static_cast<size_t>(4 * u) * k + kq * k + cc];
        return t;
    }
    const int c = 16 * J + cc;
    const unsigned cin = static_cast<unsigned>(c - k) >> 31;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = 16 * I + 4 * u + kq;
        const unsigned inside = (static_cast<unsigned>(i - k) >> 31) & cin;
        const unsigned diag = 1u - min(1u, static_cast<unsigned>(i ^ c));
        const double g = G[static_cast<unsigned>(min(i, k - 1) * k + min(c, k - 1))];
        t[u] = keep_if(g, inside) + static_cast<double>(diag) * (inside ? shift : 1.0);
    }
    return t;
}

// Lout: KP x KP row-major, the blocks below the diagonal blocks written (the
// triangular inverse reads nothing else).  LIout: NB blocks of 32 x 32, the
// inverses of the diagonal blocks of L (zeros above the diagonal).
// status[0]: number of shifted restarts (7 = gave up, L = I).
//
// Right-looking by 32-column panels with look-ahead.  Wave 0 only factors the
// diagonal blocks (factor_diag_block).  The lower 16 x 16 tiles (I >= J) of
// the padded matrix in block columns 0 and 1 go straight from G to LDS
// (block 0 -> Dg, panel 0 -> X); the other tiles are held in the accumulator
// layout of v_mfma_f64_16x16x4f64 (register u of lane l holds tile element
// (4u + l / 16, l % 16)) by the 12 waves that do not share wave 0's SIMD (a
// workgroup's waves are dealt to the four SIMDs in turn, so waves 4, 8, 12
// run beside wave 0: left without tiles, they keep the matrix core free for
// the factorisation), ordered by column then row, so every trailing matrix
// is a suffix of that order and each step's tiles are spread over the 12
// waves to within one.  Step jb:
//   B1  wave 0 has factored block jb (LI); waves 1..15 copy LI to LIout and
//       form the panel L_I,jb = A_I,jb L_jj^{-T} on the matrix cores (A from
//       the LDS panel X, result to the LDS panel Y and to Lout), its tiles
//       dealt over all 15 waves;
//   B2  the diagonal block jb + 1 takes its update A -= L L^T first and goes
//       to Dg;
//   B3  wave 0 factors block jb + 1 while the tile holders update the rest of
//       the trailing matrix and copy the next panel into X.
// The products read their operands from LDS: two 8-byte reads per
// 16 x 16 x 4 product.  The barriers are on LDS only: the held tiles load
// while block 0 is factored, and the stores of L drain behind the next steps.
template <int NB>
__global__ __launch_bounds__(kCholThreads) void chol_blocked_kernel(const double *__restrict__ G, int k,
                                                                     double *__restrict__ Lout,
                                                                     double *__restrict__ LIout,
                                                                     int *__restrict__ status,
                                                                     const int *__restrict__ run) {
    if (run && run[0] == 0) return;  // uniform: the refinement step replaced this pass
    constexpr int KP = NB * 32, NT = 2 * NB, NTILES = NT * (NT + 1) / 2;
    constexpr int C01 = 2 * NT - 1;  // tiles in block columns 0 and 1
    constexpr int OW = 12;           // tile-holding waves
    constexpr int HS = (NTILES - C01 + OW - 1) / OW, LS = (C01 + 3) / 4;  // held, loaded-only tiles per wave
    constexpr int SLOTS = HS > LS ? HS : LS;
    constexpr int PSLOTS = (2 * (NT - 2) + 14) / 15 > 0 ? (2 * (NT - 2) + 14) / 15 : 1;  // panel tiles per wave
    constexpr int PR = (NB > 1) ? (NB - 1) * 32 : 1;
    static_assert(kCholThreads == 1024, "16 waves: wave 0 and three tile-free waves on one SIMD");
    // pitch 33 (odd): the MFMA operand reads (16 rows, one column each) and the
    // tile stores (one row, 16 columns) hit 32 distinct banks per 16 lanes
    constexpr int PITCH = 33;
    __shared__ double Dg[32][PITCH];  // diagonal block: its three lower 16 x 16 tiles
    __shared__ double LI[32][PITCH];  // L_jj^{-1}, zeros above the diagonal
    __shared__ double X[PR][PITCH];   // panel rows below the diagonal block, before the solve
    __shared__ double Y[PR][PITCH];   // the same rows of L
    __shared__ double red[kCholThreads / 64];
    __shared__ int broke;

    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    double shift = 0.0, dmax = 0.0, tiny = 0.0;
    int attempt = 0;
    bool identity = false;
    for (;; ++attempt) {
        if (threadIdx.x == 0) broke = 0;
        bool failed = false;
        // slots: waves w % 4 != 0 hold tiles C01 + OW m + (w - 1 - w / 4) for the
        // whole factorisation; waves 0, 4, 8, 12 load the tiles 4 m + w / 4 of
        // block columns 0, 1 into LDS
        int tI[SLOTS], tJ[SLOTS];
#pragma unroll
        for (int m = 0; m < SLOTS; ++m) {
            const int idx = ((wave & 3) == 0) ? (4 * m + (wave >> 2) < C01 ? 4 * m + (wave >> 2) : NTILES)
                                              : C01 + OW * m + wave - 1 - (wave >> 2);
            tile_coords<NT>(idx < NTILES ? idx : 0, tI[m], tJ[m]);
            if (idx >= NTILES) tJ[m] = -1;  // no tile in this slot
        }
        f64x4 acc[SLOTS];
        if (wave == 0) __builtin_amdgcn_s_setprio(3);  // its loads and the factorisation are the critical path
        {
            const int lane = opaque(static_cast<int>(threadIdx.x)) & 63, kq = lane >> 4, cc = lane & 15;
            // waves 0, 4, 8, 12 load first: their tiles (block columns 0, 1) go to
            // LDS before P0; the other waves issue the loads of their held
            // tiles after P0, so those do not delay block 0 and stay in flight
            // across the LDS-only barriers while wave 0 factors block 0 (each
            // wave passes one barrier here)
            if ((wave & 3) != 0) lds_barrier();  // P0
#pragma unroll
            for (int m = 0; m < SLOTS; ++m)
                acc[m] = (tJ[m] < 0) ? f64x4{0.0, 0.0, 0.0, 0.0}  // uniform
                                     : load_tile(G, k, tI[m], tJ[m], shift, kq, cc);
            if (attempt == 0 && wave == 0) {
                // breakdown scale max |G_ii|, for wave 0 (tiny) and, through
                // LDS, the others (the shift of a restart); issued after the
                // tile loads, so both memory round trips overlap
                double dm = 0.0;
#pragma unroll
                for (int m = 0; m < (KP + 63) / 64; ++m) {
                    const int i = lane + 64 * m;
                    const double g = G[static_cast<unsigned>(min(i, k - 1)) * static_cast<unsigned>(k + 1)];
                    dm = fmax(dm, keep_if(fabs(g), static_cast<unsigned>(i - k) >> 31));
                }
                for (int off = 32; off >= 1; off >>= 1) dm = fmax(dm, __shfl_xor(dm, off));
                dmax = dm;
                tiny = (dmax > 0.0 ? dmax : 1.0) * 1e-15;
                if (lane == 0) red[0] = dm;
            }
            if ((wave & 3) == 0) {
#pragma unroll
                for (int m = 0; m < SLOTS; ++m) {
                    const int I = tI[m], J = tJ[m];
                    if (J >= 0) {  // uniform
                        if (I < 2) {
#pragma unroll
                            for (int u = 0; u < 4; ++u) Dg[16 * I + 4 * u + kq][16 * J + cc] = acc[m][u];
                        } else {
#pragma unroll
                            for (int u = 0; u < 4; ++u) X[16 * (I - 2) + 4 * u + kq][16 * J + cc] = acc[m][u];
                        }
                    }
                }
                lds_barrier();  // P0: block 0 is in Dg, panel 0 in X, max |G_ii| in red[0]
            }
        }
        if (attempt == 0) dmax = red[0];
        if (wave == 0) {
            // the factorisation wave (issued first on its SIMD: it is the
            // critical path); the same barrier sequence as the other waves
#pragma unroll 1
            for (int jb = 0; jb < NB; ++jb) {
                const int lane = opaque(static_cast<int>(threadIdx.x)) & 63;
                const bool bad = factor_diag_block<PITCH>(Dg, LI, tiny, lane);
                if (bad && lane == 0) broke = 1;
                lds_barrier();  // B1
                if (broke) {
                    failed = true;
                    break;
                }
                if (jb + 1 < NB) {
                    lds_barrier();  // B2
                    lds_barrier();  // B3
                }
            }
            __builtin_amdgcn_s_setprio(0);
        } else {
            // jb stays a loop: the tile registers are indexed by slot only
#pragma unroll 1
            for (int jb = 0; jb < NB; ++jb) {
                const int lane = opaque(static_cast<int>(threadIdx.x)) & 63, kq = lane >> 4, cc = lane & 15;
                lds_barrier();  // B1: LI holds block jb's inverse
                if (broke) {
                    failed = true;
                    break;
                }
                {
                    // LI -> LIout block jb (32 x 32 row-major): 960 lanes, e and e + 960
                    double *LIblk = LIout + static_cast<uint64_t>(jb) * 1024;
                    const int e = 64 * (wave - 1) + lane;
                    LIblk[e] = LI[e >> 5][e & 31];
                    if (e < 1024 - 960) LIblk[e + 960] = LI[(e + 960) >> 5][e & 31];
                }
                if (jb + 1 < NB) {
                    // panel tiles q = 15 m + wave - 1: column 2 jb + (q & 1), row
                    // 2 jb + 2 + (q >> 1); A[r][q] = X[row r][4s + q], B[q][c] =
                    // LI[c][4s + q] (LI is lower triangular: its first 16 rows end
                    // at column 15)
#pragma unroll
                    for (int m = 0; m < PSLOTS; ++m) {
                        const int q = 15 * m + wave - 1, J = 2 * jb + (q & 1), I = 2 * jb + 2 + (q >> 1);
                        if (q < 2 * (NT - 2 * jb - 2)) {  // uniform
                            const int pr = 16 * (I - 2 * jb - 2), lc16 = 16 * (J - 2 * jb);
                            f64x4 t = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
                            for (int s = 0; s < 8; ++s)
                                if (s < 4 || (q & 1))
                                    t = __builtin_amdgcn_mfma_f64_16x16x4f64(X[pr + cc][4 * s + kq],
                                                                             LI[lc16 + cc][4 * s + kq], t, 0, 0, 0);
#pragma unroll
                            for (int u = 0; u < 4; ++u) {
                                Y[pr + 4 * u + kq][lc16 + cc] = t[u];
                                Lout[static_cast<uint64_t>(16 * I + 4 * u + kq) * KP + 16 * J + cc] = t[u];
                            }
                        }
                    }
                    lds_barrier();  // B2: Y holds the panel of L
                    // trailing update A_IJ -= L_I,jb L_J,jb^T (2 jb + 2 <= J <= I):
                    // first the diagonal block jb + 1, which goes to Dg
                    const int nb0 = 2 * jb + 2;
#pragma unroll
                    for (int m = 0; m < SLOTS; ++m) {
                        const int I = tI[m], J = tJ[m];
                        if (J >= nb0 && I < nb0 + 2) {
                            const int pa = 16 * (I - nb0), pb = 16 * (J - nb0);
                            f64x4 t = acc[m];
#pragma unroll
                            for (int s = 0; s < 8; ++s)
                                t = __builtin_amdgcn_mfma_f64_16x16x4f64(-Y[pa + cc][4 * s + kq], Y[pb + cc][4 * s + kq],
                                                                         t, 0, 0, 0);
#pragma unroll
                            for (int u = 0; u < 4; ++u) Dg[pa + 4 * u + kq][pb + cc] = t[u];
                        }
                    }
                    lds_barrier();  // B3: wave 0 factors block jb + 1 meanwhile
#pragma unroll
                    for (int m = 0; m < SLOTS; ++m) {
                        const int I = tI[m], J = tJ[m];
                        if (J >= nb0 && I >= nb0 + 2) {
                            const int pa = 16 * (I - nb0), pb = 16 * (J - nb0);
                            f64x4 t = acc[m];
#pragma unroll
                            for (int s = 0; s < 8; ++s)
                                t = __builtin_amdgcn_mfma_f64_16x16x4f64(-Y[pa + cc][4 * s + kq], Y[pb + cc][4 * s + kq],
                                                                         t, 0, 0, 0);
                            acc[m] = t;
                            if (J < nb0 + 2) {  // the next panel
#pragma unroll
                                for (int u = 0; u < 4; ++u) X[pa - 32 + 4 * u + kq][pb + cc] = t[u];
                            }
                        }
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
// Output B = L^{-T} (k x k FP32 row-major): B[c][r] = L^{-1}[r][c]; or, with
// B64, L^{-1} itself in FP64 (k x k row-major, zeros above the diagonal).
constexpr int kTrinvThreads = 1024;

template <int NB>
__global__ __launch_bounds__(kTrinvThreads) void trinv_kernel(const double *__restrict__ Lin,
                                                              const double *__restrict__ LIin, int k,
                                                              float *__restrict__ B, const int *__restrict__ run,
                                                              double *__restrict__ B64 = nullptr) {
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
    // X is read by other waves: by the first block row's products, or, in the
    // last column block (no block rows below it), by the output loop directly
    __syncthreads();
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
    if (B64) {  // uniform
        for (int t = tid; t < 16 * k; t += kTrinvThreads) {
            const int r = t >> 4, jj = t & 15, c = c0 + jj;
            if (c < k) B64[static_cast<uint64_t>(r) * k + c] = (r >= c) ? X[r][jj] : 0.0;
        }
        return;
    }
    for (int jj = 0; jj < 16 && c0 + jj < k; ++jj) {
        float *brow = B + static_cast<uint64_t>(c0 + jj) * k;
        for (int r = tid; r < k; r += kTrinvThreads)
            brow[r] = (r >= cb * 32) ? static_cast<float>(X[r][jj]) : 0.0f;
    }
}

// Q = X L^{-T} by blocked forward substitution (Q L^T = X), for the
// orthonormalisation step of CholeskyQR: with L's blocks below the diagonal
// (Lin) and the inverses of its 32 x 32 diagonal blocks (LIin), both FP64 from
// the factorisation and rounded to FP32 as they are staged, block column J of
// Q is
//     Q_J = (X_J - sum_{I < J} Q_I L_JI^T) LI_J^T.
// One workgroup per 32 rows of X (76 KB of LDS: two workgroups per CU).  Wave
// w works on row group g = w / 2 (16 rows) and column half h = w % 2 of each
// 32-wide block column; the group's rows of -Q stay in LDS (they are the A
// operand of the later block columns, and the sign makes the update a plain
// accumulation).  Per block column, two barriers:
//   A  panel L_J,0..J-1 and LI_J staged (LI double-buffered: its last reader
//      is the diagonal product after B); -Q_{J-1} of both halves visible;
//   B  both halves of T = X_J - Q L^T in the group's LDS tile (the panel's
//      last reader is the update before B, so the next staging, after B,
//      may overwrite it).
// The global loads of the next panel, LI and X block are issued after A and
// are in flight during the products.  The products run on the FP32 matrix
// cores (v_mfma_f32_16x16x4f32: operand lane 16 kk + i holds row / column i;
// accumulator register u of lane l holds row 4 (l / 16) + u, column l % 16);
// the reduction index is permuted within each 32-column block so that lane
// group kk holds columns 8 kk .. 8 kk + 7 (two 16-byte LDS reads per
// operand), and even and odd steps accumulate in two chains.  Replaces the
// triangular inverse and the X * L^{-T} product (two launches, one of them
// latency-bound on k / 16 CUs).
// pv[i] = src[8 i] for i < 2 J (J <= 7): constant slot indices on every path,
// so that the slots stay in registers.
template <int PV>
__device__ __forceinline__ void fetch_panel(double2 (&pv)[PV], const double2 *__restrict__ src, int J) {
#define BSQ_PANEL_PAIR(j)                                   \
    case j:                                                 \
        if constexpr (PV >= 2 * (j)) {                      \
            pv[2 * (j) - 1] = src[8 * (2 * (j) - 1)];       \
            pv[2 * (j) - 2] = src[8 * (2 * (j) - 2)];       \
        }                                                   \
        [[fallthrough]];
    switch (J) {
        BSQ_PANEL_PAIR(7)
        BSQ_PANEL_PAIR(6)
        BSQ_PANEL_PAIR(5)
        BSQ_PANEL_PAIR(4)
        BSQ_PANEL_PAIR(3)
        BSQ_PANEL_PAIR(2)
        BSQ_PANEL_PAIR(1)
        default: break;
    }
#undef BSQ_PANEL_PAIR
}
constexpr int kSolveRows = 32;
template <int NB>
__global__ __launch_bounds__(256, 2) void chol_solve_kernel(const float *__restrict__ X, int M, int k,
                                                            const double *__restrict__ Lin,
                                                            const double *__restrict__ LIin, float *__restrict__ Q) {
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    constexpr int KP = NB * 32, QP = KP + 4, LP = (NB > 1 ? (NB - 1) * 32 : 32) + 4, TP = 36;
    constexpr int PV = NB > 1 ? 2 * (NB - 1) : 1;  // 16-byte panel loads per thread, widest panel
    __shared__ __align__(16) float Qs[2][16][QP];   // -Q of this workgroup's rows, per row group
    __shared__ __align__(16) float Ls[32][LP];      // L_J,0..J-1
    __shared__ __align__(16) float LIs[2][32][TP];  // LI_J (buffer J % 2)
    __shared__ __align__(16) float Ts[2][16][TP];   // T of each row group in operand layout
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kk = lane >> 4, cc = lane & 15, g = wave >> 1, h = wave & 1;
    const int r0 = blockIdx.x * kSolveRows + 16 * g;  // this wave's first row
    const int pr = tid >> 3, pc = tid & 7;             // panel row, 16-byte column phase
    const double2 *Lv = reinterpret_cast<const double2 *>(Lin);
    const double2 *LIv = reinterpret_cast<const double2 *>(LIin);
    double2 pv[PV], lv[2];
    float xv[4];
    // loads of block column J (panel rows: PV slots, the first J used)
#define BSQ_SOLVE_FETCH(J)                                                                          \
    do {                                                                                            \
        const double2 *src = Lv + (static_cast<uint64_t>(32 * (J) + pr) * KP) / 2 + pc;            \
        fetch_panel<PV>(pv, src, (J));                                                              \
        lv[0] = LIv[static_cast<uint64_t>(J) * 512 + tid];                                          \
        lv[1] = LIv[static_cast<uint64_t>(J) * 512 + 256 + tid];                                    \
        _Pragma("unroll") for (int u = 0; u < 4; ++u) {                                             \
            const int row = r0 + 4 * kk + u, col = 32 * (J) + 16 * h + cc;                          \
            xv[u] = (row < M && col < k) ? X[static_cast<uint64_t>(row) * k + col] : 0.0f;          \
        }                                                                                           \
    } while (0)
    for (int i = 0; i < PV; ++i) pv[i] = make_double2(0.0, 0.0);
    BSQ_SOLVE_FETCH(0);
    // unrolled: every trip count and LDS offset below is a constant
#pragma unroll
    for (int J = 0; J < NB; ++J) {
        const int b = J & 1;
#pragma unroll
        for (int i = 0; i < PV; ++i)  // slots >= 2 J land in columns the update does not use
            *reinterpret_cast<float2 *>(&Ls[pr][2 * (pc + 8 * i)]) =
                make_float2(static_cast<float>(pv[i].x), static_cast<float>(pv[i].y));
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int t = 2 * tid + 512 * e;
            *reinterpret_cast<float2 *>(&LIs[b][t >> 5][t & 31]) =
                make_float2(static_cast<float>(lv[e].x), static_cast<float>(lv[e].y));
        }
        f32x4v acc = {xv[0], xv[1], xv[2], xv[3]}, acc1 = {0.f, 0.f, 0.f, 0.f};
        __syncthreads();  // A
        if (J + 1 < NB) BSQ_SOLVE_FETCH(J + 1);
        // T = X_J - Q_{0..J-1} L_J,0..J-1^T  (K = 32 J)
#pragma unroll
        for (int I = 0; I < J; ++I) {
            const int o = 32 * I + 8 * kk;
            const float4 c0 = *reinterpret_cast<const float4 *>(&Qs[g][cc][o]);
            const float4 c1 = *reinterpret_cast<const float4 *>(&Qs[g][cc][o + 4]);
            const float4 d0 = *reinterpret_cast<const float4 *>(&Ls[16 * h + cc][o]);
            const float4 d1 = *reinterpret_cast<const float4 *>(&Ls[16 * h + cc][o + 4]);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.x, d0.x, acc, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.y, d0.y, acc1, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.z, d0.z, acc, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.w, d0.w, acc1, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.x, d1.x, acc, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.y, d1.y, acc1, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.z, d1.z, acc, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.w, d1.w, acc1, 0, 0, 0);
        }
        acc += acc1;
#pragma unroll
        for (int u = 0; u < 4; ++u) Ts[g][4 * kk + u][16 * h + cc] = acc[u];
        __syncthreads();  // B
        f32x4v q = {0.f, 0.f, 0.f, 0.f}, q1 = {0.f, 0.f, 0.f, 0.f};
        {
            const float4 *ta = reinterpret_cast<const float4 *>(&Ts[g][cc][8 * kk]);
            const float4 *lb = reinterpret_cast<const float4 *>(&LIs[b][16 * h + cc][8 * kk]);
            const float4 c0 = ta[0], c1 = ta[1], d0 = lb[0], d1 = lb[1];
            q = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.x, d0.x, q, 0, 0, 0);
            q1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.y, d0.y, q1, 0, 0, 0);
            q = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.z, d0.z, q, 0, 0, 0);
            q1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.w, d0.w, q1, 0, 0, 0);
            q = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.x, d1.x, q, 0, 0, 0);
            q1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.y, d1.y, q1, 0, 0, 0);
            q = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.z, d1.z, q, 0, 0, 0);
            q1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.w, d1.w, q1, 0, 0, 0);
        }
        q += q1;
        // -Q_J -> LDS (operand of the later block columns), Q_J to the output
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int rl = 4 * kk + u, col = 32 * J + 16 * h + cc, row = r0 + rl;
            Qs[g][rl][col] = -q[u];
            if (row < M && col < k) Q[static_cast<uint64_t>(row) * k + col] = q[u];
        }
    }
}

template <int NB>
void chol_solve(const double *G, int k, double *Lbuf, const float *X, int M, float *Q, int *status,
                hipStream_t stream) {
    constexpr uint64_t KP = NB * 32;
    double *L = Lbuf, *LI = Lbuf + KP * KP;
    chol_blocked_kernel<NB><<<1, kCholThreads, 0, stream>>>(G, k, L, LI, status, nullptr);
    BSQ_HIP(hipGetLastError());
    chol_solve_kernel<NB><<<static_cast<unsigned>(ceil_div(M, kSolveRows)), 256, 0, stream>>>(X, M, k, L, LI, Q);
    BSQ_HIP(hipGetLastError());
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

// C = alpha op(A) op(B) + (D ? D : 0), FP64, for the k x k blocks of the
// two-level Cholesky below (M, N, K <= a few hundred).  op(A) is M x K (A
// stored K x M when TA), op(B) is K x N (B stored N x K when TB).  One 32 x 32
// tile of C per workgroup of 256 lanes, 2 x 2 outputs per lane.  K is staged
// through LDS 128 at a time, every load of a chunk issued before any is
// stored (16-deep chunks, one memory round trip each, took 30 us for a
// 256^3 product); entries outside the operands read as zero.
constexpr int kDgemmKc = 128;
template <bool TA, bool TB>
__global__ __launch_bounds__(256) void dgemm_small_kernel(int M, int N, int K, double alpha,
                                                          const double *__restrict__ A, int lda,
                                                          const double *__restrict__ B, int ldb,
                                                          const double *__restrict__ D, int ldd,
                                                          double *__restrict__ C, int ldc) {
    __shared__ double As[kDgemmKc][33];  // As[kk][m]
    __shared__ double Bs[kDgemmKc][33];  // Bs[kk][n]
    constexpr int kPer = 32 * kDgemmKc / 256;  // chunk elements per lane and operand
    const int tid = threadIdx.x, m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
    const int tr = 2 * (tid >> 4), tc = 2 * (tid & 15);
    double acc[2][2] = {{0.0, 0.0}, {0.0, 0.0}};
    for (int k0 = 0; k0 < K; k0 += kDgemmKc) {
        // element (kk, i) of the A and B chunks: consecutive lanes read
        // consecutive addresses in either storage order
        double a[kPer], b[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int t = tid + 256 * q;
            const int kk = TA ? (t >> 5) : (t & (kDgemmKc - 1)), i = TA ? (t & 31) : (t / kDgemmKc);
            const int gk = k0 + kk, gm = m0 + i;
            a[q] = (gk < K && gm < M)
                       ? (TA ? A[static_cast<uint64_t>(gk) * lda + gm] : A[static_cast<uint64_t>(gm) * lda + gk])
                       : 0.0;
            const int kb = TB ? (t & (kDgemmKc - 1)) : (t >> 5), j = TB ? (t / kDgemmKc) : (t & 31);
            const int gkb = k0 + kb, gnb = n0 + j;
            b[q] = (gkb < K && gnb < N)
                       ? (TB ? B[static_cast<uint64_t>(gnb) * ldb + gkb] : B[static_cast<uint64_t>(gkb) * ldb + gnb])
                       : 0.0;
        }
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int t = tid + 256 * q;
            const int kk = TA ? (t >> 5) : (t & (kDgemmKc - 1)), i = TA ? (t & 31) : (t / kDgemmKc);
            As[kk][i] = a[q];
            const int kb = TB ? (t & (kDgemmKc - 1)) : (t >> 5), j = TB ? (t / kDgemmKc) : (t & 31);
            Bs[kb][j] = b[q];
        }
        __syncthreads();
        const int kn = min(kDgemmKc, K - k0);
        for (int kk = 0; kk < kn; ++kk) {
            const double a0 = As[kk][tr], a1 = As[kk][tr + 1], b0 = Bs[kk][tc], b1 = Bs[kk][tc + 1];
            acc[0][0] = fma(a0, b0, acc[0][0]);
            acc[0][1] = fma(a0, b1, acc[0][1]);
            acc[1][0] = fma(a1, b0, acc[1][0]);
            acc[1][1] = fma(a1, b1, acc[1][1]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const int r = m0 + tr + u, c = n0 + tc + v;
            if (r < M && c < N) {
                double x = alpha * acc[u][v];
                if (D) x += D[static_cast<uint64_t>(r) * ldd + c];
                C[static_cast<uint64_t>(r) * ldc + c] = x;
            }
        }
}

template <bool TA, bool TB>
void dgemm_small(int M, int N, int K, double alpha, const double *A, int lda, const double *B, int ldb,
                 const double *D, int ldd, double *C, int ldc, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(ceil_div(N, 32)), static_cast<unsigned>(ceil_div(M, 32)));
    dgemm_small_kernel<TA, TB><<<grid, 256, 0, stream>>>(M, N, K, alpha, A, lda, B, ldb, D, ldd, C, ldc);
    BSQ_HIP(hipGetLastError());
}

// dst (rows x cols, ld dld) = src (ld sld) in FP64, or zeros when src is
// null; with dst32, the values rounded to FP32 go there instead.  (A kernel,
// not a memset: the no-allocation SVD entry point may run under graph
// capture.)
__global__ void dcopy_block_kernel(const double *__restrict__ src, int sld, int rows, int cols,
                                   double *__restrict__ dst, int dld, float *__restrict__ dst32) {
    const uint64_t n = static_cast<uint64_t>(rows) * cols;
    for (uint64_t t = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < n;
         t += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const int r = static_cast<int>(t / cols), c = static_cast<int>(t % cols);
        const double v = src ? src[static_cast<uint64_t>(r) * sld + c] : 0.0;
        if (dst32) dst32[static_cast<uint64_t>(r) * dld + c] = static_cast<float>(v);
        else dst[static_cast<uint64_t>(r) * dld + c] = v;
    }
}

void dcopy_block(const double *src, int sld, int rows, int cols, double *dst, int dld, float *dst32,
                 hipStream_t stream) {
    const uint64_t n = static_cast<uint64_t>(rows) * cols;
    dcopy_block_kernel<<<static_cast<unsigned>(std::min<uint64_t>(ceil_div(n, 256), 1024)), 256, 0, stream>>>(
        src, sld, rows, cols, dst, dld, dst32);
    BSQ_HIP(hipGetLastError());
}

// G = L L^T and L^{-1} (FP64, k x k) on the blocked one-workgroup kernels
// (k <= 256): the factorisation, then the triangular inverse.
void chol_inverse_f64(const double *G, int k, double *Lbuf, double *Linv, int *status, hipStream_t stream) {
    const int nb = static_cast<int>(ceil_div(k, 32));
    auto go = [&](auto nbc) {
        constexpr int NB = decltype(nbc)::value;
        double *L = Lbuf, *LI = Lbuf + static_cast<uint64_t>(NB) * 32 * NB * 32;
        chol_blocked_kernel<NB><<<1, kCholThreads, 0, stream>>>(G, k, L, LI, status, nullptr);
        BSQ_HIP(hipGetLastError());
        trinv_kernel<NB><<<static_cast<unsigned>(ceil_div(k, 16)), kTrinvThreads, 0, stream>>>(L, LI, k, nullptr,
                                                                                               nullptr, Linv);
        BSQ_HIP(hipGetLastError());
    };
    switch (nb) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 3: go(std::integral_constant<int, 3>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        case 5: go(std::integral_constant<int, 5>{}); break;
        case 6: go(std::integral_constant<int, 6>{}); break;
        case 7: go(std::integral_constant<int, 7>{}); break;
        default: go(std::integral_constant<int, 8>{}); break;
    }
}

}  // namespace

// FP64 doubles needed by the L buffer of launch_chol_blocked and
// launch_chol_solve for rank k: L and the diagonal-block inverses.
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

// G = L L^T (with shifted restarts on breakdown) and Q = X L^{-T} for the
// M x k FP32 matrix X (row-major, leading dimension k) whose Gram G is.
void launch_chol_solve(const double *G, int k, double *Lbuf, const float *X, int M, float *Q, int *status,
                       hipStream_t stream) {
    BSQ_REQUIRE(chol_blocked_supported(k) && M > 0 && X && Q && X != Q, "chol solve: bad arguments");
    switch (ceil_div(k, 32)) {
        case 1: chol_solve<1>(G, k, Lbuf, X, M, Q, status, stream); break;
        case 2: chol_solve<2>(G, k, Lbuf, X, M, Q, status, stream); break;
        case 3: chol_solve<3>(G, k, Lbuf, X, M, Q, status, stream); break;
        case 4: chol_solve<4>(G, k, Lbuf, X, M, Q, status, stream); break;
        case 5: chol_solve<5>(G, k, Lbuf, X, M, Q, status, stream); break;
        case 6: chol_solve<6>(G, k, Lbuf, X, M, Q, status, stream); break;
        case 7: chol_solve<7>(G, k, Lbuf, X, M, Q, status, stream); break;
        default: chol_solve<8>(G, k, Lbuf, X, M, Q, status, stream); break;
    }
}

// Two-level Cholesky for 256 < k <= 512: with G = [[G11, G21^T], [G21, G22]]
// split at k1 = 256,
//   L11 = chol(G11);  L21 = G21 L11^{-T};  L22 = chol(G22 - L21 L21^T);
//   L^{-1} = [[L11^{-1}, 0], [-L22^{-1} L21 L11^{-1}, L22^{-1}]],
// both diagonal factorisations on the blocked one-workgroup kernels (each
// shifted and restarted on its own block when it breaks down: L L^T then
// equals G plus a non-negative diagonal, still a basis change of the same
// column space for CholeskyQR), the off-diagonal products in FP64.  Linv gets
// L^{-1} in FP32 (k x k row-major, zeros above the diagonal), as
// launch_chol_inv writes it.  `work` holds chol_inv_2x2_work_doubles(k)
// doubles; status[0] and status[1] count the two blocks' restarts.
bool chol_inv_2x2_supported(int k) { return k > 256 && k <= 512; }

uint64_t chol_inv_2x2_work_doubles(int k) {
    const uint64_t k1 = 256, k2 = static_cast<uint64_t>(k) - k1;
    return 2 * chol_blocked_buffer_doubles(256) + k1 * k1 * 2 + k2 * k2 * 2 + k2 * k1 * 3;
}

void launch_chol_inv_2x2(const double *G, int k, double *work, float *Linv, int *status, hipStream_t stream) {
    BSQ_REQUIRE(chol_inv_2x2_supported(k) && G && work && Linv && status, "chol 2x2: bad arguments");
    const int k1 = 256, k2 = k - k1;
    double *w = work;
    auto take = [&](uint64_t n) {
        double *p = w;
        w += n;
        return p;
    };
    double *Lb1 = take(chol_blocked_buffer_doubles(256)), *Lb2 = take(chol_blocked_buffer_doubles(256));
    double *G11 = take(static_cast<uint64_t>(k1) * k1), *Li1 = take(static_cast<uint64_t>(k1) * k1);
    double *S = take(static_cast<uint64_t>(k2) * k2), *Li2 = take(static_cast<uint64_t>(k2) * k2);
    double *L21 = take(static_cast<uint64_t>(k2) * k1), *T = take(static_cast<uint64_t>(k2) * k1);
    double *I21 = take(static_cast<uint64_t>(k2) * k1);
    const double *G21 = G + static_cast<uint64_t>(k1) * k, *G22 = G21 + k1;
    dcopy_block(G, k, k1, k1, G11, k1, nullptr, stream);
    chol_inverse_f64(G11, k1, Lb1, Li1, status, stream);
    // L21 = G21 Li1^T;  S = G22 - L21 L21^T
    dgemm_small<false, true>(k2, k1, k1, 1.0, G21, k, Li1, k1, nullptr, 0, L21, k1, stream);
    dgemm_small<false, true>(k2, k2, k1, -1.0, L21, k1, L21, k1, G22, k, S, k2, stream);
    chol_inverse_f64(S, k2, Lb2, Li2, status + 1, stream);
    // (L^{-1})21 = -Li2 (L21 Li1)
    dgemm_small<false, false>(k2, k1, k1, 1.0, L21, k1, Li1, k1, nullptr, 0, T, k1, stream);
    dgemm_small<false, false>(k2, k1, k2, -1.0, Li2, k2, T, k1, nullptr, 0, I21, k1, stream);
    // Linv = [[Li1, 0], [I21, Li2]] in FP32
    dcopy_block(Li1, k1, k1, k1, nullptr, k, Linv, stream);
    dcopy_block(nullptr, 0, k1, k2, nullptr, k, Linv + k1, stream);
    dcopy_block(I21, k1, k2, k1, nullptr, k, Linv + static_cast<uint64_t>(k1) * k, stream);
    dcopy_block(Li2, k2, k2, k2, nullptr, k, Linv + static_cast<uint64_t>(k1) * k + k1, stream);
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
