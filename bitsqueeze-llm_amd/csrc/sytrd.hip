// Householder tridiagonalisation of the k x k FP64 Gram matrix of the
// randomised SVD's core (k <= 256), one workgroup of 1024 lanes.
//
// The lower triangle of the padded KP x KP matrix (KP = 32 * NB) lives in
// registers, lane (ty, tx) holding element (32a + ty, 32b + tx) of every lower
// 32 x 32 block (a >= b).  Step j (LAPACK dsytd2 order):
//   1. the lanes holding column j copy it to LDS;
//   2. wave 0 forms the reflector v (v[j+1] = 1), tau and e[j];
//   3. every lane forms partial sums of p = A v over its elements, row sums
//      and (by symmetry) column sums, plus its share of v^T A v; the partials
//      land in LDS and four lanes per index finish p;
//   4. w = tau p - (tau^2 / 2) (v^T A v) v, then A -= v w^T + w v^T.
// Four workgroup barriers per step; blocks left of column j are skipped
// (v vanishes there).  Output: d, e, tau and the reflectors row-wise,
// H[j][i] = v_j[i] (zero for i <= j, one at i = j + 1).
#include "bsq_internal.hpp"
#include "wave_ops.hpp"

namespace bsq {
namespace {

constexpr int kTrdThreads = 1024;

__device__ __forceinline__ constexpr int tri(int a, int b) { return a * (a + 1) / 2 + b; }

__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

template <int NB>
__global__ __launch_bounds__(kTrdThreads) void sytrd_blocked_kernel(const double *__restrict__ G, int k,
                                                                     double *__restrict__ d, double *__restrict__ e,
                                                                     double *__restrict__ tau,
                                                                     double *__restrict__ H) {
    // PP pitch 65 (odd): the column-partial writes (16 lanes down a column)
    // and the finishing reads (four lanes per index, 8 banks apart) are free
    // of LDS bank conflicts with 8-byte accesses
    constexpr int KP = NB * 32, NE = NB * (NB + 1) / 2, PITCH = 65;
    __shared__ double xs[KP], vs[KP], ws[KP];
    __shared__ double PP[NB][32][PITCH];  // [blk][y][0..31 row, 32..63 col partials]
    __shared__ double red[kTrdThreads / 64];
    __shared__ double s_tau;

    double r[NE];
    {
        const int tid = threadIdx.x, tx = tid & 31, ty = tid >> 5;
#pragma unroll
        for (int a = 0; a < NB; ++a)
#pragma unroll
            for (int b = 0; b <= a; ++b) {
                // branch-free: G inside (both triangles of the diagonal blocks), 0 in the padding
                const int i = a * 32 + ty, c = b * 32 + tx;
                const bool inside = (i < k) && (c < k);
                const double g = G[inside ? static_cast<uint64_t>(i) * k + c : 0];
                r[tri(a, b)] = inside ? g : 0.0;
            }
    }
    const int steps = k - 2;  // reflectors j = 0 .. k-3
#pragma unroll
    for (int jb = 0; jb < NB; ++jb) {
#pragma unroll 1
        for (int jt = 0; jt < 32; ++jt) {
            const int j = jb * 32 + jt;
            if (j >= steps) break;  // uniform
            const int tid = opaque(static_cast<int>(threadIdx.x));
            const int tx = tid & 31, ty = tid >> 5, lane = tid & 63, wave = tid >> 6;
            // 1. column j (rows > j) -> xs, d[j]
            if (tx == jt) {
#pragma unroll
                for (int a = jb; a < NB; ++a) xs[a * 32 + ty] = r[tri(a, jb)];
                if (ty == jt) d[j] = r[tri(jb, jb)];
            }
            __syncthreads();
            // 2. reflector (wave 0, every lane computes the scalars)
            if (wave == 0) {
                double sig = 0.0;
#pragma unroll
                for (int m = 0; m < KP / 64 + (KP % 64 ? 1 : 0); ++m) {
                    const int i = lane + 64 * m;
                    const double xv = (i < KP) ? xs[min(i, KP - 1)] : 0.0;
                    sig = (i >= j + 2 && i < k) ? fma(xv, xv, sig) : sig;
                }
                sig = wave_sum_dpp(sig);
                const double alpha = xs[j + 1];
                double t = 0.0, beta = alpha, scal = 0.0;
                if (sig > 0.0) {
                    const double nrm = sqrt(fma(alpha, alpha, sig));
                    beta = (alpha >= 0.0) ? -nrm : nrm;
                    t = (beta - alpha) / beta;
                    scal = 1.0 / (alpha - beta);
                }
#pragma unroll
                for (int m = 0; m < KP / 64 + (KP % 64 ? 1 : 0); ++m) {
                    const int i = lane + 64 * m;
                    if (i < KP) {
                        const double v = (i == j + 1) ? 1.0 : ((i > j + 1 && i < k) ? xs[i] * scal : 0.0);
                        vs[i] = v;
                        if (i < k) H[static_cast<uint64_t>(j) * k + i] = v;
                    }
                }
                if (lane == 0) {
                    e[j] = beta;
                    tau[j] = t;
                    s_tau = t;
                }
            }
            __syncthreads();
            const double t = s_tau;
            if (t == 0.0) continue;  // uniform: A is already reduced in column j
            // 3. partial sums of p = A v (rows: sum over this lane's columns;
            // columns: by symmetry) and of v^T A v.  Diagonal blocks: an element
            // counts for its row when tx <= ty and for its column when tx < ty.
            const double mrow = static_cast<double>(1u - (static_cast<unsigned>(ty - tx) >> 31));
            const double mcol = static_cast<double>(static_cast<unsigned>(tx - ty) >> 31);
            // v at this lane's row and column indices, kept in registers for the
            // update below (which then reads mostly w from LDS: LDS bytes per
            // step bound this kernel)
            double va[NB], vb[NB];
#pragma unroll
            for (int a = jb; a < NB; ++a) {
                va[a] = vs[a * 32 + ty];
                vb[a] = vs[a * 32 + tx];
            }
            double quad = 0.0;
#pragma unroll
            for (int a = jb; a < NB; ++a) {
                double rowp = 0.0;
#pragma unroll
                for (int b = jb; b <= a; ++b) rowp = fma(r[tri(a, b)], (a == b) ? vb[b] * mrow : vb[b], rowp);
                PP[a][ty][tx] = rowp;
                quad = fma(rowp, va[a], quad);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int b = jb; b < NB; ++b) {
                double colp = 0.0;
#pragma unroll
                for (int a = b; a < NB; ++a) colp = fma(r[tri(a, b)], (a == b) ? va[a] * mcol : va[a], colp);
                PP[b][tx][32 + ty] = colp;
                quad = fma(colp, vb[b], quad);
            }
            quad = wave_sum_dpp(quad);
            if (lane == 0) red[wave] = quad;
            __syncthreads();
            // finish p: four lanes per index, 16 partials each; blocks left
            // of block jb are skipped (whole waves: 128 lanes per block), the
            // update reads w only at indices in blocks >= jb
            if (tid < 4 * KP && (tid >> 7) >= jb) {
                const int idx = tid >> 2, qq = tid & 3;  // idx = 32 * blk + y
                const int blk = idx >> 5, y = idx & 31;
                // this lane's 16 partials: slots 16 m + 4 qq + s
                double s = 0.0;
#pragma unroll
                for (int m = 0; m < 4; ++m)
#pragma unroll
                    for (int u = 0; u < 4; u += 2) s += PP[blk][y][16 * m + 4 * qq + u] + PP[blk][y][16 * m + 4 * qq + u + 1];
                s = quad_sum(s);
                // K = sum of the 16 wave partials: one LDS read per lane and a
                // 16-lane DPP sum instead of 16 reads per lane
                double K = red[lane & 15];
                K = quad_sum(K);
                K += dpp_read<0x141>(K);  // row_half_mirror: 8-lane sums
                K += dpp_read<0x140>(K);  // row_mirror: 16-lane sums in every lane
                // v^T A v counted every off-diagonal pair twice through rows and
                // columns, which is exactly the symmetric sum
                if (qq == 0) ws[idx] = (idx > j) ? fma(-0.5 * t * t * K, vs[idx], t * s) : 0.0;
            }
            __syncthreads();
            // 4. A -= v w^T + w v^T (v and w vanish at indices <= j)
#pragma unroll
            for (int a = jb; a < NB; ++a) {
                // at NB = 8 the row values are read again instead (holding both
                // vectors through the finish phase spills there)
                const double w_a = ws[a * 32 + ty], v_a = (NB < 8) ? va[a] : vs[a * 32 + ty];
#pragma unroll
                for (int b = jb; b <= a; ++b)
                    r[tri(a, b)] = fma(-v_a, ws[b * 32 + tx], fma(-w_a, vb[b], r[tri(a, b)]));
            }
        }
    }
    // trailing 2 x 2 (or 1 x 1) block
    const int tid = threadIdx.x, tx = tid & 31, ty = tid >> 5;
    const int j2 = k - 2;
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
        for (int b = 0; b <= a; ++b) {
            const int i = a * 32 + ty, c = b * 32 + tx;
            if (i == c && i >= (j2 > 0 ? j2 : 0) && i < k) d[i] = r[tri(a, b)];
            if (j2 >= 0 && i == j2 + 1 && c == j2) e[j2] = r[tri(a, b)];
        }
    if (tid == 0) {
        if (k >= 2) tau[k - 2] = 0.0;
        tau[k - 1] = 0.0;
    }
}

template <int NB>
void sytrd_blocked(const double *G, int k, double *d, double *e, double *tau, double *H, hipStream_t stream) {
    sytrd_blocked_kernel<NB><<<1, kTrdThreads, 0, stream>>>(G, k, d, e, tau, H);
    BSQ_HIP(hipGetLastError());
}

}  // namespace

bool sytrd_blocked_supported(int k) { return k >= 3 && k <= 256; }

// d[0..k), e[0..k-1), tau[0..k) and reflector rows H (k x k) of the symmetric G.
void launch_sytrd_blocked(const double *G, int k, double *d, double *e, double *tau, double *H, hipStream_t stream) {
    BSQ_REQUIRE(sytrd_blocked_supported(k), "sytrd: rank outside the register kernel's range");
    switch (ceil_div(k, 32)) {
        case 1: sytrd_blocked<1>(G, k, d, e, tau, H, stream); break;
        case 2: sytrd_blocked<2>(G, k, d, e, tau, H, stream); break;
        case 3: sytrd_blocked<3>(G, k, d, e, tau, H, stream); break;
        case 4: sytrd_blocked<4>(G, k, d, e, tau, H, stream); break;
        case 5: sytrd_blocked<5>(G, k, d, e, tau, H, stream); break;
        case 6: sytrd_blocked<6>(G, k, d, e, tau, H, stream); break;
        case 7: sytrd_blocked<7>(G, k, d, e, tau, H, stream); break;
        default: sytrd_blocked<8>(G, k, d, e, tau, H, stream); break;
    }
}

}  // namespace bsq
