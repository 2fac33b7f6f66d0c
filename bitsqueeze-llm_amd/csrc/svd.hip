// Randomised rank-q SVD (range finder with power iterations), the low-rank
// reconstruction and the Gaussian sketch generator.
//
// Algorithm (reference modules/svd_lowrank_cuda/src/svd_lowrank_cuda.cu:
// 129-137, 284-426, 478-524): with A_w = A (m >= n) or A^T (m < n), of size
// M_w x N_w, and k = max(1, min(q, m, n)) (no oversampling):
//     X = A_w R; Q = orth(X)
//     repeat niter: Q' = orth(A_w^T Q); Q = orth(A_w Q')
//     B = Q^T A_w = U_hat S V_hat^T;  U_w = Q U_hat
//     outputs (row-major): U = U_w, V = V_hat, or swapped when m < n.
// Design on MI355X: the big matrix is read in place (row-major, as op(A) or
// op(A)^T inside the MFMA GEMM, no transposed copy); orth() is CholeskyQR
// with the Gram matrix formed in FP64 (twice for the final basis); the SVD of
// B is taken from the FP64 eigen-decomposition of B B^T = Y^T Y with
// Y = A_w^T Q, so that U_hat comes from a k x k problem and
// V_hat = Y U_hat / S by one more GEMM.  Signs are normalised so that the
// largest-magnitude entry of every column of U is positive.
#include "bsq_internal.hpp"

#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>

namespace bsq {

// launchers from gemm.hip / linalg.hip
uint64_t gemm_workspace_bytes(int M, int N, int K);
void launch_gemm(bool ta, bool tb, int M, int N, int K, const float *A, int lda, const float *B, int ldb, float *C,
                 int ldc, const float *a_colscale, const float *minuend, float *workspace, uint64_t workspace_bytes,
                 hipStream_t stream);
uint64_t gram_workspace_bytes(int M, int k);
void launch_gram(const float *X, int M, int k, int ld, double *G, double *workspace, hipStream_t stream,
                 double *rowsq = nullptr);
void launch_chol_inv(const double *G, int k, double *W, float *Linv, int *status, double *ext, hipStream_t stream);
bool chol_inv_2x2_supported(int k);
uint64_t chol_inv_2x2_work_doubles(int k);
void launch_chol_inv_2x2(const double *G, int k, double *work, float *Linv, int *status, hipStream_t stream);
uint64_t chol_blocked_buffer_doubles(int k);
bool chol_blocked_supported(int k);
void launch_chol_blocked(const double *G, int k, double *Lbuf, float *B, int *status, hipStream_t stream,
                         const int *run = nullptr);
void launch_orth_refine(const double *G, const double *rowsq, int k, double *Lbuf, float *B, int *status, int *run,
                        hipStream_t stream);
void launch_chol_solve(const double *G, int k, double *Lbuf, const float *X, int M, float *Q, int *status,
                       hipStream_t stream);
void launch_syev(const double *G, int k, double *W, double *Z, double *small, double *scratch, int *iscratch,
                 double *lambda, float *Uh, hipStream_t stream);

namespace {

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC'11): counter = element group index, key = seed.
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
    constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(M0, c.x), lo0 = M0 * c.x;
        const uint32_t hi1 = __umulhi(M1, c.z), lo1 = M1 * c.z;
        c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
        k.x += W0;
        k.y += W1;
    }
    return c;
}

__global__ void gaussian_fill_kernel(float *__restrict__ out, uint64_t n, uint64_t seed) {
    const uint64_t groups = (n + 3) / 4;
    for (uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < groups;
         g += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint4 r = philox4x32_10(make_uint4(static_cast<uint32_t>(g), static_cast<uint32_t>(g >> 32), 0u, 0u),
                                      make_uint2(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)));
        // Box-Muller on (r.x, r.y) and (r.z, r.w); u1 in (0, 1]
        constexpr float kInv32 = 2.3283064365386963e-10f;
        constexpr float kTwoPi = 6.283185307179586f;
        const float u1 = (static_cast<float>(r.x) + 1.0f) * kInv32, u2 = static_cast<float>(r.y) * kInv32;
        const float u3 = (static_cast<float>(r.z) + 1.0f) * kInv32, u4 = static_cast<float>(r.w) * kInv32;
        const float ra = sqrtf(-2.0f * logf(fminf(u1, 1.0f))), rb = sqrtf(-2.0f * logf(fminf(u3, 1.0f)));
        float s1, c1, s2, c2;
        sincosf(kTwoPi * u2, &s1, &c1);
        sincosf(kTwoPi * u4, &s2, &c2);
        const float v[4] = {ra * c1, ra * s1, rb * c2, rb * s2};
        const uint64_t e0 = g * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (e0 + i < n) out[e0 + i] = v[i];
    }
}

// S[t] = sqrt(max(lambda[t], 0))
__global__ void sqrt_eig_kernel(const double *__restrict__ lambda, int k, float *__restrict__ S) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < k) S[t] = static_cast<float>(sqrt(fmax(lambda[t], 0.0)));
}

// Column t of V (rows x k, row-major) divided by its 2-norm (FP64 sum).
// Column statistics for the final normalisation, row-chunk by row-chunk with
// coalesced row reads (lane t = column t): over chunk c of the rows,
//   U:  largest |U[i][t]| and its first row (the sign reference),
//   Vh: sum of Vh[i][t]^2 (FP64).
constexpr int kColChunks = 64;

__global__ __launch_bounds__(256) void colstat_kernel(const float *__restrict__ U, int mu,
                                                       const float *__restrict__ Vh, int nv, int k,
                                                       float *__restrict__ pbest, int *__restrict__ pidx,
                                                       double *__restrict__ psum) {
    const int chunk = blockIdx.x;
    if (blockIdx.y == 0) {
        const int r0 = static_cast<int>((static_cast<int64_t>(mu) * chunk) / kColChunks);
        const int r1 = static_cast<int>((static_cast<int64_t>(mu) * (chunk + 1)) / kColChunks);
        for (int t = threadIdx.x; t < k; t += blockDim.x) {
            float best = -1.0f;
            int bidx = 0x7FFFFFFF;
#pragma unroll 8
            for (int i = r0; i < r1; ++i) {
                const float a = fabsf(U[static_cast<uint64_t>(i) * k + t]);
                if (a > best) {  // strict: the first row wins ties
                    best = a;
                    bidx = i;
                }
            }
            pbest[static_cast<uint64_t>(chunk) * k + t] = best;
            pidx[static_cast<uint64_t>(chunk) * k + t] = bidx;
        }
    } else {
        const int r0 = static_cast<int>((static_cast<int64_t>(nv) * chunk) / kColChunks);
        const int r1 = static_cast<int>((static_cast<int64_t>(nv) * (chunk + 1)) / kColChunks);
        for (int t = threadIdx.x; t < k; t += blockDim.x) {
            double s = 0.0;
#pragma unroll 8
            for (int i = r0; i < r1; ++i) {
                const double v = Vh[static_cast<uint64_t>(i) * k + t];
                s = fma(v, v, s);
            }
            psum[static_cast<uint64_t>(chunk) * k + t] = s;
        }
    }
}

// Per column (one wave, lane c holding chunk c's statistics): the sign that
// makes the first largest-|.| entry of U[:, t] non-negative, and
// 1 / ||Vh[:, t]|| (1 for a zero column).  The chunks combine by a butterfly:
// largest value first, lowest index among equals; the squared norms by the
// same fixed tree in every lane.
__global__ __launch_bounds__(256) void colfinal_kernel(const float *__restrict__ U, int k,
                                                       const float *__restrict__ pbest, const int *__restrict__ pidx,
                                                       const double *__restrict__ psum, float *__restrict__ usign,
                                                       float *__restrict__ vscale) {
    static_assert(kColChunks == 64, "one lane per chunk");
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= k) return;  // whole waves
    const uint64_t e = static_cast<uint64_t>(lane) * k + t;
    float best = pbest[e];
    int bidx = pidx[e];
    double s = psum[e];
    for (int off = 32; off >= 1; off >>= 1) {
        const float ob = __shfl_xor(best, off);
        const int oi = __shfl_xor(bidx, off);
        const double os = __shfl_xor(s, off);
        if (ob > best || (ob == best && oi < bidx)) {
            best = ob;
            bidx = oi;
        }
        s += os;
    }
    if (lane == 0) {
        const float sg = (bidx != 0x7FFFFFFF && U[static_cast<uint64_t>(bidx) * k + t] < 0.0f) ? -1.0f : 1.0f;
        usign[t] = sg;
        vscale[t] = (s > 0.0) ? sg * static_cast<float>(1.0 / sqrt(s)) : sg;
    }
}

// Uw[:, t] *= usign[t];  Vh[:, t] *= vscale[t]  (coalesced rows)
__global__ void colscale_kernel(float *__restrict__ Uw, uint64_t nu, float *__restrict__ Vh, uint64_t nv, int k,
                                const float *__restrict__ usign, const float *__restrict__ vscale) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < nu; e += stride)
        Uw[e] *= usign[e % k];
    for (uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < nv; e += stride)
        Vh[e] *= vscale[e % k];
}

template <typename T>
T *alloc(uint64_t count) {
    if (count == 0) return nullptr;
    void *p = nullptr;
    BSQ_HIP(hipMalloc(&p, count * sizeof(T)));
    return static_cast<T *>(p);
}

template <typename T>
void release(T *&p) noexcept {
    if (p) (void)hipFree(p);
    p = nullptr;
}

}  // namespace

struct SvdPlan {
    int m = 0, n = 0, k = 0, niter = 0;
    bool transposed = false;
    int Mw = 0, Nw = 0;
    float *R = nullptr, *X = nullptr, *X2 = nullptr, *Y = nullptr, *Y2 = nullptr;
    float *Linv = nullptr, *Uh = nullptr;
    double *G = nullptr, *W = nullptr, *Z = nullptr, *small = nullptr, *scratch = nullptr, *lambda = nullptr;
    double *Lbuf = nullptr;  // blocked Cholesky: L and the inverses of its diagonal blocks
    float *cbest = nullptr, *csign = nullptr;  // column statistics of the final normalisation
    int *cidx = nullptr;
    double *csum = nullptr;
    double *rowsq = nullptr;  // per-row squared distance of the final Gram from I
    int *iscratch = nullptr, *status = nullptr;
    double *gram_ws = nullptr;
    float *gemm_ws = nullptr;
    uint64_t gemm_ws_bytes = 0;
    bool owns = true;  // buffers from hipMalloc (freed here), else carved from a caller's arena

    ~SvdPlan() {
        if (!owns) return;
        release(R);
        release(X);
        release(X2);
        release(Y);
        release(Y2);
        release(Linv);
        release(Uh);
        release(G);
        release(W);
        release(Lbuf);
        release(cbest);
        release(csign);
        release(cidx);
        release(csum);
        release(rowsq);
        release(Z);
        release(small);
        release(scratch);
        release(lambda);
        release(iscratch);
        release(status);
        release(gram_ws);
        release(gemm_ws);
    }
};

namespace {

// Shape fields of a plan (k = max(1, min(q, m, n)), svd_lowrank_cuda.cu:129-137).
void plan_shape(SvdPlan &p, int m, int n, int q, int niter) {
    BSQ_REQUIRE(m > 0 && n > 0 && q > 0 && niter >= 0, "svd: bad arguments");
    p.m = m;
    p.n = n;
    p.k = std::max(1, std::min(q, std::min(m, n)));
    p.niter = niter;
    p.transposed = m < n;
    p.Mw = p.transposed ? n : m;
    p.Nw = p.transposed ? m : n;
}

// Every device buffer of the plan, in one place: `get(ptr, count)` sets each
// pointer (hipMalloc per buffer, or a bump pointer over an arena).
template <class Get>
void plan_buffers(SvdPlan &p, Get &&get) {
    const uint64_t k = p.k;
    get(p.R, p.Nw * k);
    get(p.X, p.Mw * k);
    get(p.X2, p.Mw * k);
    get(p.Y, p.Nw * k);
    get(p.Y2, p.Nw * k);
    get(p.Linv, k * k);
    get(p.Uh, k * k);
    get(p.G, k * k);
    get(p.W, k * k);
    if (chol_blocked_supported(static_cast<int>(k))) get(p.Lbuf, chol_blocked_buffer_doubles(static_cast<int>(k)));
    get(p.Z, k * k);
    get(p.small, 4 * k + 8);
    get(p.cbest, kColChunks * k);
    get(p.cidx, kColChunks * k);
    get(p.csum, kColChunks * k);
    get(p.rowsq, k);
    get(p.csign, 2 * k);
    get(p.scratch, std::max<uint64_t>(9 * k * k + 2 * k,
                                      chol_inv_2x2_supported(static_cast<int>(k))
                                          ? chol_inv_2x2_work_doubles(static_cast<int>(k))
                                          : 0));
    get(p.lambda, k);
    get(p.iscratch, 2 * k * k);
    get(p.status, 4);
    const uint64_t gw = std::max(gram_workspace_bytes(p.Mw, p.k), gram_workspace_bytes(p.Nw, p.k));
    get(p.gram_ws, gw / sizeof(double) + 1);
    uint64_t ws = 0;
    ws = std::max(ws, gemm_workspace_bytes(p.Mw, p.k, p.Nw));
    ws = std::max(ws, gemm_workspace_bytes(p.Nw, p.k, p.Mw));
    p.gemm_ws_bytes = ws;
    if (ws) get(p.gemm_ws, ws / sizeof(float));
}

constexpr uint64_t kArenaAlign = 256;

}  // namespace

SvdPlan *svd_plan_create(int m, int n, int q, int niter) {
    auto *p = new SvdPlan;
    try {
        plan_shape(*p, m, n, q, niter);
        plan_buffers(*p, [](auto *&ptr, uint64_t count) {
            using T = std::remove_reference_t<decltype(*ptr)>;
            ptr = alloc<T>(count);
        });
    } catch (...) {
        delete p;
        throw;
    }
    return p;
}

uint64_t svd_plan_arena_bytes(int m, int n, int q, int niter) {
    SvdPlan p;
    p.owns = false;
    plan_shape(p, m, n, q, niter);
    uint64_t total = 0;
    plan_buffers(p, [&](auto *&ptr, uint64_t count) {
        using T = std::remove_reference_t<decltype(*ptr)>;
        total += ceil_div(count * sizeof(T), kArenaAlign) * kArenaAlign;
        ptr = nullptr;
    });
    return total;
}

void svd_plan_init_arena(SvdPlan &p, int m, int n, int q, int niter, void *arena, uint64_t arena_bytes) {
    BSQ_REQUIRE(arena && (reinterpret_cast<uintptr_t>(arena) % kArenaAlign) == 0, "svd: arena not 256-byte aligned");
    p.owns = false;
    plan_shape(p, m, n, q, niter);
    const uint64_t need = svd_plan_arena_bytes(m, n, q, niter);
    BSQ_REQUIRE(need <= arena_bytes, "svd: shape needs more scratch than the arena holds");
    auto *base = static_cast<uint8_t *>(arena);
    uint64_t off = 0;
    plan_buffers(p, [&](auto *&ptr, uint64_t count) {
        using T = std::remove_reference_t<decltype(*ptr)>;
        ptr = reinterpret_cast<T *>(base + off);
        off += ceil_div(count * sizeof(T), kArenaAlign) * kArenaAlign;
    });
}

void svd_plan_destroy(SvdPlan *plan) noexcept { delete plan; }

int svd_plan_rank(const SvdPlan *plan) { return plan ? plan->k : 0; }

void svd_run(SvdPlan *p, const float *A, const float *sketch, uint64_t seed, float *U, float *S, float *V,
             hipStream_t st) {
    BSQ_REQUIRE(p && A && U && S && V, "svd: null argument");
    const int m = p->m, n = p->n, k = p->k, Mw = p->Mw, Nw = p->Nw;
    const float *R = sketch;
    if (!R) {
        launch_gaussian_fill(p->R, static_cast<uint64_t>(Nw) * k, seed, st);
        R = p->R;
    }
    // X (Mw x k) = A_w * B (B is Nw x k)
    auto aw_times = [&](const float *Bm, float *out) {
        timed_launch(kTimeRangeFinder, st, [&] {
            if (!p->transposed) launch_gemm(false, false, m, k, n, A, n, Bm, k, out, k, nullptr, nullptr, p->gemm_ws,
                                            p->gemm_ws_bytes, st);
            else launch_gemm(true, false, n, k, m, A, n, Bm, k, out, k, nullptr, nullptr, p->gemm_ws,
                             p->gemm_ws_bytes, st);
        });
    };
    // Y (Nw x k) = A_w^T * B (B is Mw x k)
    auto awt_times = [&](const float *Bm, float *out) {
        timed_launch(kTimeRangeFinder, st, [&] {
            if (!p->transposed) launch_gemm(true, false, n, k, m, A, n, Bm, k, out, k, nullptr, nullptr, p->gemm_ws,
                                            p->gemm_ws_bytes, st);
            else launch_gemm(false, false, m, k, n, A, n, Bm, k, out, k, nullptr, nullptr, p->gemm_ws,
                             p->gemm_ws_bytes, st);
        });
    };
    // one CholeskyQR pass: out = in * L^{-T}, G = in^T in = L L^T
    auto orth = [&](const float *in, float *out, int rows) {
        launch_gram(in, rows, k, k, p->G, p->gram_ws, st);
        if (p->Lbuf) {  // out L^T = in, by blocked forward substitution
            launch_chol_solve(p->G, k, p->Lbuf, in, rows, out, p->status, st);
            return;
        }
        if (chol_inv_2x2_supported(k))  // Linv holds L^{-1}
            launch_chol_inv_2x2(p->G, k, p->scratch, p->Linv, p->status, st);
        else
            launch_chol_inv(p->G, k, p->W, p->Linv, p->status, p->scratch, st);
        launch_gemm(false, true, rows, k, k, in, k, p->Linv, k, out, k, nullptr, nullptr, p->gemm_ws,
                    p->gemm_ws_bytes, st);
    };
    float *Xa = p->X, *Xb = p->X2, *Ya = p->Y, *Yb = p->Y2;
    aw_times(R, Xa);
    orth(Xa, Xb, Mw);
    std::swap(Xa, Xb);
    for (int it = 0; it < p->niter; ++it) {
        awt_times(Xa, Ya);
        orth(Ya, Yb, Nw);
        std::swap(Ya, Yb);
        aw_times(Ya, Xa);
        orth(Xa, Xb, Mw);
        std::swap(Xa, Xb);
    }
    // second pass on the final basis: CholeskyQR2, or, when the first pass
    // left it orthonormal to working accuracy, one Newton-Schulz step
    if (p->Lbuf) {
        launch_gram(Xa, Mw, k, k, p->G, p->gram_ws, st, p->rowsq);
        launch_orth_refine(p->G, p->rowsq, k, p->Lbuf, p->Linv, p->status, p->status + 1, st);
        launch_gemm(false, false, Mw, k, k, Xa, k, p->Linv, k, Xb, k, nullptr, nullptr, p->gemm_ws,
                    p->gemm_ws_bytes, st);
    } else {
        orth(Xa, Xb, Mw);
    }
    std::swap(Xa, Xb);
    // Y = A_w^T Q = B^T;  B B^T = Y^T Y = U_hat diag(S^2) U_hat^T
    awt_times(Xa, Ya);
    launch_gram(Ya, Nw, k, k, p->G, p->gram_ws, st);
    launch_syev(p->G, k, p->W, p->Z, p->small, p->scratch, p->iscratch, p->lambda, p->Uh, st);
    sqrt_eig_kernel<<<static_cast<unsigned>(ceil_div(k, 256)), 256, 0, st>>>(p->lambda, k, S);
    BSQ_HIP(hipGetLastError());
    float *Uw_out = p->transposed ? V : U;  // Mw x k
    float *Vh_out = p->transposed ? U : V;  // Nw x k
    launch_gemm(false, false, Mw, k, k, Xa, k, p->Uh, k, Uw_out, k, nullptr, nullptr, p->gemm_ws, p->gemm_ws_bytes,
                st);
    launch_gemm(false, false, Nw, k, k, Ya, k, p->Uh, k, Vh_out, k, nullptr, nullptr, p->gemm_ws, p->gemm_ws_bytes,
                st);
    // V_hat = Y U_hat / S (columns normalised), then the sign convention: the
    // first largest-|.| entry of every column of U is non-negative (U and V
    // flipped together).  Positive scaling does not move that entry, so both
    // come from one pass of column statistics.
    const float *Usrc = p->transposed ? Vh_out : Uw_out;  // U in the output orientation
    colstat_kernel<<<dim3(kColChunks, 2), 256, 0, st>>>(Usrc, m, Vh_out, Nw, k, p->cbest, p->cidx, p->csum);
    BSQ_HIP(hipGetLastError());
    colfinal_kernel<<<static_cast<unsigned>(ceil_div(k, 4)), 256, 0, st>>>(Usrc, k, p->cbest, p->cidx, p->csum,
                                                                           p->csign, p->csign + k);
    BSQ_HIP(hipGetLastError());
    {
        const uint64_t nu = static_cast<uint64_t>(Mw) * k, nvh = static_cast<uint64_t>(Nw) * k;
        uint64_t grid = ceil_div(std::max(nu, nvh), 256);
        grid = std::min<uint64_t>(grid, static_cast<uint64_t>(cu_count()) * 8);
        colscale_kernel<<<static_cast<unsigned>(grid), 256, 0, st>>>(Uw_out, nu, Vh_out, nvh, k, p->csign,
                                                                     p->csign + k);
        BSQ_HIP(hipGetLastError());
    }
}

void launch_reconstruct(const float *U, const float *S, const float *V, int m, int n, int k, const float *minuend,
                        float *out, hipStream_t stream) {
    BSQ_REQUIRE(m > 0 && n > 0 && k > 0 && U && S && V && out, "reconstruct: bad arguments");
    // out = (minuend -) (U diag(S)) V^T: A = U with columns scaled by S, B = V^T
    launch_gemm(false, true, m, n, k, U, k, V, k, out, n, S, minuend, nullptr, 0, stream);
}

void launch_gaussian_fill(float *out, uint64_t n, uint64_t seed, hipStream_t stream) {
    if (n == 0) return;
    BSQ_REQUIRE(out != nullptr, "gaussian fill: null output");
    const uint64_t groups = (n + 3) / 4;
    uint64_t grid = (groups + 255) / 256;
    const uint64_t cap = static_cast<uint64_t>(cu_count()) * 8;
    if (grid > cap) grid = cap;
    gaussian_fill_kernel<<<static_cast<unsigned>(grid), 256, 0, stream>>>(out, n, seed);
    BSQ_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// No-allocation variant of the standalone SVD (bsq_svd_lowrank_noalloc): the
// plan's buffers are carved out of one file-scope device array instead of
// hipMalloc'ed per call, for callers that cannot allocate (code under HIP
// graph capture, allocation-free serving loops).  Every call on a GPU uses
// that GPU's copy of the array, so calls that overlap on one GPU race.  The
// SVD kernels write every scratch word before reading it (nothing needs to
// start at zero), so the contents a previous call left behind do not matter.
// ---------------------------------------------------------------------------
constexpr uint64_t kNoAllocScratchBytes = 256ull << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device with that device current (each GPU holds its own copy at its own
// address; the host-side name is not a device address).
void *scratch_address() {
    int dev = 0;
    BSQ_HIP(hipGetDevice(&dev));
    BSQ_REQUIRE(dev >= 0 && dev < kMaxDevices, "svd noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        BSQ_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        BSQ_REQUIRE(p != nullptr, "svd noalloc: scratch symbol has no device address");
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

void svd_run_noalloc(const float *A, int m, int n, int q, int niter, const float *sketch, uint64_t seed, float *U,
                     float *S, float *V, hipStream_t stream) {
    BSQ_REQUIRE(A && U && S && V, "svd noalloc: null argument");
    BSQ_REQUIRE(m > 0 && n > 0 && q > 0 && niter >= 0, "svd noalloc: bad shape");
    const uint64_t need = svd_plan_arena_bytes(m, n, q, niter);
    if (need > kNoAllocScratchBytes)
        fail("svd noalloc: this shape needs " + std::to_string(need) + " bytes of scratch, above the " +
             std::to_string(kNoAllocScratchBytes) + " bytes the no-allocation entry point holds");
    void *arena = scratch_address();
    SvdPlan plan;
    svd_plan_init_arena(plan, m, n, q, niter, arena, kNoAllocScratchBytes);
    svd_run(&plan, A, sketch, seed, U, S, V, stream);
}

uint64_t svd_noalloc_scratch_bytes() { return kNoAllocScratchBytes; }

}  // namespace bsq
