// Randomised low-rank SVD (placeholder plan) + reconstruction + sketch generator.
#include "bsq_internal.hpp"

namespace bsq {
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

// out[i, j] = (minuend[i, j] -) sum_k (U[i, k] * S[k]) * V[j, k]
constexpr int kT = 16;
__global__ void reconstruct_simple_kernel(const float *__restrict__ U, const float *__restrict__ S,
                                          const float *__restrict__ V, int m, int n, int k,
                                          const float *__restrict__ minuend, float *__restrict__ out) {
    __shared__ float us[kT][kT + 1];
    __shared__ float vs[kT][kT + 1];
    const int i = blockIdx.y * kT + threadIdx.y, j = blockIdx.x * kT + threadIdx.x;
    float acc = 0.0f;
    for (int k0 = 0; k0 < k; k0 += kT) {
        const int ku = k0 + threadIdx.x;
        const int iu = blockIdx.y * kT + threadIdx.y;
        us[threadIdx.y][threadIdx.x] = (iu < m && ku < k) ? U[static_cast<uint64_t>(iu) * k + ku] * S[ku] : 0.0f;
        const int jv = blockIdx.x * kT + threadIdx.y;
        vs[threadIdx.y][threadIdx.x] = (jv < n && ku < k) ? V[static_cast<uint64_t>(jv) * k + ku] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int t = 0; t < kT; ++t) acc = fmaf(us[threadIdx.y][t], vs[threadIdx.x][t], acc);
        __syncthreads();
    }
    if (i < m && j < n) {
        const uint64_t e = static_cast<uint64_t>(i) * n + j;
        out[e] = minuend ? minuend[e] - acc : acc;
    }
}

}  // namespace

struct SvdPlan {
    int m = 0, n = 0, q = 0, niter = 0;
};

SvdPlan *svd_plan_create(int m, int n, int q, int niter) {
    BSQ_REQUIRE(m > 0 && n > 0 && q > 0 && niter >= 0, "svd: bad arguments");
    auto *p = new SvdPlan;
    p->m = m;
    p->n = n;
    p->q = std::max(1, std::min(q, std::min(m, n)));
    p->niter = niter;
    return p;
}

void svd_plan_destroy(SvdPlan *plan) noexcept { delete plan; }

int svd_plan_rank(const SvdPlan *plan) { return plan ? plan->q : 0; }

void svd_run(SvdPlan *, const float *, const float *, uint64_t, float *, float *, float *, hipStream_t) {
    fail("svd_lowrank: not implemented yet");
}

void launch_reconstruct(const float *U, const float *S, const float *V, int m, int n, int k, const float *minuend,
                        float *out, hipStream_t stream) {
    BSQ_REQUIRE(m > 0 && n > 0 && k > 0 && U && S && V && out, "reconstruct: bad arguments");
    dim3 grid((n + kT - 1) / kT, (m + kT - 1) / kT);
    reconstruct_simple_kernel<<<grid, dim3(kT, kT), 0, stream>>>(U, S, V, m, n, k, minuend, out);
    BSQ_HIP(hipGetLastError());
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

}  // namespace bsq
