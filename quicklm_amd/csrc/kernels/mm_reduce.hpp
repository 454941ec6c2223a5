// Ordered reduction of K-split partial sums, shared by the split-K matmuls
// (gemm.hip, gemm_t.hip): slice partials part[ks, m, n] summed in slice order
// (deterministic), then the epilogue.
#pragma once

#include "common.hpp"

namespace {

enum { MMR_STORE = 0, MMR_RESID = 1, MMR_SWIGLU = 2 };
constexpr int kReduceThreads = 256;

// y[m, n] (=, +=) sum over slices of part[ks, m, n], or for SwiGLU
// y[m, n] = silu(gate) * up with gate/up the sums at columns n and F + n.
// Workgroup (bx, m) takes columns bx*256.. of row m. NORM: the slices hold
// (x * (1 + w)) . W and the row's RMSNorm factor 1/sqrt(mean(x^2) + eps) is
// computed here from x and multiplies the sums.
template <int EPI, bool NORM>
__global__ __launch_bounds__(kReduceThreads) void k_mm_reduce(const float* __restrict__ part, int ks,
                                                        int M, int NR, int N,
                                                        float* __restrict__ y, int ldy,
                                                        const float* __restrict__ x, int ldx,
                                                        int K, float eps) {
    const int m = blockIdx.y, n = blockIdx.x * kReduceThreads + threadIdx.x;
    float rsv = 1.0f;
    if constexpr (NORM) {
        __shared__ float red[kReduceThreads / QLM_WAVE];
        const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * ldx);
        float ss = 0.0f;
        for (int i = threadIdx.x; i < (K >> 2); i += kReduceThreads) {
            const float4 v = xr[i];
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
        rsv = 1.0f / sqrtf(block_sum(ss, red) / (float)K + eps);
    }
    if (n >= N) return;
    // slices summed in order; 8 slices' loads issued together
    float g = 0.0f, u = 0.0f;
    const size_t sstride = (size_t)M * NR;
    const float* pr = part + (size_t)m * NR + n;
    int k = 0;
    for (; k + 8 <= ks; k += 8) {
        float vg[8], vu[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            vg[j] = pr[(k + j) * sstride];
            vu[j] = EPI == MMR_SWIGLU ? pr[(k + j) * sstride + N] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            g += vg[j];
            u += vu[j];
        }
    }
    for (; k < ks; ++k) {
        g += pr[k * sstride];
        if constexpr (EPI == MMR_SWIGLU) u += pr[k * sstride + N];
    }
    if constexpr (NORM) {
        g *= rsv;
        u *= rsv;
    }
    float* dst = y + (size_t)m * ldy + n;
    if constexpr (EPI == MMR_SWIGLU)
        *dst = silu_f(g) * u;
    else if constexpr (EPI == MMR_RESID)
        *dst += g;
    else
        *dst = g;
}

}  // namespace
