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
// Every operand of a thread is requested before the first one is used: the
// residual, kReduceBatch slices at a time and kNormPer float4 of x at a time
// (indices clamped, so no load sits under a branch; the clamped copies are
// masked out of the sums). A runtime-bounded loop of loads would wait for
// each load before issuing the next, one memory round trip per slice past
// the first batch. The sums keep their order: slices 0, 1, .., ks - 1, and
// each thread's x elements in the order of the strided loop, so the results
// are those of one load at a time.
constexpr int kReduceBatch = 16;
constexpr int kNormPer = 4;  // float4 of x per thread and round (K <= 4096 in one)

template <int EPI, bool NORM>
__global__ __launch_bounds__(kReduceThreads) void k_mm_reduce(const float* __restrict__ part, int ks,
                                                        int M, int NR, int N,
                                                        float* __restrict__ y, int ldy,
                                                        const float* __restrict__ x, int ldx,
                                                        int K, float eps) {
    const int m = blockIdx.y, n = blockIdx.x * kReduceThreads + threadIdx.x;
    const int nc = min(n, N - 1);
    float* dst = y + (size_t)m * ldy + nc;
    const float resid = EPI == MMR_RESID ? *dst : 0.0f;
    const size_t sstride = (size_t)M * NR;
    const float* pr = part + (size_t)m * NR + nc;
    float vg[kReduceBatch], vu[kReduceBatch];
    auto request = [&](int k0) {
#pragma unroll
        for (int j = 0; j < kReduceBatch; ++j) {
            const size_t o = (size_t)min(k0 + j, ks - 1) * sstride;
            vg[j] = pr[o];
            vu[j] = EPI == MMR_SWIGLU ? pr[o + N] : 0.0f;
        }
    };
    float rsv = 1.0f;
    if constexpr (NORM) {
        // the first kNormPer float4 of x per thread go out before the slices
        // (K <= 4 * kNormPer * kReduceThreads needs no more); later rounds
        // wait for everything requested before them
        __shared__ float red[kReduceThreads / QLM_WAVE];
        const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * ldx);
        const int K4 = K >> 2;
        float4 v[kNormPer];
        auto load_x = [&](int i0) {
#pragma unroll
            for (int j = 0; j < kNormPer; ++j)
                v[j] = xr[min(i0 + j * kReduceThreads + (int)threadIdx.x, K4 - 1)];
        };
        float ss = 0.0f;
        auto add_x = [&](int i0) {
#pragma unroll
            for (int j = 0; j < kNormPer; ++j) {
                // a clamped copy adds +0 to a sum that is >= +0: unchanged
                const bool in = i0 + j * kReduceThreads + (int)threadIdx.x < K4;
                const float4 e = in ? v[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                ss = fmaf(e.x, e.x, ss);
                ss = fmaf(e.y, e.y, ss);
                ss = fmaf(e.z, e.z, ss);
                ss = fmaf(e.w, e.w, ss);
            }
        };
        load_x(0);
        request(0);
        add_x(0);
        for (int i0 = kNormPer * kReduceThreads; i0 < K4; i0 += kNormPer * kReduceThreads) {
            load_x(i0);
            add_x(i0);
        }
        rsv = 1.0f / sqrtf(block_sum(ss, red) / (float)K + eps);
    } else {
        request(0);
    }
    // slices summed in order (g starts at +0 and never becomes -0, so adding
    // +0 for a masked slot leaves it unchanged)
    float g = 0.0f, u = 0.0f;
    for (int k0 = 0;;) {
#pragma unroll
        for (int j = 0; j < kReduceBatch; ++j) {
            const bool in = k0 + j < ks;
            g += in ? vg[j] : 0.0f;
            if constexpr (EPI == MMR_SWIGLU) u += in ? vu[j] : 0.0f;
        }
        k0 += kReduceBatch;
        if (k0 >= ks) break;
        request(k0);
    }
    if (n >= N) return;
    if constexpr (NORM) {
        g *= rsv;
        u *= rsv;
    }
    if constexpr (EPI == MMR_SWIGLU)
        *dst = silu_f(g) * u;
    else if constexpr (EPI == MMR_RESID)
        *dst = resid + g;
    else
        *dst = g;
}

}  // namespace
