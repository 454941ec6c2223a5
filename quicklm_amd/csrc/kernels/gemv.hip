// int8 weight-only GEMV for decode (M <= 4 activation rows per launch):
//   y[m, n] = sum_k x[m, k] * q[n, k] * s[n, k / G]
// Replaces math::matmul's int8 branch (reference math_ops.cpp:820-900,
// int8_gemv_range :558-579, dot8_avx2_int8 :448-494).
//
// Layout and mapping (HBM-bound; one pass over the weights):
//   - A workgroup is 4 waves; each wave is two half-waves of 32 lanes. A
//     half-wave owns R output rows and walks K in 16-byte chunks, so one
//     load instruction of a half-wave covers 512 contiguous weight bytes of
//     one row (every K of the model family is a multiple of 512, so no lane
//     idles on a ragged tail).
//   - The next step's weight chunks are loaded before the current step is
//     computed (two steps of R x 16 B per lane in flight).
//   - Activations are staged once per workgroup in LDS, sub-chunk-major
//     ([m][j][chunk][4], j = 0..3) so that a half-wave's 16-byte LDS reads
//     hit consecutive addresses (conflict-free). When M*K floats do not fit
//     the LDS budget the chunks are read from global memory (L1/L2).
//   - Group scales (G = 32) are applied per 16-element partial with one FMA;
//     per-row scales (G = K) once after the reduction.
//   - Partial sums are reduced with butterflies inside each half-wave.
//   - Fused prologue (RMSNorm with zero-centred gain) and epilogues (residual
//     add, SiLU(gate)*up) remove separate elementwise launches.

#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / QLM_WAVE;
constexpr int kLdsBudget = 64 * 1024;

enum { PRO_NONE = 0, PRO_RMSNORM = 1 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

__device__ __forceinline__ float dot16(const int4 w, const float4 a, const float4 b,
                                       const float4 c, const float4 d) {
    float f0, f1, f2, f3;
    i8x4_to_f32(w.x, f0, f1, f2, f3);
    float p0 = a.x * f0;
    p0 = fmaf(a.y, f1, p0);
    p0 = fmaf(a.z, f2, p0);
    p0 = fmaf(a.w, f3, p0);
    i8x4_to_f32(w.y, f0, f1, f2, f3);
    float p1 = b.x * f0;
    p1 = fmaf(b.y, f1, p1);
    p1 = fmaf(b.z, f2, p1);
    p1 = fmaf(b.w, f3, p1);
    i8x4_to_f32(w.z, f0, f1, f2, f3);
    float p2 = c.x * f0;
    p2 = fmaf(c.y, f1, p2);
    p2 = fmaf(c.z, f2, p2);
    p2 = fmaf(c.w, f3, p2);
    i8x4_to_f32(w.w, f0, f1, f2, f3);
    float p3 = d.x * f0;
    p3 = fmaf(d.y, f1, p3);
    p3 = fmaf(d.z, f2, p3);
    p3 = fmaf(d.w, f3, p3);
    return (p0 + p1) + (p2 + p3);
}

__device__ __forceinline__ float4 norm4(float4 v, float rs, float4 w) {
    // Reference order: (x * s) * (1 + w)  (math_ops.cpp:1021-1031).
    v.x = (v.x * rs) * (1.0f + w.x);
    v.y = (v.y * rs) * (1.0f + w.y);
    v.z = (v.z * rs) * (1.0f + w.z);
    v.w = (v.w * rs) * (1.0f + w.w);
    return v;
}

template <int R, int M, bool ROWSCALE, int PRO, int EPI, bool XLDS>
__global__ __launch_bounds__(kThreads) void k_gemv_i8(
    const float* __restrict__ x, int ldx, int mr, const float* __restrict__ nw, float eps,
    const int8_t* __restrict__ q, const float* __restrict__ sc, float* __restrict__ y, int ldy,
    int N, int K, int F) {
    extern __shared__ float4 xs4[];  // [M][4][nchunk] float4 when XLDS
    __shared__ float red[kWaves * M];

    const int tid = threadIdx.x;
    const int lane = tid & (QLM_WAVE - 1);
    const int wave = tid / QLM_WAVE;
    const int half = lane >> 5;
    const int hl = lane & 31;
    const int nchunk = K >> 4;
    const int nblk = K >> 5;

    // ---- prologue: per-row RMS scale and activation staging ----
    float rs[M];
#pragma unroll
    for (int m = 0; m < M; ++m) rs[m] = 1.0f;
    if constexpr (PRO == PRO_RMSNORM) {
        float ss[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            ss[m] = 0.0f;
            if (m < mr) {
                const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * ldx);
                for (int i = tid; i < (K >> 2); i += kThreads) {
                    float4 v = xr[i];
                    ss[m] = fmaf(v.x, v.x, ss[m]);
                    ss[m] = fmaf(v.y, v.y, ss[m]);
                    ss[m] = fmaf(v.z, v.z, ss[m]);
                    ss[m] = fmaf(v.w, v.w, ss[m]);
                }
            }
            ss[m] = wave_sum(ss[m]);
        }
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < M; ++m) red[wave * M + m] = ss[m];
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float t = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) t += red[w * M + m];
            rs[m] = 1.0f / sqrtf(t / (float)K + eps);
        }
    }
    if constexpr (XLDS) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * ldx);
            const float4* wr = reinterpret_cast<const float4*>(nw);
            for (int i = tid; i < (K >> 2); i += kThreads) {
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (m < mr) {
                    v = xr[i];
                    if constexpr (PRO == PRO_RMSNORM) v = norm4(v, rs[m], wr[i]);
                }
                const int c = i >> 2, j = i & 3;
                xs4[(m * 4 + j) * nchunk + c] = v;
            }
        }
        __syncthreads();
    }

    // ---- row ownership ----
    int wrow[R];   // weight row per slot
    int orow[R];   // output row per slot
    bool rv[R];
    if constexpr (EPI == EPI_SWIGLU) {
        const int base = (blockIdx.x * kWaves + wave) * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            orow[r] = base + r;
            rv[r] = orow[r] < N;
            wrow[r] = half * F + orow[r];
        }
    } else {
        const int base = ((blockIdx.x * kWaves + wave) * 2 + half) * R;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            orow[r] = base + r;
            rv[r] = orow[r] < N;
            wrow[r] = orow[r];
        }
    }

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

    auto load_w = [&](int c, int4 (&wv)[R], float (&sv)[R]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (rv[r] && c < nchunk) {
                wv[r] = *reinterpret_cast<const int4*>(q + (size_t)wrow[r] * K + ((size_t)c << 4));
                if constexpr (!ROWSCALE) sv[r] = sc[(size_t)wrow[r] * nblk + (c >> 1)];
            } else {
                wv[r] = make_int4(0, 0, 0, 0);
                sv[r] = 0.0f;
            }
        }
    };

    int4 cw[R], nwv[R];
    float cs[R], ns[R];
    int c = hl;
    load_w(c, cw, cs);
    while (c < nchunk) {
        const int cn = c + 32;
        load_w(cn, nwv, ns);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float4 a, b, cc, d;
            if constexpr (XLDS) {
                a = xs4[(m * 4 + 0) * nchunk + c];
                b = xs4[(m * 4 + 1) * nchunk + c];
                cc = xs4[(m * 4 + 2) * nchunk + c];
                d = xs4[(m * 4 + 3) * nchunk + c];
            } else {
                const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * ldx) + c * 4;
                if (m < mr) {
                    a = xr[0];
                    b = xr[1];
                    cc = xr[2];
                    d = xr[3];
                    if constexpr (PRO == PRO_RMSNORM) {
                        const float4* wr = reinterpret_cast<const float4*>(nw) + c * 4;
                        a = norm4(a, rs[m], wr[0]);
                        b = norm4(b, rs[m], wr[1]);
                        cc = norm4(cc, rs[m], wr[2]);
                        d = norm4(d, rs[m], wr[3]);
                    }
                } else {
                    a = b = cc = d = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float p = dot16(cw[r], a, b, cc, d);
                if constexpr (ROWSCALE)
                    acc[r][m] += p;
                else
                    acc[r][m] = fmaf(p, cs[r], acc[r][m]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            cw[r] = nwv[r];
            cs[r] = ns[r];
        }
        c = cn;
    }

    // ---- reduction inside each half-wave, then epilogue ----
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = group_sum<32>(acc[r][m]);

    if constexpr (ROWSCALE) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = rv[r] ? sc[wrow[r]] : 0.0f;
#pragma unroll
            for (int m = 0; m < M; ++m) acc[r][m] *= s;
        }
    }

    if constexpr (EPI == EPI_SWIGLU) {
        // half 0 holds gate rows, half 1 the matching up rows.
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float up = __shfl_xor(acc[r][m], 32, QLM_WAVE);
                if (lane == r && rv[r] && m < mr) {
                    const float g = acc[r][m];
                    y[(size_t)m * ldy + orow[r]] = silu_f(g) * up;
                }
            }
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if (hl == r && rv[r] && m < mr) {
                    float* dst = y + (size_t)m * ldy + orow[r];
                    if constexpr (EPI == EPI_RESID)
                        *dst = *dst + acc[r][m];
                    else
                        *dst = acc[r][m];
                }
            }
    }
}

template <int R, int M, bool ROWSCALE, int PRO, int EPI, bool XLDS>
int launch_one(const float* x, int ldx, int mr, const float* nw, float eps, const int8_t* q,
               const float* sc, float* y, int ldy, int N, int K, int F, hipStream_t st) {
    const int rows_per_wg = (EPI == EPI_SWIGLU) ? kWaves * R : kWaves * 2 * R;
    const int grid = (N + rows_per_wg - 1) / rows_per_wg;
    const size_t lds = XLDS ? (size_t)M * K * sizeof(float) : 0;
    hipLaunchKernelGGL((k_gemv_i8<R, M, ROWSCALE, PRO, EPI, XLDS>), dim3(grid), dim3(kThreads),
                       lds, st, x, ldx, mr, nw, eps, q, sc, y, ldy, N, K, F);
    return qlm_launch_status();
}

template <int M, bool ROWSCALE, int PRO, int EPI>
int launch_r(int R, bool xlds, const float* x, int ldx, int mr, const float* nw, float eps,
             const int8_t* q, const float* sc, float* y, int ldy, int N, int K, int F,
             hipStream_t st) {
#define QLM_GEMV_CASE(RR)                                                                    \
    if (R == RR) {                                                                           \
        if (xlds)                                                                            \
            return launch_one<RR, M, ROWSCALE, PRO, EPI, true>(x, ldx, mr, nw, eps, q, sc, y, \
                                                               ldy, N, K, F, st);            \
        return launch_one<RR, M, ROWSCALE, PRO, EPI, false>(x, ldx, mr, nw, eps, q, sc, y,   \
                                                            ldy, N, K, F, st);               \
    }
    QLM_GEMV_CASE(4)
    QLM_GEMV_CASE(2)
    QLM_GEMV_CASE(1)
#undef QLM_GEMV_CASE
    return QLM_ERR_ARG;
}

template <bool ROWSCALE, int PRO, int EPI>
int launch_m(int Mt, int R, bool xlds, const float* x, int ldx, int mr, const float* nw,
             float eps, const int8_t* q, const float* sc, float* y, int ldy, int N, int K, int F,
             hipStream_t st) {
    if (Mt == 1)
        return launch_r<1, ROWSCALE, PRO, EPI>(R, xlds, x, ldx, mr, nw, eps, q, sc, y, ldy, N, K,
                                               F, st);
    if (Mt == 2)
        return launch_r<2, ROWSCALE, PRO, EPI>(R, xlds, x, ldx, mr, nw, eps, q, sc, y, ldy, N, K,
                                               F, st);
    return launch_r<4, ROWSCALE, PRO, EPI>(R, xlds, x, ldx, mr, nw, eps, q, sc, y, ldy, N, K, F,
                                           st);
}

int gemv_dispatch(int pro, int epi, const float* x, int ldx, const float* nw, float eps,
                  const int8_t* q, const float* sc, int group, float* y, int ldy, int M, int N,
                  int K, void* stream) {
    if (!x || !q || !sc || !y || (pro == PRO_RMSNORM && !nw)) return QLM_ERR_ARG;
    if (M <= 0 || N <= 0 || K <= 0 || M > 64) return QLM_ERR_ARG;
    if (K % 16 != 0) return QLM_ERR_SHAPE;
    const bool rowscale = (group == K);
    if (!rowscale && (group != 32 || K % 32 != 0)) return QLM_ERR_SHAPE;
    if (ldx < K || ldy < N || ldx % 4 != 0) return QLM_ERR_SHAPE;
    // 16-byte vector loads of activations, weights and norm gains
    if (((uintptr_t)x | (uintptr_t)q | (uintptr_t)nw) & 15u) return QLM_ERR_SHAPE;
    hipStream_t st = as_stream(stream);
    const int F = N;  // swiglu: up rows start at F
    for (int m0 = 0; m0 < M; m0 += 4) {
        const int mr = (M - m0) < 4 ? (M - m0) : 4;
        const int Mt = mr == 1 ? 1 : (mr == 2 ? 2 : 4);
        const bool xlds = (size_t)Mt * K * sizeof(float) <= (size_t)kLdsBudget;
        const int per_r = (epi == EPI_SWIGLU) ? kWaves : kWaves * 2;
        int R = 1;
        if ((N + per_r * 4 - 1) / (per_r * 4) >= 1024)
            R = 4;
        else if ((N + per_r * 2 - 1) / (per_r * 2) >= 1024)
            R = 2;
        const float* xm = x + (size_t)m0 * ldx;
        float* ym = y + (size_t)m0 * ldy;
        int rc;
#define QLM_GEMV_CALL(RS, P, E) \
    rc = launch_m<RS, P, E>(Mt, R, xlds, xm, ldx, mr, nw, eps, q, sc, ym, ldy, N, K, F, st)
        if (rowscale) {
            if (pro == PRO_NONE && epi == EPI_STORE) QLM_GEMV_CALL(true, PRO_NONE, EPI_STORE);
            else if (pro == PRO_RMSNORM && epi == EPI_STORE) QLM_GEMV_CALL(true, PRO_RMSNORM, EPI_STORE);
            else if (pro == PRO_NONE && epi == EPI_RESID) QLM_GEMV_CALL(true, PRO_NONE, EPI_RESID);
            else QLM_GEMV_CALL(true, PRO_RMSNORM, EPI_SWIGLU);
        } else {
            if (pro == PRO_NONE && epi == EPI_STORE) QLM_GEMV_CALL(false, PRO_NONE, EPI_STORE);
            else if (pro == PRO_RMSNORM && epi == EPI_STORE) QLM_GEMV_CALL(false, PRO_RMSNORM, EPI_STORE);
            else if (pro == PRO_NONE && epi == EPI_RESID) QLM_GEMV_CALL(false, PRO_NONE, EPI_RESID);
            else QLM_GEMV_CALL(false, PRO_RMSNORM, EPI_SWIGLU);
        }
#undef QLM_GEMV_CALL
        if (rc != QLM_OK) return rc;
    }
    return QLM_OK;
}

}  // namespace

extern "C" int qlm_gemv_i8(const float* x, int ldx, const int8_t* q, const float* scales,
                           int group, float* y, int ldy, int M, int N, int K, void* stream) {
    return gemv_dispatch(PRO_NONE, EPI_STORE, x, ldx, nullptr, 0.0f, q, scales, group, y, ldy, M,
                         N, K, stream);
}

extern "C" int qlm_gemv_i8_rmsnorm(const float* x, int ldx, const float* norm_w, float eps,
                                   const int8_t* q, const float* scales, int group, float* y,
                                   int ldy, int M, int N, int K, void* stream) {
    return gemv_dispatch(PRO_RMSNORM, EPI_STORE, x, ldx, norm_w, eps, q, scales, group, y, ldy, M,
                         N, K, stream);
}

extern "C" int qlm_gemv_i8_residual(const float* x, int ldx, const int8_t* q,
                                    const float* scales, int group, float* y, int ldy, int M,
                                    int N, int K, void* stream) {
    return gemv_dispatch(PRO_NONE, EPI_RESID, x, ldx, nullptr, 0.0f, q, scales, group, y, ldy, M,
                         N, K, stream);
}

extern "C" int qlm_gemv_i8_swiglu_rmsnorm(const float* x, int ldx, const float* norm_w,
                                          float eps, const int8_t* q, const float* scales,
                                          int group, float* y, int ldy, int M, int F, int K,
                                          void* stream) {
    return gemv_dispatch(PRO_RMSNORM, EPI_SWIGLU, x, ldx, norm_w, eps, q, scales, group, y, ldy,
                         M, F, K, stream);
}
