// int8 weight-only matmul for M > 1 on the gfx950 matrix cores:
//   y[m, n] = sum_k x[m, k] * q[n, k] * s[n, k / G]
// Replaces math::matmul's int8 branch with M > 1 (reference
// math_ops.cpp:845-871: batched decode M = B, prefill M = T - 1).
//
// Arithmetic. The int8 weights are exact in bf16 (|q| <= 127 fits the 8-bit
// significand). Each activation is split into bf16 hi + lo (hi = RNE(x),
// lo = RNE(x - hi)), so hi + lo carries 16 significant bits and the only
// rounding left is |x - hi - lo| <= 2^-17 |x|; the products and sums run in
// fp32 inside v_mfma_f32_16x16x32_bf16. With 32-wide groups each group is
// exactly one MFMA k-step: its two MFMAs (hi, lo) start from zero and the
// 16x16 result is scaled by s[n, group] in fp32 and accumulated, so the
// weights are never rounded. Per-row scales (G = K) chain the MFMAs and
// scale once at the end. Normwise error vs the fp32 reference is ~1e-6.
//
// Tiling. A workgroup is 4 waves arranged WM x WN x WK; a wave owns TM x TN
// 16x16 output tiles (16*TM activation rows x 16*TN weight rows) and the
// WK waves of a (wm, wn) pair split each K chunk by 32-groups, their partial
// tiles summed through LDS in a fixed order at the end. Per chunk of
// KC = 32*WK, x [BM, KC] is staged in LDS as bf16 hi/lo and the weights
// [BN, KC] as bf16; the next chunk is loaded into registers while the
// current one is multiplied.
//   M <= 64 (batched decode): BM = 16..64, BN = 16 (32 for SwiGLU), WK = 4:
//     one pass over the weights, grid = N/16 workgroups.
//   M > 64 (prefill): BM = BN = 128, WK = 1.
// Epilogues: store, residual add, SwiGLU (weights [2F, K]; a wave's first
// TN/2 tiles are gate rows, the last TN/2 the matching up rows, so
// silu(gate)*up is formed in registers).

#include "common.hpp"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

__device__ __forceinline__ unsigned bf16_rne_bits(float x) {
    unsigned u = __float_as_uint(x);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// hi/lo bf16 pair of x packed as (hi, lo) 16-bit halves
__device__ __forceinline__ void split_bf16(float x, unsigned short& hi, unsigned short& lo) {
    const unsigned h = bf16_rne_bits(x);
    hi = (unsigned short)h;
    lo = (unsigned short)bf16_rne_bits(x - __uint_as_float(h << 16));
}

// int8 -> bf16 bits (exact): the float's upper half
__device__ __forceinline__ unsigned short i8_bf16(int v) {
    return (unsigned short)(__float_as_uint((float)v) >> 16);
}

template <int WM, int WN, int WK, int TM, int TN, bool ROWSCALE, int EPI>
__global__ __launch_bounds__(kThreads) void k_mm_i8(const float* __restrict__ x, int ldx,
                                                    const int8_t* __restrict__ q,
                                                    const float* __restrict__ sc,
                                                    float* __restrict__ y, int ldy, int M, int N,
                                                    int K, int F) {
    static_assert(WM * WN * WK == 4, "4 waves");
    static_assert(EPI != EPI_SWIGLU || TN % 2 == 0, "SwiGLU pairs gate and up tiles");
    constexpr int BM = WM * TM * 16;
    constexpr int BN = WN * TN * 16;  // weight rows staged per chunk
    constexpr int KC = 32 * WK;
    constexpr int XP = KC + 8;        // padded LDS rows (bf16 elements)
    constexpr int WP = KC + 8;
    constexpr int XV = BM * KC / 4;   // float4 per x chunk
    constexpr int WV = BN * KC / 16;  // int4 per weight chunk
    constexpr int XPT = (XV + kThreads - 1) / kThreads;
    constexpr int WPT = (WV + kThreads - 1) / kThreads;
    constexpr int NT = TM * TN;
    constexpr int OUT_TN = EPI == EPI_SWIGLU ? TN / 2 : TN;  // output tiles per wave
    constexpr int BN_OUT = WN * OUT_TN * 16;                  // output columns per workgroup
    // LDS: staged chunk (x hi, x lo, w) during the K loop; the same bytes
    // then hold the K-split partial tiles.
    constexpr size_t kStage = (size_t)(2 * BM * XP + BN * WP) * sizeof(unsigned short);
    constexpr size_t kRed = WK > 1 ? (size_t)(WK - 1) * WM * WN * 64 * NT * sizeof(f32x4) : 0;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kStage > kRed ? kStage : kRed];
    unsigned short* xs_hi = reinterpret_cast<unsigned short*>(smem);
    unsigned short* xs_lo = xs_hi + BM * XP;
    unsigned short* ws = xs_lo + BM * XP;
    f32x4* red = reinterpret_cast<f32x4*>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int kw = wave % WK;
    const int wn = (wave / WK) % WN;
    const int wm = wave / (WK * WN);
    const int m0 = blockIdx.y * BM;
    const int nout0 = blockIdx.x * BN_OUT;  // first output column of the workgroup
    const int nblk = K >> 5;

    // staged weight row r -> global weight row (clamped into the matrix)
    auto w_row = [&](int r) -> int {
        int n;
        if constexpr (EPI == EPI_SWIGLU) {
            const int half = BN / 2;
            n = r < half ? nout0 + r : F + nout0 + (r - half);
            const int lim = r < half ? F - 1 : 2 * F - 1;
            return n < lim ? n : lim;
        } else {
            n = nout0 + r;
            return n < N - 1 ? n : N - 1;
        }
    };
    // a wave's tile tn -> first staged row of that tile
    auto tile_row = [&](int tn) -> int {
        if constexpr (EPI == EPI_SWIGLU)
            return tn < TN / 2 ? (wn * (TN / 2) + tn) * 16 : BN / 2 + (wn * (TN / 2) + tn - TN / 2) * 16;
        else
            return (wn * TN + tn) * 16;
    };

    float4 xr[XPT];
    int4 wr[WPT];
    float sr[TN];
    auto load_chunk = [&](int c) {
        const int k0 = c * KC;
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < XV) {
                const int r = i / (KC / 4), c4 = i % (KC / 4);
                const int m = min(m0 + r, M - 1);
                xr[u] = *reinterpret_cast<const float4*>(x + (size_t)m * ldx + k0 + c4 * 4);
            }
        }
#pragma unroll
        for (int u = 0; u < WPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < WV) {
                const int r = i / (KC / 16), c16 = i % (KC / 16);
                wr[u] = *reinterpret_cast<const int4*>(q + (size_t)w_row(r) * K + k0 + c16 * 16);
            }
        }
        if constexpr (!ROWSCALE) {
            const int g = (k0 >> 5) + kw;
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
                sr[tn] = sc[(size_t)w_row(tile_row(tn) + (lane & 15)) * nblk + g];
        }
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < XV) {
                const int r = i / (KC / 4), c4 = i % (KC / 4);
                unsigned short h[4], l[4];
                split_bf16(xr[u].x, h[0], l[0]);
                split_bf16(xr[u].y, h[1], l[1]);
                split_bf16(xr[u].z, h[2], l[2]);
                split_bf16(xr[u].w, h[3], l[3]);
                uint2 ph, pl;
                ph.x = (unsigned)h[0] | ((unsigned)h[1] << 16);
                ph.y = (unsigned)h[2] | ((unsigned)h[3] << 16);
                pl.x = (unsigned)l[0] | ((unsigned)l[1] << 16);
                pl.y = (unsigned)l[2] | ((unsigned)l[3] << 16);
                *reinterpret_cast<uint2*>(&xs_hi[r * XP + c4 * 4]) = ph;
                *reinterpret_cast<uint2*>(&xs_lo[r * XP + c4 * 4]) = pl;
            }
        }
#pragma unroll
        for (int u = 0; u < WPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < WV) {
                const int r = i / (KC / 16), c16 = i % (KC / 16);
                const int wv[4] = {wr[u].x, wr[u].y, wr[u].z, wr[u].w};
                uint4 o[2];
                unsigned* ow = reinterpret_cast<unsigned*>(o);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const unsigned v = (unsigned)wv[j];
                    const int b0 = (int8_t)(v & 0xffu), b1 = (int8_t)((v >> 8) & 0xffu);
                    const int b2 = (int8_t)((v >> 16) & 0xffu), b3 = (int8_t)(v >> 24);
                    ow[2 * j] = (unsigned)i8_bf16(b0) | ((unsigned)i8_bf16(b1) << 16);
                    ow[2 * j + 1] = (unsigned)i8_bf16(b2) | ((unsigned)i8_bf16(b3) << 16);
                }
                uint4* dst = reinterpret_cast<uint4*>(&ws[r * WP + c16 * 16]);
                dst[0] = o[0];
                dst[1] = o[1];
            }
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nch = K / KC;
    load_chunk(0);
    for (int c = 0; c < nch; ++c) {
        float s_cur[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) s_cur[tn] = sr[tn];
        __syncthreads();  // the previous chunk's LDS reads are done
        store_chunk();
        __syncthreads();
        if (c + 1 < nch) load_chunk(c + 1);
        const int kofs = kw * 32 + (lane >> 4) * 8;
        bf16x8 ah[TM], al[TM], bw[TN];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            const int r = (wm * TM + tm) * 16 + (lane & 15);
            ah[tm] = *reinterpret_cast<const bf16x8*>(&xs_hi[r * XP + kofs]);
            al[tm] = *reinterpret_cast<const bf16x8*>(&xs_lo[r * XP + kofs]);
        }
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
            bw[tn] = *reinterpret_cast<const bf16x8*>(&ws[(tile_row(tn) + (lane & 15)) * WP + kofs]);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                if constexpr (ROWSCALE) {
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[tm], bw[tn], acc[tm][tn], 0, 0, 0);
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[tm], bw[tn], acc[tm][tn], 0, 0, 0);
                } else {
                    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[tm], bw[tn], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[tm], bw[tn], d, 0, 0, 0);
                    const float s = s_cur[tn];
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[tm][tn][i] = fmaf(d[i], s, acc[tm][tn][i]);
                }
            }
    }

    // ---- sum the WK partial tiles (fixed order) ----
    if constexpr (WK > 1) {
        const int pair = wm * WN + wn;
        __syncthreads();  // the last chunk's LDS reads are done before red reuses the bytes
        if (kw > 0) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
                    red[(((kw - 1) * WM * WN + pair) * 64 + lane) * NT + tm * TN + tn] = acc[tm][tn];
        }
        __syncthreads();
        if (kw > 0) return;
#pragma unroll
        for (int k2 = 1; k2 < WK; ++k2)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    const f32x4 o = red[(((k2 - 1) * WM * WN + pair) * 64 + lane) * NT + tm * TN + tn];
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[tm][tn][i] += o[i];
                }
    }
    if constexpr (ROWSCALE) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const float s = sc[w_row(tile_row(tn) + (lane & 15))];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[tm][tn][i] *= s;
        }
    }

    // ---- epilogue: lane holds rows (lane/16)*4 + i, column lane%16 of each tile ----
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < OUT_TN; ++tn) {
            const int n = nout0 + (wn * OUT_TN + tn) * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + (wm * TM + tm) * 16 + (lane >> 4) * 4 + i;
                if (m < M && n < N) {
                    float* dst = y + (size_t)m * ldy + n;
                    if constexpr (EPI == EPI_SWIGLU)
                        *dst = silu_f(acc[tm][tn][i]) * acc[tm][tn + TN / 2][i];
                    else if constexpr (EPI == EPI_RESID)
                        *dst += acc[tm][tn][i];
                    else
                        *dst = acc[tm][tn][i];
                }
            }
        }
}

template <int WM, int WN, int WK, int TM, int TN, bool RS, int EPI>
int launch_mm(const float* x, int ldx, const int8_t* q, const float* sc, float* y, int ldy, int M,
              int N, int K, hipStream_t st) {
    constexpr int BM = WM * TM * 16;
    constexpr int BN_OUT = WN * (EPI == EPI_SWIGLU ? TN / 2 : TN) * 16;
    const dim3 grid((N + BN_OUT - 1) / BN_OUT, (M + BM - 1) / BM);
    hipLaunchKernelGGL((k_mm_i8<WM, WN, WK, TM, TN, RS, EPI>), grid, dim3(kThreads), 0, st, x,
                       ldx, q, sc, y, ldy, M, N, K, N);
    return qlm_launch_status();
}

template <bool RS, int EPI>
int mm_dispatch(const float* x, int ldx, const int8_t* q, const float* sc, float* y, int ldy,
                int M, int N, int K, hipStream_t st) {
    constexpr int TNS = EPI == EPI_SWIGLU ? 2 : 1;  // weight tiles per wave, small M
    if (M <= 64 && K % 128 == 0) {
        if (M <= 16) return launch_mm<1, 1, 4, 1, TNS, RS, EPI>(x, ldx, q, sc, y, ldy, M, N, K, st);
        if (M <= 32) return launch_mm<1, 1, 4, 2, TNS, RS, EPI>(x, ldx, q, sc, y, ldy, M, N, K, st);
        return launch_mm<1, 1, 4, 4, TNS, RS, EPI>(x, ldx, q, sc, y, ldy, M, N, K, st);
    }
    return launch_mm<2, 2, 1, 4, 4, RS, EPI>(x, ldx, q, sc, y, ldy, M, N, K, st);
}

}  // namespace

extern "C" int qlm_matmul_i8(const float* x, int ldx, const int8_t* q, const float* scales,
                             int group, float* y, int ldy, int M, int N, int K, int epilogue,
                             void* stream) {
    if (!x || !q || !scales || !y) return QLM_ERR_ARG;
    if (M <= 0 || N <= 0 || K <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    if (K % 32 != 0) return QLM_ERR_SHAPE;
    const bool rowscale = (group == K);
    if (!rowscale && group != 32) return QLM_ERR_SHAPE;
    if (ldx < K || ldy < N || ldx % 4 != 0) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)q) & 15u) return QLM_ERR_SHAPE;
    hipStream_t st = as_stream(stream);
    if (rowscale) {
        if (epilogue == EPI_STORE) return mm_dispatch<true, EPI_STORE>(x, ldx, q, scales, y, ldy, M, N, K, st);
        if (epilogue == EPI_RESID) return mm_dispatch<true, EPI_RESID>(x, ldx, q, scales, y, ldy, M, N, K, st);
        return mm_dispatch<true, EPI_SWIGLU>(x, ldx, q, scales, y, ldy, M, N, K, st);
    }
    if (epilogue == EPI_STORE) return mm_dispatch<false, EPI_STORE>(x, ldx, q, scales, y, ldy, M, N, K, st);
    if (epilogue == EPI_RESID) return mm_dispatch<false, EPI_RESID>(x, ldx, q, scales, y, ldy, M, N, K, st);
    return mm_dispatch<false, EPI_SWIGLU>(x, ldx, q, scales, y, ldy, M, N, K, st);
}
