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
#include "mm_reduce.hpp"

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

// RMSNorm of a staged activation: (x * s) * (1 + w), the reference's order
// (math_ops.cpp:1021-1031), s = 1/sqrt(mean(x^2) + eps) of the row.
__device__ __forceinline__ float4 norm4(float4 v, float s, float4 w) {
    v.x = (v.x * s) * (1.0f + w.x);
    v.y = (v.y * s) * (1.0f + w.y);
    v.z = (v.z * s) * (1.0f + w.z);
    v.w = (v.w * s) * (1.0f + w.w);
    return v;
}

__device__ __forceinline__ void store_hilo(unsigned short* hi, unsigned short* lo, float4 v) {
    unsigned short h[4], l[4];
    split_bf16(v.x, h[0], l[0]);
    split_bf16(v.y, h[1], l[1]);
    split_bf16(v.z, h[2], l[2]);
    split_bf16(v.w, h[3], l[3]);
    *reinterpret_cast<uint2*>(hi) = make_uint2((unsigned)h[0] | ((unsigned)h[1] << 16),
                                               (unsigned)h[2] | ((unsigned)h[3] << 16));
    *reinterpret_cast<uint2*>(lo) = make_uint2((unsigned)l[0] | ((unsigned)l[1] << 16),
                                               (unsigned)l[2] | ((unsigned)l[3] << 16));
}

// 16 int8 -> 16 bf16 (exact), as two 16-byte LDS stores
__device__ __forceinline__ void store_w16(unsigned short* dst, int4 w) {
    const int wv[4] = {w.x, w.y, w.z, w.w};
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
    reinterpret_cast<uint4*>(dst)[0] = o[0];
    reinterpret_cast<uint4*>(dst)[1] = o[1];
}

// Tile-major weights (qlm_mx_swizzle: 16-row x 64-column fragments of 1 KB
// in lane order, each half of a [gate; up] matrix tiled on its own; group-32
// scales as [fragment][h][n]). Row r of the stacked matrix is row r - half F
// of half `half`; its 16 columns k .. k + 15 (k a multiple of 16) are one
// lane's 16 bytes of fragment (tile, k / 64). Per-row scales keep their
// [rows] layout.
struct TileMap {
    int F;           // rows per half (all rows when the matrix has one half)
    int tiles_half;  // 16-row tiles per half
    int nblk64;      // 64-column blocks per row
};
__device__ __forceinline__ int tm_frag(const TileMap& t, int r, int k, int& n) {
    const int half = r >= t.F ? 1 : 0;
    const int rh = r - half * t.F;
    n = rh & 15;
    return (half * t.tiles_half + (rh >> 4)) * t.nblk64 + (k >> 6);
}
// byte offset of row r's 16 columns k .. k + 15
__device__ __forceinline__ size_t tm_off(const TileMap& t, int r, int k) {
    int n;
    const int fb = tm_frag(t, r, k, n);
    return ((size_t)fb * 64 + ((k >> 4) & 3) * 16 + n) * 16;
}
// index of row r's scale for the 32-column group g
__device__ __forceinline__ size_t tm_scale(const TileMap& t, int r, int g) {
    int n;
    const int fb = tm_frag(t, r, g * 32, n);
    return (size_t)fb * 32 + (g & 1) * 16 + n;
}

// WB16: the weights are bf16 rows (the native --precision bf16 form, no
// scales): copied to LDS as they are, the MFMAs chained over K.
// XS: x is already split (k_split_rows): x points at the bf16 hi plane
// [M, ldx] and the lo plane follows it (M * ldx further); any RMSNorm has
// been applied there, so NORM is false.
// KG: 32-column scale groups per staged chunk and wave (more matrix-core work
// between the chunk's load and its use).
// TL: q and sc are tile-major (TileMap tmap); otherwise row-major.
template <int WM, int WN, int WK, int TM, int TN, bool ROWSCALE, int EPI, bool NORM,
          bool WB16 = false, bool XS = false, int KG = 1, bool TL = false>
__global__ __launch_bounds__(kThreads) void k_mm_i8(const float* __restrict__ x, int ldx,
                                                    const float* __restrict__ rs,
                                                    const float* __restrict__ nw,
                                                    const int8_t* __restrict__ q,
                                                    const float* __restrict__ sc,
                                                    float* __restrict__ y, int ldy, int M, int N,
                                                    int K, int F, TileMap tmap) {
    static_assert(WM * WN * WK == 4, "4 waves");
    static_assert(EPI != EPI_SWIGLU || TN % 2 == 0, "SwiGLU pairs gate and up tiles");
    constexpr int BM = WM * TM * 16;
    constexpr int BN = WN * TN * 16;  // weight rows staged per chunk
    constexpr int KC = 32 * WK * KG;
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
    float4 gr[NORM ? XPT : 1];  // RMSNorm gain of the same columns
    float rr[NORM ? XPT : 1];   // RMSNorm row scale
    int4 wr[WPT];
    int4 wr2[WB16 ? WPT : 1];  // bf16 rows: the second 16 bytes of a unit
    // XS: hi and lo bf16 quadruples, kept in integer registers (as floats a
    // pair could read as a denormal and be flushed)
    uint4 xq[XS ? XPT : 1];
    float sr[KG][TN];
    auto load_chunk = [&](int c) {
        const int k0 = c * KC;
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < XV) {
                const int r = i / (KC / 4), c4 = i % (KC / 4);
                const int m = min(m0 + r, M - 1);
                if constexpr (XS) {
                    const uint16_t* xh = reinterpret_cast<const uint16_t*>(x);
                    const size_t o = (size_t)m * ldx + k0 + c4 * 4;
                    const uint2 h = *reinterpret_cast<const uint2*>(xh + o);
                    const uint2 l = *reinterpret_cast<const uint2*>(xh + (size_t)M * ldx + o);
                    xq[u] = make_uint4(h.x, h.y, l.x, l.y);
                } else {
                    xr[u] = *reinterpret_cast<const float4*>(x + (size_t)m * ldx + k0 + c4 * 4);
                }
                if constexpr (NORM) {
                    gr[u] = *reinterpret_cast<const float4*>(nw + k0 + c4 * 4);
                    rr[u] = rs[m];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < WPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < WV) {
                const int r = i / (KC / 16), c16 = i % (KC / 16);
                if constexpr (WB16) {
                    const int4* p = reinterpret_cast<const int4*>(
                        reinterpret_cast<const uint16_t*>(q) + (size_t)w_row(r) * K + k0 + c16 * 16);
                    wr[u] = p[0];
                    wr2[u] = p[1];
                } else if constexpr (TL) {
                    wr[u] = *reinterpret_cast<const int4*>(q + tm_off(tmap, w_row(r), k0 + c16 * 16));
                } else {
                    wr[u] = *reinterpret_cast<const int4*>(q + (size_t)w_row(r) * K + k0 + c16 * 16);
                }
            }
        }
        if constexpr (!ROWSCALE && !WB16) {
#pragma unroll
            for (int gg = 0; gg < KG; ++gg) {
                const int g = (k0 >> 5) + kw * KG + gg;
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    const int wr_ = w_row(tile_row(tn) + (lane & 15));
                    sr[gg][tn] = TL ? sc[tm_scale(tmap, wr_, g)] : sc[(size_t)wr_ * nblk + g];
                }
            }
        }
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < XV && XS) {
                const int r = i / (KC / 4), c4 = i % (KC / 4);
                const uint4 v = xq[XS ? u : 0];
                *reinterpret_cast<uint2*>(&xs_hi[r * XP + c4 * 4]) = make_uint2(v.x, v.y);
                *reinterpret_cast<uint2*>(&xs_lo[r * XP + c4 * 4]) = make_uint2(v.z, v.w);
            } else if (i < XV) {
                const int r = i / (KC / 4), c4 = i % (KC / 4);
                float4 v = xr[u];
                if constexpr (NORM) v = norm4(v, rr[u], gr[u]);
                unsigned short h[4], l[4];
                split_bf16(v.x, h[0], l[0]);
                split_bf16(v.y, h[1], l[1]);
                split_bf16(v.z, h[2], l[2]);
                split_bf16(v.w, h[3], l[3]);
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
            if (i < WV && WB16) {
                const int r = i / (KC / 16), c16 = i % (KC / 16);
                uint4* dst = reinterpret_cast<uint4*>(&ws[r * WP + c16 * 16]);
                dst[0] = __builtin_bit_cast(uint4, wr[u]);
                dst[1] = __builtin_bit_cast(uint4, wr2[WB16 ? u : 0]);
            } else if (i < WV) {
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
        float s_cur[KG][TN];
#pragma unroll
        for (int gg = 0; gg < KG; ++gg)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) s_cur[gg][tn] = sr[gg][tn];
        __syncthreads();  // the previous chunk's LDS reads are done
        store_chunk();
        __syncthreads();
        if (c + 1 < nch) load_chunk(c + 1);
#pragma unroll
        for (int gg = 0; gg < KG; ++gg) {
        const int kofs = (kw * KG + gg) * 32 + (lane >> 4) * 8;
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
                if constexpr (ROWSCALE || WB16) {
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[tm], bw[tn], acc[tm][tn], 0, 0, 0);
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[tm], bw[tn], acc[tm][tn], 0, 0, 0);
                } else {
                    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[tm], bw[tn], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[tm], bw[tn], d, 0, 0, 0);
                    const float s = s_cur[gg][tn];
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[tm][tn][i] = fmaf(d[i], s, acc[tm][tn][i]);
                }
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
    if constexpr (ROWSCALE && !WB16) {
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

// ---------------------------------------------------------------------------
// Prefill (M > 64) over the tile-major int8 weights and the pre-split
// activation (bf16 hi plane [M, ldx], lo plane after it): the arithmetic of
// k_mm_i8<2, 2, 1, 4, 4, ...> (the same operands in the same lane positions,
// the same per-group MFMA pairs, scale FMAs and order, so the same bits), with
// the staging rebuilt:
//   - LDS in operand order: each 16-row x 32-column operand (a 16x16x32 MFMA
//     input) is 1 KB with lane l's 16 bytes at 16 l, for the activation
//     hi/lo tiles and the converted weight tiles alike, so every ds_read_b128
//     and every staging store is lane-contiguous (no bank conflicts; the
//     padded rows measured a third of the LDS cycles in conflicts);
//   - two stages, one barrier per 32-column group: group g + 1 is converted
//     and stored while group g is multiplied, and group g + 2 requested;
//   - addresses advance by constants (a group is 512 bytes of a weight
//     fragment and 16 scales), none recomputed in the loop;
//   - every load unconditional (clamped rows, tiles and groups).
// Workgroup: 2 x WNW waves, each 64 activation rows x 64 staged weight rows
// (SwiGLU: 32 gate + the matching 32 up rows); 128 x 64 WNW staged per group
// (WNW = 4 halves the activation bytes a product against WNW = 2).
template <bool RS, int EPI, int WNW>
__global__ __launch_bounds__(128 * WNW, WNW == 2 ? 2 : 1) void k_mm_pf(
    const uint16_t* __restrict__ xh, int ldx,
                                                       const int8_t* __restrict__ q,
                                                       const float* __restrict__ sc,
                                                       float* __restrict__ y, int ldy, int M,
                                                       int N, int K, TileMap tmap) {
    constexpr int TM = 4, TN = 4;
    constexpr int NTH = 128 * WNW;            // threads
    constexpr int NBT = 4 * WNW;              // staged weight tiles
    constexpr int AS = 512 / NTH;             // activation slots a thread, each plane
    constexpr int OUT_TN = EPI == EPI_SWIGLU ? TN / 2 : TN;
    constexpr int BN_OUT = WNW * OUT_TN * 16;
    constexpr int A_LO = 8192, B_OFS = 16384, STAGE = 16384 + NBT * 1024;
    __shared__ __attribute__((aligned(16))) unsigned char smem[2 * STAGE];
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WNW, wn = wave % WNW;
    const int m0 = blockIdx.y * 128;
    const int nout0 = blockIdx.x * BN_OUT;
    const int ngrp = K >> 5;
    const size_t plane = (size_t)M * ldx;

    // staged weight tile t (0..NBT-1) -> tile of the tile-major matrix (clamped)
    auto gtile = [&](int t) -> int {
        if constexpr (EPI == EPI_SWIGLU) {
            const int th = min(nout0 / 16 + t % (NBT / 2), tmap.tiles_half - 1);
            return (t / (NBT / 2)) * tmap.tiles_half + th;
        } else {
            return min(nout0 / 16 + t, tmap.tiles_half - 1);
        }
    };
    // a wave's tile tn -> staged tile
    auto stile = [&](int tn) -> int {
        if constexpr (EPI == EPI_SWIGLU)
            return tn < TN / 2 ? wn * (TN / 2) + tn : NBT / 2 + wn * (TN / 2) + (tn - TN / 2);
        else
            return wn * TN + tn;
    };

    // activation operand slots s = tid + NTH u of 8 tiles x 64 lanes:
    // row 16 (s >> 6) + (s & 15), columns 8 ((s >> 4) & 3) .. + 7 of a group
    const uint16_t* ap[AS];
#pragma unroll
    for (int u = 0; u < AS; ++u) {
        const int sl_ = tid + NTH * u;
        const int row = min(m0 + 16 * (sl_ >> 6) + (sl_ & 15), M - 1);
        ap[u] = xh + (size_t)row * ldx + 8 * ((sl_ >> 4) & 3);
    }
    // weights: thread tid takes staged tile tid >> 5 and the 16 bytes of its
    // fragment lane 32 (g & 1) + (tid & 31) (row tid & 15, columns 16 ((tid >> 4)
    // & 1) .. + 15 of the group): group g is at + 512 g
    const int bt = tid >> 5, bn = tid & 15, bo = 2 * ((tid >> 4) & 1);
    const int8_t* bp = q + (size_t)gtile(bt) * tmap.nblk64 * 1024 + (size_t)(tid & 31) * 16;
    // group-32 scales of the wave's tiles, row lane & 15: group g at + 16 g
    const float* sp[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
        sp[tn] = sc + (size_t)gtile(stile(tn)) * tmap.nblk64 * 32 + (lane & 15);

    u32x4 xa_h[AS], xa_l[AS];
    int4 wb;
    float sl[TN];
    auto load = [&](int g) {
#pragma unroll
        for (int u = 0; u < AS; ++u) {
            xa_h[u] = *reinterpret_cast<const u32x4*>(ap[u] + 32 * g);
            xa_l[u] = *reinterpret_cast<const u32x4*>(ap[u] + plane + 32 * g);
        }
        wb = *reinterpret_cast<const int4*>(bp + (size_t)512 * g);
        if constexpr (!RS) {
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) sl[tn] = sp[tn][16 * g];
        }
    };
    auto store = [&](int stage) {
        unsigned char* st = smem + stage * STAGE;
#pragma unroll
        for (int u = 0; u < AS; ++u) {
            *reinterpret_cast<u32x4*>(st + (tid + NTH * u) * 16) = xa_h[u];
            *reinterpret_cast<u32x4*>(st + A_LO + (tid + NTH * u) * 16) = xa_l[u];
        }
        // 16 int8 -> 16 bf16 (exact): columns 0-7 to operand lane bo*16 + bn,
        // 8-15 to the next k-octet's lane
        const int wv[4] = {wb.x, wb.y, wb.z, wb.w};
        unsigned ow[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const unsigned v = (unsigned)wv[j];
            const int b0 = (int8_t)(v & 0xffu), b1 = (int8_t)((v >> 8) & 0xffu);
            const int b2 = (int8_t)((v >> 16) & 0xffu), b3 = (int8_t)(v >> 24);
            ow[2 * j] = (unsigned)i8_bf16(b0) | ((unsigned)i8_bf16(b1) << 16);
            ow[2 * j + 1] = (unsigned)i8_bf16(b2) | ((unsigned)i8_bf16(b3) << 16);
        }
        unsigned char* bd = st + B_OFS + bt * 1024 + (bo * 16 + bn) * 16;
        *reinterpret_cast<u32x4*>(bd) = u32x4{ow[0], ow[1], ow[2], ow[3]};
        *reinterpret_cast<u32x4*>(bd + 256) = u32x4{ow[4], ow[5], ow[6], ow[7]};
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = f32x4{0.f, 0.f, 0.f, 0.f};

    float s_cur[TN];
    load(0);
    store(0);
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) s_cur[tn] = sl[tn];
    load(min(1, ngrp - 1));
    __syncthreads();
    for (int g = 0; g < ngrp; ++g) {
        const unsigned char* st = smem + (g & 1) * STAGE;
        bf16x8 ah[TM], al[TM], bw[TN];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            ah[tm] = *reinterpret_cast<const bf16x8*>(st + (wm * TM + tm) * 1024 + lane * 16);
            al[tm] = *reinterpret_cast<const bf16x8*>(st + A_LO + (wm * TM + tm) * 1024 + lane * 16);
        }
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
            bw[tn] = *reinterpret_cast<const bf16x8*>(st + B_OFS + stile(tn) * 1024 + lane * 16);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                if constexpr (RS) {
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[tm], bw[tn], acc[tm][tn], 0, 0, 0);
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[tm], bw[tn], acc[tm][tn], 0, 0, 0);
                } else {
                    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[tm], bw[tn], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[tm], bw[tn], d, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[tm][tn][i] = fmaf(d[i], s_cur[tn], acc[tm][tn][i]);
                }
            }
        // group g + 1 into the other stage (its last reads ended at the
        // previous barrier); past the end a copy of the last group nobody reads
        store((g + 1) & 1);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) s_cur[tn] = sl[tn];
        load(min(g + 2, ngrp - 1));
        __syncthreads();
    }

    if constexpr (RS) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            int r;
            const int t = stile(tn);
            if constexpr (EPI == EPI_SWIGLU)
                r = t < NBT / 2 ? min(nout0 + t * 16 + (lane & 15), N - 1)
                                : N + min(nout0 + (t - NBT / 2) * 16 + (lane & 15), N - 1);
            else
                r = min(nout0 + t * 16 + (lane & 15), N - 1);
            const float s = sc[r];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[tm][tn][i] *= s;
        }
    }
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

// ---------------------------------------------------------------------------
// M <= 64 (batched decode): weight streaming with K split across workgroups.
//
// A workgroup owns 64 weight rows (wave w: rows 16w..16w+15 as one MFMA
// n-tile) and 16*TM activation rows, over a K slice of kper columns; per
// 128-column chunk (4 groups) x [BM, 128] is staged as bf16 hi/lo (with the
// RMSNorm applied when NORM) and the weights [64, 128] as bf16, the next
// chunk being loaded into registers meanwhile. Each slice writes its fp32
// partial tile to part[ks, m, n]; k_mm_reduce sums the slices in order and
// applies the epilogue. With a single slice and a plain store the partial
// is the output itself.
constexpr int kSkRows = 64;
constexpr int kSkKc = 128;
// chunks in flight per workgroup (register ring), by activation tiles
constexpr int sk_ring(int tm) { return tm <= 2 ? 2 : 1; }

// DEFER (with NORM): the activation is staged as x * (1 + w) and the row's
// 1/rms multiplies the reduced sums instead (k_mm_reduce<..., true>), so no
// separate row-scale launch precedes the matmul.
// TL: q and sc are tile-major (TileMap tmap); otherwise row-major.
template <int TM, bool ROWSCALE, bool NORM, bool DEFER, bool TL = false>
__global__ __launch_bounds__(kThreads) void k_mm_i8_sk(
    const float* __restrict__ x, int ldx, const float* __restrict__ rs,
    const float* __restrict__ nw, const int8_t* __restrict__ q, const float* __restrict__ sc,
    float* __restrict__ part, int ldp, int M, int NR, int K, int kper, TileMap tmap) {
    constexpr int BM = 16 * TM;
    constexpr int KC = kSkKc;
    constexpr int XP = KC + 8, WP = KC + 8;
    constexpr int XV = BM * KC / 4, WV = kSkRows * KC / 16;
    constexpr int XPT = (XV + kThreads - 1) / kThreads;
    constexpr int WPT = (WV + kThreads - 1) / kThreads;
    constexpr int CPF = sk_ring(TM);
    __shared__ __attribute__((aligned(16))) unsigned short xs_hi[BM * XP];
    __shared__ __attribute__((aligned(16))) unsigned short xs_lo[BM * XP];
    __shared__ __attribute__((aligned(16))) unsigned short ws[kSkRows * WP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * kSkRows;
    const int ks = blockIdx.y;
    const int m0 = blockIdx.z * BM;
    const int kb = ks * kper;
    const int nblk = K >> 5;
    const int ncol = n0 + wave * 16 + (lane & 15);      // this lane's weight row (output column)
    const int nrow = ncol < NR ? ncol : NR - 1;

    // a ring of CPF chunk buffers in registers: a chunk's registers are
    // refilled with chunk c + CPF as soon as chunk c is staged to LDS, so a
    // workgroup's whole K slice (<= CPF chunks) is requested at once
    float4 xr[CPF][XPT];
    float4 gr[CPF][NORM ? XPT : 1];
    float rr[CPF][NORM ? XPT : 1];
    int4 wr[CPF][WPT];
    float4 sr[CPF];  // group scales of this lane's row for a chunk's 4 groups
    auto load_chunk = [&](int c, int j) {
        const int k0 = kb + c * KC;
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < XV) {
                const int r = i / (KC / 4), c4 = i % (KC / 4);
                const int m = min(m0 + r, M - 1);
                xr[j][u] = *reinterpret_cast<const float4*>(x + (size_t)m * ldx + k0 + c4 * 4);
                if constexpr (NORM) {
                    gr[j][u] = *reinterpret_cast<const float4*>(nw + k0 + c4 * 4);
                    rr[j][u] = DEFER ? 1.0f : rs[m];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < WPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < WV) {
                const int r = i / (KC / 16), c16 = i % (KC / 16);
                const int n = min(n0 + r, NR - 1);
                if constexpr (TL)
                    wr[j][u] = *reinterpret_cast<const int4*>(q + tm_off(tmap, n, k0 + c16 * 16));
                else
                    wr[j][u] = *reinterpret_cast<const int4*>(q + (size_t)n * K + k0 + c16 * 16);
            }
        }
        if constexpr (!ROWSCALE) {
            if constexpr (TL) {
                const int g0 = k0 >> 5;
                sr[j] = make_float4(sc[tm_scale(tmap, nrow, g0)], sc[tm_scale(tmap, nrow, g0 + 1)],
                                    sc[tm_scale(tmap, nrow, g0 + 2)],
                                    sc[tm_scale(tmap, nrow, g0 + 3)]);
            } else {
                sr[j] = *reinterpret_cast<const float4*>(sc + (size_t)nrow * nblk + (k0 >> 5));
            }
        }
    };
    auto store_chunk = [&](int j) {
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < XV) {
                const int r = i / (KC / 4), c4 = i % (KC / 4);
                float4 v = xr[j][u];
                if constexpr (NORM) v = norm4(v, rr[j][u], gr[j][u]);
                store_hilo(&xs_hi[r * XP + c4 * 4], &xs_lo[r * XP + c4 * 4], v);
            }
        }
#pragma unroll
        for (int u = 0; u < WPT; ++u) {
            const int i = tid + u * kThreads;
            if (i < WV) {
                const int r = i / (KC / 16), c16 = i % (KC / 16);
                store_w16(&ws[r * WP + c16 * 16], wr[j][u]);
            }
        }
    };

    f32x4 acc[TM];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) acc[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nch = kper / KC;
#pragma unroll
    for (int j = 0; j < CPF; ++j)
        if (j < nch) load_chunk(j, j);
    for (int c0 = 0; c0 < nch; c0 += CPF)
#pragma unroll
    for (int j = 0; j < CPF; ++j) {
        const int c = c0 + j;
        if (c >= nch) break;  // uniform
        const float4 s_cur = sr[j];
        __syncthreads();
        store_chunk(j);
        __syncthreads();
        if (c + CPF < nch) load_chunk(c + CPF, j);
        const float sg[4] = {s_cur.x, s_cur.y, s_cur.z, s_cur.w};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int kofs = g * 32 + (lane >> 4) * 8;
            const bf16x8 bw = *reinterpret_cast<const bf16x8*>(&ws[(wave * 16 + (lane & 15)) * WP + kofs]);
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const int r = tm * 16 + (lane & 15);
                const bf16x8 ah = *reinterpret_cast<const bf16x8*>(&xs_hi[r * XP + kofs]);
                const bf16x8 al = *reinterpret_cast<const bf16x8*>(&xs_lo[r * XP + kofs]);
                if constexpr (ROWSCALE) {
                    acc[tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bw, acc[tm], 0, 0, 0);
                    acc[tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bw, acc[tm], 0, 0, 0);
                } else {
                    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bw, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bw, d, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[tm][i] = fmaf(d[i], sg[g], acc[tm][i]);
                }
            }
        }
    }
    if constexpr (ROWSCALE) {
        const float s = sc[nrow];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[tm][i] *= s;
    }
    if (ncol < NR) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + tm * 16 + (lane >> 4) * 4 + i;
                if (m < M) part[((size_t)ks * M + m) * ldp + ncol] = acc[tm][i];
            }
    }
}


// RMSNorm row scales rs[m] = 1/sqrt(mean(x[m]^2) + eps): every load of the
// row is issued before the sum (K <= 4096 per pass of 256 x float4).
__global__ __launch_bounds__(kThreads) void k_row_rs(const float* __restrict__ x, int ldx, int K,
                                                     float eps, float* __restrict__ rs) {
    __shared__ float red[kThreads / QLM_WAVE];
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)blockIdx.x * ldx);
    const int n4 = K >> 2;
    float ss = 0.0f;
    for (int b = 0; b < n4; b += 4 * kThreads) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = b + u * kThreads + threadIdx.x;
            v[u] = i < n4 ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            ss = fmaf(v[u].x, v[u].x, ss);
            ss = fmaf(v[u].y, v[u].y, ss);
            ss = fmaf(v[u].z, v[u].z, ss);
            ss = fmaf(v[u].w, v[u].w, ss);
        }
    }
    ss = block_sum(ss, red);
    if (threadIdx.x == 0) rs[blockIdx.x] = 1.0f / sqrtf(ss / (float)K + eps);
}

// The activation of the prefill GEMM split once into bf16 hi and lo planes
// ([M, K] each, the lo plane after the hi one), with the RMSNorm applied when
// NORM (rs from k_row_rs): the GEMM's workgroups along N then copy them
// instead of each converting the same chunk again.
template <bool NORM>
__global__ __launch_bounds__(kThreads) void k_split_rows(const float* __restrict__ x, int ldx,
                                                        const float* __restrict__ rs,
                                                        const float* __restrict__ nw, int M,
                                                        int K, uint16_t* __restrict__ xh) {
    const int k4 = K >> 2;
    const size_t n4 = (size_t)M * k4;
    for (size_t i = blockIdx.x * (size_t)kThreads + threadIdx.x; i < n4;
         i += (size_t)gridDim.x * kThreads) {
        const int m = (int)(i / k4), c4 = (int)(i % k4);
        float4 v = *reinterpret_cast<const float4*>(x + (size_t)m * ldx + c4 * 4);
        if constexpr (NORM)
            v = norm4(v, rs[m], *reinterpret_cast<const float4*>(nw + c4 * 4));
        unsigned short h[4], l[4];
        split_bf16(v.x, h[0], l[0]);
        split_bf16(v.y, h[1], l[1]);
        split_bf16(v.z, h[2], l[2]);
        split_bf16(v.w, h[3], l[3]);
        const size_t o = (size_t)m * K + c4 * 4;
        *reinterpret_cast<uint2*>(xh + o) = make_uint2((unsigned)h[0] | ((unsigned)h[1] << 16),
                                                       (unsigned)h[2] | ((unsigned)h[3] << 16));
        *reinterpret_cast<uint2*>(xh + (size_t)M * K + o) =
            make_uint2((unsigned)l[0] | ((unsigned)l[1] << 16),
                       (unsigned)l[2] | ((unsigned)l[3] << 16));
    }
}

template <bool NORM>
int launch_split(const float* x, int ldx, const float* rs, const float* nw, int M, int K,
                 uint16_t* xh, hipStream_t st) {
    const size_t n4 = (size_t)M * (K >> 2);
    const size_t g = (n4 + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(k_split_rows<NORM>, dim3((unsigned)(g < 2048 ? g : 2048)),
                       dim3(kThreads), 0, st, x, ldx, rs, nw, M, K, xh);
    return qlm_launch_status();
}

// K slices for the M <= 64 path: the fewest that divide the 128-column
// chunk count and give each workgroup at most 6 chunks and the launch at
// least ~640 workgroups (up to 16 rows); above 16 rows (four times the work
// a workgroup) at most 8 chunks a workgroup, ~320 workgroups and at least 8
// slices. A tall matrix (>= 1024 row tiles) is one slice. Measured on the
// config-1 shapes (graph replays): 4096 x 12288 at 4 / 16 rows 21.4 / 23.1
// us with the former rule (at most 4 chunks a workgroup) against 18.2 /
// 20.4 us; 64 rows 40.9 against 38.5 us; 4096 x 4096 at 64 rows 22.4
// against 20.7 us; 12288 x 4096 at 64 rows 42.6 us in 8 slices, 43.1 in 4.
int sk_splits(int M, int NR, int K) {
    const int nt = (NR + kSkRows - 1) / kSkRows;
    const int nch = K / kSkKc;
    if (nt >= 1024) return 1;
    const bool tall = M > 16;
    const int per = tall ? 8 : 6;
    const int wgs = tall ? 320 : 640;
    int want = (nch + per - 1) / per;
    want = want > (wgs + nt - 1) / nt ? want : (wgs + nt - 1) / nt;
    if (tall && want < 8) want = 8;
    for (int d = 1; d <= nch; ++d)
        if (nch % d == 0 && d >= want) return d;
    return nch;
}

bool use_sk(int M, int K) { return M <= 64 && K % kSkKc == 0; }

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace
extern "C" size_t qlm_matmul_i8_rows64_workspace_bytes(int M, int N, int K, int epilogue);
extern "C" int qlm_matmul_i8_rows64(const float* x, int ldx, const float* norm_w, float eps,
                                    const int8_t* q_tiles, const float* s_rows, float* y,
                                    int ldy, int M, int N, int K, int epilogue, void* work,
                                    size_t work_bytes, void* stream);
namespace {

// the tile-major 2..64-row form with one scale per weight row (gemm_mx.hip),
// where measured faster than the K-sliced bf16 form: N >= 8192 (32 or more
// 256-row tile groups), or more than 16 rows and K > 4096. With fewer groups
// its K slices and their reduction launch cost more (4096 x 4096: 15.4
// against 12.6 us at 16 rows, 27.5 against 23.3 us at 64)
bool rows64_applies(int M, int N, int K, int group, int epi) {
    if (N < 8192 && (M <= 16 || K <= 4096)) return false;
    return group == K && M >= 2 && M <= 64 && K % 64 == 0 && epi != EPI_SWIGLU;
}

size_t mm_workspace(int M, int N, int K, int epi) {
    size_t b = align256((size_t)M * sizeof(float));  // row scales
    if (use_sk(M, K)) {
        const int NR = epi == EPI_SWIGLU ? 2 * N : N;
        const int ks = sk_splits(M, NR, K);
        if (!(ks == 1 && epi == EPI_STORE)) b += (size_t)ks * M * NR * sizeof(float);
    } else {
        b += align256((size_t)4 * M * K);  // the split activation (bf16 hi, lo)
    }
    // room for the 2..64-row digit form of qlm_matmul_i8_tm (one scale per
    // weight row); the query cannot tell which scales a caller holds
    if (M >= 2 && M <= 64 && K % 64 == 0 && epi != EPI_SWIGLU) {
        const size_t r = qlm_matmul_i8_rows64_workspace_bytes(M, N, K, epi);
        if (r > b) b = r;
    }
    return b;
}

template <int TM, bool RS, bool NORM, bool DEFER, bool TL>
void launch_sk(const float* x, int ldx, const float* rs, const float* nw, const int8_t* q,
               const float* sc, float* part, int ldp, int M, int NR, int K, int ks,
               const TileMap& tm, hipStream_t st) {
    const dim3 grid((NR + kSkRows - 1) / kSkRows, ks, (M + 16 * TM - 1) / (16 * TM));
    hipLaunchKernelGGL((k_mm_i8_sk<TM, RS, NORM, DEFER, TL>), grid, dim3(kThreads), 0, st, x, ldx,
                       rs, nw, q, sc, part, ldp, M, NR, K, K / ks, tm);
}

template <bool RS, bool NORM, bool DEFER, bool TL>
void launch_sk_tm(const float* x, int ldx, const float* rs, const float* nw, const int8_t* q,
                  const float* sc, float* part, int ldp, int M, int NR, int K, int ks,
                  const TileMap& tm, hipStream_t st) {
    if (M <= 16)
        launch_sk<1, RS, NORM, DEFER, TL>(x, ldx, rs, nw, q, sc, part, ldp, M, NR, K, ks, tm, st);
    else if (M <= 32)
        launch_sk<2, RS, NORM, DEFER, TL>(x, ldx, rs, nw, q, sc, part, ldp, M, NR, K, ks, tm, st);
    else
        launch_sk<4, RS, NORM, DEFER, TL>(x, ldx, rs, nw, q, sc, part, ldp, M, NR, K, ks, tm, st);
}

template <int EPI, bool NORM>
void launch_reduce(const float* part, int ks, int M, int NR, int N, float* y, int ldy,
                   const float* x, int ldx, int K, float eps, hipStream_t st) {
    const dim3 grid((N + kThreads - 1) / kThreads, M);
    hipLaunchKernelGGL((k_mm_reduce<EPI, NORM>), grid, dim3(kThreads), 0, st, part, ks, M, NR, N,
                       y, ldy, x, ldx, K, eps);
}

template <int WM, int WN, int WK, int TM, int TN, bool RS, int EPI, bool NORM, bool XS, bool TL>
int launch_mm(const float* x, int ldx, const float* rs, const float* nw, const int8_t* q,
              const float* sc, float* y, int ldy, int M, int N, int K, const TileMap& tm,
              hipStream_t st) {
    constexpr int BM = WM * TM * 16;
    constexpr int BN_OUT = WN * (EPI == EPI_SWIGLU ? TN / 2 : TN) * 16;
    const dim3 grid((N + BN_OUT - 1) / BN_OUT, (M + BM - 1) / BM);
    if (K % (64 * WK) == 0)  // two scale groups a chunk
        hipLaunchKernelGGL((k_mm_i8<WM, WN, WK, TM, TN, RS, EPI, NORM, false, XS, 2, TL>), grid,
                           dim3(kThreads), 0, st, x, ldx, rs, nw, q, sc, y, ldy, M, N, K, N, tm);
    else if constexpr (!TL)  // tile-major weights have whole 64-column blocks
        hipLaunchKernelGGL((k_mm_i8<WM, WN, WK, TM, TN, RS, EPI, NORM, false, XS>), grid,
                           dim3(kThreads), 0, st, x, ldx, rs, nw, q, sc, y, ldy, M, N, K, N, tm);
    else
        return QLM_ERR_SHAPE;
    return qlm_launch_status();
}

template <bool RS, int EPI, int WNW = 4>
int launch_pf(const uint16_t* xh, int ldx, const int8_t* q, const float* sc, float* y, int ldy,
              int M, int N, int K, const TileMap& tm, hipStream_t st) {
    constexpr int BN_OUT = (EPI == EPI_SWIGLU ? 32 : 64) * WNW;
    const dim3 grid((N + BN_OUT - 1) / BN_OUT, (M + 127) / 128);
    hipLaunchKernelGGL((k_mm_pf<RS, EPI, WNW>), grid, dim3(128 * WNW), 0, st, xh, ldx, q, sc, y,
                       ldy, M, N, K, tm);
    return qlm_launch_status();
}

template <int EPI, bool NORM, bool XS>
int launch_mm16(const float* x, int ldx, const float* rs, const float* nw, const uint16_t* w,
                float* y, int ldy, int M, int N, int K, hipStream_t st) {
    constexpr int BM = 2 * 4 * 16;
    constexpr int BN_OUT = 2 * (EPI == EPI_SWIGLU ? 2 : 4) * 16;
    const dim3 grid((N + BN_OUT - 1) / BN_OUT, (M + BM - 1) / BM);
    const int8_t* wq = reinterpret_cast<const int8_t*>(w);
    const TileMap none{N, 0, 0};
    if (K % 64 == 0)
        hipLaunchKernelGGL((k_mm_i8<2, 2, 1, 4, 4, false, EPI, NORM, true, XS, 2>), grid,
                           dim3(kThreads), 0, st, x, ldx, rs, nw, wq, nullptr, y, ldy, M, N, K, N,
                           none);
    else
        hipLaunchKernelGGL((k_mm_i8<2, 2, 1, 4, 4, false, EPI, NORM, true, XS>), grid,
                           dim3(kThreads), 0, st, x, ldx, rs, nw, wq, nullptr, y, ldy, M, N, K, N,
                           none);
    return qlm_launch_status();
}

template <bool RS, bool NORM, bool TL>
int mm_run(const float* x, int ldx, float* rs, const float* nw, float eps, const int8_t* q,
           const float* sc, float* y, int ldy, int M, int N, int K, int epi, float* part,
           hipStream_t st) {
    const TileMap tm{N, (N + 15) / 16, K / 64};  // a SwiGLU matrix: gate rows, then up rows
    if (use_sk(M, K)) {
        const int NR = epi == EPI_SWIGLU ? 2 * N : N;
        const int ks = sk_splits(M, NR, K);
        const bool direct = ks == 1 && epi == EPI_STORE;
        float* dst = direct ? y : part;
        const int ldp = direct ? ldy : NR;
        if (direct) {  // the matmul writes y itself: row scales first
            if constexpr (NORM) {
                hipLaunchKernelGGL(k_row_rs, dim3(M), dim3(kThreads), 0, st, x, ldx, K, eps, rs);
                const int rc = qlm_launch_status();
                if (rc != QLM_OK) return rc;
            }
            launch_sk_tm<RS, NORM, false, TL>(x, ldx, rs, nw, q, sc, dst, ldp, M, NR, K, ks, tm,
                                              st);
            return qlm_launch_status();
        }
        // row scales folded into the reduction (no separate launch)
        launch_sk_tm<RS, NORM, NORM, TL>(x, ldx, rs, nw, q, sc, dst, ldp, M, NR, K, ks, tm, st);
        int rc = qlm_launch_status();
        if (rc != QLM_OK) return rc;
        if (epi == EPI_STORE)
            launch_reduce<EPI_STORE, NORM>(part, ks, M, NR, N, y, ldy, x, ldx, K, eps, st);
        else if (epi == EPI_RESID)
            launch_reduce<EPI_RESID, false>(part, ks, M, NR, N, y, ldy, x, ldx, K, eps, st);
        else
            launch_reduce<EPI_SWIGLU, NORM>(part, ks, M, NR, N, y, ldy, x, ldx, K, eps, st);
        return qlm_launch_status();
    }
    if constexpr (NORM) {
        hipLaunchKernelGGL(k_row_rs, dim3(M), dim3(kThreads), 0, st, x, ldx, K, eps, rs);
        const int rc = qlm_launch_status();
        if (rc != QLM_OK) return rc;
    }
    // the activation split once (RMSNorm applied), then the GEMM copies it
    uint16_t* xh = reinterpret_cast<uint16_t*>(part);
    const int rc = launch_split<NORM>(x, ldx, rs, nw, M, K, xh, st);
    if (rc != QLM_OK) return rc;
    if constexpr (TL) {  // tile-major weights: the double-buffered operand-order form
        // 256 weight rows a workgroup where that still gives 1024 workgroups
        // or more (four rounds of the GPU), else 128, two workgroups a CU.
        // Measured at 2047 rows (graph replays): gate/up 509 us wide against
        // 515 narrow; the DeltaNet in-projection 306 against 278 us (528
        // workgroups wide: two rounds and 16 more), attention q/k/v 213
        // against 197, down 415 against 360 us
        const int bn = epi == EPI_SWIGLU ? 128 : 256;
        const bool wide = (long)((N + bn - 1) / bn) * ((M + 127) / 128) >= 1024;
        if (epi == EPI_STORE)
            return wide ? launch_pf<RS, EPI_STORE, 4>(xh, K, q, sc, y, ldy, M, N, K, tm, st)
                        : launch_pf<RS, EPI_STORE, 2>(xh, K, q, sc, y, ldy, M, N, K, tm, st);
        if (epi == EPI_RESID)
            return wide ? launch_pf<RS, EPI_RESID, 4>(xh, K, q, sc, y, ldy, M, N, K, tm, st)
                        : launch_pf<RS, EPI_RESID, 2>(xh, K, q, sc, y, ldy, M, N, K, tm, st);
        return wide ? launch_pf<RS, EPI_SWIGLU, 4>(xh, K, q, sc, y, ldy, M, N, K, tm, st)
                    : launch_pf<RS, EPI_SWIGLU, 2>(xh, K, q, sc, y, ldy, M, N, K, tm, st);
    }
    const float* xs = reinterpret_cast<const float*>(xh);
    if (epi == EPI_STORE)
        return launch_mm<2, 2, 1, 4, 4, RS, EPI_STORE, false, true, TL>(
            xs, K, nullptr, nullptr, q, sc, y, ldy, M, N, K, tm, st);
    if (epi == EPI_RESID)
        return launch_mm<2, 2, 1, 4, 4, RS, EPI_RESID, false, true, TL>(
            xs, K, nullptr, nullptr, q, sc, y, ldy, M, N, K, tm, st);
    return launch_mm<2, 2, 1, 4, 4, RS, EPI_SWIGLU, false, true, TL>(
        xs, K, nullptr, nullptr, q, sc, y, ldy, M, N, K, tm, st);
}

}  // namespace

extern "C" size_t qlm_matmul_i8_workspace_bytes(int M, int N, int K, int epilogue) {
    if (M <= 0 || N <= 0 || K <= 0 || epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return 0;
    return mm_workspace(M, N, K, epilogue);
}

extern "C" size_t qlm_matmul_bf16_workspace_bytes(int M, int K) {
    if (M <= 0 || K <= 0) return 0;
    return align256((size_t)M * sizeof(float)) + align256((size_t)4 * M * K);
}

extern "C" int qlm_matmul_bf16(const float* x, int ldx, const float* norm_w, float eps,
                               const uint16_t* w, float* y, int ldy, int M, int N, int K,
                               int epilogue, void* work, size_t work_bytes, void* stream) {
    if (!x || !w || !y || M <= 0 || N <= 0 || K <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    if (epilogue == EPI_SWIGLU && !norm_w) return QLM_ERR_ARG;
    if (epilogue == EPI_RESID && norm_w) return QLM_ERR_ARG;
    if (K % 32 != 0 || ldx < K || ldx % 4 != 0 || ldy < N) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)norm_w | (uintptr_t)work) & 15u)
        return QLM_ERR_SHAPE;
    hipStream_t st = as_stream(stream);
    const size_t rsb = align256((size_t)M * sizeof(float));
    if (norm_w && (!work || work_bytes < rsb)) return QLM_ERR_ARG;
    float* rs = static_cast<float*>(work);
    if (norm_w) {
        hipLaunchKernelGGL(k_row_rs, dim3(M), dim3(kThreads), 0, st, x, ldx, K, eps, rs);
        const int rc = qlm_launch_status();
        if (rc != QLM_OK) return rc;
    }
    if (work && work_bytes >= qlm_matmul_bf16_workspace_bytes(M, K)) {
        // the activation split once (RMSNorm applied), then the GEMM copies it
        uint16_t* xh = reinterpret_cast<uint16_t*>(static_cast<char*>(work) + rsb);
        const int rc = norm_w ? launch_split<true>(x, ldx, rs, norm_w, M, K, xh, st)
                              : launch_split<false>(x, ldx, nullptr, nullptr, M, K, xh, st);
        if (rc != QLM_OK) return rc;
        const float* xs = reinterpret_cast<const float*>(xh);
        if (epilogue == EPI_SWIGLU)
            return launch_mm16<EPI_SWIGLU, false, true>(xs, K, nullptr, nullptr, w, y, ldy, M, N,
                                                        K, st);
        if (epilogue == EPI_RESID)
            return launch_mm16<EPI_RESID, false, true>(xs, K, nullptr, nullptr, w, y, ldy, M, N, K,
                                                       st);
        return launch_mm16<EPI_STORE, false, true>(xs, K, nullptr, nullptr, w, y, ldy, M, N, K,
                                                   st);
    }
    // a smaller workspace: each workgroup converts its activation chunks itself
    if (epilogue == EPI_SWIGLU)
        return launch_mm16<EPI_SWIGLU, true, false>(x, ldx, rs, norm_w, w, y, ldy, M, N, K, st);
    if (epilogue == EPI_RESID)
        return launch_mm16<EPI_RESID, false, false>(x, ldx, nullptr, nullptr, w, y, ldy, M, N, K,
                                                    st);
    if (norm_w)
        return launch_mm16<EPI_STORE, true, false>(x, ldx, rs, norm_w, w, y, ldy, M, N, K, st);
    return launch_mm16<EPI_STORE, false, false>(x, ldx, nullptr, nullptr, w, y, ldy, M, N, K, st);
}

namespace {
template <bool TL>
int matmul_i8_entry(const float* x, int ldx, const float* norm_w, float eps, const int8_t* q,
                    const float* scales, int group, float* y, int ldy, int M, int N, int K,
                    int epilogue, void* work, size_t work_bytes, void* stream) {
    if (!x || !q || !scales || !y) return QLM_ERR_ARG;
    if (M <= 0 || N <= 0 || K <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    if (K % (TL ? 64 : 32) != 0) return QLM_ERR_SHAPE;
    const bool rowscale = (group == K);
    if (!rowscale && group != 32) return QLM_ERR_SHAPE;
    if (ldx < K || ldy < N || ldx % 4 != 0) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)q | (uintptr_t)norm_w | (uintptr_t)scales) & 15u)
        return QLM_ERR_SHAPE;
    const size_t need = mm_workspace(M, N, K, epilogue);
    if (!work || work_bytes < need || ((uintptr_t)work & 15u)) return QLM_ERR_ARG;
    if constexpr (TL) {
        // 2..64 rows with one scale per weight row: int8 digits on the int8
        // matrix cores (its workspace needs 256-byte alignment)
        if (rows64_applies(M, N, K, group, epilogue) && !(epilogue == EPI_RESID && norm_w) &&
            ((uintptr_t)work & 255u) == 0) {
            const int rc = qlm_matmul_i8_rows64(x, ldx, norm_w, eps, q, scales, y, ldy, M, N, K,
                                                epilogue, work, work_bytes, stream);
            if (rc != QLM_ERR_SHAPE) return rc;
        }
    }
    hipStream_t st = as_stream(stream);
    float* rs = reinterpret_cast<float*>(work);
    float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(work) + align256((size_t)M * 4));
    if (norm_w)
        return rowscale ? mm_run<true, true, TL>(x, ldx, rs, norm_w, eps, q, scales, y, ldy, M, N,
                                                 K, epilogue, part, st)
                        : mm_run<false, true, TL>(x, ldx, rs, norm_w, eps, q, scales, y, ldy, M,
                                                  N, K, epilogue, part, st);
    return rowscale ? mm_run<true, false, TL>(x, ldx, nullptr, nullptr, eps, q, scales, y, ldy, M,
                                              N, K, epilogue, part, st)
                    : mm_run<false, false, TL>(x, ldx, nullptr, nullptr, eps, q, scales, y, ldy,
                                               M, N, K, epilogue, part, st);
}
}  // namespace

extern "C" int qlm_matmul_i8(const float* x, int ldx, const float* norm_w, float eps,
                             const int8_t* q, const float* scales, int group, float* y, int ldy,
                             int M, int N, int K, int epilogue, void* work, size_t work_bytes,
                             void* stream) {
    return matmul_i8_entry<false>(x, ldx, norm_w, eps, q, scales, group, y, ldy, M, N, K,
                                  epilogue, work, work_bytes, stream);
}

extern "C" int qlm_matmul_i8_tm(const float* x, int ldx, const float* norm_w, float eps,
                                const int8_t* q_tiles, const float* s_tiles, int group, float* y,
                                int ldy, int M, int N, int K, int epilogue, void* work,
                                size_t work_bytes, void* stream) {
    return matmul_i8_entry<true>(x, ldx, norm_w, eps, q_tiles, s_tiles, group, y, ldy, M, N, K,
                                 epilogue, work, work_bytes, stream);
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_gemm() {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(k_row_rs));
}
