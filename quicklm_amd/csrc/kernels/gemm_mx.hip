// Batched decode matmul (2 <= M <= 16 activation rows) on the int8 matrix
// cores, over the tile-major weights of the one-row GEMV (gemv.hip,
// k_mx_swizzle):
//   y[m, n] = sum_k x[m, k] * q[n, k] * s[n, k / G]
// The same product as math::matmul's int8 branch with M rows
// (math_ops.cpp:845-871), which batched decode runs once per step.
//
// Two launches:
//   k_act_digits: per activation row m (one workgroup each), the optional
//     RMSNorm (zero-centred gain) and the int8 digit vectors of the row with
//     its own power-of-two scale, x_m = 2^E_m (d0 + d1 2^-7 + d2 2^-14 +
//     d3 2^-21) to within 2^-27 max|x_m| (the one-row GEMV's decomposition),
//     written as planes [m][d][K] plus E_m.
//   k_gemm_mx: one v_mfma_i32_16x16x64_i8 per pair of activation rows and
//     64-column block of a 16-row weight tile. A row r = 8 m' + 4 h + d of
//     the pair's operand holds digit d of row m' over the elements of group
//     2b + h (zero for the other group), so lane l = 16q + n of the result
//     holds the four digit sums of weight row n, activation row 2j + (q >> 1),
//     group 2b + (q & 1): combined exactly in int32, scaled by the group scale
//     in fp32. With one scale per weight row (G = K) A rows 4 m' + d carry
//     every element and the int32 sums accumulate across blocks.
//
// k_gemm_mx keeps K inside a workgroup, so no partial sums leave it: NW
// waves split each tile's 64-column blocks (wave w: blocks w + NW u, u < U;
// blocks past K meet zero digits), the digits of one block column per wave
// (a "phase", M x 4 x 64 NW bytes) are staged through double-buffered LDS
// from registers loaded one phase ahead, a ring of R weight blocks per wave
// (R divides U) stays in flight, refilled R blocks ahead (into the next
// tile), and the waves' partial sums meet in LDS at the end of each tile.

#include "common.hpp"
#include "mm_reduce.hpp"

namespace {

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kPrepThreads = 256;
constexpr int kMaxRows = 16;

// Activation digits of one row per gridDim.y workgroups; rows m >= M
// (padding up to the products' row count) are written as zeros. Two passes
// over the row: sum of squares (RMSNorm) and max|x * (1 + w)| over the whole
// row (by every workgroup of the row), then the digits of this workgroup's
// share of the columns (blockIdx.y). Each thread keeps kDigitLoads loads in
// flight (indices clamped, so the loads are unconditional; elements past
// the row are then dropped); the sum of squares accumulates in the same
// order for any split.
constexpr int kDigitLoads = 4;

template <bool NORM>
__global__ __launch_bounds__(kPrepThreads) void k_act_digits(const float* __restrict__ x,
                                                              int ldx, const float* __restrict__ nw,
                                                              float eps, int M, int K,
                                                              int8_t* __restrict__ digits,
                                                              int* __restrict__ dexp) {
    __shared__ float rsum[kPrepThreads / QLM_WAVE], rmax[kPrepThreads / QLM_WAVE];
    const int m = blockIdx.x, tid = threadIdx.x, lane = tid & (QLM_WAVE - 1);
    const int wave = tid / QLM_WAVE;
    const int n4 = K >> 2;
    // float4 columns [c0, c1) get their digits here
    const int per = (n4 + (int)gridDim.y - 1) / (int)gridDim.y;
    const int c0 = (int)blockIdx.y * per, c1 = min(n4, c0 + per);
    constexpr int U = kDigitLoads, STEP = U * kPrepThreads;
    unsigned* planes = reinterpret_cast<unsigned*>(digits + (size_t)m * 4 * K);
    if (m >= M) {
        for (int i = c0 + tid; i < c1; i += kPrepThreads)
#pragma unroll
            for (int d = 0; d < 4; ++d) planes[(size_t)d * n4 + i] = 0u;
        if (blockIdx.y == 0 && tid == 0) dexp[m] = 0;
        return;
    }
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * ldx);
    const float4* wr = reinterpret_cast<const float4*>(nw);
    float ss = 0.0f, mx = 0.0f;
    for (int i = tid; i < n4; i += STEP) {
        float4 v[U], g[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = min(i + u * kPrepThreads, n4 - 1);
            v[u] = xr[k];
            if constexpr (NORM) g[u] = wr[k];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (i + u * kPrepThreads >= n4) break;
            float4 a = v[u];
            if constexpr (NORM) {
                ss = fmaf(a.x, a.x, ss);
                ss = fmaf(a.y, a.y, ss);
                ss = fmaf(a.z, a.z, ss);
                ss = fmaf(a.w, a.w, ss);
                a.x *= 1.0f + g[u].x;
                a.y *= 1.0f + g[u].y;
                a.z *= 1.0f + g[u].z;
                a.w *= 1.0f + g[u].w;
            }
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        }
    }
    if constexpr (NORM) ss = wave_sum(ss);
    mx = wave_max(mx);
    if (lane == 0) {
        rsum[wave] = ss;
        rmax[wave] = mx;
    }
    __syncthreads();
    float tot = rsum[0], mm = rmax[0];
#pragma unroll
    for (int i = 1; i < kPrepThreads / QLM_WAVE; ++i) {
        tot += rsum[i];
        mm = fmaxf(mm, rmax[i]);
    }
    const float rs = NORM ? 1.0f / sqrtf(tot / (float)K + eps) : 1.0f;
    int e2 = 0;
    frexpf(mm * rs, &e2);
    const int E = e2 - 6;  // max|x| / 2^E < 64 (one rounding of slack: digits <= 64)
    if (blockIdx.y == 0 && tid == 0) dexp[m] = E;
    for (int i = c0 + tid; i < c1; i += STEP) {
        float4 v[U], g[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = min(i + u * kPrepThreads, c1 - 1);
            v[u] = xr[k];
            if constexpr (NORM) g[u] = wr[k];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = i + u * kPrepThreads;
            if (k >= c1) break;
            float4 a = v[u];
            if constexpr (NORM) {
                a.x = (a.x * (1.0f + g[u].x)) * rs;
                a.y = (a.y * (1.0f + g[u].y)) * rs;
                a.z = (a.z * (1.0f + g[u].z)) * rs;
                a.w = (a.w * (1.0f + g[u].w)) * rs;
            }
            const float vv[4] = {a.x, a.y, a.z, a.w};
            unsigned pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float t0 = ldexpf(vv[c], -E);
                const float d0 = rintf(t0);
                float t = (t0 - d0) * 128.0f;
                const float d1 = rintf(t);
                t = (t - d1) * 128.0f;
                const float d2 = rintf(t);
                t = (t - d2) * 128.0f;
                const float d3 = rintf(t);
                pk[0] |= ((unsigned)(int)d0 & 0xffu) << (8 * c);
                pk[1] |= ((unsigned)(int)d1 & 0xffu) << (8 * c);
                pk[2] |= ((unsigned)(int)d2 & 0xffu) << (8 * c);
                pk[3] |= ((unsigned)(int)d3 & 0xffu) << (8 * c);
            }
#pragma unroll
            for (int d = 0; d < 4; ++d) planes[(size_t)d * n4 + k] = pk[d];
        }
    }
}

// Workgroups per activation row of k_act_digits: about 256 in all, at most 8
// a row.
int act_digit_splits(int rows) {
    int s = 1;
    while (s < 8 && rows * s < 256) s *= 2;
    return s;
}

// NW waves, T = 2 for the [gate; up] pair of SwiGLU, U >= K / 64 / NW blocks
// per wave and tile, R ring slots (U % R == 0), MP pairs of activation rows
// (2 MP >= M).
template <int NW, int T, int U, int R, int MP, bool ROWSCALE, int EPI>
__global__ __launch_bounds__(NW * QLM_WAVE) void k_gemm_mx(
    const int8_t* __restrict__ digits, const int* __restrict__ dexp,
    const int8_t* __restrict__ q, const float* __restrict__ sc, float* __restrict__ y, int ldy,
    int M, int N, int K, int F, int ntiles) {
    constexpr int NT = NW * QLM_WAVE;
    constexpr int MR = 2 * MP;               // activation rows with padding
    constexpr int PHB = MR * 4 * 64 * NW;    // bytes of one phase of digits
    constexpr int CPT = (PHB / 16 + NT - 1) / NT;  // 16-byte staging chunks per thread
    __shared__ __align__(16) unsigned char dig[2][PHB];
    __shared__ __align__(16) unsigned char zero16[16];
    __shared__ int red[2][NW][T][MR][16];
    __shared__ int esh[MR];

    const int tid = threadIdx.x, lane = tid & (QLM_WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / QLM_WAVE);
    const int n = lane & 15, qd = lane >> 4;
    const int nblk = K >> 6;
    // this wave's last block (a wave past the last block reads block nblk-1,
    // which then meets zero digits)
    const int blast = w < nblk ? nblk - 1 - ((nblk - 1 - w) % NW) : nblk - 1;

    // ---- digits of phase u (block column u, 64 NW columns) into registers
    int4 stg[CPT];
    auto stage = [&](int u) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * NT;  // chunk of the phase: (row-plane, 16-column)
            int4 v = make_int4(0, 0, 0, 0);
            if (c < PHB / 16) {
                const int rp = c / (4 * NW), c16 = c % (4 * NW);  // rp = 4 m + d
                const int col = (u * NW) * 64 + c16 * 16;
                if (col < K)
                    v = *reinterpret_cast<const int4*>(digits + (size_t)rp * K + col);
            }
            stg[i] = v;
        }
    };
    auto commit = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + i * NT;
            if (c < PHB / 16) reinterpret_cast<int4*>(dig[buf])[c] = stg[i];
        }
    };

    // ---- weight ring: block u of a tile lives in slot u % R (blocks past K
    // repeat the wave's last block and meet zero digits)
    static_assert(U % R == 0, "ring slots must divide the blocks per tile");
    int4 wb[R][T];
    float sb[R][T];
    auto issue = [&](int tile, int u, int sl) {
        const int b = min(w + NW * u, blast);
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            const size_t fb = (size_t)(tile + tt * ntiles) * nblk + b;
            wb[sl][tt] = reinterpret_cast<const int4*>(q)[fb * QLM_WAVE + lane];
            if constexpr (!ROWSCALE) sb[sl][tt] = sc[fb * 32 + (qd & 1) * 16 + n];
        }
    };
    stage(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < R; ++u) issue(blockIdx.x, u, u);
    if (tid < MR) esh[tid] = dexp[tid];
    if (tid < 4) reinterpret_cast<unsigned*>(zero16)[tid] = 0u;

    // A-fragment of this lane for pair j: LDS offset aoff + j * APAIR within
    // a phase buffer
    constexpr int APAIR = 2 * 4 * 64 * NW;
    int aoff;
    bool active;
    {
        int mloc, d;
        if constexpr (ROWSCALE) {
            active = n < 8;
            mloc = n >> 2;
            d = n & 3;
        } else {
            active = ((n >> 2) & 1) == (qd >> 1);
            mloc = n >> 3;
            d = n & 3;
        }
        aoff = (mloc * 4 + d) * (64 * NW) + w * 64 + qd * 16;
    }

    float accf[T][MP];
    v4i acci[T][MP];
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
        for (int j = 0; j < MP; ++j) {
            accf[tt][j] = 0.0f;
            acci[tt][j] = v4i{0, 0, 0, 0};
        }

    auto consume = [&](int sl, int u, int buf) {
        const bool real = w + NW * u < nblk;
#pragma unroll
        for (int j = 0; j < MP; ++j) {
            const unsigned char* ap = active && real ? dig[buf] + aoff + j * APAIR : zero16;
            const v4i a = *reinterpret_cast<const v4i*>(ap);
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
                const v4i bw = v4i{wb[sl][tt].x, wb[sl][tt].y, wb[sl][tt].z, wb[sl][tt].w};
                if constexpr (ROWSCALE) {
                    acci[tt][j] =
                        __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bw, acci[tt][j], 0, 0, 0);
                } else {
                    const v4i dd =
                        __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bw, v4i{0, 0, 0, 0}, 0, 0, 0);
                    const int pp = (dd[0] << 7) + dd[1];
                    const int qq = (dd[2] << 7) + dd[3];
                    const float v = fmaf((float)qq, 0x1p-14f, (float)pp);
                    accf[tt][j] = fmaf(v, sb[sl][tt], accf[tt][j]);
                }
            }
        }
    };

    int par = 0;
    // cross-wave sums of a tile and its epilogue (every thread takes outputs)
    auto tile_end = [&](int tile) {
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
#pragma unroll
            for (int j = 0; j < MP; ++j) {
                if constexpr (ROWSCALE) {
                    // lanes q = 0, 1: rows 2j + q, four digit sums (exact int32)
                    const v4i s = acci[tt][j];
                    const float v = fmaf((float)s[3], 0x1p-21f,
                                         fmaf((float)s[2], 0x1p-14f,
                                              fmaf((float)s[1], 0x1p-7f, (float)s[0])));
                    if (qd < 2) red[par][w][tt][2 * j + qd][n] = __float_as_int(v);
                    acci[tt][j] = v4i{0, 0, 0, 0};
                } else {
                    // lanes q and q ^ 1 hold groups 2b and 2b + 1 of the same row
                    const float p = accf[tt][j] + __shfl_xor(accf[tt][j], 16, QLM_WAVE);
                    if ((qd & 1) == 0) red[par][w][tt][2 * j + (qd >> 1)][n] = __float_as_int(p);
                    accf[tt][j] = 0.0f;
                }
            }
        }
        __syncthreads();
        for (int o = tid; o < M * 16; o += NT) {
            const int m = o >> 4, nn = o & 15;
            const int row = tile * 16 + nn;
            if (row >= N) continue;
            float val[T];
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
                float v = __int_as_float(red[par][0][tt][m][nn]);
                for (int ww = 1; ww < NW; ++ww) v += __int_as_float(red[par][ww][tt][m][nn]);
                if constexpr (ROWSCALE) {
                    const int r = EPI == EPI_SWIGLU && tt == 1 ? F + row : row;
                    val[tt] = ldexpf(v, esh[m]) * sc[r];
                } else {
                    val[tt] = ldexpf(v, esh[m] - 7);
                }
            }
            float* dst = y + (size_t)m * ldy + row;
            if constexpr (EPI == EPI_SWIGLU)
                *dst = silu_f(val[0]) * val[1];
            else if constexpr (EPI == EPI_RESID)
                *dst += val[0];
            else
                *dst = val[0];
        }
        par ^= 1;
    };

    // ---- tiles x phases. Phase u: commit its staged digits to LDS buffer
    // (u & 1), stage phase u + 1 (the next tile's phase 0 after the last),
    // one barrier, consume block u, refill its slot with block u + R (of the
    // next tile once past U).
    for (int tile = blockIdx.x;; tile += gridDim.x) {
        const int next = tile + (int)gridDim.x;
        if (next < ntiles) {
#pragma unroll 1
            for (int u0 = 0; u0 < U; u0 += R) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int u = u0 + r;
                    commit(u & 1);
                    stage(u + 1 < U ? u + 1 : 0);
                    __syncthreads();
                    consume(r, u, u & 1);
                    if (u + R < U)
                        issue(tile, u + R, r);
                    else
                        issue(next, u + R - U, r);
                }
            }
        } else {
#pragma unroll 1
            for (int u0 = 0; u0 < U; u0 += R) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int u = u0 + r;
                    commit(u & 1);
                    if (u + 1 < U) stage(u + 1);
                    __syncthreads();
                    consume(r, u, u & 1);
                    if (u + R < U) issue(tile, u + R, r);
                }
            }
        }
        tile_end(tile);
        if (next >= ntiles) break;
    }
}

// Instantiated (waves per workgroup, blocks per wave, ring slots) shapes;
// a shape serves the K with ceil(K / 64 / waves) in (U - R, U] (a wave's last
// ring round may hold zero-digit blocks). LDS per workgroup: 2 x 2MP x 4 x
// 64 NW bytes of digits + 2 x NW x T x 2MP x 16 partial sums.
constexpr int kGmShapes[][3] = {{4, 2, 2},  {4, 4, 4},   {4, 8, 2},  {4, 10, 2},
                                {4, 14, 2}, {8, 20, 2},  {16, 2, 2}, {16, 4, 2},
                                {16, 10, 2}};

struct GmConfig {
    int nw, u, r, grid;
};

size_t gm_lds(int nw, int mp, int t) {
    return (size_t)2 * 2 * mp * 4 * 64 * nw + (size_t)2 * nw * t * 2 * mp * 16 * 4;
}

int mp_for(int M) { return M <= 2 ? 1 : (M <= 4 ? 2 : (M <= 8 ? 4 : 8)); }

// The fewest waves per workgroup that cover K and give >= 2048 waves in all
// (more waves split each tile's K when the matrix has few tiles), within
// 96 KB of LDS; one tile per workgroup up to 2048 workgroups, grid-stride
// beyond. nw = 0 when no shape fits.
GmConfig gm_config(int M, int N, int K, int t) {
    const int tiles = (N + 15) / 16, nblk = K / 64, mp = mp_for(M);
    GmConfig c{0, 0, 0, tiles < 2048 ? tiles : 2048};
    if (K <= 0 || K % 64 != 0) return c;
    for (int nw = 4; nw <= 16; nw *= 2) {
        if (gm_lds(nw, mp, t) > 96 * 1024 || nblk < nw) break;  // every wave has a block
        for (const auto& sh : kGmShapes) {
            if (sh[0] != nw) continue;
            const int need = (nblk + nw - 1) / nw;
            if (need <= sh[1] && need > sh[1] - sh[2]) {
                c.nw = sh[0];
                c.u = sh[1];
                c.r = sh[2];
                break;
            }
        }
        if (c.nw && tiles * c.nw >= 2048) break;
    }
    return c;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t digits_bytes(int M, int K) { return (size_t)2 * mp_for(M) * 4 * K; }

template <int NW, int U, int R, int MP, bool RS, int EPI>
int launch_gm(const GmConfig& c, const int8_t* dg, const int* de, const int8_t* q,
              const float* sc, float* y, int ldy, int M, int N, int K, hipStream_t st) {
    constexpr int T = EPI == EPI_SWIGLU ? 2 : 1;
    // shapes whose LDS exceeds the configuration limit are never chosen
    // (gm_config) and not instantiated
    constexpr size_t kLds = (size_t)2 * 2 * MP * 4 * 64 * NW + (size_t)2 * NW * T * 2 * MP * 16 * 4;
    if constexpr (kLds > 96 * 1024) {
        return QLM_ERR_SHAPE;
    } else {
        const int ntiles = (N + 15) / 16;
        int grid = c.grid < ntiles ? c.grid : ntiles;
        if (grid < 1) grid = 1;
        hipLaunchKernelGGL((k_gemm_mx<NW, T, U, R, MP, RS, EPI>), dim3(grid),
                           dim3(NW * QLM_WAVE), 0, st, dg, de, q, sc, y, ldy, M, N, K, N, ntiles);
        return qlm_launch_status();
    }
}

template <int MP, bool RS, int EPI>
int launch_gm_pair(const GmConfig& c, const int8_t* dg, const int* de, const int8_t* q,
                   const float* sc, float* y, int ldy, int M, int N, int K, hipStream_t st) {
#define QLM_GM(W, UU, RR)                                                                 \
    if (c.nw == W && c.u == UU && c.r == RR)                                               \
        return launch_gm<W, UU, RR, MP, RS, EPI>(c, dg, de, q, sc, y, ldy, M, N, K, st);
    QLM_GM(4, 2, 2) QLM_GM(4, 4, 4) QLM_GM(4, 8, 2) QLM_GM(4, 10, 2) QLM_GM(4, 14, 2)
    QLM_GM(8, 20, 2) QLM_GM(16, 2, 2) QLM_GM(16, 4, 2) QLM_GM(16, 10, 2)
#undef QLM_GM
    return QLM_ERR_SHAPE;
}

template <bool RS, int EPI>
int launch_gm_mp(const GmConfig& c, const int8_t* dg, const int* de, const int8_t* q,
                 const float* sc, float* y, int ldy, int M, int N, int K, hipStream_t st) {
    switch (mp_for(M)) {
        case 1: return launch_gm_pair<1, RS, EPI>(c, dg, de, q, sc, y, ldy, M, N, K, st);
        case 2: return launch_gm_pair<2, RS, EPI>(c, dg, de, q, sc, y, ldy, M, N, K, st);
        case 4: return launch_gm_pair<4, RS, EPI>(c, dg, de, q, sc, y, ldy, M, N, K, st);
        default: return launch_gm_pair<8, RS, EPI>(c, dg, de, q, sc, y, ldy, M, N, K, st);
    }
}


// ---- 2 <= M <= 64 activation rows, one scale per weight row ----
//
// y[m, n] = s[n] * sum_k x[m, k] q[n, k]. The rows are written as int8 digit
// planes by k_act_digits (x_m = 2^E_m (d0 + d1 2^-7 + d2 2^-14 + d3 2^-21),
// RMSNorm folded in) and multiplied on v_mfma_i32_16x16x64_i8 with B = a
// tile-major weight fragment as stored (lane 16q + n: weight row n, columns
// 16q .. 16q+15) and A = 16 digit rows over the block's 64 columns, in one of
// two orders:
//   interleaved (2 <= M <= 8): A row 4 m' + d of product a holds digit d of
//       activation row 4a + m'; NP = 1 or 2 products cover 4 NP rows, all
//       four digits;
//   digit-major (9 <= M <= 64): product 3g + d holds digit d of activation
//       rows 16g .. 16g+15; NP = 3 ceil(M / 16) products, three digits
//       (x_m to within 2^(E_m - 15), at most 2^-20 of the row's largest
//       magnitude: a quarter fewer products and digit bytes than four
//       digits, at the precision of a bf16 hi/lo split).
// D lane (q', n) then holds, for weight row n, the four digit sums of
// activation row 4a + q' (interleaved) or digit d's sums of rows 16g + 4q' ..
// +3 (digit-major, so a row's digits meet in one lane and register slot);
// with one scale per weight row nothing is scaled inside the K loop, so the
// products accumulate exact int32 sums over all of the workgroup's blocks
// (|sum| <= 64 * 127 * K < 2^31 for K <= 2^18) and are combined once at the
// end, in fp32: (D0 + 2^-7 (D1 + 2^-7 (D2 [+ 2^-7 D3]))) 2^E_m s[n].
//
// Work split: a workgroup of 8 waves owns 8 x 2 tiles (16 weight rows each)
// and one K slice; wave w owns 2 of the tiles, so the waves share
// every digit block, which the workgroup stages once through double-
// buffered LDS in operand order (product a's 1 KB holds lane l's 16 bytes at
// 16 l, so both the stores and the ds_read_b128 of an operand are lane-
// contiguous and free of bank conflicts; rows padded to 80 bytes measured
// half of the LDS cycles in conflicts) while each wave streams its 2
// fragments a block; both are requested three
// blocks ahead (a block's products take well under one load latency). The
// digit traffic from L2 is then one block per workgroup and block, shared by
// 16 tiles.
//
// Scheduling: a workgroup fills a CU (two waves a SIMD), so the tile groups
// run in rounds of 256. Whole rounds take whole K ("full" units, results
// stored directly); the groups of the last, partial round are split into K
// slices so that it fills the chip too (on 151936 x 2560 the third round
// would otherwise hold 82 workgroups and take as long as a whole one). The
// slices write fp32 partial sums of their columns, added in slice order by
// k_mm_reduce.
constexpr int kR64Waves = 8;   // waves per workgroup (two a SIMD)
constexpr int kR64Tiles = 2;   // tiles per wave

template <int NP, bool DM, int EPI>
__global__ __launch_bounds__(kR64Waves * QLM_WAVE) void k_mm_rows64(
    const int8_t* __restrict__ digits, const int* __restrict__ dexp,
    const int8_t* __restrict__ qz, const float* __restrict__ srow, float* __restrict__ y, int ldy,
    float* __restrict__ part, int M, int N, int K, int tiles, int full, int ks, int bps) {
    constexpr int NT = kR64Waves * QLM_WAVE;
    constexpr int AR = 16 * NP;       // A rows of a block
    constexpr int CH = AR * 4;        // 16-byte chunks of a block
    static_assert(!DM || NP % 3 == 0, "digit-major blocks hold three digits a row group");
    // chunks per thread; when the threads do not divide the chunks (whole
    // waves of them: CH is a multiple of 64) every thread still loads its
    // last chunk (index clamped, so the loads stay unconditional) and only
    // the threads with a chunk there store it
    constexpr int CPT = (CH + NT - 1) / NT;
    constexpr bool PART = CH % NT != 0;
    typedef int v4i __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) unsigned char abuf[2][AR * 64];

    const int tid = threadIdx.x, lane = tid & (QLM_WAVE - 1);
    const int w = tid / QLM_WAVE, qd = lane >> 4, n = lane & 15;
    const int nblk = K >> 6;
    // unit -> tile group, K range: whole K below `full`, then ks slices a group
    const int u = blockIdx.x;
    int g = u, b0 = 0, nb = nblk, slice = -1;
    if (u >= full) {
        const int v = u - full;
        g = full + v / ks;
        slice = v - (v / ks) * ks;
        b0 = slice * bps;
        nb = min(bps, nblk - b0);
    }
    const bool to_part = slice >= 0 && ks > 1;
    const int tile0 = (g * kR64Waves + w) * kR64Tiles;

    // Blocks are requested three ahead: digit block j goes through staging
    // registers st[j & 3] into LDS buffer j & 1 at the end of iteration j - 1,
    // weight block j into wr[j & 3] (rings of four, so that the slot of every
    // access is a compile-time constant in the loop unrolled by four). Digit
    // chunk c = tid + NT i is operand lane p = c & 63 (A row p & 15, bytes
    // 16 (p >> 4)) of product c >> 6, at LDS byte 16 c; A row i of product a
    // is digit plane 16 a + i (interleaved) or 4 (16 (a / 3) + i) + a % 3
    // (digit-major) of the [row][digit][K] planes. Vector types: an
    // aggregate copy into LDS would keep the staging array in scratch memory.
    constexpr int RING = 4;
    v4i st[RING][CPT];
    v4i wr[RING][kR64Tiles];
    auto issue = [&](int slot, int b) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = PART ? min(tid + NT * i, CH - 1) : tid + NT * i;
            const int a = c >> 6, ar = c & 15;
            const int r = DM ? 4 * (16 * (a / 3) + ar) + a % 3 : 16 * a + ar;
            st[slot][i] = *reinterpret_cast<const v4i*>(digits + (size_t)r * K + 64 * b +
                                                        16 * ((c >> 4) & 3));
        }
        // weight fragments of this wave's tiles (tile index clamped: a ragged
        // last group recomputes the last tile and stores nothing for it)
#pragma unroll
        for (int t = 0; t < kR64Tiles; ++t) {
            const int tl = min(tile0 + t, tiles - 1);
            wr[slot][t] = *reinterpret_cast<const v4i*>(
                qz + ((size_t)tl * nblk + b) * 1024 + (size_t)lane * 16);
        }
    };
    auto store_digits = [&](int slot, int buf) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = tid + NT * i;
            if (!PART || c < CH) *reinterpret_cast<v4i*>(&abuf[buf][16 * c]) = st[slot][i];
        }
    };

    v4i acc[kR64Tiles][NP];
#pragma unroll
    for (int t = 0; t < kR64Tiles; ++t)
#pragma unroll
        for (int a = 0; a < NP; ++a) acc[t][a] = v4i{0, 0, 0, 0};

    // iteration i: request block i + 3, multiply block i, stage block i + 1.
    // The requests are unconditional (past the slice they repeat its last
    // block, an L2 hit): a load under a branch leaves the compiler unsure of
    // how many loads are in flight, and it then waits for all of them.
    auto mul = [&](int i, int slot) {
        const int buf = i & 1;
#pragma unroll
        for (int a = 0; a < NP; ++a) {
            const v4i av = *reinterpret_cast<const v4i*>(&abuf[buf][1024 * a + 16 * lane]);
#pragma unroll
            for (int t = 0; t < kR64Tiles; ++t)
                acc[t][a] =
                    __builtin_amdgcn_mfma_i32_16x16x64_i8(av, wr[slot][t], acc[t][a], 0, 0, 0);
        }
    };
    // Block i + 1's digits go to LDS first (its buffer was last read by the
    // products of block i - 1, which every wave finished before the barrier
    // ending step i - 1), then block i + 3 is requested, then block i is
    // multiplied; the barrier ending step i publishes block i + 1. The store
    // is unconditional: at the last block it writes a clamped copy nobody
    // reads, and a conditional store lets the compiler move the slot's load
    // into the branch, where it is waited on at once.
    auto step = [&](int i, int slot) {
        store_digits((slot + 1) & (RING - 1), (i & 1) ^ 1);
        issue((slot + RING - 1) & (RING - 1), b0 + min(i + RING - 1, nb - 1));
        // the requests go out before the products (left to itself the
        // scheduler sinks them below, shortening the prefetch to ~1 block)
        __builtin_amdgcn_sched_barrier(0);
        mul(i, slot);
        __syncthreads();
    };
    auto tail = [&](int i, int slot) {  // the last blocks: nothing left to request
        store_digits((slot + 1) & (RING - 1), (i & 1) ^ 1);
        mul(i, slot);
        __syncthreads();
    };

#pragma unroll
    for (int j = 0; j < RING - 1; ++j) issue(j, b0 + min(j, nb - 1));
    store_digits(0, 0);
    __syncthreads();
    int i0 = 0;
    for (; i0 + RING <= nb; i0 += RING) {  // workgroup-uniform bounds
        step(i0, 0);
        step(i0 + 1, 1);
        step(i0 + 2, 2);
        step(i0 + 3, 3);
    }
    if (i0 < nb) tail(i0, 0);
    if (i0 + 1 < nb) tail(i0 + 1, 1);
    if (i0 + 2 < nb) tail(i0 + 2, 2);

    // ---- lane (qd, n), weight row 16 tile + n: its activation rows i are
    // 4 i + qd (interleaved) or 16 (i / 4) + 4 qd + i % 4 (digit-major) ----
    constexpr int NR = DM ? 4 * (NP / 3) : NP;
    auto row_m = [&](int i) { return DM ? 16 * (i >> 2) + 4 * qd + (i & 3) : 4 * i + qd; };
    const int row0 = full * kR64Waves * kR64Tiles * 16, nt = N - row0;
    float ex[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) ex[i] = ldexpf(1.0f, dexp[min(row_m(i), M - 1)]);
#pragma unroll
    for (int t = 0; t < kR64Tiles; ++t) {
        const int tile = tile0 + t;
        const int row = tile * 16 + n;
        if (tile >= tiles || row >= N) continue;
        const float sn = srow[row];
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int m = row_m(i);
            if (m >= M) continue;
            float v;
            if constexpr (DM) {
                const int g = i >> 2, j = i & 3;
                v = fmaf(fmaf((float)acc[t][3 * g + 2][j], 0x1p-7f, (float)acc[t][3 * g + 1][j]),
                         0x1p-7f, (float)acc[t][3 * g][j]);
            } else {
                const v4i dd = acc[t][i];
                v = fmaf(fmaf(fmaf((float)dd[3], 0x1p-7f, (float)dd[2]), 0x1p-7f, (float)dd[1]),
                         0x1p-7f, (float)dd[0]);
            }
            const float r = (v * ex[i]) * sn;
            if (to_part)  // tail columns only: [slice][m][N - row0]
                part[((size_t)slice * M + m) * nt + (row - row0)] = r;
            else if constexpr (EPI == EPI_RESID)
                y[(size_t)m * ldy + row] += r;
            else
                y[(size_t)m * ldy + row] = r;
        }
    }
}

constexpr int kR64MaxRows = 64;

struct R64Plan {
    int np, groups, full, ks, bps, units;
};

// Whole rounds of 256 groups (one workgroup a CU) take whole K; the last
// partial round's groups are cut into ks slices of bps blocks (about one
// workgroup a CU again).
R64Plan r64_plan(int M, int N, int K) {
    R64Plan p;
    // products a block: 4 interleaved rows each up to 8 rows, then three
    // digit-major products per 16 rows
    p.np = M <= 4 ? 1 : (M <= 8 ? 2 : 3 * ((M + 15) / 16));
    const int tiles = (N + 15) / 16, nblk = K / 64;
    p.groups = (tiles + kR64Waves * kR64Tiles - 1) / (kR64Waves * kR64Tiles);
    p.full = (p.groups / 256) * 256;
    const int tail = p.groups - p.full;
    int ks = tail > 0 ? 256 / tail : 1;
    ks = ks < 1 ? 1 : (ks > nblk ? nblk : ks);
    p.bps = (nblk + ks - 1) / ks;
    p.ks = (nblk + p.bps - 1) / p.bps;
    p.units = p.full + tail * p.ks;
    return p;
}

size_t r64_digits_bytes(int K) { return (size_t)kR64MaxRows * 4 * K; }

// columns of the partial round (the ones that go through partial sums)
int r64_tail_rows(const R64Plan& p, int N) { return N - p.full * kR64Waves * kR64Tiles * 16; }

size_t r64_work_bytes(int M, int N, int K, int epi) {
    const R64Plan p = r64_plan(M, N, K);
    size_t b = align256(r64_digits_bytes(K)) + align256((size_t)kR64MaxRows * sizeof(int));
    if (p.ks > 1) b += (size_t)p.ks * M * r64_tail_rows(p, N) * sizeof(float);
    (void)epi;
    return b;
}

template <int NP, bool DM>
int launch_r64(const R64Plan& p, const int8_t* dg, const int* de, const int8_t* qz,
               const float* sr, float* y, int ldy, float* part, int M, int N, int K, int epi,
               hipStream_t st) {
    const int tiles = (N + 15) / 16;
    if (epi == EPI_RESID)
        hipLaunchKernelGGL((k_mm_rows64<NP, DM, EPI_RESID>), dim3(p.units), dim3(kR64Waves * QLM_WAVE),
                           0, st, dg, de, qz, sr, y, ldy, part, M, N, K, tiles, p.full, p.ks,
                           p.bps);
    else
        hipLaunchKernelGGL((k_mm_rows64<NP, DM, EPI_STORE>), dim3(p.units), dim3(kR64Waves * QLM_WAVE),
                           0, st, dg, de, qz, sr, y, ldy, part, M, N, K, tiles, p.full, p.ks,
                           p.bps);
    int rc = qlm_launch_status();
    if (rc != QLM_OK || p.ks == 1) return rc;
    const int row0 = N - r64_tail_rows(p, N), nt = N - row0;
    const dim3 rgrid((nt + kReduceThreads - 1) / kReduceThreads, M);
    if (epi == EPI_RESID)
        hipLaunchKernelGGL((k_mm_reduce<MMR_RESID, false>), rgrid, dim3(kReduceThreads), 0, st,
                           part, p.ks, M, nt, nt, y + row0, ldy, nullptr, 0, K, 0.0f);
    else
        hipLaunchKernelGGL((k_mm_reduce<MMR_STORE, false>), rgrid, dim3(kReduceThreads), 0, st,
                           part, p.ks, M, nt, nt, y + row0, ldy, nullptr, 0, K, 0.0f);
    return qlm_launch_status();
}
}  // namespace

extern "C" size_t qlm_matmul_i8_mx_workspace_bytes(int M, int K) {
    if (M <= 0 || M > kMaxRows || K <= 0) return 0;
    return align256(digits_bytes(M, K)) + align256((size_t)kMaxRows * sizeof(int));
}

extern "C" int qlm_matmul_i8_mx_shape(int M, int N, int K, int epilogue, int* waves,
                                      int* blocks, int* ring, int* grid) {
    if (M <= 0 || N <= 0 || K <= 0 || !waves || !blocks || !ring || !grid) return QLM_ERR_ARG;
    if (M > kMaxRows) return QLM_ERR_SHAPE;
    const GmConfig c = gm_config(M, N, K, epilogue == EPI_SWIGLU ? 2 : 1);
    if (c.nw == 0) return QLM_ERR_SHAPE;
    *waves = c.nw;
    *blocks = c.u;
    *ring = c.r;
    *grid = c.grid;
    return QLM_OK;
}

extern "C" int qlm_matmul_i8_mx(const float* x, int ldx, const float* norm_w, float eps,
                                const int8_t* q_tiles, const float* s_tiles, int group, float* y,
                                int ldy, int M, int N, int K, int epilogue, void* work,
                                size_t work_bytes, void* stream) {
    if (!x || !q_tiles || !s_tiles || !y || M <= 0 || N <= 0 || K <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    if (M > kMaxRows) return QLM_ERR_SHAPE;
    const bool rowscale = (group == K);
    if (!rowscale && group != 32) return QLM_ERR_SHAPE;
    if (ldx < K || ldy < N || ldx % 4 != 0) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)q_tiles | (uintptr_t)norm_w) & 15u) return QLM_ERR_SHAPE;
    const GmConfig c = gm_config(M, N, K, epilogue == EPI_SWIGLU ? 2 : 1);
    if (c.nw == 0) return QLM_ERR_SHAPE;
    const size_t need = qlm_matmul_i8_mx_workspace_bytes(M, K);
    if (!work || work_bytes < need || ((uintptr_t)work & 255u)) return QLM_ERR_ARG;
    hipStream_t st = as_stream(stream);
    int8_t* dg = reinterpret_cast<int8_t*>(work);
    int* de = reinterpret_cast<int*>(reinterpret_cast<char*>(work) + align256(digits_bytes(M, K)));
    const int rows = 2 * mp_for(M);
    const dim3 dgrid(rows, act_digit_splits(rows));
    if (norm_w)
        hipLaunchKernelGGL(k_act_digits<true>, dgrid, dim3(kPrepThreads), 0, st, x, ldx, norm_w,
                           eps, M, K, dg, de);
    else
        hipLaunchKernelGGL(k_act_digits<false>, dgrid, dim3(kPrepThreads), 0, st, x, ldx, nullptr,
                           eps, M, K, dg, de);
    int rc = qlm_launch_status();
    if (rc != QLM_OK) return rc;
#define QLM_GM_CALL(RS, E) \
    return launch_gm_mp<RS, E>(c, dg, de, q_tiles, s_tiles, y, ldy, M, N, K, st)
    if (rowscale) {
        if (epilogue == EPI_STORE) QLM_GM_CALL(true, EPI_STORE);
        if (epilogue == EPI_RESID) QLM_GM_CALL(true, EPI_RESID);
        QLM_GM_CALL(true, EPI_SWIGLU);
    }
    if (epilogue == EPI_STORE) QLM_GM_CALL(false, EPI_STORE);
    if (epilogue == EPI_RESID) QLM_GM_CALL(false, EPI_RESID);
    QLM_GM_CALL(false, EPI_SWIGLU);
#undef QLM_GM_CALL
}

extern "C" size_t qlm_matmul_i8_rows64_workspace_bytes(int M, int N, int K, int epilogue) {
    if (M < 2 || M > kR64MaxRows || N <= 0 || K <= 0 || K % 64 != 0) return 0;
    if (epilogue != EPI_STORE && epilogue != EPI_RESID) return 0;
    return r64_work_bytes(M, N, K, epilogue);
}

extern "C" int qlm_matmul_i8_rows64(const float* x, int ldx, const float* norm_w, float eps,
                                    const int8_t* q_tiles, const float* s_rows, float* y,
                                    int ldy, int M, int N, int K, int epilogue, void* work,
                                    size_t work_bytes, void* stream) {
    if (!x || !q_tiles || !s_rows || !y || M <= 0 || N <= 0 || K <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    if (epilogue == EPI_RESID && norm_w) return QLM_ERR_ARG;
    if (epilogue == EPI_SWIGLU || M < 2 || M > kR64MaxRows || K % 64 != 0 || K > (1 << 18))
        return QLM_ERR_SHAPE;
    if (ldx < K || ldy < N || ldx % 4 != 0) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)q_tiles | (uintptr_t)norm_w) & 15u) return QLM_ERR_SHAPE;
    const size_t need = r64_work_bytes(M, N, K, epilogue);
    if (!work || work_bytes < need || ((uintptr_t)work & 255u)) return QLM_ERR_ARG;
    hipStream_t st = as_stream(stream);
    int8_t* dg = reinterpret_cast<int8_t*>(work);
    int* de = reinterpret_cast<int*>(reinterpret_cast<char*>(work) +
                                     align256(r64_digits_bytes(K)));
    float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(de) +
                                           align256((size_t)kR64MaxRows * sizeof(int)));
    const R64Plan p = r64_plan(M, N, K);
    // activation rows the products read (digits of the rows past M are zeros)
    const int rows = p.np <= 2 ? 4 * p.np : 16 * (p.np / 3);
    const dim3 dgrid(rows, act_digit_splits(rows));
    if (norm_w)
        hipLaunchKernelGGL(k_act_digits<true>, dgrid, dim3(kPrepThreads), 0, st, x, ldx, norm_w,
                           eps, M, K, dg, de);
    else
        hipLaunchKernelGGL(k_act_digits<false>, dgrid, dim3(kPrepThreads), 0, st, x, ldx, nullptr,
                           eps, M, K, dg, de);
    int rc = qlm_launch_status();
    if (rc != QLM_OK) return rc;
#define QLM_R64(NP, DM) \
    return launch_r64<NP, DM>(p, dg, de, q_tiles, s_rows, y, ldy, part, M, N, K, epilogue, st)
    switch (p.np) {
        case 1: QLM_R64(1, false);
        case 2: QLM_R64(2, false);
        case 3: QLM_R64(3, true);
        case 6: QLM_R64(6, true);
        case 9: QLM_R64(9, true);
        default: QLM_R64(12, true);
    }
#undef QLM_R64
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_gemm_mx() {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>((k_act_digits<false>)));
}
