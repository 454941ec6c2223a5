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

namespace {

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kPrepThreads = 256;
constexpr int kMaxRows = 16;

// Activation digits of one row per workgroup; rows m >= M (padding up to an
// even count) are written as zeros. Two passes over the row: sum of squares
// (RMSNorm) and max|x * (1 + w)|, then the digits.
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
    unsigned* planes = reinterpret_cast<unsigned*>(digits + (size_t)m * 4 * K);
    if (m >= M) {
        for (int i = tid; i < n4; i += kPrepThreads)
#pragma unroll
            for (int d = 0; d < 4; ++d) planes[(size_t)d * n4 + i] = 0u;
        if (tid == 0) dexp[m] = 0;
        return;
    }
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * ldx);
    const float4* wr = reinterpret_cast<const float4*>(nw);
    float ss = 0.0f, mx = 0.0f;
    for (int i = tid; i < n4; i += kPrepThreads) {
        float4 v = xr[i];
        if constexpr (NORM) {
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
            const float4 g = wr[i];
            v.x *= 1.0f + g.x;
            v.y *= 1.0f + g.y;
            v.z *= 1.0f + g.z;
            v.w *= 1.0f + g.w;
        }
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
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
    if (tid == 0) dexp[m] = E;
    for (int i = tid; i < n4; i += kPrepThreads) {
        float4 v = xr[i];
        if constexpr (NORM) {
            const float4 g = wr[i];
            v.x = (v.x * (1.0f + g.x)) * rs;
            v.y = (v.y * (1.0f + g.y)) * rs;
            v.z = (v.z * (1.0f + g.z)) * rs;
            v.w = (v.w * (1.0f + g.w)) * rs;
        }
        const float vv[4] = {v.x, v.y, v.z, v.w};
        unsigned pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float u = ldexpf(vv[c], -E);
            const float d0 = rintf(u);
            float t = (u - d0) * 128.0f;
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
        for (int d = 0; d < 4; ++d) planes[(size_t)d * n4 + i] = pk[d];
    }
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
    if (norm_w)
        hipLaunchKernelGGL(k_act_digits<true>, dim3(rows), dim3(kPrepThreads), 0, st, x, ldx,
                           norm_w, eps, M, K, dg, de);
    else
        hipLaunchKernelGGL(k_act_digits<false>, dim3(rows), dim3(kPrepThreads), 0, st, x, ldx,
                           nullptr, eps, M, K, dg, de);
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
