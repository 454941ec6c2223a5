// Matmul over native (unquantised) weights, the reference's --precision bf16:
// the checkpoint's own dtype is kept, fp32 rows for F32 tensors and bf16 rows
// for BF16 ones (get_tensor_keep_bf16, safetensors.cpp:248-273), and
// math::matmul computes fp32 dot products against them (dot_avx2 /
// bf16_gemv_range, math_ops.cpp:209-400, :820-900):
//   y[m, n] = sum_k x[m, k] * W[n, k],   m < M <= 16 per launch.
//
// On the fp32 matrix cores (v_mfma_f32_16x16x4f32; bf16 weights are widened
// exactly): lane l = 16q + r of a wave supplies A = W[row r of a 16-row tile]
// [4 columns] and B = x[activation row r][the same 4 columns], and holds
// D[4q + i][r] = the tile's output row 4q + i for activation row r. The four
// columns a lane loads (one 16-byte load: k0 + 4q .. +3) are spread over
// four MFMAs (element e in MFMA e), so each MFMA sums over the column set
// {k0 + 4q + e}; the same set for A and B, which is all a product needs.
//
// A workgroup of NW waves owns one 16-row tile at a time (grid-stride); wave
// w takes the 16-column chunks w, w + NW, ... of it. Work items (tile,
// chunk) of a wave form one sequence whose loads stay R items ahead in a
// register ring (weights and activation chunk together, so every wait is
// for the item about to be used); at the end of a tile the waves' partial
// tiles meet in LDS and the epilogue writes 16 x M outputs. RMSNorm is
// prepared by k_w_rows (rs[m] and x * (1 + w) once per launch) and 1/rms
// multiplies the finished sums.

#include "common.hpp"

namespace {

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWRows = 16;   // activation rows per launch
constexpr int kPrepT = 256;

// Four consecutive weights of a row as fp32 (bf16: exact widening).
template <typename WT>
struct WLoad;
template <>
struct WLoad<float> {
    typedef float4 raw;
    static __device__ __forceinline__ raw load(const float* p) {
        return *reinterpret_cast<const float4*>(p);
    }
    static __device__ __forceinline__ float4 widen(raw v) { return v; }
};
template <>
struct WLoad<uint16_t> {
    typedef uint2 raw;
    static __device__ __forceinline__ raw load(const uint16_t* p) {
        return *reinterpret_cast<const uint2*>(p);
    }
    static __device__ __forceinline__ float4 widen(raw v) {
        return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                           __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
    }
};

// Row preparation for the RMSNorm prologue: rs[m] = 1/sqrt(mean(x^2) + eps)
// and xg[m] = x[m] * (1 + w) (zero-centred gain), one workgroup per row.
__global__ __launch_bounds__(kPrepT) void k_w_rows(const float* __restrict__ x, int ldx, int K,
                                                   const float* __restrict__ nw, float eps,
                                                   float* __restrict__ rs,
                                                   float* __restrict__ xg) {
    __shared__ float red[kPrepT / QLM_WAVE];
    const int m = blockIdx.x;
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)m * ldx);
    const float4* wr = reinterpret_cast<const float4*>(nw);
    float4* out = reinterpret_cast<float4*>(xg + (size_t)m * K);
    float ss = 0.0f;
    for (int i = threadIdx.x; i < (K >> 2); i += kPrepT) {
        const float4 v = xr[i], g = wr[i];
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
        out[i] = make_float4(v.x * (1.0f + g.x), v.y * (1.0f + g.y), v.z * (1.0f + g.z),
                             v.w * (1.0f + g.w));
    }
    ss = block_sum(ss, red);
    if (threadIdx.x == 0) rs[m] = 1.0f / sqrtf(ss / (float)K + eps);
}

template <typename WT, int NW, int R, int T, int EPI, bool NORM>
__global__ __launch_bounds__(NW * QLM_WAVE) void k_gemv_w(
    const float* __restrict__ x, int ldx, const float* __restrict__ rs,
    const WT* __restrict__ W, float* __restrict__ y, int ldy, int M, int N, int K, int F,
    int ntiles) {
    using L = WLoad<WT>;
    __shared__ float red[2][NW][T][16][16];  // [parity][wave][half][tile row][activation row]

    const int tid = threadIdx.x, lane = tid & (QLM_WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / QLM_WAVE);
    const int r16 = lane & 15, q = lane >> 4;
    const int nch = K >> 4;                  // 16-column chunks
    const int per = (nch + NW - 1) / NW;     // chunks per wave and tile
    // this wave's last chunk (a wave past the last chunk repeats chunk nch-1,
    // masked to zero)
    const int clast = w < nch ? nch - 1 - ((nch - 1 - w) % NW) : nch - 1;
    const float* xrow = x + (size_t)min(r16, M - 1) * ldx;
    const bool mval = r16 < M;

    typename L::raw wb[R][T];
    float4 xb[R];
    // work item s of this wave: tile blockIdx.x + (s / per) * gridDim.x, chunk
    // w + NW * (s % per). Loads are unconditional (items past the last tile
    // reload its rows and are masked): a load under a branch would be waited
    // for where the branch ends.
    auto issue = [&](int s, int sl) {
        const int tile = min((int)blockIdx.x + (s / per) * (int)gridDim.x, ntiles - 1);
        const int c = min(w + NW * (s % per), clast);
        const int k = c * 16 + 4 * q;
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            const int row = min(tile * 16 + r16, N - 1) + tt * F;
            wb[sl][tt] = L::load(W + (size_t)row * K + k);
        }
        xb[sl] = *reinterpret_cast<const float4*>(xrow + k);
    };

    f32x4 acc[T];
#pragma unroll
    for (int tt = 0; tt < T; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    int par = 0;

    auto consume = [&](int s, int sl, int items) {
        const bool real = mval && (w + NW * (s % per) < nch) && s < items;
        float4 xv = xb[sl];
        if (!real) xv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            const float4 a = L::widen(wb[sl][tt]);
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, xv.x, acc[tt], 0, 0, 0);
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, xv.y, acc[tt], 0, 0, 0);
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, xv.z, acc[tt], 0, 0, 0);
            acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, xv.w, acc[tt], 0, 0, 0);
        }
    };

    // cross-wave sums of a finished tile and its epilogue; every thread takes
    // outputs (n, m) of the 16 x 16 block
    auto tile_end = [&](int tile) {
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) red[par][w][tt][4 * q + i][r16] = acc[tt][i];
            acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        __syncthreads();
        for (int o = tid; o < 256; o += NW * QLM_WAVE) {
            const int n = o >> 4, m = o & 15;
            const int row = tile * 16 + n;
            if (m >= M || row >= N) continue;
            float val[T];
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
                float v = red[par][0][tt][n][m];
                for (int ww = 1; ww < NW; ++ww) v += red[par][ww][tt][n][m];
                if constexpr (NORM) v *= rs[m];
                val[tt] = v;
            }
            float* dst = y + (size_t)m * ldy + row;
            if constexpr (EPI == EPI_SWIGLU)
                *dst = silu_f(val[0]) * val[1];
            else if constexpr (EPI == EPI_RESID)
                *dst += val[0];
            else
                *dst = val[0];
        }
        par ^= 1;  // a buffer is rewritten two tiles later, after another barrier
    };

    // items in rounds of R (ring slot = item % R, compile-time within a round)
#pragma unroll
    for (int r = 0; r < R; ++r) issue(r, r);
    const int my_tiles = ((int)ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int items = my_tiles * per;
#pragma unroll 1
    for (int s0 = 0; s0 < items; s0 += R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int s = s0 + r;
            consume(s, r, items);  // items past the end add zeros
            issue(s + R, r);
            if (s < items && s % per == per - 1)  // the same for every wave
                tile_end((int)blockIdx.x + (s / per) * (int)gridDim.x);
        }
    }
}

// One activation row on the vector ALUs (the matrix-core form above would
// spend 15 of its 16 activation columns on nothing and cost about as much
// time as the weight stream). The workgroup stages x (times 1 + gain for the
// RMSNorm prologue, whose 1/rms it also computes) in LDS once. A tile is
// RT = G * RG rows (G = NW / KS row groups): wave w owns row group w % G (RG
// rows, both halves for SwiGLU) and the column chunks (w / G) + KS * j of
// every tile it visits, so one x chunk read from LDS serves RG * T weight
// loads. Chunk c of a row is
// the 64 lanes' 16-byte loads, columns c * CW + EL * lane .. + EL - 1. Work
// items (tile, chunk) stream through a ring of R register slots as in
// k_gemv_w; a finished tile's partial sums meet in LDS (KS > 1) or are
// reduced inside the wave (KS == 1), and lanes of the first wave write the
// epilogue. Columns past K (a ragged last chunk) read an in-row clamped
// address and multiply staged zeros.
template <typename WT, int NW, int RG, int KS, int R, int EPI, bool NORM, int XL>
__global__ __launch_bounds__(NW * QLM_WAVE) void k_gemv_wv(
    const float* __restrict__ x, const float* __restrict__ gain, float eps,
    const WT* __restrict__ W, float* __restrict__ y, int N, int K, int F, int ntiles) {
    constexpr int T = EPI == EPI_SWIGLU ? 2 : 1;
    constexpr int G = NW / KS;           // row groups per tile
    constexpr int RT = G * RG;           // rows per tile
    constexpr int EL = 16 / sizeof(WT);  // weights per 16-byte load
    constexpr int XV = EL / 4;           // float4 of x per load
    constexpr int CW = QLM_WAVE * EL;    // columns per chunk
    constexpr int NT = NW * QLM_WAVE;
    static_assert(NW % KS == 0, "KS must divide the wave count");
    static_assert(R >= 2, "the x prefetch needs two ring slots");
    // x chunks, each as XV planes of 64 float4, then one chunk of zeros that
    // masked items read
    extern __shared__ float4 xs4[];
    __shared__ float red[KS > 1 ? 2 : 1][KS > 1 ? KS : 1][T][RT][4];
    __shared__ float bred[NW];

    const int tid = threadIdx.x, lane = tid & (QLM_WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / QLM_WAVE);
    const int rg = w % G, ph = w / G;
    const int nch = (K + CW - 1) / CW;
    const int per = (nch + KS - 1) / KS;  // items per tile and wave
    const int clast = ph < nch ? ph + KS * ((nch - 1 - ph) / KS) : nch - 1;
    const int K4 = K >> 2, KP4 = (nch + 1) * (CW / 4);

    // x and gain: loads first (clamped, unconditional, their values used
    // unconditionally so that none is sunk behind the ring's loads)
    float4 xr[XL], gr[XL];
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* g4 = reinterpret_cast<const float4*>(gain);
#pragma unroll
    for (int u = 0; u < XL; ++u) {
        const int i = min(tid + u * NT, K4 - 1);
        xr[u] = x4[i];
        if constexpr (NORM) gr[u] = g4[i];
    }
    __builtin_amdgcn_sched_barrier(0);

    // work item s of this wave: tile blockIdx.x + (s / per) * gridDim.x, chunk
    // ph + KS * (s % per); items past the wave's last chunk or last tile
    // reload a clamped chunk and read the zero chunk of x
    uint4 wb[R][T][RG];
    auto issue = [&](int s, int sl) {
        const int tile = min((int)blockIdx.x + (s / per) * (int)gridDim.x, ntiles - 1);
        const int c = min(ph + KS * (s % per), clast);
        const int col = min(c * CW + lane * EL, K - EL);
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
#pragma unroll
            for (int i = 0; i < RG; ++i) {
                const int row = min(tile * RT + rg * RG + i, N - 1) + tt * F;
                wb[sl][tt][i] = *reinterpret_cast<const uint4*>(W + (size_t)row * K + col);
            }
    };
#pragma unroll
    for (int r = 0; r < R; ++r) issue(r, r);

    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < XL; ++u) {
        const int i = tid + u * NT;  // float4 index in the staged x
        float4 v = xr[u];
        if (i >= K4) v = make_float4(0.f, 0.f, 0.f, 0.f);
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
        if constexpr (NORM) {
            const float4 g = gr[u];
            v = make_float4(v.x * (1.0f + g.x), v.y * (1.0f + g.y), v.z * (1.0f + g.z),
                            v.w * (1.0f + g.w));
        }
        // lane l's float4 p (< XV) of chunk c sits at plane p, slot l
        const int c = i / (CW / 4), o = i % (CW / 4);
        if (i < KP4) xs4[c * (CW / 4) + (o % XV) * QLM_WAVE + o / XV] = v;
    }
    float rs = 1.0f;
    if constexpr (NORM) {
        ss = block_sum(ss, bred);  // also the barrier that publishes xs4
        rs = 1.0f / sqrtf(ss / (float)K + eps);
    } else {
        __syncthreads();
    }

    float acc[T][RG];
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
#pragma unroll
        for (int i = 0; i < RG; ++i) acc[tt][i] = 0.0f;

    // x of an item is read from LDS one item ahead of its use
    float4 xq[R][XV];
    auto xread = [&](int s, int sl, int items) {
        const bool real = (ph + KS * (s % per) < nch) && s < items;
        const int c = real ? ph + KS * (s % per) : nch;
#pragma unroll
        for (int p = 0; p < XV; ++p) xq[sl][p] = xs4[c * (CW / 4) + p * QLM_WAVE + lane];
    };

    auto consume = [&](int sl) {
        float xe[EL];
#pragma unroll
        for (int p = 0; p < XV; ++p) {
            xe[4 * p] = xq[sl][p].x;
            xe[4 * p + 1] = xq[sl][p].y;
            xe[4 * p + 2] = xq[sl][p].z;
            xe[4 * p + 3] = xq[sl][p].w;
        }
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
#pragma unroll
            for (int i = 0; i < RG; ++i) {
                const uint4 q = wb[sl][tt][i];
                const uint32_t u4[4] = {q.x, q.y, q.z, q.w};
                float a = acc[tt][i];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (sizeof(WT) == 2) {
                        a = fmaf(__uint_as_float(u4[e] << 16), xe[2 * e], a);
                        a = fmaf(__uint_as_float(u4[e] & 0xffff0000u), xe[2 * e + 1], a);
                    } else {
                        a = fmaf(__uint_as_float(u4[e]), xe[e], a);
                    }
                }
                acc[tt][i] = a;
            }
    };

    auto epilogue = [&](int row, const float* v) {
        float* dst = y + row;
        if constexpr (EPI == EPI_SWIGLU)
            *dst = silu_f(v[0] * rs) * (v[1] * rs);
        else if constexpr (EPI == EPI_RESID)
            *dst += v[0] * rs;
        else
            *dst = v[0] * rs;
    };

    int par = 0;
    auto tile_end = [&](int tile) {
        if constexpr (KS == 1) {
            // whole rows in this wave: reduce inside it, lane i writes row i
            float tot[T][RG];
#pragma unroll
            for (int tt = 0; tt < T; ++tt)
#pragma unroll
                for (int i = 0; i < RG; ++i) {
                    tot[tt][i] = wave_sum(acc[tt][i]);
                    acc[tt][i] = 0.0f;
                }
#pragma unroll
            for (int i = 0; i < RG; ++i) {
                const int row = tile * RT + rg * RG + i;
                if (lane == i && row < N) {
                    float v[T];
#pragma unroll
                    for (int tt = 0; tt < T; ++tt) v[tt] = tot[tt][i];
                    epilogue(row, v);
                }
            }
        } else {
            // 16-lane sums meet in LDS: [parity][phase][half][tile row][lane group]
#pragma unroll
            for (int tt = 0; tt < T; ++tt)
#pragma unroll
                for (int i = 0; i < RG; ++i) {
                    const float v = group_sum<16>(acc[tt][i]);
                    acc[tt][i] = 0.0f;
                    if ((lane & 15) == 0) red[par][ph][tt][rg * RG + i][lane >> 4] = v;
                }
            __syncthreads();
            if (tid < RT) {
                const int row = tile * RT + tid;
                if (row < N) {
                    float v[T];
#pragma unroll
                    for (int tt = 0; tt < T; ++tt) {
                        float s = 0.0f;
#pragma unroll
                        for (int p = 0; p < KS; ++p) {
                            const float* r4 = red[par][p][tt][tid];
                            s += (r4[0] + r4[1]) + (r4[2] + r4[3]);
                        }
                        v[tt] = s;
                    }
                    epilogue(row, v);
                }
            }
            par ^= 1;  // a buffer is rewritten two tiles later, after another barrier
        }
    };

    const int my_tiles = (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int items = my_tiles * per;
    xread(0, 0, items);
#pragma unroll 1
    for (int s0 = 0; s0 < items; s0 += R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int s = s0 + r;
            xread(s + 1, (r + 1) % R, items);
            consume(r);
            issue(s + R, r);
            if (s < items && s % per == per - 1)
                tile_end((int)blockIdx.x + (s / per) * (int)gridDim.x);
        }
    }
}

struct WConfig {
    int nw, r, grid;
};

// 16 waves per workgroup (each a K slice of the tile), 6 items in flight
// per wave; about one workgroup per CU.
WConfig w_config(int N, int K) {
    const int tiles = (N + 15) / 16;
    (void)K;
    return WConfig{16, 6, tiles < 256 ? tiles : 256};
}

template <typename WT, int T, int EPI, bool NORM>
int launch_w(const WConfig& c, const float* x, int ldx, const float* rs, const WT* W, float* y,
             int ldy, int M, int N, int K, int F, hipStream_t st) {
    const int ntiles = (N + 15) / 16;
    const int grid = c.grid < ntiles ? c.grid : ntiles;
    hipLaunchKernelGGL((k_gemv_w<WT, 16, 6, T, EPI, NORM>), dim3(grid), dim3(16 * QLM_WAVE), 0,
                       st, x, ldx, rs, W, y, ldy, M, N, K, F, ntiles);
    return qlm_launch_status();
}

template <typename WT>
int w_dispatch(const float* x, int ldx, const float* norm_w, float eps, const WT* W, float* y,
               int ldy, int M, int N, int K, int epi, void* work, size_t work_bytes,
               hipStream_t st) {
    const WConfig c = w_config(N, K);
    const int F = N;
    for (int m0 = 0; m0 < M; m0 += kWRows) {  // 16 activation rows per launch
        const int mr = M - m0 < kWRows ? M - m0 : kWRows;
        const float* xs = x + (size_t)m0 * ldx;
        float* ys = y + (size_t)m0 * ldy;
        int rc;
        if (norm_w) {
            float* rs = reinterpret_cast<float*>(work);
            float* xg = rs + 64;  // 256 bytes in
            hipLaunchKernelGGL(k_w_rows, dim3(mr), dim3(kPrepT), 0, st, xs, ldx, K, norm_w, eps,
                               rs, xg);
            rc = qlm_launch_status();
            if (rc != QLM_OK) return rc;
            rc = epi == EPI_SWIGLU
                     ? launch_w<WT, 2, EPI_SWIGLU, true>(c, xg, K, rs, W, ys, ldy, mr, N, K, F, st)
                     : launch_w<WT, 1, EPI_STORE, true>(c, xg, K, rs, W, ys, ldy, mr, N, K, F, st);
        } else if (epi == EPI_RESID) {
            rc = launch_w<WT, 1, EPI_RESID, false>(c, xs, ldx, nullptr, W, ys, ldy, mr, N, K, F,
                                                   st);
        } else {
            rc = launch_w<WT, 1, EPI_STORE, false>(c, xs, ldx, nullptr, W, ys, ldy, mr, N, K, F,
                                                   st);
        }
        if (rc != QLM_OK) return rc;
    }
    (void)work_bytes;
    return QLM_OK;
}

// ---- one-row launch shapes ---------------------------------------------------
struct WvConfig {
    int nw, rg, ks, r, grid;
};

// x staged by XL float4 loads per thread: 2 or 5 (up to 8 or 20 columns of
// the padded x per thread), 0 if K needs more (the matrix-core kernel then
// serves).
int wv_xl(int K, int elt, int nw) {
    const int cw = QLM_WAVE * (16 / elt);
    const int kp4 = ((K + cw - 1) / cw + 1) * (cw / 4);  // chunks + the zero chunk
    const int nt = nw * QLM_WAVE;
    return kp4 <= 2 * nt ? 2 : kp4 <= 5 * nt ? 5 : 0;
}

template <typename WT, int NW, int RG, int KS, int R, int EPI, bool NORM>
int launch_wv_e(const WvConfig& c, int xl, const float* x, const float* gain, float eps,
                const WT* W, float* y, int N, int K, hipStream_t st) {
    constexpr int RT = NW / KS * RG;
    const int ntiles = (N + RT - 1) / RT;
    const int grid = c.grid > 0 && c.grid < ntiles ? c.grid : ntiles;
    constexpr int CW = QLM_WAVE * (16 / (int)sizeof(WT));
    const size_t lds = (size_t)((K + CW - 1) / CW + 1) * CW * sizeof(float);
    if (xl == 2)
        hipLaunchKernelGGL((k_gemv_wv<WT, NW, RG, KS, R, EPI, NORM, 2>), dim3(grid),
                           dim3(NW * QLM_WAVE), lds, st, x, gain, eps, W, y, N, K, N, ntiles);
    else
        hipLaunchKernelGGL((k_gemv_wv<WT, NW, RG, KS, R, EPI, NORM, 5>), dim3(grid),
                           dim3(NW * QLM_WAVE), lds, st, x, gain, eps, W, y, N, K, N, ntiles);
    return qlm_launch_status();
}

template <typename WT, int NW, int RG, int KS, int R>
int launch_wv_t(const WvConfig& c, const float* x, const float* gain, float eps, const WT* W,
                float* y, int N, int K, int epi, hipStream_t st) {
    const int xl = wv_xl(K, (int)sizeof(WT), NW);
    constexpr int CW = QLM_WAVE * (16 / (int)sizeof(WT));
    if (!xl || ((size_t)K + 2 * CW) * sizeof(float) > 65536) return QLM_ERR_SHAPE;
    if (epi == EPI_SWIGLU)
        return launch_wv_e<WT, NW, RG, KS, R, EPI_SWIGLU, true>(c, xl, x, gain, eps, W, y, N, K,
                                                                 st);
    if (epi == EPI_RESID)
        return launch_wv_e<WT, NW, RG, KS, R, EPI_RESID, false>(c, xl, x, gain, eps, W, y, N, K,
                                                                 st);
    if (gain)
        return launch_wv_e<WT, NW, RG, KS, R, EPI_STORE, true>(c, xl, x, gain, eps, W, y, N, K,
                                                                st);
    return launch_wv_e<WT, NW, RG, KS, R, EPI_STORE, false>(c, xl, x, gain, eps, W, y, N, K, st);
}

// The built shapes (waves, rows per wave, K phases, ring).
template <typename WT>
int launch_wv(const WvConfig& c, const float* x, const float* gain, float eps, const WT* W,
              float* y, int N, int K, int epi, hipStream_t st) {
#define QLM_WV(NW_, RG_, KS_, R_)                                                          \
    if (c.nw == NW_ && c.rg == RG_ && c.ks == KS_ && c.r == R_)                            \
        return launch_wv_t<WT, NW_, RG_, KS_, R_>(c, x, gain, eps, W, y, N, K, epi, st);
    QLM_WV(4, 1, 1, 4)
    QLM_WV(8, 1, 1, 4)
    QLM_WV(4, 2, 1, 3)
    QLM_WV(8, 2, 1, 3)
    QLM_WV(4, 4, 1, 2)
    QLM_WV(8, 2, 4, 3)
    QLM_WV(8, 1, 4, 4)
    QLM_WV(16, 1, 8, 4)
#undef QLM_WV
    return QLM_ERR_ARG;
}

// Measured per projection of the 4B model (bf16 rows; the tied lm_head is
// the fp32 embedding table), graph-replayed over rotating weight copies.
struct WvTuned {
    int N, K, epi, elt;
    WvConfig c;
};
constexpr WvTuned kWvTuned[] = {
    {9728, 2560, EPI_SWIGLU, 2, {4, 1, 1, 4, 768}},  // gate/up: 19.2 us, 5.2 TB/s
    {2560, 9728, EPI_RESID, 2, {8, 2, 4, 3, 256}},   // down: 11.4 us, 4.4 TB/s
    {8224, 2560, EPI_STORE, 2, {4, 2, 1, 3, 512}},   // DeltaNet in-projection: 10.0 us
    {5120, 2560, EPI_STORE, 2, {4, 2, 1, 3, 512}},   // attention q/k/v: 7.6 us
    {2560, 2048, EPI_RESID, 2, {4, 4, 1, 2, 160}},   // output projections: 5.2 us
    {151936, 2560, EPI_STORE, 4, {4, 2, 1, 3, 256}}, // lm_head (fp32): 240 us, 6.5 TB/s
};

WvConfig wv_config(int N, int K, int epi, int elt) {
    for (const WvTuned& t : kWvTuned)
        if (t.N == N && t.K == K && t.epi == epi && t.elt == elt) return t.c;
    return WvConfig{4, 2, 1, 3, 512};
}

template <typename WT>
int wv_auto(const float* x, const float* gain, float eps, const WT* W, float* y, int N, int K,
            int epi, hipStream_t st) {
    return launch_wv<WT>(wv_config(N, K, epi, (int)sizeof(WT)), x, gain, eps, W, y, N, K, epi,
                         st);
}

}  // namespace

extern "C" int qlm_gemv_w_config(const float* x, const float* norm_w, float eps, const void* w,
                                 int w_bf16, float* y, int N, int K, int epilogue, int waves,
                                 int rows_per_wave, int k_phases, int ring, int grid,
                                 void* stream) {
    if (!x || !w || !y || N <= 0 || K <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    if (epilogue == EPI_SWIGLU && !norm_w) return QLM_ERR_ARG;
    if (epilogue == EPI_RESID && norm_w) return QLM_ERR_ARG;
    if (K % 16 != 0) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)norm_w) & 15u) return QLM_ERR_SHAPE;
    const WvConfig c{waves, rows_per_wave, k_phases, ring, grid};
    hipStream_t st = as_stream(stream);
    return w_bf16 ? launch_wv<uint16_t>(c, x, norm_w, eps, static_cast<const uint16_t*>(w), y, N,
                                        K, epilogue, st)
                  : launch_wv<float>(c, x, norm_w, eps, static_cast<const float*>(w), y, N, K,
                                     epilogue, st);
}

extern "C" size_t qlm_matmul_w_workspace_bytes(int K) {
    if (K <= 0) return 0;
    return 256 + (size_t)kWRows * K * sizeof(float);
}

extern "C" int qlm_matmul_w(const float* x, int ldx, const float* norm_w, float eps,
                            const void* w, int w_bf16, float* y, int ldy, int M, int N, int K,
                            int epilogue, void* work, size_t work_bytes, void* stream) {
    if (!x || !w || !y || M <= 0 || N <= 0 || K <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    if (epilogue == EPI_SWIGLU && !norm_w) return QLM_ERR_ARG;  // only the fused-norm form
    if (epilogue == EPI_RESID && norm_w) return QLM_ERR_ARG;
    if (K % 16 != 0 || ldx < K || ldy < N || ldx % 4 != 0) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)norm_w) & 15u) return QLM_ERR_SHAPE;
    if (norm_w && (!work || work_bytes < qlm_matmul_w_workspace_bytes(K) ||
                   ((uintptr_t)work & 15u)))
        return QLM_ERR_ARG;
    hipStream_t st = as_stream(stream);
    if (w_bf16 && M > kWRows && K % 32 == 0)  // bf16 rows, many rows: the tiled GEMM
        return qlm_matmul_bf16(x, ldx, norm_w, eps, static_cast<const uint16_t*>(w), y, ldy, M, N,
                               K, epilogue, work, work_bytes, stream);
    if (M == 1) {  // one row: the vector-ALU GEMV (QLM_ERR_SHAPE: K too long for it)
        const int rc = w_bf16 ? wv_auto<uint16_t>(x, norm_w, eps, static_cast<const uint16_t*>(w),
                                                  y, N, K, epilogue, st)
                              : wv_auto<float>(x, norm_w, eps, static_cast<const float*>(w), y,
                                               N, K, epilogue, st);
        if (rc != QLM_ERR_SHAPE) return rc;
    }
    return w_bf16 ? w_dispatch<uint16_t>(x, ldx, norm_w, eps, static_cast<const uint16_t*>(w),
                                         y, ldy, M, N, K, epilogue, work, work_bytes, st)
                  : w_dispatch<float>(x, ldx, norm_w, eps, static_cast<const float*>(w), y, ldy,
                                      M, N, K, epilogue, work, work_bytes, st);
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_gemm_w() {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(k_w_rows));
}
