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

}  // namespace

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
    return w_bf16 ? w_dispatch<uint16_t>(x, ldx, norm_w, eps, static_cast<const uint16_t*>(w),
                                         y, ldy, M, N, K, epilogue, work, work_bytes, st)
                  : w_dispatch<float>(x, ldx, norm_w, eps, static_cast<const float*>(w), y, ldy,
                                      M, N, K, epilogue, work, work_bytes, st);
}
