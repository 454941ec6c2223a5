// Batched decode matmul (2 <= M <= 16 activation rows) on the bf16 matrix
// cores, streaming the tile-major int8 weights of the one-row GEMV
// (gemv.hip, k_mx_swizzle) straight from registers:
//   y[m, n] = sum_k x[m, k] * q[n, k] * s[n, k / 32]
// math::matmul's int8 branch with M rows (math_ops.cpp:845-871), which
// batched decode runs once per projection and step.
//
// Arithmetic (as gemm.hip's split-K path): int8 weights are exact in bf16,
// each activation is split into bf16 hi + lo (RNE both, |x - hi - lo| <=
// 2^-17 |x|), products and sums run in fp32 in v_mfma_f32_16x16x32_bf16,
// and each 32-column group's product is scaled by s[n, group] in fp32.
//
// Operands. A weight fragment (16 rows x 64 columns, 1 KB) gives lane
// l = 16q + n row n, columns 16q .. 16q + 15. One v_permlane32_swap per
// dword pair regroups it so that the first two dwords of every lane hold
// group 0 (lane quarter q: columns c0(q) .. +7, c0 = 0, 16, 8, 24) and the
// last two group 1 (32 + c0(q) .. +7): each group is then one MFMA k-step of
// 32, B = weights (column n = weight row), A = the activation rows over the
// same column order, D[m][n] in lane (m / 4, n). Lane (q, m) loads its
// activation columns with the weights (times 1 + gain for a deferred
// RMSNorm) and splits them into bf16 hi and lo once per block: each block
// is converted by one wave and serves the NT tiles.
//
// Work split. A workgroup owns NT 16-row tiles and one K slice of the 64-
// column blocks; wave w takes blocks w, w + NW, ... of the slice, each
// block's NT weight fragments, their group scales and the activation
// columns streaming through a ring of P register slots; the waves' partial tiles meet in LDS and the
// slice's partial sums go to part[ks, m, n]; k_mm_reduce sums the slices in
// order and applies the epilogue (and the RMSNorm's 1/rms).

#include "common.hpp"
#include "mm_reduce.hpp"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };
constexpr int kMaxRowsT = 16;
constexpr int kMaxSliceBlocks = 64;  // blocks of one K slice

// eight fp32 as bf16 (RNE) hi and lo planes, x = hi + lo + O(2^-17 |x|)
__device__ __forceinline__ void split8(const float (&v)[8], uint4& hi, uint4& lo) {
    unsigned h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __bf16 a = (__bf16)v[2 * i], b = (__bf16)v[2 * i + 1];
        const __bf16 la = (__bf16)(v[2 * i] - (float)a), lb = (__bf16)(v[2 * i + 1] - (float)b);
        h[i] = (unsigned)__builtin_bit_cast(unsigned short, a) |
               ((unsigned)__builtin_bit_cast(unsigned short, b) << 16);
        l[i] = (unsigned)__builtin_bit_cast(unsigned short, la) |
               ((unsigned)__builtin_bit_cast(unsigned short, lb) << 16);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// eight int8 (two dwords, little-endian) as bf16 (exact)
__device__ __forceinline__ bf16x8 i8x8_bf16(unsigned w0, unsigned w1) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r[i] = (__bf16)(float)(signed char)(w0 >> (8 * i));
        r[4 + i] = (__bf16)(float)(signed char)(w1 >> (8 * i));
    }
    return r;
}

template <int NW, int NT, int P, bool NORM>
__global__ __launch_bounds__(NW * QLM_WAVE) void k_mm_t(
    const float* __restrict__ x, int ldx, const float* __restrict__ gain,
    const int8_t* __restrict__ qz, const float* __restrict__ sz, float* __restrict__ part,
    int M, int NR, int rows_half, int tiles_half, int tiles_total, int nblk, int bps) {
    constexpr int NTH = NW * QLM_WAVE;
    __shared__ f32x4 red[NW * NT * QLM_WAVE];  // the waves' partial tiles

    const int tid = threadIdx.x, lane = tid & (QLM_WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / QLM_WAVE);
    const int tg = blockIdx.x, ks = blockIdx.y;
    const int b0 = ks * bps;
    const int nb = min(bps, nblk - b0);  // blocks of this slice
    const int per = (nb + NW - 1) / NW;  // items per wave (the last ones may be masked)
    // this lane's activation row and column offset within a group:
    // quarter q holds columns c0(q) .. +7, c0 = 0, 16, 8, 24
    const int q = lane >> 4;
    const float* xrow = x + (size_t)min(lane & 15, M - 1) * ldx + (q & 1) * 16 + (q >> 1) * 8;
    const float* grow = gain + (q & 1) * 16 + (q >> 1) * 8;

    // ring of P items (item j: local block w + NW j): NT weight fragments,
    // their group scales and this lane's 2 x 8 activation columns (+ gains).
    // Every load is unconditional (clamped), so none waits behind a branch.
    uint4 wq[P][NT];
    float ws0[P][NT], ws1[P][NT];
    float4 xa[P][4], ga[P][NORM ? 4 : 1];
    auto issue = [&](int j, int sl) {
        const int lb = min(w + NW * j, nb - 1);
        const int b = b0 + lb;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tile = min(tg * NT + t, tiles_total - 1);
            const size_t fb = (size_t)tile * nblk + b;
            wq[sl][t] = *reinterpret_cast<const uint4*>(qz + (fb * QLM_WAVE + lane) * 16);
            ws0[sl][t] = sz[fb * 32 + (lane & 15)];
            ws1[sl][t] = sz[fb * 32 + 16 + (lane & 15)];
        }
        const float4* xp = reinterpret_cast<const float4*>(xrow + 64 * b);
        xa[sl][0] = xp[0];
        xa[sl][1] = xp[1];
        xa[sl][2] = xp[8];  // + 32 columns: group 1
        xa[sl][3] = xp[9];
        if constexpr (NORM) {
            const float4* gp = reinterpret_cast<const float4*>(grow + 64 * b);
            ga[sl][0] = gp[0];
            ga[sl][1] = gp[1];
            ga[sl][2] = gp[8];
            ga[sl][3] = gp[9];
        }
    };
#pragma unroll
    for (int r = 0; r < P; ++r) issue(r, r);

    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](int j, int sl) {
        const bool real = w + NW * j < nb;  // masked items add zeros
        uint4 ah[2], al[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            float4 u = xa[sl][2 * g], v = xa[sl][2 * g + 1];
            if constexpr (NORM) {
                const float4 gu = ga[sl][2 * g], gv = ga[sl][2 * g + 1];
                u = make_float4(u.x * (1.0f + gu.x), u.y * (1.0f + gu.y), u.z * (1.0f + gu.z),
                                u.w * (1.0f + gu.w));
                v = make_float4(v.x * (1.0f + gv.x), v.y * (1.0f + gv.y), v.z * (1.0f + gv.z),
                                v.w * (1.0f + gv.w));
            }
            float e[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = real ? e[i] : 0.0f;
            split8(e, ah[g], al[g]);
        }
        const bf16x8 a0h = __builtin_bit_cast(bf16x8, ah[0]), a0l = __builtin_bit_cast(bf16x8, al[0]);
        const bf16x8 a1h = __builtin_bit_cast(bf16x8, ah[1]), a1l = __builtin_bit_cast(bf16x8, al[1]);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint4 v = wq[sl][t];
            // upper half of (x, y) <-> lower half of (z, w): group 0 in x, y
            const auto s0 = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
            const bf16x8 b0v = i8x8_bf16(s0[0], s1[0]);
            const bf16x8 b1v = i8x8_bf16(s0[1], s1[1]);
            f32x4 t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0h, b0v, f32x4{0.f, 0.f, 0.f, 0.f},
                                                               0, 0, 0);
            t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0l, b0v, t0, 0, 0, 0);
            f32x4 t1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1h, b1v, f32x4{0.f, 0.f, 0.f, 0.f},
                                                               0, 0, 0);
            t1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1l, b1v, t1, 0, 0, 0);
            const float s0f = ws0[sl][t], s1f = ws1[sl][t];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(t1[i], s1f, fmaf(t0[i], s0f, acc[t][i]));
        }
    };

#pragma unroll 1
    for (int j0 = 0; j0 < per; j0 += P) {
#pragma unroll
        for (int r = 0; r < P; ++r) {
            consume(j0 + r, r);
            issue(j0 + r + P, r);
        }
    }

    // waves' partial tiles meet in LDS; lane l holds D[4 (l / 16) + i][l % 16]
#pragma unroll
    for (int t = 0; t < NT; ++t) red[(w * NT + t) * QLM_WAVE + lane] = acc[t];
    __syncthreads();
    for (int o = tid; o < NT * QLM_WAVE * 4; o += NTH) {
        const int t = o / (QLM_WAVE * 4), rem = o % (QLM_WAVE * 4);
        const int l2 = rem >> 2, i = rem & 3;
        const int m = 4 * (l2 >> 4) + i, n = l2 & 15;
        const int tile = tg * NT + t;
        if (m >= M || tile >= tiles_total) continue;
        const int half = tile / tiles_half, th = tile % tiles_half;
        const int rh = th * 16 + n;
        if (rh >= rows_half) continue;
        float s = 0.0f;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) s += red[(ww * NT + t) * QLM_WAVE + l2][i];
        part[((size_t)ks * M + m) * NR + (size_t)half * rows_half + rh] = s;
    }
}

struct TConfig {
    int nw, nt, p, ks;
};

// Launch shapes measured per 4B projection at M = 16 (graph replays over
// rotating weight copies, the ordered reduction included); other shapes take
// 4 waves x 8 tiles, one ring slot, and the fewest K slices (while every
// wave keeps a block) that give ~2 workgroups per CU.
struct TTuned {
    int N, K, epi;
    TConfig c;
};
constexpr TTuned kTTuned[] = {
    {9728, 2560, EPI_SWIGLU, {4, 8, 1, 5}},  // gate/up: 21.5 us (split-K 28.2)
    {2560, 9728, EPI_RESID, {8, 8, 1, 10}},  // down: 13.2 us (16.2)
    {8224, 2560, EPI_STORE, {8, 8, 1, 3}},   // DeltaNet in-projection: 15.4 us (17.5)
    {5120, 2560, EPI_STORE, {8, 4, 2, 3}},   // attention q/k/v: 11.3 us (14.0)
    {2560, 2048, EPI_RESID, {8, 2, 2, 2}},   // output projections: 7.2 us (7.9)
    {151936, 2560, EPI_STORE, {4, 8, 1, 1}}, // lm_head: 110 us (180)
};

TConfig t_config(int N, int K, int epi) {
    for (const TTuned& t : kTTuned)
        if (t.N == N && t.K == K && t.epi == epi) return t.c;
    TConfig c{4, 8, 1, 1};
    const int tiles_total = (epi == EPI_SWIGLU ? 2 : 1) * ((N + 15) / 16);
    const int groups = (tiles_total + c.nt - 1) / c.nt;
    const int nblk = K / 64;
    int ks = (nblk + kMaxSliceBlocks - 1) / kMaxSliceBlocks;
    while (groups * ks < 512 && (nblk + ks) / (ks + 1) >= c.nw) ++ks;
    c.ks = ks;
    return c;
}

// slices a launch shape really uses (ceil over the blocks per slice)
int t_slices(const TConfig& c, int K) {
    const int nblk = K / 64;
    const int bps = (nblk + c.ks - 1) / c.ks;
    return (nblk + bps - 1) / bps;
}

template <int NW, int NT, int P, bool NORM>
void launch_t(int ks, const float* x, int ldx, const float* gain, const int8_t* qz,
              const float* sz, float* part, int M, int NR, int rows_half, int tiles_half,
              int tiles_total, int nblk, hipStream_t st) {
    const int bps = (nblk + ks - 1) / ks;
    const int groups = (tiles_total + NT - 1) / NT;
    hipLaunchKernelGGL((k_mm_t<NW, NT, P, NORM>), dim3(groups, (nblk + bps - 1) / bps),
                       dim3(NW * QLM_WAVE), 0, st, x, ldx, gain, qz, sz, part, M, NR,
                       rows_half, tiles_half, tiles_total, nblk, bps);
}

// built shapes (waves, tiles per workgroup, ring slots)
template <bool NORM>
int launch_t_shape(const TConfig& c, const float* x, int ldx, const float* gain,
                   const int8_t* qz, const float* sz, float* part, int M, int NR, int rows_half,
                   int tiles_half, int tiles_total, int nblk, hipStream_t st) {
#define QLM_T(NW_, NT_, P_)                                                                    \
    if (c.nw == NW_ && c.nt == NT_ && c.p == P_) {                                             \
        launch_t<NW_, NT_, P_, NORM>(c.ks, x, ldx, gain, qz, sz, part, M, NR, rows_half,        \
                                     tiles_half, tiles_total, nblk, st);                        \
        return qlm_launch_status();                                                            \
    }
    QLM_T(4, 4, 2)
    QLM_T(4, 2, 3)
    QLM_T(8, 2, 2)
    QLM_T(8, 4, 2)
    QLM_T(4, 8, 1)
    QLM_T(4, 8, 2)
    QLM_T(8, 8, 1)
#undef QLM_T
    return QLM_ERR_ARG;
}

int t_run(const TConfig& c, const float* x, int ldx, const float* norm_w, float eps,
          const int8_t* qz, const float* sz, float* y, int ldy, int M, int N, int K, int epi,
          void* work, size_t work_bytes, hipStream_t st) {
    const int halves = epi == EPI_SWIGLU ? 2 : 1;
    const int NR = halves * N;
    const int tiles_half = (N + 15) / 16, tiles_total = halves * tiles_half;
    const int nblk = K / 64;
    const int bps = (nblk + c.ks - 1) / c.ks;
    if (c.ks < 1 || bps > kMaxSliceBlocks || bps < 1) return QLM_ERR_SHAPE;
    const int ks = (nblk + bps - 1) / bps;
    if (work_bytes < (size_t)ks * M * NR * sizeof(float)) return QLM_ERR_ARG;
    float* part = static_cast<float*>(work);
    const int rc = norm_w ? launch_t_shape<true>(c, x, ldx, norm_w, qz, sz, part, M, NR, N,
                                                 tiles_half, tiles_total, nblk, st)
                          : launch_t_shape<false>(c, x, ldx, nullptr, qz, sz, part, M, NR, N,
                                                  tiles_half, tiles_total, nblk, st);
    if (rc != QLM_OK) return rc;
    const dim3 grid((N + kReduceThreads - 1) / kReduceThreads, M);
    if (epi == EPI_SWIGLU)
        hipLaunchKernelGGL((k_mm_reduce<MMR_SWIGLU, true>), grid, dim3(kReduceThreads), 0, st,
                           part, ks, M, NR, N, y, ldy, x, ldx, K, eps);
    else if (epi == EPI_RESID)
        hipLaunchKernelGGL((k_mm_reduce<MMR_RESID, false>), grid, dim3(kReduceThreads), 0, st,
                           part, ks, M, NR, N, y, ldy, x, ldx, K, eps);
    else if (norm_w)
        hipLaunchKernelGGL((k_mm_reduce<MMR_STORE, true>), grid, dim3(kReduceThreads), 0, st,
                           part, ks, M, NR, N, y, ldy, x, ldx, K, eps);
    else
        hipLaunchKernelGGL((k_mm_reduce<MMR_STORE, false>), grid, dim3(kReduceThreads), 0, st,
                           part, ks, M, NR, N, y, ldy, x, ldx, K, eps);
    return qlm_launch_status();
}

int t_check(const float* x, int ldx, const float* norm_w, const int8_t* qz, const float* sz,
            int group, float* y, int ldy, int M, int N, int K, int epi) {
    if (!x || !qz || !sz || !y || M < 1 || N < 1 || K < 64) return QLM_ERR_ARG;
    if (epi < EPI_STORE || epi > EPI_SWIGLU) return QLM_ERR_ARG;
    if (epi == EPI_SWIGLU && !norm_w) return QLM_ERR_ARG;
    if (epi == EPI_RESID && norm_w) return QLM_ERR_ARG;
    if (group != 32 || K % 64 != 0 || M > kMaxRowsT) return QLM_ERR_SHAPE;
    if (ldx < K || ldx % 4 != 0 || ldy < N) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)qz | (uintptr_t)norm_w) & 15u) return QLM_ERR_SHAPE;
    return QLM_OK;
}

}  // namespace

extern "C" size_t qlm_matmul_i8_t_workspace_bytes(int M, int N, int K, int epilogue) {
    if (M < 1 || N < 1 || K < 64) return 0;
    const int halves = epilogue == EPI_SWIGLU ? 2 : 1;
    const TConfig c = t_config(N, K, epilogue);
    return (size_t)t_slices(c, K) * M * halves * N * sizeof(float);
}

extern "C" int qlm_matmul_i8_t_config(const float* x, int ldx, const float* norm_w, float eps,
                                      const int8_t* q_tiles, const float* s_tiles, int group,
                                      float* y, int ldy, int M, int N, int K, int epilogue,
                                      int waves, int tiles, int ring, int k_slices, void* work,
                                      size_t work_bytes, void* stream) {
    const int rc = t_check(x, ldx, norm_w, q_tiles, s_tiles, group, y, ldy, M, N, K, epilogue);
    if (rc != QLM_OK) return rc;
    if (!work) return QLM_ERR_ARG;
    return t_run(TConfig{waves, tiles, ring, k_slices}, x, ldx, norm_w, eps, q_tiles, s_tiles, y,
                 ldy, M, N, K, epilogue, work, work_bytes, as_stream(stream));
}

extern "C" int qlm_matmul_i8_t(const float* x, int ldx, const float* norm_w, float eps,
                               const int8_t* q_tiles, const float* s_tiles, int group, float* y,
                               int ldy, int M, int N, int K, int epilogue, void* work,
                               size_t work_bytes, void* stream) {
    const int rc = t_check(x, ldx, norm_w, q_tiles, s_tiles, group, y, ldy, M, N, K, epilogue);
    if (rc != QLM_OK) return rc;
    if (!work) return QLM_ERR_ARG;
    const TConfig c = t_config(N, K, epilogue);
    return t_run(c, x, ldx, norm_w, eps, q_tiles, s_tiles, y, ldy, M, N, K, epilogue, work,
                 work_bytes, as_stream(stream));
}
