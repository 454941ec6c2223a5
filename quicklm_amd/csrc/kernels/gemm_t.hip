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
constexpr int kMaxGainK = 4096;  // K of the whole-K form's staged RMSNorm gains
// Word 3 of a gfx9 buffer resource for untyped (raw) loads.
constexpr int kBufferWord3 = 0x00020000;
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
    // every argument read in one batch (otherwise the compiler reads some,
    // waits, branches and reads the rest: a second round trip)
    asm volatile("" ::"s"(x), "s"(ldx), "s"(gain), "s"(qz), "s"(sz), "s"(part), "s"(M), "s"(NR),
                 "s"(rows_half), "s"(tiles_half), "s"(tiles_total), "s"(nblk), "s"(bps));
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

// Whole-K form for K <= 64 * NW * PX (no partial sums, no second launch):
// the NW waves of a workgroup split K (wave w takes the blocks w, w + NW,
// ..., PX of them) and the workgroup walks tile groups grid-stride, NTH
// 16-row tiles per half at a time (both halves of a [gate; up] matrix). A
// wave's blocks are the same for every tile group, so its activation
// columns are loaded, multiplied by 1 + gain (deferred RMSNorm) and split
// into bf16 hi + lo once, at kernel start, and stay in registers; the ring
// holds weight fragments and their group scales only, one slot per block,
// each slot refilled with the next group's fragment as soon as it is
// consumed (the loads of the first group are issued before the activation
// arithmetic). At a group's end the waves' partial tiles meet in LDS
// (double-buffered by group parity) and every thread of the workgroup takes
// a share of the outputs: partials summed in wave order, then 1/rms (from
// the waves' sums of squares of x), the epilogue and the store.
// K-sliced use (part non-null, gridDim.y slices of bps blocks): the same
// arithmetic over slice blockIdx.y's blocks only, the waves' sums written
// raw to part[slice, m, n] (both halves of a SwiGLU matrix, the up rows at
// n + N) for k_mm_reduce to add in slice order and finish (RMSNorm
// included), for K whose activation does not fit the registers at once.
template <int NW, int NTH, int PX, bool NORM, int EPI>
__global__ __launch_bounds__(NW * QLM_WAVE) void k_mm_b(
    const float* __restrict__ x, int ldx, const float* __restrict__ gain, float eps,
    const int8_t* __restrict__ qz, const float* __restrict__ sz, float* __restrict__ y, int ldy,
    int M, int N, int tiles_half, int nblk, int bps, float* __restrict__ part) {
    // every argument read in one batch, as in k_mm_t
    asm volatile("" ::"s"(x), "s"(ldx), "s"(gain), "s"(eps), "s"(qz), "s"(sz), "s"(y), "s"(ldy),
                 "s"(M), "s"(N), "s"(tiles_half), "s"(nblk), "s"(bps), "s"(part));
    constexpr int H2 = EPI == EPI_SWIGLU ? 2 : 1;
    constexpr int NT = NTH * H2;  // fragments per ring slot
    constexpr int NTHR = NW * QLM_WAVE;
    __shared__ f32x4 red[2][NW][NT][QLM_WAVE];
    __shared__ float rsum[NW][kMaxRowsT];
    __shared__ float4 gsh[NORM ? kMaxGainK / 4 : 1];  // 1 + gain, staged once

    const int tid = threadIdx.x, lane = tid & (QLM_WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / QLM_WAVE);
    const int q = lane >> 4, mr = lane & 15;
    const int ngroups = (tiles_half + NTH - 1) / NTH;
    // this workgroup's blocks: b0 .. b0 + nb - 1 (all of K when not sliced)
    const int b0 = blockIdx.y * bps;
    const int nb = min(bps, nblk - b0);
    // this wave's last block (a wave past the slice's last block repeats
    // block nb - 1, which then meets zero activations)
    const int blast = w < nb ? nb - 1 - ((nb - 1 - w) % NW) : nb - 1;

    // ---- activation of this wave's blocks: lane (q, m) holds row m's columns
    // c0(q) .. +7 and 32 + c0(q) .. +7 of each block (c0 = 0, 16, 8, 24), the
    // order the weights take after the lane swaps. Unconditional loads (row
    // and block clamped), issued before the weight ring.
    // The RMSNorm gains are the same for every row: the workgroup stages
    // 1 + gain in LDS once (kGainPer float4 per thread) instead of every
    // lane holding its columns' gains in registers.
    const int coff = (q & 1) * 16 + (q >> 1) * 8;
    const int K4 = nblk * 16;
    constexpr int kGainPer = NORM ? (kMaxGainK / 4 + NTHR - 1) / NTHR : 1;
    float4 gl[kGainPer];
    if constexpr (NORM) {
#pragma unroll
        for (int j = 0; j < kGainPer; ++j)
            gl[j] = reinterpret_cast<const float4*>(gain)[min(tid + j * NTHR, K4 - 1)];
    }
    // Operands are read through buffer resources: the per-lane part of each
    // address is a constant register offset and the rest a wave-uniform
    // scalar offset, so no vector arithmetic is spent on addresses (and a
    // read past a resource's extent returns zero instead of faulting).
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x), 0, ((M - 1) * ldx + nblk * 64) * 4, kBufferWord3);
    const int xoff = (min(mr, M - 1) * ldx + coff) * 4;
    float4 xa[PX][4];
#pragma unroll
    for (int u = 0; u < PX; ++u) {
        const int b = b0 + min(w + NW * u, nb - 1);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            xa[u][j] = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(rx, xoff, 256 * b + 16 * (j & 1) +
                                                                            128 * (j >> 1), 0));
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- weight ring: slot u holds block w + NW u of the current group's
    // NT tiles (tile index clamped for a ragged last group; its rows are not
    // stored)
    const int nfrag = H2 * tiles_half * nblk;
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(qz), 0, nfrag * 1024, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(sz), 0, nfrag * 128, kBufferWord3);
    uint4 wq[PX][NT];
    float s0[PX][NT], s1[PX][NT];
    auto issue = [&](int g, int u) {
        const int b = min(w + NW * u, blast);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int th = min(g * NTH + (t % NTH), tiles_half - 1);
            const int fb = (th + (t / NTH) * tiles_half) * nblk + b0 + b;
            wq[u][t] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, lane * 16, fb * 1024, 0));
            s0[u][t] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rs, mr * 4, fb * 128, 0));
            s1[u][t] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rs, 64 + mr * 4, fb * 128, 0));
        }
    };
    int g = blockIdx.x;
    const int G = (int)gridDim.x;
#pragma unroll
    for (int u = 0; u < PX; ++u) issue(g, u);

    if constexpr (NORM) {
#pragma unroll
        for (int j = 0; j < kGainPer; ++j) {
            // unconditional store (entries past K hold a clamped copy, never
            // read; the mask is the identity for tid < NTHR): under a branch
            // the compiler sinks the gain load into it, behind the weight
            // ring, and then waits for the whole ring
            const int i = (tid + j * NTHR) & (kMaxGainK / 4 - 1);
            gsh[i] = make_float4(1.0f + gl[j].x, 1.0f + gl[j].y, 1.0f + gl[j].z, 1.0f + gl[j].w);
        }
        __syncthreads();
    }

    // ---- split the activation once (zero past K and past row M - 1)
    uint4 xh[PX][2], xl[PX][2];
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < PX; ++u) {
        const bool real = w + NW * u < nb && mr < M;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float4 a = xa[u][2 * h], c = xa[u][2 * h + 1];
            if (!real) {
                a = make_float4(0.f, 0.f, 0.f, 0.f);
                c = a;
            }
            if constexpr (NORM) {
                ss = fmaf(a.x, a.x, ss);
                ss = fmaf(a.y, a.y, ss);
                ss = fmaf(a.z, a.z, ss);
                ss = fmaf(a.w, a.w, ss);
                ss = fmaf(c.x, c.x, ss);
                ss = fmaf(c.y, c.y, ss);
                ss = fmaf(c.z, c.z, ss);
                ss = fmaf(c.w, c.w, ss);
                const int gi = (coff + 64 * (b0 + min(w + NW * u, nb - 1))) / 4 + 8 * h;
                const float4 ha = gsh[gi], hc = gsh[gi + 1];
                a = make_float4(a.x * ha.x, a.y * ha.y, a.z * ha.z, a.w * ha.w);
                c = make_float4(c.x * hc.x, c.y * hc.y, c.z * hc.z, c.w * hc.w);
            }
            const float e[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
            split8(e, xh[u][h], xl[u][h]);
        }
    }
    if constexpr (NORM) {
        // row m's sum over the wave's columns: the four quarters of the wave
        ss += __shfl_xor(ss, 16, QLM_WAVE);
        ss += __shfl_xor(ss, 32, QLM_WAVE);
        if (lane < kMaxRowsT) rsum[w][lane] = ss;
    }

    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int u) {
        const bf16x8 a0h = __builtin_bit_cast(bf16x8, xh[u][0]);
        const bf16x8 a0l = __builtin_bit_cast(bf16x8, xl[u][0]);
        const bf16x8 a1h = __builtin_bit_cast(bf16x8, xh[u][1]);
        const bf16x8 a1l = __builtin_bit_cast(bf16x8, xl[u][1]);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint4 v = wq[u][t];
            // upper half of (x, y) <-> lower half of (z, w): group 0 in x, y
            const auto p0 = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
            const auto p1 = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
            const bf16x8 b0v = i8x8_bf16(p0[0], p1[0]);
            const bf16x8 b1v = i8x8_bf16(p0[1], p1[1]);
            f32x4 t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0h, b0v, f32x4{0.f, 0.f, 0.f, 0.f},
                                                               0, 0, 0);
            t0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0l, b0v, t0, 0, 0, 0);
            f32x4 t1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1h, b1v, f32x4{0.f, 0.f, 0.f, 0.f},
                                                               0, 0, 0);
            t1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1l, b1v, t1, 0, 0, 0);
            const float f0 = s0[u][t], f1 = s1[u][t];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(t1[i], f1, fmaf(t0[i], f0, acc[t][i]));
        }
    };

    const int K = nblk * 64;
    int par = 0;
    for (;;) {
        const int next = g + G;
        if (next < ngroups) {
#pragma unroll
            for (int u = 0; u < PX; ++u) {
                consume(u);
                issue(next, u);
            }
        } else {
#pragma unroll
            for (int u = 0; u < PX; ++u) consume(u);
        }
        // the waves' partial tiles meet in LDS; lane l holds D[4 (l / 16) + i][l % 16]
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            red[par][w][t][lane] = acc[t];
            acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        __syncthreads();
        for (int o = tid; o < NTH * QLM_WAVE * 4; o += NTHR) {
            const int t = o / (QLM_WAVE * 4), rem = o % (QLM_WAVE * 4);
            const int l2 = rem >> 2, i = rem & 3;
            const int m = 4 * (l2 >> 4) + i, n = l2 & 15;
            const int th = g * NTH + t;
            const int row = th * 16 + n;
            if (m >= M || th >= tiles_half || row >= N) continue;
            float v = 0.0f, up = 0.0f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww) {
                v += red[par][ww][t][l2][i];
                if constexpr (EPI == EPI_SWIGLU) up += red[par][ww][t + NTH][l2][i];
            }
            if (part) {  // a K slice: raw sums, finished by k_mm_reduce
                float* pp = part + ((size_t)blockIdx.y * M + m) * (H2 * N) + row;
                pp[0] = v;
                if constexpr (EPI == EPI_SWIGLU) pp[N] = up;
                continue;
            }
            if constexpr (NORM) {
                float tot = 0.0f;
#pragma unroll
                for (int ww = 0; ww < NW; ++ww) tot += rsum[ww][m];
                const float rs = 1.0f / sqrtf(tot / (float)K + eps);
                v *= rs;
                up *= rs;
            }
            float* dst = y + (size_t)m * ldy + row;
            if constexpr (EPI == EPI_SWIGLU)
                *dst = silu_f(v) * up;
            else if constexpr (EPI == EPI_RESID)
                *dst += v;
            else
                *dst = v;
        }
        par ^= 1;
        if (next >= ngroups) break;
        g = next;
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
    // config-1 4096 x 12288: 17.0 / 18.2 us at 4 / 16 rows (19.2 / 19.4)
    {4096, 12288, EPI_STORE, {8, 8, 1, 8}},
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

// Whole-K launch shapes (waves, tiles per half per group, grid, K slices)
// measured per 4B projection at 16 rows (graph replays over rotating weight
// copies, the K-sliced form's reduction included in its time); the other
// shapes take the K-sliced form above: the attention q/k/v (12.1 us here
// against 11.6) and the 9728-column down projection, whose activation does
// not fit the registers at once (16.4 us in 3 slices against 13.3: every
// slice's workgroup loads and splits its 16 x 2432 activation block for one
// or two tiles, where the K-sliced form shares it across 8).
struct BConfig {
    int nw, nth, grid;
    int ks;  // K slices (1: whole K in one launch)
};
struct BTuned {
    int N, K, epi;
    BConfig c;
};
constexpr BTuned kBTuned[] = {
    {9728, 2560, EPI_SWIGLU, {8, 1, 224, 1}},   // gate/up: 19.1 us (K-sliced 23.5)
    {8224, 2560, EPI_STORE, {8, 1, 256, 1}},    // DeltaNet in-projection: 13.8 us (15.5)
    {2560, 2048, EPI_RESID, {16, 1, 160, 1}},   // output projections: 6.5 us (7.9)
    {151936, 2560, EPI_STORE, {8, 2, 256, 1}},  // lm_head: 87.9 us (113.5)
    // the config-1 shapes with K = 4096, in 4 K slices (then the ordered
    // reduction), at 4 / 16 rows: 4096 x 4096 8.7 / 10.0 us (K-sliced form
    // 11.6 / 13.0), 12288 x 4096 14.7 / 17.6 us (21.8 / 23.3)
    {4096, 4096, EPI_STORE, {8, 2, 128, 4}},
    {12288, 4096, EPI_STORE, {8, 2, 128, 4}},
};

bool b_lookup(int N, int K, int epi, BConfig* c) {
    for (const BTuned& t : kBTuned)
        if (t.N == N && t.K == K && t.epi == epi) {
            *c = t.c;
            return true;
        }
    return false;
}

// blocks per K slice, and the slices that then exist
int b_bps(const BConfig& c, int K) {
    const int nblk = K / 64, ks = c.ks < 1 ? 1 : c.ks;
    return (nblk + ks - 1) / ks;
}
int b_slices(const BConfig& c, int K) {
    const int bps = b_bps(c, K);
    return (K / 64 + bps - 1) / bps;
}
size_t b_work_bytes(const BConfig& c, int M, int N, int K, int epi) {
    const int s = b_slices(c, K);
    return s > 1 ? (size_t)s * M * (epi == EPI_SWIGLU ? 2 : 1) * N * sizeof(float) : 0;
}

struct BLaunch {
    int grid, slices, bps;
    float* part;  // partial sums of the slices (null: whole K)
};

template <int NW, int NTH, int PX, bool NORM, int EPI>
void launch_b(const BLaunch& l, const float* x, int ldx, const float* gain, float eps,
              const int8_t* qz, const float* sz, float* y, int ldy, int M, int N, int tiles_half,
              int nblk, hipStream_t st) {
    hipLaunchKernelGGL((k_mm_b<NW, NTH, PX, NORM, EPI>), dim3(l.grid, l.slices),
                       dim3(NW * QLM_WAVE), 0, st, x, ldx, gain, eps, qz, sz, y, ldy, M, N,
                       tiles_half, nblk, l.bps, l.part);
}

template <int NW, int NTH, int PX>
int launch_b_epi(const BLaunch& l, const float* x, int ldx, const float* norm_w, float eps,
                 const int8_t* qz, const float* sz, float* y, int ldy, int M, int N, int epi,
                 int tiles_half, int nblk, hipStream_t st) {
    if (epi == EPI_SWIGLU)
        launch_b<NW, NTH, PX, true, EPI_SWIGLU>(l, x, ldx, norm_w, eps, qz, sz, y, ldy, M, N,
                                                  tiles_half, nblk, st);
    else if (epi == EPI_RESID)
        launch_b<NW, NTH, PX, false, EPI_RESID>(l, x, ldx, nullptr, eps, qz, sz, y, ldy, M, N,
                                                  tiles_half, nblk, st);
    else if (norm_w)
        launch_b<NW, NTH, PX, true, EPI_STORE>(l, x, ldx, norm_w, eps, qz, sz, y, ldy, M, N,
                                                 tiles_half, nblk, st);
    else
        launch_b<NW, NTH, PX, false, EPI_STORE>(l, x, ldx, nullptr, eps, qz, sz, y, ldy, M, N,
                                                  tiles_half, nblk, st);
    return qlm_launch_status();
}

// Shapes whose registers do not fit (the compiler spills; counts from the
// gfx950 build): 7 blocks a wave with the RMSNorm gains; SwiGLU with two
// tiles per half at 5 blocks a wave (8 waves) or 2 (16 waves).
bool b_spills(int nw, int nth, int px, bool norm, bool swiglu) {
    if (px >= 7 && norm) return true;
    if (swiglu && nth == 2 && (nw == 16 || px >= 5)) return true;
    return false;
}

// Built: (waves, blocks per wave) = (8, 2) (8, 4) (8, 5) (8, 7) (16, 2),
// with 1 or 2 tiles per half; blocks per wave = ceil(blocks per slice /
// waves). A slice count above 1 writes partial sums to work and adds the
// ordered reduction (k_mm_reduce, with the RMSNorm when norm_w is given).
int b_run(const BConfig& c, const float* x, int ldx, const float* norm_w, float eps,
          const int8_t* qz, const float* sz, float* y, int ldy, int M, int N, int K, int epi,
          void* work, size_t work_bytes, hipStream_t st) {
    const int nblk = K / 64;
    const int tiles_half = (N + 15) / 16;
    if ((c.nw != 8 && c.nw != 16) || (c.nth != 1 && c.nth != 2) || c.ks < 1) return QLM_ERR_ARG;
    const int bps = b_bps(c, K), slices = b_slices(c, K);
    const int px = (bps + c.nw - 1) / c.nw;
    if (b_spills(c.nw, c.nth, px, norm_w != nullptr, epi == EPI_SWIGLU)) return QLM_ERR_SHAPE;
    if (norm_w && K > kMaxGainK) return QLM_ERR_SHAPE;
    const int groups = (tiles_half + c.nth - 1) / c.nth;
    const int grid = c.grid < groups ? c.grid : groups;
    if (grid < 1) return QLM_ERR_ARG;
    float* part = nullptr;
    if (slices > 1) {
        if (!work || work_bytes < b_work_bytes(c, M, N, K, epi)) return QLM_ERR_ARG;
        part = static_cast<float*>(work);
    }
    const BLaunch l{grid, slices, bps, part};
    int rc = QLM_ERR_SHAPE;
#define QLM_B(NW_, NTH_, PX_)                                                                 \
    if (c.nw == NW_ && c.nth == NTH_ && px == PX_)                                            \
        rc = launch_b_epi<NW_, NTH_, PX_>(l, x, ldx, norm_w, eps, qz, sz, y, ldy, M, N, epi,     \
                                          tiles_half, nblk, st);
    QLM_B(8, 1, 2)
    else QLM_B(8, 1, 4)
    else QLM_B(8, 1, 5)
    else QLM_B(8, 1, 7)
    else QLM_B(8, 2, 2)
    else QLM_B(8, 2, 4)
    else QLM_B(8, 2, 5)
    else QLM_B(8, 2, 7)
    else QLM_B(16, 1, 2)
    else QLM_B(16, 2, 2)
#undef QLM_B
    if (rc != QLM_OK || slices == 1) return rc;
    const int NR = (epi == EPI_SWIGLU ? 2 : 1) * N;
    const dim3 rgrid((N + kReduceThreads - 1) / kReduceThreads, M);
    if (epi == EPI_SWIGLU)
        hipLaunchKernelGGL((k_mm_reduce<MMR_SWIGLU, true>), rgrid, dim3(kReduceThreads), 0, st,
                           part, slices, M, NR, N, y, ldy, x, ldx, K, eps);
    else if (epi == EPI_RESID)
        hipLaunchKernelGGL((k_mm_reduce<MMR_RESID, false>), rgrid, dim3(kReduceThreads), 0, st,
                           part, slices, M, NR, N, y, ldy, x, ldx, K, eps);
    else if (norm_w)
        hipLaunchKernelGGL((k_mm_reduce<MMR_STORE, true>), rgrid, dim3(kReduceThreads), 0, st,
                           part, slices, M, NR, N, y, ldy, x, ldx, K, eps);
    else
        hipLaunchKernelGGL((k_mm_reduce<MMR_STORE, false>), rgrid, dim3(kReduceThreads), 0, st,
                           part, slices, M, NR, N, y, ldy, x, ldx, K, eps);
    return qlm_launch_status();
}

}  // namespace

extern "C" size_t qlm_matmul_i8_t_workspace_bytes(int M, int N, int K, int epilogue) {
    if (M < 1 || N < 1 || K < 64) return 0;
    BConfig bc;
    if (b_lookup(N, K, epilogue, &bc)) return b_work_bytes(bc, M, N, K, epilogue);
    const int halves = epilogue == EPI_SWIGLU ? 2 : 1;
    const TConfig c = t_config(N, K, epilogue);
    return (size_t)t_slices(c, K) * M * halves * N * sizeof(float);
}

extern "C" size_t qlm_matmul_i8_t_whole_workspace_bytes(int M, int N, int K, int epilogue,
                                                       int k_slices) {
    if (M < 1 || N < 1 || K < 64 || k_slices < 1) return 0;
    return b_work_bytes(BConfig{8, 1, 1, k_slices}, M, N, K, epilogue);
}

extern "C" int qlm_matmul_i8_t_whole_config(const float* x, int ldx, const float* norm_w,
                                            float eps, const int8_t* q_tiles,
                                            const float* s_tiles, int group, float* y, int ldy,
                                            int M, int N, int K, int epilogue, int waves,
                                            int tiles, int grid, int k_slices, void* work,
                                            size_t work_bytes, void* stream) {
    const int rc = t_check(x, ldx, norm_w, q_tiles, s_tiles, group, y, ldy, M, N, K, epilogue);
    if (rc != QLM_OK) return rc;
    return b_run(BConfig{waves, tiles, grid, k_slices}, x, ldx, norm_w, eps, q_tiles, s_tiles, y,
                 ldy, M, N, K, epilogue, work, work_bytes, as_stream(stream));
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
    BConfig bc;
    if (b_lookup(N, K, epilogue, &bc))
        return b_run(bc, x, ldx, norm_w, eps, q_tiles, s_tiles, y, ldy, M, N, K, epilogue, work,
                     work_bytes, as_stream(stream));
    if (!work) return QLM_ERR_ARG;
    const TConfig c = t_config(N, K, epilogue);
    return t_run(c, x, ldx, norm_w, eps, q_tiles, s_tiles, y, ldy, M, N, K, epilogue, work,
                 work_bytes, as_stream(stream));
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_gemm_t() {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>((k_mm_t<8, 8, 1, false>)));
}
