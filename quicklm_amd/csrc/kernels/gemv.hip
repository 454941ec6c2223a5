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

#include <type_traits>

#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / QLM_WAVE;
constexpr int kLdsBudget = 64 * 1024;

// PRO_HEADNORM (k_gemv_mx only): x is the column-split DeltaNet mixer's
// u, and each 128-column head of it is scaled by 1/sqrt(sum of the head's
// eight partial sums of squares / 128 + eps), the head RMSNorm the mixer
// left to its consumer (nw then points at the partial sums [K / 128][8]).
enum { PRO_NONE = 0, PRO_RMSNORM = 1, PRO_HEADNORM = 2 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

// Greedy tail of a decode step (EPI_ARGMAX, M = 1): the logits are stored and
// each workgroup writes its rows' maximum (first index wins ties, as
// DecoderModel::sample, model.cpp:263-274) as a 64-bit key into its own slot
// keys[blockIdx.x]; a one-workgroup kernel then reduces the slots, advances
// the sequence (token written unless position p+1 is still prompt, pos += 1)
// and gathers the embedding of the token now at pos into h for the next
// step. The kernel boundary orders the two, so no workgroup of the GEMV
// pays for a device-scope fence (on MI355X each one writes back and
// invalidates its XCD's L2, ~0.3 us apiece over a 2048-workgroup grid).
// One 64-bit key slot per workgroup of the logits GEMV (grid <= kMaxXsGrid).
constexpr int kMaxXsGrid = 2048;
constexpr int kEmbPer = 4;  // float4 of the next embedding row per thread and round

struct GreedyTail {
    unsigned long long* keys;
    int* tokens;
    int ld_tokens;
    int* pos;
    const int* prompt_len;
    const float* embed;
    int H;
    int vocab;
    float* h;
};

__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    unsigned u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // monotone in v (non-NaN)
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)idx);
}

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

// ---------------------------------------------------------------------------
// M = 1, activation-stationary form (the batch-1 decode path).
//
// A row is shared by `lpr` lanes (16..256, a power of two); lane li of a row
// group owns the 16-byte chunks c = li + s*lpr, s < SLOTS, of EVERY row, so
// its slice of the activation vector (SLOTS x 16 floats, normalised once when
// the RMSNorm prologue is fused) stays in registers for the whole kernel and
// is never re-read. A workgroup (256 lanes = 256/lpr row groups) walks row
// blocks of (256/lpr)*R rows with a grid-stride loop; the next block's weight
// chunks (and group scales) are loaded before the current block is reduced,
// so 2*R*SLOTS 16-byte loads per lane are in flight. With lpr chosen so that
// SLOTS*lpr*16 >= K, every chunk of a row is loaded by exactly one lane.
// Partial sums are reduced across the lpr lanes of the row (butterfly inside
// a wave, then through LDS when lpr > 64) in a fixed order.
template <int SLOTS, int R, bool ROWSCALE, int PRO, int EPI>
__global__ __launch_bounds__(kThreads) void k_gemv_xs(
    const float* __restrict__ x, const float* __restrict__ nw, float eps,
    const int8_t* __restrict__ q, const float* __restrict__ sc, float* __restrict__ y, int N,
    int K, int F, int lpr, int nblocks, GreedyTail tail) {
    __shared__ float red[kWaves][R];
    __shared__ float ssr[kWaves];
    float best_v = -INFINITY;  // EPI_ARGMAX: this lane's best stored logit
    int best_i = 0x7fffffff;
    const int tid = threadIdx.x;
    const int lane = tid & (QLM_WAVE - 1);
    const int wave = tid / QLM_WAVE;
    const int li = tid & (lpr - 1);
    const int grp = tid / lpr;
    const int groups = kThreads / lpr;
    const int nchunk = K >> 4;
    const int nblk = K >> 5;
    const int wpg = lpr > QLM_WAVE ? lpr / QLM_WAVE : 1;  // waves per row group

    // ---- row blocks ----
    // Loads never branch: a lane's chunk index is clamped into the row (the
    // matching activation slot is zero, so the duplicate contributes 0) and
    // rows past N are clamped to N-1 (computed, never stored).
    constexpr int OUT_PER_GRP = (EPI == EPI_SWIGLU) ? R / 2 : R;
    const int out_per_block = groups * OUT_PER_GRP;
    int soff[SLOTS], coff[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int c = min(li + s * lpr, nchunk - 1);
        soff[s] = c << 4;
        coff[s] = c >> 1;
    }
    auto out_row = [&](int rb, int r) -> int {
        return rb * out_per_block + grp * OUT_PER_GRP + ((EPI == EPI_SWIGLU) ? (r % (R / 2)) : r);
    };
    // Weight chunks and group scales (row scale in sv[r][0] when ROWSCALE) of
    // block rb; for EPI_RESID also the residual values the block adds to
    // (read long before they are needed).
    auto load = [&](int rb, int4 (&w)[R][SLOTS], float (&sv)[R][SLOTS],
                    float (&res)[OUT_PER_GRP]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int o = min(out_row(rb, r), N - 1);
            if constexpr (EPI == EPI_SWIGLU)
                if (r >= R / 2) o += F;
            const int8_t* rp = q + (size_t)o * K;
            const float* sp = sc + (size_t)o * nblk;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                w[r][s] = *reinterpret_cast<const int4*>(rp + soff[s]);
                if constexpr (!ROWSCALE) sv[r][s] = sp[coff[s]];
            }
            if constexpr (ROWSCALE) sv[r][0] = sc[o];  // the row's one scale
        }
        if constexpr (EPI == EPI_RESID) {
#pragma unroll
            for (int r = 0; r < OUT_PER_GRP; ++r) res[r] = y[min(out_row(rb, r), N - 1)];
        }
    };

    // The first two blocks' weights are requested before anything else, so
    // their HBM latency overlaps the activation load and the RMSNorm prologue.
    // Blocks b0, b1, b2, ... (stride gridDim.x) alternate between the two
    // register buffers; a buffer is refilled as soon as its block is reduced.
    int4 wa[R][SLOTS], wb[R][SLOTS];
    float sa[R][SLOTS], sb[R][SLOTS];
    float ra[OUT_PER_GRP], rbv[OUT_PER_GRP];
    int rb = blockIdx.x;
    if (EPI != EPI_ARGMAX && rb >= nblocks) return;  // uniform per workgroup
    if (rb < nblocks) load(rb, wa, sa, ra);
    if (rb + (int)gridDim.x < nblocks) load(rb + gridDim.x, wb, sb, rbv);

    // ---- activation (+ gain) staged once per workgroup through LDS ----
    // Coalesced 16-byte loads by all 256 lanes (x is read once per
    // workgroup, not once per row group), the RMSNorm sum of squares folded
    // into the same pass; then each lane takes its slice into registers,
    // normalised there. xsh holds x [K] and, with the RMSNorm prologue, the
    // gain [K] behind it.
    extern __shared__ float4 xsh[];
    float ss = 0.0f;
    for (int i = tid; i < (K >> 2); i += kThreads) {
        const float4 v = reinterpret_cast<const float4*>(x)[i];
        xsh[i] = v;
        if constexpr (PRO == PRO_RMSNORM) {
            xsh[(K >> 2) + i] = reinterpret_cast<const float4*>(nw)[i];
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
    }
    if constexpr (PRO == PRO_RMSNORM) {
        ss = wave_sum(ss);
        if (lane == 0) ssr[wave] = ss;
    }
    __syncthreads();
    float rs = 1.0f;
    if constexpr (PRO == PRO_RMSNORM) {
        float tot = ssr[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) tot += ssr[w];
        rs = 1.0f / sqrtf(tot / (float)K + eps);
    }
    float4 xv[SLOTS][4];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int c = li + s * lpr;
        if (c < nchunk) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xv[s][j] = xsh[c * 4 + j];
                if constexpr (PRO == PRO_RMSNORM)
                    xv[s][j] = norm4(xv[s][j], rs, xsh[(K >> 2) + c * 4 + j]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[s][j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }

    auto finish = [&](int rb, const int4 (&w)[R][SLOTS], const float (&sv)[R][SLOTS],
                      const float (&res)[OUT_PER_GRP]) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.0f;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const float p = dot16(w[r][s], xv[s][0], xv[s][1], xv[s][2], xv[s][3]);
                if constexpr (ROWSCALE)
                    acc[r] += p;
                else
                    acc[r] = fmaf(p, sv[r][s], acc[r]);
            }
        }
        // reduce each row over its lpr lanes (fixed order)
        if (lpr <= QLM_WAVE) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                for (int m = lpr >> 1; m >= 1; m >>= 1) acc[r] += __shfl_xor(acc[r], m, QLM_WAVE);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) red[wave][r] = acc[r];
            }
            __syncthreads();
            const int w0 = grp * wpg;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float t = red[w0][r];
                for (int w2 = 1; w2 < wpg; ++w2) t += red[w0 + w2][r];
                acc[r] = t;
            }
            __syncthreads();  // red is rewritten by the next block
        }
        if constexpr (ROWSCALE) {
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] *= sv[r][0];
        }
        // epilogue: lane li == r of each row group stores output r
        const int o0 = rb * out_per_block + grp * OUT_PER_GRP;
#pragma unroll
        for (int r = 0; r < OUT_PER_GRP; ++r) {
            if (li == r && o0 + r < N) {
                float* dst = y + o0 + r;
                if constexpr (EPI == EPI_SWIGLU)
                    *dst = silu_f(acc[r]) * acc[r + R / 2];
                else if constexpr (EPI == EPI_RESID)
                    *dst = res[r] + acc[r];
                else
                    *dst = acc[r];
                if constexpr (EPI == EPI_ARGMAX) {
                    if (acc[r] > best_v || (acc[r] == best_v && o0 + r < best_i)) {
                        best_v = acc[r];
                        best_i = o0 + r;
                    }
                }
            }
        }
    };

    const int gs = gridDim.x;
    while (rb < nblocks) {
        finish(rb, wa, sa, ra);
        if (rb + 2 * gs < nblocks) load(rb + 2 * gs, wa, sa, ra);
        rb += gs;
        if (rb >= nblocks) break;
        finish(rb, wb, sb, rbv);
        if (rb + 2 * gs < nblocks) load(rb + 2 * gs, wb, sb, rbv);
        rb += gs;
    }

    if constexpr (EPI == EPI_ARGMAX) {
        // workgroup maximum into this workgroup's key slot (0 = no rows)
        unsigned long long k = argmax_key(best_v, best_i);
        if (best_i == 0x7fffffff) k = 0ull;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const unsigned long long o = __shfl_xor(k, m, QLM_WAVE);
            k = o > k ? o : k;
        }
        __shared__ unsigned long long wk[kWaves];
        if (lane == 0) wk[wave] = k;
        __syncthreads();
        if (tid == 0) {
            unsigned long long m = wk[0];
            for (int w2 = 1; w2 < kWaves; ++w2) m = wk[w2] > m ? wk[w2] : m;
            tail.keys[blockIdx.x] = m;
        }
    }
}

// Second half of the greedy tail: reduce the nkeys workgroup keys, advance
// the sequence and gather the next embedding (one workgroup).
__global__ __launch_bounds__(kThreads) void k_greedy_finish(GreedyTail tail, int nkeys, int N) {
    __shared__ unsigned long long wk[kWaves];
    __shared__ int tok;
    const int tid = threadIdx.x, lane = tid & (QLM_WAVE - 1), wave = tid / QLM_WAVE;
    // the position and prompt length travel with the keys (one round trip)
    const int p = tail.pos[0], plen = tail.prompt_len[0];
    // nkeys <= kMaxXsGrid: every slot is requested before any is compared
    unsigned long long v[kMaxXsGrid / kThreads];
#pragma unroll
    for (int u = 0; u < kMaxXsGrid / kThreads; ++u) {
        const int i = tid + u * kThreads;
        v[u] = i < nkeys ? tail.keys[i] : 0ull;
    }
    unsigned long long k = 0ull;
#pragma unroll
    for (int u = 0; u < kMaxXsGrid / kThreads; ++u) k = v[u] > k ? v[u] : k;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(k, m, QLM_WAVE);
        k = o > k ? o : k;
    }
    if (lane == 0) wk[wave] = k;
    __syncthreads();
    if (tid == 0) {
        unsigned long long m = wk[0];
        for (int w2 = 1; w2 < kWaves; ++w2) m = wk[w2] > m ? wk[w2] : m;
        int idx = m ? (int)(0xFFFFFFFFu - (unsigned)(m & 0xFFFFFFFFull)) : 0;
        if (idx < 0 || idx >= N) idx = 0;
        if (p + 1 < tail.ld_tokens && p + 1 >= plen) tail.tokens[p + 1] = idx;
        // the token now at p + 1: the prompt's there, else the pick (no
        // reload of what was just stored)
        int t = (p + 1 < tail.ld_tokens && p + 1 < plen) ? tail.tokens[p + 1] : idx;
        t = t < 0 ? 0 : (t >= tail.vocab ? tail.vocab - 1 : t);
        tok = t;
        tail.pos[0] = p + 1;
    }
    __syncthreads();
    // the embedding row: every float4 of a round (kEmbPer a thread) is
    // requested before any is stored; a strided copy loop with a runtime
    // bound waits for each load before issuing the next
    const float* src = tail.embed + (size_t)tok * tail.H;
    if ((tail.H & 3) == 0) {
        const int H4 = tail.H >> 2;
        const float4* s4 = reinterpret_cast<const float4*>(src);
        float4* d4 = reinterpret_cast<float4*>(tail.h);
        for (int i0 = 0; i0 < H4; i0 += kEmbPer * kThreads) {
            float4 v[kEmbPer];
#pragma unroll
            for (int j = 0; j < kEmbPer; ++j) v[j] = s4[min(i0 + j * kThreads + tid, H4 - 1)];
#pragma unroll
            for (int j = 0; j < kEmbPer; ++j)
                if (i0 + j * kThreads + tid < H4) d4[i0 + j * kThreads + tid] = v[j];
        }
    } else {
        for (int i = tid; i < tail.H; i += kThreads) tail.h[i] = src[i];
    }
}

// ---------------------------------------------------------------------------
// M = 1 on the int8 matrix cores (v_mfma_i32_16x16x64_i8), weights in the
// tile-major layout below.
//
// The activation is written as four int8 digit vectors, with one exponent
// per wave over the elements that wave multiplies (its K blocks): with E
// chosen from their max|x| so that |x| / 2^E < 64,
//     x = 2^E * (d0 + d1 2^-7 + d2 2^-14 + d3 2^-21) + e,   |e| <= 2^-27 max|x|,
// every |d| <= 64. A weight group's dot products with the four digit vectors
// are exact int32 sums on the matrix cores, so per 1024 weights a wave spends
// one MFMA and about six VALU operations (two shift-adds, two conversions,
// two FMAs) instead of a conversion and an FMA per weight.
//
// Operands of one K = 64 block b of a tile of 16 weight rows (lane l,
// n = l & 15, q = l >> 4):
//   B (weights) lane l: row n, bytes 64b + 16q .. +15. The tile-major layout
//               stores these 64 fragments as one contiguous 1 KB span, so a
//               wave's load is a linear 1 KB read (row-major rows would make
//               it 16 scattered 64-byte pieces, which streams ~30% slower).
//   A (digits)  lane l: A row n, elements 64b + 16q .. +15. A row 4h + d
//               holds digit d of the elements of group 2b + h (zero for the
//               other group; rows 8..15 are zero).
//   D           lane l: D[4q + i][n], i = 0..3. Lanes q = 0, 1 hold the four
//               digit sums of row n over group 2b + q, combined as
//               P = (D0 << 7) + D1, Q = (D2 << 7) + D3 (exact int32) and
//               accumulated as (P + Q 2^-14) * s[n][2b + q] in fp32; the
//               wave's sum is then scaled by 2^(E - 7) (with one scale per
//               row, s = 1 there and the row scale multiplies the result).
//
// A workgroup of NW waves owns one tile at a time (grid-stride over tiles);
// wave w takes the P = ceil(K / 64 / NW) blocks w, w + NW, ... of every tile.
// A wave requests the activation (and gain) of its own blocks first, then all
// P weight blocks of its first tile (and their scales); each slot is refilled
// with the next tile's block as soon as it is consumed. A wave's digits
// depend only on its own blocks, so it starts on its weights as soon as its
// own activation has arrived, with no workgroup barrier before the first
// MFMA (an exponent shared by the workgroup would wait for the whole vector,
// whose loads queue behind the flood of weight loads: measured, that wait
// was the largest part of a launch). RMSNorm is linear in 1/rms, so the
// digits are taken of x * (1 + w) and 1/rms multiplies the finished sums;
// the waves' sums of squares meet at the first tile end. At the end of a tile the waves' partial
// sums meet in LDS (one barrier per tile) and wave 0 applies the epilogue and
// the stores.

// Tile-major weight layout: the rows are cut into halves (2 for the
// [gate; up] matrix of SwiGLU) of `rows` rows each, each half padded with
// zero rows to 16-row tiles; fragment (tile g, block b) is the 1 KB B operand
// above in lane order (lane l = 16q + n: row 16t + n, bytes 64b + 16q .. +15).
// Group-32 scales of the fragment follow as 32 floats [h][n] (group 2b + h of
// row n). One thread per 16 bytes.
__global__ __launch_bounds__(256) void k_mx_swizzle(const int8_t* __restrict__ q,
                                                    const float* __restrict__ sc, int rows,
                                                    int K, int tiles, int halves,
                                                    int8_t* __restrict__ qz,
                                                    float* __restrict__ sz) {
    const int nblk = K >> 6, nsb = K >> 5;
    const size_t total = (size_t)halves * tiles * nblk * QLM_WAVE;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % QLM_WAVE);
        const size_t fb = i / QLM_WAVE;
        const int b = (int)(fb % nblk);
        const int g = (int)(fb / nblk);
        const int half = g / tiles, t = g % tiles;
        const int n = lane & 15, qd = lane >> 4;
        const int rh = t * 16 + n;  // row within the half
        int4 v = make_int4(0, 0, 0, 0);
        if (rh < rows)
            v = *reinterpret_cast<const int4*>(q + ((size_t)half * rows + rh) * K + b * 64 +
                                               qd * 16);
        reinterpret_cast<int4*>(qz)[i] = v;
        if (sz && lane < 32) {
            const int h = lane >> 4;
            sz[fb * 32 + lane] =
                rh < rows ? sc[((size_t)half * rows + rh) * nsb + 2 * b + h] : 0.0f;
        }
    }
}

// int4 tile-major layout: the same fragments as the int8 one (lane l = 16q +
// n: row 16t + n, columns 64b + 16q .. +15) at 8 bytes a lane, 512 B a
// fragment, each column as the nibble value + 8 (8 for padded rows): byte i
// of the lane's first word holds columns i (low nibble) and 4 + i (high),
// of its second word columns 8 + i and 12 + i. Scales as in the int8 layout.
__global__ __launch_bounds__(256) void k_mx4_swizzle(const uint8_t* __restrict__ q4,
                                                     const float* __restrict__ sc, int rows,
                                                     int K, int tiles, int halves,
                                                     uint8_t* __restrict__ qz,
                                                     float* __restrict__ sz) {
    const int nblk = K >> 6, nsb = K >> 5;
    const size_t total = (size_t)halves * tiles * nblk * QLM_WAVE;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % QLM_WAVE);
        const size_t fb = i / QLM_WAVE;
        const int b = (int)(fb % nblk);
        const int g = (int)(fb / nblk);
        const int half = g / tiles, t = g % tiles;
        const int n = lane & 15, qd = lane >> 4;
        const int rh = t * 16 + n;  // row within the half
        unsigned wa = 0x88888888u, wb = 0x88888888u;
        if (rh < rows) {
            // columns 64b + 16q .. +15: 8 packed bytes (low nibble = even column)
            const uint2 src = *reinterpret_cast<const uint2*>(
                q4 + ((size_t)half * rows + rh) * (K / 2) + 32 * b + 8 * qd);
            unsigned v[16];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const unsigned byte = ((j < 4 ? src.x : src.y) >> (8 * (j % 4))) & 0xffu;
                v[2 * j] = byte & 15u;
                v[2 * j + 1] = byte >> 4;
            }
            wa = 0u;
            wb = 0u;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                wa |= (v[j] | (v[4 + j] << 4)) << (8 * j);
                wb |= (v[8 + j] | (v[12 + j] << 4)) << (8 * j);
            }
        }
        reinterpret_cast<uint2*>(qz)[i] = make_uint2(wa, wb);
        if (lane < 32) {
            const int h = lane >> 4;
            sz[fb * 32 + lane] =
                rh < rows ? sc[((size_t)half * rows + rh) * nsb + 2 * b + h] : 0.0f;
        }
    }
}

// A lane's 16 int4 weights (int4 tile-major layout) as the int8 B operand:
// nibbles to bytes, then value = nibble - 8 per byte without borrows
// ((x | 0x80) - 8 stays >= 0x78; the xor restores the sign).
__device__ __forceinline__ int unbias4(unsigned w) {
    return (int)(((w | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
}
typedef int v4i_w4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4i_w4 unpack_w4(int2 w) {
    const unsigned a = (unsigned)w.x, b = (unsigned)w.y;
    return v4i_w4{unbias4(a & 0x0F0F0F0Fu), unbias4((a >> 4) & 0x0F0F0F0Fu),
                  unbias4(b & 0x0F0F0F0Fu), unbias4((b >> 4) & 0x0F0F0F0Fu)};
}

template <int NW, int T, int P, bool ROWSCALE, int PRO, int EPI, bool W4>
__global__ __launch_bounds__(NW * QLM_WAVE) void k_gemv_mx(
    const float* __restrict__ x, const float* __restrict__ nw, float eps,
    const int8_t* __restrict__ q, const float* __restrict__ sc, float* __restrict__ y, int N,
    int K, int F, int ntiles, GreedyTail tail, int gtiles) {
    constexpr int XL = (P + 3) / 4;  // activation float4 per lane (16 lanes per block)
    typedef int v4i __attribute__((ext_vector_type(4)));
    // dynamic LDS: the digits [wave][slot][digit][64 B], then the partial
    // sums of gtiles tiles [tile][wave][T][16] (floats)
    extern __shared__ __align__(16) unsigned char mx_lds[];
    __shared__ float rsum[NW];

    const int tid = threadIdx.x, lane = tid & (QLM_WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / QLM_WAVE);
    const int n = lane & 15, qd = lane >> 4;
    const int nblk = K >> 6;
    unsigned char* dig = mx_lds + (size_t)w * P * 256;

    // ---- this wave's activation (and gain) first: load i of lane l is
    // elements 4n .. 4n+3 of slot u = 4i + q (block w + NW*u). The loads are
    // unconditional (block clamped into K; lanes past the wave's blocks are
    // zeroed once the values are used): a load under a branch makes the
    // compiler wait for it at the branch's end, before the weight loads.
    float4 xr[XL], gr[XL], hn[XL];
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        const int b = min(w + NW * (4 * i + qd), nblk - 1);
        xr[i] = reinterpret_cast<const float4*>(x)[b * 16 + n];
        if constexpr (PRO == PRO_RMSNORM) gr[i] = reinterpret_cast<const float4*>(nw)[b * 16 + n];
        if constexpr (PRO == PRO_HEADNORM) {
            // the head (two 64-column blocks) of block b: its eight partials
            const float4* hp = reinterpret_cast<const float4*>(nw) + (size_t)(b >> 1) * 2;
            gr[i] = hp[0];
            hn[i] = hp[1];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    auto row_of = [&](int tile, int tt) {
        int r = min(tile * 16 + n, N - 1);
        if constexpr (EPI == EPI_SWIGLU)
            if (tt == 1) r += F;
        return r;
    };
    // Epilogue operands (residual, row scales) of the first tile, requested
    // by every lane before the ring (row clamped, unconditional). Later tiles
    // read theirs in the epilogue, after their ring loads have drained: a
    // load issued behind the ring could only be waited for by draining it
    // (loads retire in order).
    float res0 = 0.0f, rsc0[T];
    if constexpr (EPI == EPI_RESID) res0 = y[min((int)blockIdx.x * 16 + n, N - 1)];
#pragma unroll
    for (int tt = 0; tt < T; ++tt) rsc0[tt] = ROWSCALE ? sc[row_of(blockIdx.x, tt)] : 1.0f;

    // ---- weight ring: slot u holds block w + NW*u of the current tile.
    // P = ceil(blocks / NW), so a wave's last slot may lie past K: it then
    // repeats the wave's last block (a cache hit) and meets zero digits. The
    // next tile's slot u is requested as soon as slot u is consumed.
    // this wave's last block (a wave past the last block reads block nblk-1,
    // which then meets zero digits)
    const int blast = w < nblk ? nblk - 1 - ((nblk - 1 - w) % NW) : nblk - 1;
    using WT = typename std::conditional<W4, int2, int4>::type;  // a lane's 16 weights
    WT wb[P][T];
    float sb[P][T];
    auto issue = [&](int tile, int u) {
        const int b = min(w + NW * u, blast);
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            // fragment (tile of half tt, block b): 1 KB (512 B at int4) in lane order
            const size_t fb = (size_t)(tile + tt * ntiles) * nblk + b;
            wb[u][tt] = reinterpret_cast<const WT*>(q)[fb * QLM_WAVE + lane];
            if constexpr (!ROWSCALE) sb[u][tt] = sc[fb * 32 + (qd & 1) * 16 + n];
        }
    };
#pragma unroll
    for (int u = 0; u < P; ++u) issue(blockIdx.x, u);

    // ---- digits of this wave's blocks, one exponent per wave
    float ss = 0.0f, m = 0.0f;
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        float4& v = xr[i];
        const int u = 4 * i + qd;
        if (u >= P || w + NW * u >= nblk) v = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (PRO == PRO_RMSNORM) {
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
            const float4 g = gr[i];
            v.x *= 1.0f + g.x;
            v.y *= 1.0f + g.y;
            v.z *= 1.0f + g.z;
            v.w *= 1.0f + g.w;
        }
        if constexpr (PRO == PRO_HEADNORM) {
            const float4 a = gr[i], c = hn[i];
            const float tot = ((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w));
            const float sn = 1.0f / sqrtf(tot / 128.0f + eps);
            v.x *= sn;
            v.y *= sn;
            v.z *= sn;
            v.w *= sn;
        }
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    int e2 = 0;
    frexpf(wave_max(m), &e2);
    const int E = __builtin_amdgcn_readfirstlane(e2 - 6);  // max|x| / 2^E < 64 (digits <= 64)
    const float fx = ldexpf(1.0f, E - 7);  // 2^(E - 7): multiplies the wave's sums
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        const float vv[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
        unsigned pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float s0 = ldexpf(vv[c], -E);
            const float d0 = rintf(s0);
            float t = (s0 - d0) * 128.0f;
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
        const int u = 4 * i + qd;
        if (u < P) {
#pragma unroll
            for (int d = 0; d < 4; ++d)
                *reinterpret_cast<unsigned*>(dig + (u * 4 + d) * 64 + n * 4) = pk[d];
        }
    }
    if constexpr (PRO == PRO_RMSNORM) {
        ss = wave_sum(ss);
        if (lane == 0) rsum[w] = ss;
    }
    // the wave's own digit stores complete before its lanes read them back
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();

    // A fragment of this lane: digit n & 3 of elements 16q .. 16q+15 when
    // A row n carries group q >> 1, zero otherwise
    const bool active = n < 8 && (n >> 2) == (qd >> 1);
    int aoff = (n & 3) * 64 + qd * 16;

    float accf[T];
#pragma unroll
    for (int tt = 0; tt < T; ++tt) accf[tt] = 0.0f;
    auto consume = [&](int u) {
        v4i a = v4i{0, 0, 0, 0};
        if (active) a = *reinterpret_cast<const v4i*>(dig + u * 256 + aoff);
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            v4i bw;
            if constexpr (W4) {
                bw = unpack_w4(wb[u][tt]);
            } else {
                bw = v4i{wb[u][tt].x, wb[u][tt].y, wb[u][tt].z, wb[u][tt].w};
            }
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bw, v4i{0, 0, 0, 0}, 0, 0, 0);
            const int pp = (d[0] << 7) + d[1];
            const int qq = (d[2] << 7) + d[3];
            const float v = fmaf((float)qq, 0x1p-14f, (float)pp);
            accf[tt] = ROWSCALE ? accf[tt] + v : fmaf(v, sb[u][tt], accf[tt]);
        }
    };

    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    // Partial sums of the waves meet in LDS, gtiles tiles at a time: after
    // each tile a wave parks its partial sums in the tile's slot, and after
    // the group's last tile one barrier precedes the epilogues, slot s by
    // wave s % NW (its lanes qd == 0, one output row each), which sums the
    // waves' partials in wave order and applies 1/rms, the row scale, the
    // epilogue and the stores. No barrier stands between the tiles of a
    // group, so a wave whose weights arrived early runs on into the next
    // tile (and requests the one after).
    float* red = reinterpret_cast<float*>(mx_lds + (size_t)NW * P * 256);
    auto park = [&](int slot) {
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            const float p = xor16_add(accf[tt]) * fx;
            if (qd == 0) red[((slot * NW + w) * T + tt) * 16 + n] = p;
            accf[tt] = 0.0f;
        }
    };
    auto epilogue = [&](int tile, int slot) {
        const int o = tile * 16 + n;
        const bool first = tile == (int)blockIdx.x;
        float rs = 1.0f;
        if constexpr (PRO == PRO_RMSNORM) {
            float tot = rsum[0];
#pragma unroll
            for (int i = 1; i < NW; ++i) tot += rsum[i];
            rs = 1.0f / sqrtf(tot / (float)K + eps);
        }
        float val[T];
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            float v = red[((slot * NW) * T + tt) * 16 + n];
            for (int ww = 1; ww < NW; ++ww) v += red[((slot * NW + ww) * T + tt) * 16 + n];
            if constexpr (PRO == PRO_RMSNORM) v *= rs;
            if constexpr (ROWSCALE) v *= first ? rsc0[tt] : sc[row_of(tile, tt)];
            val[tt] = v;
        }
        if (o < N) {
            if constexpr (EPI == EPI_SWIGLU)
                y[o] = silu_f(val[0]) * val[1];
            else if constexpr (EPI == EPI_RESID)
                y[o] = (first ? res0 : y[o]) + val[0];
            else
                y[o] = val[0];
            if constexpr (EPI == EPI_ARGMAX) {
                if (val[0] > best_v || (val[0] == best_v && o < best_i)) {
                    best_v = val[0];
                    best_i = o;
                }
            }
        }
    };
    // the epilogues of slots [0, count) of the group starting at tile0
    auto flush = [&](int tile0, int count) {
        __syncthreads();
        if (qd == 0)
            for (int sl = w; sl < count; sl += NW) epilogue(tile0 + sl * (int)gridDim.x, sl);
    };

    // ---- tiles: consume the P slots in order (each refilled with the next
    // tile's block when there is one); the cross-wave epilogues per group
    int slot = 0, tile0 = blockIdx.x;
    for (int tile = blockIdx.x;; tile += gridDim.x) {
        const int next = tile + (int)gridDim.x;
        // the digit reads stay in the loop (hoisted, P fragments would stay
        // live across it)
        asm volatile("" : "+v"(aoff));
        if (next < ntiles) {
#pragma unroll
            for (int u = 0; u < P; ++u) {
                consume(u);
                issue(next, u);
            }
        } else {
#pragma unroll
            for (int u = 0; u < P; ++u) consume(u);
        }
        park(slot);
        ++slot;
        if (next >= ntiles) {
            flush(tile0, slot);
            break;
        }
        if (slot == gtiles) {
            flush(tile0, slot);
            __syncthreads();  // the group's slots are read before they are rewritten
            slot = 0;
            tile0 = next;
        }
    }

    if constexpr (EPI == EPI_ARGMAX) {
        // each wave's best over its rows, then the workgroup's
        __shared__ unsigned long long wkey[NW];
        unsigned long long k = argmax_key(best_v, best_i);
        if (best_i == 0x7fffffff) k = 0ull;
#pragma unroll
        for (int mm = 32; mm >= 1; mm >>= 1) {
            const unsigned long long o = __shfl_xor(k, mm, QLM_WAVE);
            k = o > k ? o : k;
        }
        if (lane == 0) wkey[w] = k;
        __syncthreads();
        if (tid == 0) {
#pragma unroll
            for (int i = 0; i < NW; ++i) k = wkey[i] > k ? wkey[i] : k;
            tail.keys[blockIdx.x] = k;
        }
    }
}

GreedyTail greedy_tail(void* work, int* tokens, int ld_tokens, int* pos, const int* prompt_len,
                       const float* embed, int H, int V, float* h_next) {
    GreedyTail t;
    t.keys = reinterpret_cast<unsigned long long*>(work);
    t.tokens = tokens;
    t.ld_tokens = ld_tokens;
    t.pos = pos;
    t.prompt_len = prompt_len;
    t.embed = embed;
    t.H = H;
    t.vocab = V;
    t.h = h_next;
    return t;
}

// Dynamic LDS of the M = 1 kernel: x, plus the RMSNorm gain.
size_t xs_lds_bytes(int K, int pro) {
    return (size_t)K * sizeof(float) * (pro == PRO_RMSNORM ? 2 : 1);
}
constexpr size_t kXsLdsMax = 64 * 1024;

struct XsConfig {
    int lpr, slots, R, grid;
    bool balance;  // grid is an upper bound: fit it to residency, equal blocks per workgroup
};

// Launch-shape choice for M = 1, from a sweep of the fused forms at the
// model's decode shapes on MI355X (graph replays): the fewest lanes per row
// that leave at most 3 16-byte chunks per lane (2 for SwiGLU, whose rows come
// in gate/up pairs; 5 when K > 8192), one output row per lane group, and for
// the 151936-row logits matrix 32 lanes per row with two rows. The grid is
// then fitted to what is resident at once (balanced_grid).
// Measured best launch shapes for the 4B hybrid's decode projections
// (N, K, epilogue -> lanes per row, rows, grid), graph replays on MI355X;
// each beats the rule below by 3-12%.
struct XsTuned {
    int N, K, epi, lpr, rows, grid;
};
constexpr XsTuned kXsTuned[] = {
    {9728, 2560, EPI_SWIGLU, 128, 1, 1024},  // gate/up
    {2560, 9728, EPI_RESID, 128, 1, 512},    // down
    {8224, 2560, EPI_STORE, 64, 1, 512},     // DeltaNet in_proj [qkv|z|b|a]
    {5120, 2560, EPI_STORE, 64, 1, 512},     // GQA q(+gate)/k/v
    {2560, 2048, EPI_RESID, 64, 1, 640},     // out_proj / o_proj
    {151936, 2560, EPI_STORE, 32, 2, 1280},  // lm_head (also its greedy form)
};

XsConfig xs_config(int N, int K, int epi) {
    for (const XsTuned& t : kXsTuned) {
        const int e = epi == EPI_ARGMAX ? EPI_STORE : epi;
        if (t.N == N && t.K == K && t.epi == e) {
            XsConfig c;
            c.lpr = t.lpr;
            c.slots = ((K >> 4) + t.lpr - 1) / t.lpr;
            c.R = epi == EPI_SWIGLU ? 2 * t.rows : t.rows;
            c.grid = t.grid;
            c.balance = false;
            return c;
        }
    }
    const int nchunk = K >> 4;
    const bool tall = N >= 65536;
    const int max_slots = tall ? 6 : (K > 8192 ? 5 : (epi == EPI_SWIGLU ? 2 : 3));
    int lpr = 32;
    while (lpr < 256 && (nchunk + lpr - 1) / lpr > max_slots) lpr *= 2;
    XsConfig c;
    c.lpr = lpr;
    c.slots = (nchunk + lpr - 1) / lpr;
    const int groups = kThreads / lpr;
    c.R = (epi == EPI_SWIGLU || tall) ? 2 : 1;
    const int out_per_block = groups * ((epi == EPI_SWIGLU) ? c.R / 2 : c.R);
    const int nblocks = (N + out_per_block - 1) / out_per_block;
    c.grid = nblocks < 2048 ? nblocks : 2048;
    c.balance = true;
    return c;
}

// Compute units and LDS per compute unit of the current device.
void device_shape(int& cus, size_t& lds_per_cu) {
    int dev = 0, v = 0;
    cus = 256;
    lds_per_cu = 160 * 1024;
    if (hipGetDevice(&dev) != hipSuccess) return;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
        cus = v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) ==
            hipSuccess &&
        v > 0)
        lds_per_cu = (size_t)v;
}

// Grid for a grid-stride launch of nblocks row blocks: never more
// workgroups than are resident at once (register- and LDS-limited), so there
// is no straggler round; within that, as many as possible (bytes in flight),
// then trimmed to give every workgroup the same number of blocks.
int balanced_grid(int nblocks, int cap, int per_cu_regs, size_t lds) {
    int cus;
    size_t lds_cu;
    device_shape(cus, lds_cu);
    int per_cu = per_cu_regs > 0 ? per_cu_regs : 1;
    if (lds > 0 && (int)(lds_cu / lds) < per_cu) per_cu = (int)(lds_cu / lds);
    if (per_cu < 1) per_cu = 1;
    int lim = per_cu * cus;
    if (cap > 0 && cap < lim) lim = cap;
    const int bpw = (nblocks + lim - 1) / lim;
    return (nblocks + bpw - 1) / bpw;
}

template <int SLOTS, int R, bool ROWSCALE, int PRO, int EPI>
int launch_xs(const XsConfig& c, const float* x, const float* nw, float eps, const int8_t* q,
              const float* sc, float* y, int N, int K, int F, hipStream_t st,
              const GreedyTail& tail) {
    auto kern = k_gemv_xs<SLOTS, R, ROWSCALE, PRO, EPI>;
    const int groups = kThreads / c.lpr;
    const int out_per_block = groups * ((EPI == EPI_SWIGLU) ? R / 2 : R);
    const int nblocks = (N + out_per_block - 1) / out_per_block;
    const size_t lds = xs_lds_bytes(K, PRO);
    int grid = c.grid < nblocks ? c.grid : nblocks;
    if (c.balance) {
        // register-limited workgroups per CU of this instance (LDS aside)
        static const int per_cu = [kern] {
            int n = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, kThreads, 0) != hipSuccess)
                n = 1;
            return n;
        }();
        grid = balanced_grid(nblocks, c.grid, per_cu, lds);
    }
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, st, x, nw, eps, q, sc, y, N, K, F,
                       c.lpr, nblocks, tail);
    if constexpr (EPI == EPI_ARGMAX) {
        const int rc = qlm_launch_status();
        if (rc != QLM_OK) return rc;
        hipLaunchKernelGGL(k_greedy_finish, dim3(1), dim3(kThreads), 0, st, tail, grid, N);
    }
    return qlm_launch_status();
}

template <bool ROWSCALE, int PRO, int EPI>
int launch_xs_sr(const XsConfig& c, const float* x, const float* nw, float eps, const int8_t* q,
                 const float* sc, float* y, int N, int K, int F, hipStream_t st,
                 const GreedyTail& tail) {
#define QLM_XS(S, RR)                                                                        \
    if (c.slots <= S && c.R == RR)                                                           \
        return launch_xs<S, RR, ROWSCALE, PRO, EPI>(c, x, nw, eps, q, sc, y, N, K, F, st, tail);
    if constexpr (EPI == EPI_SWIGLU) {
        QLM_XS(2, 2) QLM_XS(3, 2) QLM_XS(4, 2) QLM_XS(5, 2) QLM_XS(6, 2)
        QLM_XS(2, 4) QLM_XS(3, 4) QLM_XS(4, 4) QLM_XS(5, 4) QLM_XS(6, 4)
    } else {
        QLM_XS(2, 1) QLM_XS(3, 1) QLM_XS(4, 1) QLM_XS(5, 1) QLM_XS(6, 1)
        QLM_XS(2, 2) QLM_XS(3, 2) QLM_XS(4, 2) QLM_XS(5, 2) QLM_XS(6, 2)
    }
#undef QLM_XS
    return QLM_ERR_SHAPE;
}

int xs_dispatch(int pro, int epi, XsConfig c, const float* x, const float* nw, float eps,
                const int8_t* q, const float* sc, bool rowscale, float* y, int N, int K,
                hipStream_t st, const GreedyTail& tail = GreedyTail{}) {
    const int F = N;
#define QLM_XS_CALL(RS, P, E) \
    return launch_xs_sr<RS, P, E>(c, x, nw, eps, q, sc, y, N, K, F, st, tail)
    if (epi == EPI_ARGMAX) {
        if (rowscale) QLM_XS_CALL(true, PRO_RMSNORM, EPI_ARGMAX);
        QLM_XS_CALL(false, PRO_RMSNORM, EPI_ARGMAX);
    }
    if (rowscale) {
        if (pro == PRO_NONE && epi == EPI_STORE) QLM_XS_CALL(true, PRO_NONE, EPI_STORE);
        if (pro == PRO_RMSNORM && epi == EPI_STORE) QLM_XS_CALL(true, PRO_RMSNORM, EPI_STORE);
        if (pro == PRO_NONE && epi == EPI_RESID) QLM_XS_CALL(true, PRO_NONE, EPI_RESID);
        QLM_XS_CALL(true, PRO_RMSNORM, EPI_SWIGLU);
    }
    if (pro == PRO_NONE && epi == EPI_STORE) QLM_XS_CALL(false, PRO_NONE, EPI_STORE);
    if (pro == PRO_RMSNORM && epi == EPI_STORE) QLM_XS_CALL(false, PRO_RMSNORM, EPI_STORE);
    if (pro == PRO_NONE && epi == EPI_RESID) QLM_XS_CALL(false, PRO_NONE, EPI_RESID);
    QLM_XS_CALL(false, PRO_RMSNORM, EPI_SWIGLU);
#undef QLM_XS_CALL
}

// ---- matrix-core M = 1 launches (tile-major weights) ----
struct MxConfig {
    int nw, ring, grid;
};

// Dynamic LDS of k_gemv_mx: per wave and slot, four 64-byte digit planes.
size_t mx_lds_bytes(int nw, int ring) { return (size_t)nw * ring * 256; }
// dynamic LDS of a k_gemv_mx workgroup, digits and parked partial sums
constexpr size_t kMxLdsMax = 60 * 1024;

// Instantiated (waves per workgroup, slots per wave) pairs; slots =
// ceil(K / 64 / waves), so each pair serves a range of K.
constexpr int kMxPairs[][2] = {{4, 1}, {4, 2},  {4, 4},  {4, 8},   {4, 10},  {8, 4},
                               {8, 5}, {8, 8},  {16, 2}, {16, 4}, {16, 10}, {16, 12}};

// Whether k_gemv_mx<nw, *, ring> runs this K: whole 64-element blocks,
// ring = ceil(blocks / nw), and the pair is instantiated.
bool mx_fits(int K, int nw, int ring) {
    if (K <= 0 || K % 64 != 0) return false;
    if (K / 64 < nw) return false;  // every wave has a block
    if (ring != (K / 64 + nw - 1) / nw) return false;
    for (const auto& pr : kMxPairs)
        if (pr[0] == nw && pr[1] == ring) return true;
    return false;
}

// Measured launch shapes of the 4B hybrid's decode projections (N, K,
// epilogue -> waves per workgroup, ring depth, grid), graph replays on MI355X.
// group: the scale group an entry is for (0: either).
struct MxTuned {
    int N, K, epi, group, nw, ring, grid;
};
constexpr MxTuned kMxTuned[] = {
    {9728, 2560, EPI_SWIGLU, 0, 8, 5, 203},     // gate/up (3 tiles per workgroup)
    {2560, 9728, EPI_RESID, 0, 16, 10, 160},    // down
    {8224, 2560, EPI_STORE, 0, 8, 5, 512},      // DeltaNet in_proj [qkv|z|b|a]
    {5120, 2560, EPI_STORE, 0, 8, 5, 160},      // GQA q(+gate)/k/v (2 tiles per workgroup)
    {2560, 2048, EPI_RESID, 0, 8, 4, 160},      // out_proj / o_proj
    {151936, 2560, EPI_STORE, 0, 8, 5, 192},  // lm_head (also its greedy form)
    {12288, 4096, EPI_STORE, 32, 16, 4, 768},   // 12288 x 4096, group-32 scales
};

// Where int4 weights (half the bytes) measured a different best shape.
constexpr MxTuned kMx4Tuned[] = {
    {151936, 2560, EPI_STORE, 0, 8, 5, 512},    // lm_head
};

// Launch shape: the tuned table (int4 overrides first), else the fewest
// waves per workgroup that give >= 2048 waves in all (each a K-slice of a
// tile) among the instantiated pairs, and one tile per workgroup up to the
// greedy tail's key slots. nw = 0 when no pair fits K.
MxConfig mx_config(int N, int K, int epi, bool w4 = false, int group = 0) {
    const int e = epi == EPI_ARGMAX ? EPI_STORE : epi;
    auto match = [&](const MxTuned& t) {
        return t.N == N && t.K == K && t.epi == e && (t.group == 0 || t.group == group);
    };
    if (w4)
        for (const MxTuned& t : kMx4Tuned)
            if (match(t)) return MxConfig{t.nw, t.ring, t.grid};
    for (const MxTuned& t : kMxTuned)
        if (match(t)) return MxConfig{t.nw, t.ring, t.grid};
    const int tiles = (N + 15) / 16, nblk = K / 64;
    MxConfig c{0, 0, tiles < kMaxXsGrid ? tiles : kMaxXsGrid};
    for (int nw = 4; nw <= 16; nw *= 2) {
        const int ring = (nblk + nw - 1) / nw;
        if (!mx_fits(K, nw, ring)) continue;
        c.nw = nw;
        c.ring = ring;
        if (tiles * nw >= 2048) break;
    }
    return c;
}

template <int NW, int P, bool ROWSCALE, int PRO, int EPI, bool W4>
int launch_mx(const MxConfig& c, const float* x, const float* nw, float eps, const int8_t* q,
              const float* sc, float* y, int N, int K, int F, hipStream_t st,
              const GreedyTail& tail) {
    constexpr int T = EPI == EPI_SWIGLU ? 2 : 1;
    const int ntiles = (N + 15) / 16;
    int grid = c.grid < ntiles ? c.grid : ntiles;
    if (grid < 1) grid = 1;
    // tiles whose partial sums wait in LDS together: all of a workgroup's
    // tiles where they fit
    const int tpw = (ntiles + grid - 1) / grid;
    const size_t per_tile = (size_t)NW * T * 16 * sizeof(float);
    int gtiles = (int)((kMxLdsMax - mx_lds_bytes(NW, P)) / per_tile);
    gtiles = gtiles < 1 ? 1 : (gtiles > tpw ? tpw : gtiles);
    hipLaunchKernelGGL((k_gemv_mx<NW, T, P, ROWSCALE, PRO, EPI, W4>), dim3(grid),
                       dim3(NW * QLM_WAVE), mx_lds_bytes(NW, P) + gtiles * per_tile, st, x, nw, eps,
                       q, sc, y, N, K, F, ntiles, tail, gtiles);
    if constexpr (EPI == EPI_ARGMAX) {
        const int rc = qlm_launch_status();
        if (rc != QLM_OK) return rc;
        hipLaunchKernelGGL(k_greedy_finish, dim3(1), dim3(kThreads), 0, st, tail, grid, N);
    }
    return qlm_launch_status();
}

template <bool ROWSCALE, int PRO, int EPI, bool W4>
int launch_mx_np(const MxConfig& c, const float* x, const float* nw, float eps, const int8_t* q,
                 const float* sc, float* y, int N, int K, int F, hipStream_t st,
                 const GreedyTail& tail) {
#define QLM_MX(W, PP)                                                                      \
    if (c.nw == W && c.ring == PP)                                                          \
        return launch_mx<W, PP, ROWSCALE, PRO, EPI, W4>(c, x, nw, eps, q, sc, y, N, K, F, st, tail);
    QLM_MX(4, 1) QLM_MX(4, 2) QLM_MX(4, 4) QLM_MX(4, 8) QLM_MX(4, 10) QLM_MX(8, 4)
    QLM_MX(8, 5) QLM_MX(8, 8) QLM_MX(16, 2) QLM_MX(16, 4) QLM_MX(16, 10) QLM_MX(16, 12)
#undef QLM_MX
    return QLM_ERR_SHAPE;
}

int mx_dispatch(int pro, int epi, const MxConfig& c, const float* x, const float* nw, float eps,
                const int8_t* q, const float* sc, bool rowscale, float* y, int N, int K,
                hipStream_t st, const GreedyTail& tail = GreedyTail{}, bool w4 = false) {
    if (!mx_fits(K, c.nw, c.ring) || c.grid < 1) return QLM_ERR_SHAPE;
    if (epi == EPI_ARGMAX && c.grid > kMaxXsGrid) return QLM_ERR_SHAPE;
    const int F = N;
#define QLM_MX_CALL(RS, P, E, W) \
    return launch_mx_np<RS, P, E, W>(c, x, nw, eps, q, sc, y, N, K, F, st, tail)
    if (w4) {  // int4 weights: group-32 scales only (the reference's Q4_0)
        if (rowscale) return QLM_ERR_SHAPE;
        if (epi == EPI_ARGMAX) QLM_MX_CALL(false, PRO_RMSNORM, EPI_ARGMAX, true);
        if (pro == PRO_NONE && epi == EPI_STORE) QLM_MX_CALL(false, PRO_NONE, EPI_STORE, true);
        if (pro == PRO_RMSNORM && epi == EPI_STORE) QLM_MX_CALL(false, PRO_RMSNORM, EPI_STORE, true);
        if (pro == PRO_NONE && epi == EPI_RESID) QLM_MX_CALL(false, PRO_NONE, EPI_RESID, true);
        if (pro == PRO_HEADNORM && epi == EPI_RESID)
            QLM_MX_CALL(false, PRO_HEADNORM, EPI_RESID, true);
        if (pro == PRO_HEADNORM) QLM_MX_CALL(false, PRO_HEADNORM, EPI_STORE, true);
        QLM_MX_CALL(false, PRO_RMSNORM, EPI_SWIGLU, true);
    }
    if (epi == EPI_ARGMAX) {
        if (rowscale) QLM_MX_CALL(true, PRO_RMSNORM, EPI_ARGMAX, false);
        QLM_MX_CALL(false, PRO_RMSNORM, EPI_ARGMAX, false);
    }
    if (rowscale) {
        if (pro == PRO_NONE && epi == EPI_STORE) QLM_MX_CALL(true, PRO_NONE, EPI_STORE, false);
        if (pro == PRO_RMSNORM && epi == EPI_STORE) QLM_MX_CALL(true, PRO_RMSNORM, EPI_STORE, false);
        if (pro == PRO_NONE && epi == EPI_RESID) QLM_MX_CALL(true, PRO_NONE, EPI_RESID, false);
        if (pro == PRO_HEADNORM && epi == EPI_RESID)
            QLM_MX_CALL(true, PRO_HEADNORM, EPI_RESID, false);
        if (pro == PRO_HEADNORM) QLM_MX_CALL(true, PRO_HEADNORM, EPI_STORE, false);
        QLM_MX_CALL(true, PRO_RMSNORM, EPI_SWIGLU, false);
    }
    if (pro == PRO_HEADNORM && epi == EPI_RESID) QLM_MX_CALL(false, PRO_HEADNORM, EPI_RESID, false);
    if (pro == PRO_HEADNORM) QLM_MX_CALL(false, PRO_HEADNORM, EPI_STORE, false);
    if (pro == PRO_NONE && epi == EPI_STORE) QLM_MX_CALL(false, PRO_NONE, EPI_STORE, false);
    if (pro == PRO_RMSNORM && epi == EPI_STORE) QLM_MX_CALL(false, PRO_RMSNORM, EPI_STORE, false);
    if (pro == PRO_NONE && epi == EPI_RESID) QLM_MX_CALL(false, PRO_NONE, EPI_RESID, false);
    QLM_MX_CALL(false, PRO_RMSNORM, EPI_SWIGLU, false);
#undef QLM_MX_CALL
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
    if (M == 1 && xs_lds_bytes(K, pro) <= kXsLdsMax)
        return xs_dispatch(pro, epi, xs_config(N, K, epi), x, nw, eps, q, sc, rowscale, y, N, K,
                           st);
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

extern "C" int qlm_gemv_i8_config(const float* x, const float* norm_w, float eps,
                                  const int8_t* q, const float* scales, int group, float* y, int N,
                                  int K, int epilogue, int lanes_per_row, int rows, int grid,
                                  void* stream) {
    if (!x || !q || !scales || !y || N <= 0 || K <= 0 || grid <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    if (K % 16 != 0) return QLM_ERR_SHAPE;
    const bool rowscale = (group == K);
    if (!rowscale && (group != 32 || K % 32 != 0)) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)q | (uintptr_t)norm_w) & 15u) return QLM_ERR_SHAPE;
    if (lanes_per_row < 16 || lanes_per_row > kThreads ||
        (lanes_per_row & (lanes_per_row - 1)) != 0 || (rows != 1 && rows != 2))
        return QLM_ERR_SHAPE;
    const int pro = norm_w ? PRO_RMSNORM : PRO_NONE;
    if (epilogue == EPI_SWIGLU && !norm_w) return QLM_ERR_ARG;  // only the fused-norm form exists
    XsConfig c;
    c.lpr = lanes_per_row;
    c.slots = ((K >> 4) + lanes_per_row - 1) / lanes_per_row;
    if (c.slots > 6) return QLM_ERR_SHAPE;
    c.R = epilogue == EPI_SWIGLU ? 2 * rows : rows;
    c.grid = grid;
    c.balance = false;
    if (xs_lds_bytes(K, pro) > kXsLdsMax) return QLM_ERR_SHAPE;
    if (epilogue == EPI_RESID && pro == PRO_RMSNORM) return QLM_ERR_ARG;
    return xs_dispatch(pro, epilogue, c, x, norm_w, eps, q, scales, rowscale, y, N, K,
                       as_stream(stream));
}

extern "C" int qlm_mx_layout_bytes(int rows, int K, int group, int halves, size_t* q_bytes,
                                   size_t* s_bytes) {
    if (rows <= 0 || K <= 0 || K % 64 != 0 || (halves != 1 && halves != 2) || !q_bytes ||
        !s_bytes)
        return QLM_ERR_ARG;
    if (group != 32 && group != K) return QLM_ERR_SHAPE;
    const size_t tiles = (size_t)(rows + 15) / 16;
    *q_bytes = halves * tiles * 16 * (size_t)K;
    *s_bytes = group == 32 ? halves * tiles * (size_t)(K / 64) * 32 * sizeof(float) : 0;
    return QLM_OK;
}

extern "C" int qlm_mx_swizzle(const int8_t* q, const float* scales, int group, int rows, int K,
                              int halves, int8_t* q_out, float* s_out, void* stream) {
    size_t qb = 0, sb = 0;
    const int rc = qlm_mx_layout_bytes(rows, K, group, halves, &qb, &sb);
    if (rc != QLM_OK) return rc;
    if (!q || !q_out || (sb && (!scales || !s_out))) return QLM_ERR_ARG;
    if (((uintptr_t)q | (uintptr_t)q_out) & 15u) return QLM_ERR_SHAPE;
    const int tiles = (rows + 15) / 16;
    const size_t chunks = qb / 16;
    const int grid = (int)((chunks + 255) / 256 < 65536 ? (chunks + 255) / 256 : 65536);
    hipLaunchKernelGGL(k_mx_swizzle, dim3(grid), dim3(256), 0, as_stream(stream), q,
                       sb ? scales : nullptr, rows, K, tiles, halves, q_out,
                       sb ? s_out : nullptr);
    return qlm_launch_status();
}

extern "C" int qlm_gemv_i8_mx_config(const float* x, const float* norm_w, float eps,
                                     const int8_t* q, const float* scales, int group, float* y,
                                     int N, int K, int epilogue, int waves, int ring, int grid,
                                     void* stream) {
    if (!x || !q || !scales || !y || N <= 0 || K <= 0 || grid <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    const bool rowscale = (group == K);
    if (!rowscale && group != 32) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)q | (uintptr_t)norm_w) & 15u) return QLM_ERR_SHAPE;
    const int pro = norm_w ? PRO_RMSNORM : PRO_NONE;
    if (epilogue == EPI_SWIGLU && !norm_w) return QLM_ERR_ARG;  // only the fused-norm form exists
    if (epilogue == EPI_RESID && pro == PRO_RMSNORM) return QLM_ERR_ARG;
    return mx_dispatch(pro, epilogue, MxConfig{waves, ring, grid}, x, norm_w, eps, q, scales,
                       rowscale, y, N, K, as_stream(stream));
}

extern "C" size_t qlm_lm_head_greedy_workspace_bytes(void) {
    return (size_t)kMaxXsGrid * sizeof(unsigned long long);
}

extern "C" int qlm_lm_head_greedy(const float* x, const float* norm_w, float eps, const int8_t* q,
                                  const float* scales, int group, float* logits, int V, int K,
                                  void* work, int* tokens, int ld_tokens, int* pos,
                                  const int* prompt_len, const float* embed, int H, float* h_next,
                                  void* stream) {
    if (!x || !norm_w || !q || !scales || !logits || !work || !tokens || !pos || !prompt_len ||
        !embed || !h_next || V <= 0 || K <= 0 || H <= 0 || ld_tokens <= 0)
        return QLM_ERR_ARG;
    if (K % 16 != 0) return QLM_ERR_SHAPE;
    const bool rowscale = (group == K);
    if (!rowscale && (group != 32 || K % 32 != 0)) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)q | (uintptr_t)norm_w | (uintptr_t)work) & 15u)
        return QLM_ERR_SHAPE;
    const XsConfig c = xs_config(V, K, EPI_STORE);
    if (c.grid > kMaxXsGrid || xs_lds_bytes(K, PRO_RMSNORM) > kXsLdsMax) return QLM_ERR_SHAPE;
    return xs_dispatch(PRO_RMSNORM, EPI_ARGMAX, c, x, norm_w, eps, q, scales, rowscale, logits, V,
                       K, as_stream(stream),
                       greedy_tail(work, tokens, ld_tokens, pos, prompt_len, embed, H, V, h_next));
}

extern "C" int qlm_lm_head_greedy_mx(const float* x, const float* norm_w, float eps,
                                     const int8_t* q_tiles, const float* s_tiles, int group,
                                     float* logits, int V, int K, void* work, int* tokens,
                                     int ld_tokens, int* pos, const int* prompt_len,
                                     const float* embed, int H, float* h_next, void* stream) {
    if (!x || !norm_w || !q_tiles || !s_tiles || !logits || !work || !tokens || !pos ||
        !prompt_len || !embed || !h_next || V <= 0 || K <= 0 || H <= 0 || ld_tokens <= 0)
        return QLM_ERR_ARG;
    const bool rowscale = (group == K);
    if (!rowscale && group != 32) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)q_tiles | (uintptr_t)norm_w | (uintptr_t)work) & 15u)
        return QLM_ERR_SHAPE;
    const MxConfig c = mx_config(V, K, EPI_ARGMAX, false, group);
    if (c.nw == 0) return QLM_ERR_SHAPE;
    return mx_dispatch(PRO_RMSNORM, EPI_ARGMAX, c, x, norm_w, eps, q_tiles, s_tiles, rowscale,
                       logits, V, K, as_stream(stream),
                       greedy_tail(work, tokens, ld_tokens, pos, prompt_len, embed, H, V, h_next));
}

extern "C" int qlm_gemv_i8_mx_shape(int N, int K, int epilogue, int* waves, int* ring,
                                    int* grid) {
    if (N <= 0 || K <= 0 || !waves || !ring || !grid) return QLM_ERR_ARG;
    const MxConfig c = mx_config(N, K, epilogue);
    if (c.nw == 0 || !mx_fits(K, c.nw, c.ring)) return QLM_ERR_SHAPE;
    *waves = c.nw;
    *ring = c.ring;
    *grid = c.grid;
    return QLM_OK;
}

extern "C" int qlm_gemv_mx_l2_plan(const void* q_tiles, const float* s_tiles, int group, int int4,
                                   int N, int K, int epilogue, int max_tiles, qlm_l2_plan* plan) {
    if (!q_tiles || !plan || N <= 0 || K <= 0 || max_tiles < 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    const bool rowscale = (group == K);
    if (!rowscale && (group != 32 || !s_tiles)) return QLM_ERR_SHAPE;
    if (int4 && rowscale) return QLM_ERR_SHAPE;
    const MxConfig c = mx_config(N, K, epilogue, int4 != 0, group);
    if (c.nw == 0 || K % 64 != 0) return QLM_ERR_SHAPE;
    const int ntiles = (N + 15) / 16, nblk = K / 64, T = epilogue == EPI_SWIGLU ? 2 : 1;
    const int grid = c.grid < ntiles ? c.grid : ntiles;  // as launch_mx
    const int tiles = max_tiles < grid ? max_tiles : grid;
    const int nseg = T * (rowscale ? 1 : 2);
    if (plan->nseg < 0 || plan->nseg + nseg > QLM_L2_PLAN_SEGMENTS) return QLM_ERR_SHAPE;
    if (tiles == 0) return QLM_OK;
    // fragment (tile t of half tt, block b) at (t + tt * ntiles) * nblk + b:
    // 1 KB of int8 (512 B of int4) and 32 scales
    const long long fq = int4 ? 512 : 1024, fs = 32 * sizeof(float);
    for (int tt = 0; tt < T; ++tt) {
        const long long f0 = (long long)tt * ntiles * nblk;
        int s = plan->nseg++;
        plan->base[s] = static_cast<const char*>(q_tiles) + f0 * fq;
        plan->stride[s] = nblk * fq;
        plan->bytes[s] = (int)(nblk * fq);
        plan->tiles[s] = tiles;
        if (rowscale) continue;
        s = plan->nseg++;
        plan->base[s] = reinterpret_cast<const char*>(s_tiles) + f0 * fs;
        plan->stride[s] = nblk * fs;
        plan->bytes[s] = (int)(nblk * fs);
        plan->tiles[s] = tiles;
    }
    return QLM_OK;
}

extern "C" int qlm_gemv_i8_mx(const float* x, const float* norm_w, float eps,
                              const int8_t* q_tiles, const float* s_tiles, int group, float* y,
                              int N, int K, int epilogue, void* stream) {
    if (!x || !q_tiles || !s_tiles || !y || N <= 0 || K <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    const bool rowscale = (group == K);
    if (!rowscale && group != 32) return QLM_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)q_tiles | (uintptr_t)norm_w) & 15u) return QLM_ERR_SHAPE;
    const int pro = norm_w ? PRO_RMSNORM : PRO_NONE;
    if (epilogue == EPI_SWIGLU && !norm_w) return QLM_ERR_ARG;
    if (epilogue == EPI_RESID && pro == PRO_RMSNORM) return QLM_ERR_ARG;
    const MxConfig c = mx_config(N, K, epilogue, false, group);
    if (c.nw == 0) return QLM_ERR_SHAPE;
    return mx_dispatch(pro, epilogue, c, x, norm_w, eps, q_tiles, s_tiles, rowscale, y, N, K,
                       as_stream(stream));
}

// The column-split DeltaNet mixer's output through a projection: x[j] =
// u[j] / sqrt(sum of ss[j / 128][0..7] / 128 + eps), per 128-column head.
namespace {
int headnorm_mx(const float* u, const float* ss, float eps, const int8_t* q, const float* s,
                int group, float* y, int N, int K, int epilogue, bool w4, void* stream) {
    if (!u || !ss || !q || !s || !y || N <= 0 || K <= 0) return QLM_ERR_ARG;
    if (epilogue != EPI_STORE && epilogue != EPI_RESID) return QLM_ERR_ARG;
    if (K % 128 != 0) return QLM_ERR_SHAPE;  // whole heads of 128 columns
    const bool rowscale = (group == K);
    if (!rowscale && group != 32) return QLM_ERR_SHAPE;
    if (((uintptr_t)u | (uintptr_t)q | (uintptr_t)ss) & 15u) return QLM_ERR_SHAPE;
    const MxConfig c = mx_config(N, K, epilogue, w4);
    if (c.nw == 0) return QLM_ERR_SHAPE;
    return mx_dispatch(PRO_HEADNORM, epilogue, c, u, ss, eps, q, s, rowscale, y, N, K,
                       as_stream(stream), GreedyTail{}, w4);
}
}  // namespace

extern "C" int qlm_gemv_i8_mx_headnorm(const float* u, const float* ss, float eps,
                                       const int8_t* q_tiles, const float* s_tiles, int group,
                                       float* y, int N, int K, int epilogue, void* stream) {
    return headnorm_mx(u, ss, eps, q_tiles, s_tiles, group, y, N, K, epilogue, false, stream);
}

extern "C" int qlm_gemv_i4_mx_headnorm(const float* u, const float* ss, float eps,
                                       const uint8_t* q_tiles, const float* s_tiles, float* y,
                                       int N, int K, int epilogue, void* stream) {
    return headnorm_mx(u, ss, eps, reinterpret_cast<const int8_t*>(q_tiles), s_tiles, 32, y, N,
                       K, epilogue, true, stream);
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

// ---- int4 (Q4_0) weights on the matrix cores ----

extern "C" int qlm_mx4_layout_bytes(int rows, int K, int halves, size_t* q_bytes,
                                    size_t* s_bytes) {
    size_t qb = 0;
    const int rc = qlm_mx_layout_bytes(rows, K, 32, halves, &qb, s_bytes);
    if (rc != QLM_OK) return rc;
    *q_bytes = qb / 2;
    return QLM_OK;
}

extern "C" int qlm_mx4_swizzle(const uint8_t* q4, const float* scales, int rows, int K,
                               int halves, uint8_t* q_out, float* s_out, void* stream) {
    size_t qb = 0, sb = 0;
    const int rc = qlm_mx4_layout_bytes(rows, K, halves, &qb, &sb);
    if (rc != QLM_OK) return rc;
    if (!q4 || !scales || !q_out || !s_out) return QLM_ERR_ARG;
    if (((uintptr_t)q4 | (uintptr_t)q_out) & 7u) return QLM_ERR_SHAPE;
    const int tiles = (rows + 15) / 16;
    const size_t lanes = qb / 8;
    const int grid = (int)((lanes + 255) / 256 < 65536 ? (lanes + 255) / 256 : 65536);
    hipLaunchKernelGGL(k_mx4_swizzle, dim3(grid), dim3(256), 0, as_stream(stream), q4, scales,
                       rows, K, tiles, halves, q_out, s_out);
    return qlm_launch_status();
}

extern "C" int qlm_gemv_i4_mx_config(const float* x, const float* norm_w, float eps,
                                     const uint8_t* q_tiles, const float* s_tiles, float* y,
                                     int N, int K, int epilogue, int waves, int ring, int grid,
                                     void* stream) {
    if (!x || !q_tiles || !s_tiles || !y || N <= 0 || K <= 0 || grid <= 0) return QLM_ERR_ARG;
    if (epilogue < EPI_STORE || epilogue > EPI_SWIGLU) return QLM_ERR_ARG;
    if (((uintptr_t)x | (uintptr_t)q_tiles | (uintptr_t)norm_w) & 15u) return QLM_ERR_SHAPE;
    const int pro = norm_w ? PRO_RMSNORM : PRO_NONE;
    if (epilogue == EPI_SWIGLU && !norm_w) return QLM_ERR_ARG;
    if (epilogue == EPI_RESID && pro == PRO_RMSNORM) return QLM_ERR_ARG;
    return mx_dispatch(pro, epilogue, MxConfig{waves, ring, grid}, x, norm_w, eps,
                       reinterpret_cast<const int8_t*>(q_tiles), s_tiles, false, y, N, K,
                       as_stream(stream), GreedyTail{}, true);
}

extern "C" int qlm_gemv_i4_mx(const float* x, const float* norm_w, float eps,
                              const uint8_t* q_tiles, const float* s_tiles, float* y, int N,
                              int K, int epilogue, void* stream) {
    if (N <= 0 || K <= 0) return QLM_ERR_ARG;
    const MxConfig c = mx_config(N, K, epilogue, true);
    if (c.nw == 0) return QLM_ERR_SHAPE;
    return qlm_gemv_i4_mx_config(x, norm_w, eps, q_tiles, s_tiles, y, N, K, epilogue, c.nw,
                                 c.ring, c.grid, stream);
}

extern "C" int qlm_lm_head_greedy_mx4(const float* x, const float* norm_w, float eps,
                                      const uint8_t* q_tiles, const float* s_tiles, float* logits,
                                      int V, int K, void* work, int* tokens, int ld_tokens,
                                      int* pos, const int* prompt_len, const float* embed, int H,
                                      float* h_next, void* stream) {
    if (!x || !norm_w || !q_tiles || !s_tiles || !logits || !work || !tokens || !pos ||
        !prompt_len || !embed || !h_next || V <= 0 || K <= 0 || H <= 0 || ld_tokens <= 0)
        return QLM_ERR_ARG;
    if (((uintptr_t)x | (uintptr_t)q_tiles | (uintptr_t)norm_w | (uintptr_t)work) & 15u)
        return QLM_ERR_SHAPE;
    const MxConfig c = mx_config(V, K, EPI_ARGMAX, true);
    if (c.nw == 0) return QLM_ERR_SHAPE;
    return mx_dispatch(PRO_RMSNORM, EPI_ARGMAX, c, x, norm_w, eps,
                       reinterpret_cast<const int8_t*>(q_tiles), s_tiles, false, logits, V, K,
                       as_stream(stream),
                       greedy_tail(work, tokens, ld_tokens, pos, prompt_len, embed, H, V, h_next),
                       true);
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_gemv() {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(k_greedy_finish));
}
