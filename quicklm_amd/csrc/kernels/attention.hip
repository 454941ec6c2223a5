// GQA decode attention over a contiguous, position-major KV cache
// [B, max_seq, n_kv, hd] (reference: Qwen3_5Attention::forward,
// attention.cpp:138-232; gqa_attend_head :54-82).
//
// Two launches (split-K "flash decoding"):
//   k_attn          one workgroup per (chunk of CH positions, kv head g,
//                   sequence b); the G = n_q/n_kv query heads of the group
//                   share every K/V row read. The chunk's K and V rows (one
//                   sub-tile of T positions at a time: 64 at hd 128, 32 at
//                   hd 256) are requested before anything else, so their HBM
//                   latency overlaps the prologue:
//     PREP          QK-norm (zero-centred gain, eps 1e-6) and partial NeoX
//                   RoPE of the group's query heads from the projection row;
//                   the workgroup whose chunk holds p = pos[b] also
//                   normalises/rotates k_p and writes k_p, v_p into the cache
//                   (attention.cpp:166-199), using the LDS copy of that row
//                   itself. Other chunks never read row p.
//     scores        s = q.k * 1/sqrt(hd) (16 lanes x 8 floats per K row).
//     softmax/PV    running max and sum across sub-tiles, P.V with float4 V
//                   rows; the chunk leaves a record [m, l, -, -, o[hd]] per
//                   query head.
//   k_attn_combine  one workgroup per (query head, sequence) merges the
//                   records and applies the sigmoid output gate
//                   (attention.cpp:216-227). The kernel boundary orders the
//                   two, so no workgroup needs a device-scope fence.
// The graph-captured decode step launches the grid for max_seq; chunks past
// pos[b] exit at once and are not counted.

#include <mutex>

#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kNW = kThreads / QLM_WAVE;

// Position reads: a launch with a position array reads pos[b], one without
// reads this zero and ignores it, so the read is one unconditional load
// (not a load under a branch, which the compiler waits for where the
// branch ends). The kernels also name every argument in an empty asm at
// their start: without it the compiler reads a few arguments, waits and
// branches, then reads the rest, one more scalar round trip before the
// first operand load.
__device__ int g_pos_zero = 0;

template <typename KV>
__device__ __forceinline__ void load8(const KV* p, float (&o)[8]);
template <>
__device__ __forceinline__ void load8<float>(const float* p, float (&o)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float (&o)[8]) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[2 * i] = __uint_as_float(w[i] << 16);
        o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

template <typename KV>
__device__ __forceinline__ float4 load4(const KV* p);
template <>
__device__ __forceinline__ float4 load4<float>(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}
template <>
__device__ __forceinline__ float4 load4<uint16_t>(const uint16_t* p) {
    const uint2 a = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(a.x << 16), __uint_as_float(a.x & 0xffff0000u),
                       __uint_as_float(a.y << 16), __uint_as_float(a.y & 0xffff0000u));
}

template <int HD, int G, int T, int NT, typename KV, bool PREP>
__global__ __launch_bounds__(kThreads) void k_attn(
    const float* __restrict__ qsrc, int ldq, int qhs, const float* __restrict__ qn_w,
    const float* __restrict__ kn_w, const float* __restrict__ cos_tab,
    const float* __restrict__ sin_tab, int rot, KV* __restrict__ kc, KV* __restrict__ vc,
    int max_seq, int n_kv, const int* __restrict__ pos, int ctx, int pstep, size_t kvb,
    float* __restrict__ work, int nchunks, int n_q, float scale) {
    static_assert(!PREP || sizeof(KV) == 4, "the fused prologue writes an fp32 cache");
    constexpr int LPP = HD / 8;            // lanes per position in the score phase
    constexpr int PPW = QLM_WAVE / LPP;    // positions per wave per score step
    constexpr int SPS = kNW * PPW;         // positions per workgroup per score step
    constexpr int NS = T / SPS;            // K rows per lane per sub-tile
    constexpr int C4 = HD / 4;             // float4 columns of a row
    constexpr int NPG = kThreads / C4;     // position groups in the PV phase
    constexpr int NV = T / NPG;            // V float4 per lane per sub-tile
    constexpr int CH = T * NT;             // positions per chunk (workgroup)
    constexpr int EPL = HD / QLM_WAVE;     // row elements per lane in the norm phase
    constexpr int RPW = (G + kNW - 1) / kNW;  // query rows per wave in the norm phase
    static_assert(T % SPS == 0 && T % NPG == 0, "sub-tile must cover whole load steps");
    __shared__ float qs[G][HD];
    __shared__ float sc[G][T];
    __shared__ float4 red[NPG][G][C4];
    __shared__ float kvp[2][HD];
    __shared__ float fsc[G], mstat[G], lstat[G];

    asm volatile("" ::"s"(qsrc), "s"(ldq), "s"(qhs), "s"(qn_w), "s"(kn_w), "s"(cos_tab),
                 "s"(sin_tab), "s"(rot), "s"(kc), "s"(vc), "s"(max_seq), "s"(n_kv), "s"(pos),
                 "s"(ctx), "s"(pstep), "s"(kvb), "s"(work), "s"(nchunks), "s"(n_q), "s"(scale));
    const int chunk = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // query row b sits at position pos[b], or ctx-1 + pstep*b (pstep = 1:
    // consecutive prompt rows over one shared cache, kvb = 0)
    const int pp = *(pos ? pos + b : &g_pos_zero);
    const int p = pos ? pp : ctx - 1 + pstep * b;
    const int L = min(p + 1, max_seq);
    const int nc = (L + CH - 1) / CH;
    if (chunk >= nc || p < 0) return;
    const int start = chunk * CH;
    const int n = min(CH, L - start);
    const float* qrow = qsrc + (size_t)b * ldq;
    const bool own_p = PREP && (p / CH == chunk);
    const int plp = own_p ? p - start : -1;  // local index of the row written this step

    // ---- sub-tile 0's K and V rows are requested first ----
    // Row indices are clamped into the chunk (duplicates are masked later),
    // so the loads never branch. Row p of the cache is stale until this
    // launch writes it; its values are taken from LDS below instead.
    const int sub = lane % LPP, pw = lane / LPP;
    const int c4 = tid % C4, pg = tid / C4;
    const size_t row0 = ((size_t)b * kvb + start) * n_kv + g;
    float kr[NS][8];
    float4 vv[NV];
    auto load_k = [&](int t0) {
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const int pl = min(t0 + u * SPS + wave * PPW + pw, n - 1);
            load8<KV>(kc + (row0 + (size_t)pl * n_kv) * HD + sub * 8, kr[u]);
        }
    };
    auto load_v = [&](int t0) {
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int pl = min(t0 + u * NPG + pg, n - 1);
            vv[u] = load4<KV>(vc + (row0 + (size_t)pl * n_kv) * HD + c4 * 4);
        }
    };
    // ---- prologue operands first: loads complete in order, so operands
    // requested after the K/V rows could only be used once those arrived.
    // Every load is unconditional (clamped or substitute address; unused
    // values are dropped later): a load under a branch makes the compiler
    // wait for it where the branch ends, ahead of the K/V requests.
    constexpr int RI = ((G + 1) * (HD / 2) + kThreads - 1) / kThreads;  // RoPE items per thread
    float qv[RPW][EPL], gq[EPL], gk[EPL], kp[EPL], vp[EPL], cr[RI], sr[RI];
    const bool k_wave = own_p && wave == kNW - 1;
    const int half = rot / 2;
    if constexpr (PREP) {
        // wave w normalises query rows w, w + kNW, ...; the last wave also
        // takes k_p when this chunk owns p
        const float* gqp = qn_w ? qn_w : qrow;
        const float* gkp = kn_w ? kn_w : qrow;
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int r = min(wave + i * kNW, G - 1);
#pragma unroll
            for (int j = 0; j < EPL; ++j)
                qv[i][j] = qrow[(size_t)(g * G + r) * qhs + lane + j * QLM_WAVE];
        }
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + j * QLM_WAVE;
            gq[j] = gqp[e];
            gk[j] = gkp[e];
            kp[j] = qrow[(size_t)n_q * qhs + (size_t)g * HD + e];
            vp[j] = qrow[(size_t)n_q * qhs + (size_t)(n_kv + g) * HD + e];
        }
        // cos/sin of this thread's RoPE items i = tid + k*kThreads (column i % half)
#pragma unroll
        for (int k = 0; k < RI; ++k) {
            const size_t o = half > 0 ? (size_t)p * half + (tid + k * kThreads) % half : 0;
            cr[k] = (half > 0 ? cos_tab : qrow)[o];
            sr[k] = (half > 0 ? sin_tab : qrow)[o];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_k(0);
    load_v(0);

    // ---- query rows (+ QK-norm, RoPE, k_p/v_p when PREP) ----
    if constexpr (PREP) {
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int r = wave + i * kNW;
            if (r < G) {  // wave-uniform
                if (qn_w) {
                    float ss = 0.0f;
#pragma unroll
                    for (int j = 0; j < EPL; ++j) ss = fmaf(qv[i][j], qv[i][j], ss);
                    ss = wave_sum(ss);
                    const float s = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
#pragma unroll
                    for (int j = 0; j < EPL; ++j) qv[i][j] = (qv[i][j] * s) * (1.0f + gq[j]);
                }
#pragma unroll
                for (int j = 0; j < EPL; ++j) qs[r][lane + j * QLM_WAVE] = qv[i][j];
            }
        }
        if (k_wave) {
            if (kn_w) {
                float ss = 0.0f;
#pragma unroll
                for (int j = 0; j < EPL; ++j) ss = fmaf(kp[j], kp[j], ss);
                ss = wave_sum(ss);
                const float s = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
#pragma unroll
                for (int j = 0; j < EPL; ++j) kp[j] = (kp[j] * s) * (1.0f + gk[j]);
            }
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                kvp[0][lane + j * QLM_WAVE] = kp[j];
                kvp[1][lane + j * QLM_WAVE] = vp[j];
            }
        }
        __syncthreads();
        // NeoX rotation of the first `rot` dims (attention.cpp:181-188)
        const int nrows = G + (own_p ? 1 : 0);
#pragma unroll
        for (int k = 0; k < RI; ++k) {
            const int i = tid + k * kThreads;
            if (i < nrows * half) {
                const int r = i / half, j = i % half;
                float* v = r < G ? qs[r] : kvp[0];
                const float x1 = v[j], x2 = v[j + half];
                v[j] = nc_mul_sub(x1, cr[k], x2, sr[k]);
                v[j + half] = nc_mul_add2(x2, cr[k], x1, sr[k]);
            }
        }
        __syncthreads();
        if (own_p) {
            const size_t off = (((size_t)b * kvb + p) * n_kv + g) * HD;
            for (int i = tid; i < HD; i += kThreads) {
                kc[off + i] = kvp[0][i];
                vc[off + i] = kvp[1][i];
            }
        }
    } else {
        for (int i = tid; i < G * HD; i += kThreads)
            qs[i / HD][i % HD] = qrow[(size_t)(g * G + i / HD) * qhs + i % HD];
        __syncthreads();
    }

    float qr[G][8];
#pragma unroll
    for (int gh = 0; gh < G; ++gh)
#pragma unroll
        for (int e = 0; e < 8; ++e) qr[gh][e] = qs[gh][sub * 8 + e];
    float4 acc[G];
#pragma unroll
    for (int gh = 0; gh < G; ++gh) acc[gh] = make_float4(0.f, 0.f, 0.f, 0.f);
    // running softmax state of head gh lives in the wave that owns it
    float m_run[RPW], l_run[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.0f;
    }

    // Sub-tile t+1's K rows are requested once sub-tile t's scores have
    // consumed kr, its V rows once t's P.V has consumed vv, so each sub-tile's
    // loads overlap the previous one's softmax and P.V.
    for (int t = 0; t < NT; ++t) {
        const int t0 = t * T;
        if (t0 >= n) break;  // uniform
        const int nt = min(T, n - t0);
        const bool more = t + 1 < NT && t0 + T < n;

        // ---- scores s = q.k * scale ----
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const int pli = u * SPS + wave * PPW + pw;
            if (t0 + pli == plp) {
#pragma unroll
                for (int e = 0; e < 8; ++e) kr[u][e] = kvp[0][sub * 8 + e];
            }
#pragma unroll
            for (int gh = 0; gh < G; ++gh) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(qr[gh][e], kr[u][e], d);
                d = group_sum<LPP>(d);
                if (sub == 0 && pli < nt) sc[gh][pli] = d * scale;
            }
        }
        if (more) load_k(t0 + T);
        __syncthreads();

        // ---- per-head max, exponentials, sums (online across sub-tiles) ----
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int gh = wave + i * kNW;
            if (gh < G) {
                float m = -INFINITY;
                for (int pl = lane; pl < nt; pl += QLM_WAVE) m = fmaxf(m, sc[gh][pl]);
                m = fmaxf(wave_max(m), m_run[i]);
                float l = 0.0f;
                for (int pl = lane; pl < nt; pl += QLM_WAVE) {
                    const float e = expf(sc[gh][pl] - m);
                    sc[gh][pl] = e;
                    l += e;
                }
                l = wave_sum(l);
                const float f = expf(m_run[i] - m);  // 0 on the first sub-tile
                l_run[i] = fmaf(l_run[i], f, l);
                m_run[i] = m;
                if (lane == 0) fsc[gh] = f;
            }
        }
        __syncthreads();

        // ---- P.V ----
#pragma unroll
        for (int gh = 0; gh < G; ++gh) {
            if (t > 0) {
                const float f = fsc[gh];
                acc[gh].x *= f;
                acc[gh].y *= f;
                acc[gh].z *= f;
                acc[gh].w *= f;
            }
        }
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int pli = u * NPG + pg;
            if (t0 + pli == plp) vv[u] = reinterpret_cast<const float4*>(kvp[1])[c4];
            if (pli < nt) {
#pragma unroll
                for (int gh = 0; gh < G; ++gh) {
                    const float e = sc[gh][pli];
                    acc[gh].x = fmaf(e, vv[u].x, acc[gh].x);
                    acc[gh].y = fmaf(e, vv[u].y, acc[gh].y);
                    acc[gh].z = fmaf(e, vv[u].z, acc[gh].z);
                    acc[gh].w = fmaf(e, vv[u].w, acc[gh].w);
                }
            }
        }
        if (more) load_v(t0 + T);
        if (NT > 1) __syncthreads();  // sc is rewritten by the next sub-tile
    }

    // ---- chunk record [m, l, -, -, o[HD]] per query head ----
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int gh = wave + i * kNW;
        if (gh < G && lane == 0) {
            mstat[gh] = m_run[i];
            lstat[gh] = l_run[i];
        }
    }
#pragma unroll
    for (int gh = 0; gh < G; ++gh) red[pg][gh][c4] = acc[gh];
    __syncthreads();
    for (int i = tid; i < G * C4; i += kThreads) {
        const int gh = i / C4, cc = i % C4;
        float4 tt = red[0][gh][cc];
#pragma unroll
        for (int p2 = 1; p2 < NPG; ++p2) {
            const float4 u = red[p2][gh][cc];
            tt.x += u.x;
            tt.y += u.y;
            tt.z += u.z;
            tt.w += u.w;
        }
        float* dst = work + (((size_t)b * n_q + g * G + gh) * nchunks + chunk) * (HD + 4);
        reinterpret_cast<float4*>(dst + 4)[cc] = tt;
        if (cc == 0) {
            dst[0] = mstat[gh];
            dst[1] = lstat[gh];
        }
    }
}

// Merge of the chunk records of one (query head, sequence), then the
// optional sigmoid output gate (attention.cpp:216-227): gate[b*ldg + h*ghs +
// HD + e]. 256 threads: thread (cg, c4) takes float4 column c4 of the
// chunks c = cg, cg + NG, ...; the chunk weights meet in LDS (their sum of
// weighted l as a block reduction), and the NG chunk groups meet at the end
// (within a wave by shuffles, then across the four waves in LDS). Everything the first pass
// needs -- (m, l) of chunk tid, the first KB records of the thread's chunks
// and the gate -- is requested at kernel start with clamped, unconditional
// loads, so a short context costs one memory round trip. Up to kCombineTile
// chunks per pass (a running maximum rescales across passes).
constexpr int kCombineThreads = 256;
constexpr int kCombineTile = 256;

template <int HD, int CS>
__global__ __launch_bounds__(kCombineThreads) void k_attn_combine(
    const float* __restrict__ work, int nchunks, int CH, int max_seq, const int* __restrict__ pos,
    int ctx, int pstep, const float* __restrict__ gate, int ldg, int ghs, float* __restrict__ out,
    int ldo, int n_q) {
    // CS workgroups (blockIdx.z) split a head's columns: few (head,
    // sequence) pairs would otherwise leave most of the GPU idle
    constexpr int C4 = HD / 4 / CS;               // float4 columns of this workgroup
    constexpr int NG = kCombineThreads / C4;      // chunk groups
    constexpr int KB = 8;                         // records per thread per request batch
    constexpr int RS = HD + 4;                    // record stride (floats)
    __shared__ float fs[kCombineTile];
    __shared__ float4 part[NG][C4];
    __shared__ float red[kCombineThreads / QLM_WAVE], red_l[kCombineThreads / QLM_WAVE];
    asm volatile("" ::"s"(work), "s"(nchunks), "s"(CH), "s"(max_seq), "s"(pos), "s"(ctx),
                 "s"(pstep), "s"(gate), "s"(ldg), "s"(ghs), "s"(out), "s"(ldo), "s"(n_q));
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int c4 = tid % C4, cg = tid / C4;
    const int cb = blockIdx.z * C4;  // first float4 column of this workgroup
    const int pp = *(pos ? pos + b : &g_pos_zero);
    const int L = min(pos ? pp + 1 : ctx + pstep * b, max_seq);
    const int nc = min(nchunks, (L + CH - 1) / CH);
    const int last = max(nc, 1) - 1;  // clamp target of the unconditional loads
    const float* base = work + ((size_t)b * n_q + h) * nchunks * RS;

    // ---- first-pass operands, all requested before any is used ----
    auto rec4 = [&](int c) {  // float4 column c4 of record c (clamped into the context)
        return reinterpret_cast<const float4*>(base + (size_t)min(c, last) * RS + 4)[cb + c4];
    };
    float mc = base[(size_t)min(tid, last) * RS];
    float lc = base[(size_t)min(tid, last) * RS + 1];
    float4 ov[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) ov[k] = rec4(cg + NG * k);
    const float* gp = (gate ? gate + (size_t)b * ldg + (size_t)h * ghs + HD : base + 4) +
                      (cb + c4) * 4;
    const float gg[4] = {gp[0], gp[1], gp[2], gp[3]};

    float M = -INFINITY, lsum = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c0 = 0; c0 < nc; c0 += kCombineTile) {
        const int nt = min(kCombineTile, nc - c0);
        if (c0 > 0) {
            mc = base[(size_t)(c0 + min(tid, nt - 1)) * RS];
            lc = base[(size_t)(c0 + min(tid, nt - 1)) * RS + 1];
        }
        if (tid >= nt) {
            mc = -INFINITY;
            lc = 0.0f;
        }
        // tile maximum
        float mt = wave_max(mc);
        if ((tid & (QLM_WAVE - 1)) == 0) red[tid / QLM_WAVE] = mt;
        __syncthreads();
        mt = red[0];
#pragma unroll
        for (int w = 1; w < kCombineThreads / QLM_WAVE; ++w) mt = fmaxf(mt, red[w]);
        const float Mn = fmaxf(M, mt);
        // chunk weights, and the pass's sum of weighted l over all threads
        const float fc = tid < nt ? expf(mc - Mn) : 0.0f;
        if (tid < nt) fs[tid] = fc;
        float lt = wave_sum(fc * lc);
        if ((tid & (QLM_WAVE - 1)) == 0) red_l[tid / QLM_WAVE] = lt;
        __syncthreads();
        lt = red_l[0];
#pragma unroll
        for (int w = 1; w < kCombineThreads / QLM_WAVE; ++w) lt += red_l[w];
        const float f0 = expf(M - Mn);  // 0 on the first pass
        lsum = fmaf(lsum, f0, lt);
        o.x *= f0;
        o.y *= f0;
        o.z *= f0;
        o.w *= f0;
        for (int k0 = 0; k0 * NG < nt; k0 += KB) {
            if (c0 > 0 || k0 > 0) {
#pragma unroll
                for (int k = 0; k < KB; ++k) ov[k] = rec4(c0 + cg + NG * (k0 + k));
            }
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                const int c = cg + NG * (k0 + k);
                const float f = c < nt ? fs[c] : 0.0f;
                o.x = fmaf(f, ov[k].x, o.x);
                o.y = fmaf(f, ov[k].y, o.y);
                o.z = fmaf(f, ov[k].z, o.z);
                o.w = fmaf(f, ov[k].w, o.w);
            }
        }
        M = Mn;
        __syncthreads();  // fs/red/red_l are rewritten by the next pass
    }
    // the chunk groups of one wave first (lanes of equal c4, by shuffles),
    // then the waves' sums in LDS
    constexpr int NP = C4 < QLM_WAVE ? kCombineThreads / QLM_WAVE : NG;  // partials left
    if constexpr (C4 < QLM_WAVE) {
#pragma unroll
        for (int m = C4; m < QLM_WAVE; m <<= 1) {
            o.x += __shfl_xor(o.x, m, QLM_WAVE);
            o.y += __shfl_xor(o.y, m, QLM_WAVE);
            o.z += __shfl_xor(o.z, m, QLM_WAVE);
            o.w += __shfl_xor(o.w, m, QLM_WAVE);
        }
        if ((tid & (QLM_WAVE - 1)) < C4) part[tid / QLM_WAVE][c4] = o;
    } else {
        part[cg][c4] = o;
    }
    __syncthreads();
    if (cg == 0) {
        float4 t = part[0][c4];
#pragma unroll
        for (int g2 = 1; g2 < NP; ++g2) {
            const float4 u = part[g2][c4];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
        float r[4] = {t.x / lsum, t.y / lsum, t.z / lsum, t.w / lsum};
        if (gate) {
#pragma unroll
            for (int i = 0; i < 4; ++i) r[i] *= 1.0f / (1.0f + expf(-gg[i]));
        }
        float* dst = out + (size_t)b * ldo + (size_t)h * HD + (cb + c4) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = r[i];
    }
}

// Prefill form of k_attn's PREP phase for T consecutive projection rows
// (positions p0 + t, one workgroup per row): QK-norm and partial NeoX RoPE of
// the query heads in place in the row, the same for each k head, and the K/V
// cache rows p0 + t of one sequence (cache [max_seq, n_kv, HD]). Same
// arithmetic as the decode prologue (attention.cpp:166-199 per row).
template <int HD>
__global__ __launch_bounds__(kThreads) void k_gqa_prep_rows(
    float* __restrict__ qkv, int ldq, int qhs, const float* __restrict__ qn_w,
    const float* __restrict__ kn_w, const float* __restrict__ cos_tab,
    const float* __restrict__ sin_tab, int rot, float* __restrict__ kc, float* __restrict__ vc,
    int n_q, int n_kv, int p0) {
    extern __shared__ float rsh[];  // (n_q + n_kv) rows of HD
    constexpr int EPL = HD / QLM_WAVE;
    const int t = blockIdx.x, p = p0 + t;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float* row = qkv + (size_t)t * ldq;
    const int nr = n_q + n_kv;
    for (int r = wave; r < nr; r += kNW) {
        const float* src = r < n_q ? row + (size_t)r * qhs : row + (size_t)n_q * qhs + (size_t)(r - n_q) * HD;
        const float* w = r < n_q ? qn_w : kn_w;
        float v[EPL], gn[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            v[j] = src[lane + j * QLM_WAVE];
            gn[j] = w ? w[lane + j * QLM_WAVE] : 0.0f;
        }
        if (w) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < EPL; ++j) ss = fmaf(v[j], v[j], ss);
            ss = wave_sum(ss);
            const float sc = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
#pragma unroll
            for (int j = 0; j < EPL; ++j) v[j] = (v[j] * sc) * (1.0f + gn[j]);
        }
#pragma unroll
        for (int j = 0; j < EPL; ++j) rsh[r * HD + lane + j * QLM_WAVE] = v[j];
    }
    __syncthreads();
    const int half = rot / 2;
    if (half > 0) {
        const float* ct = cos_tab + (size_t)p * half;
        const float* st = sin_tab + (size_t)p * half;
        for (int i = tid; i < nr * half; i += kThreads) {
            const int r = i / half, j = i % half;
            float* v = rsh + r * HD;
            const float x1 = v[j], x2 = v[j + half];
            v[j] = nc_mul_sub(x1, ct[j], x2, st[j]);
            v[j + half] = nc_mul_add2(x2, ct[j], x1, st[j]);
        }
    }
    __syncthreads();
    for (int i = tid; i < nr * HD; i += kThreads) {
        const int r = i / HD, e = i % HD;
        if (r < n_q)
            row[(size_t)r * qhs + e] = rsh[i];
        else
            kc[((size_t)p * n_kv + (r - n_q)) * HD + e] = rsh[i];
    }
    for (int i = tid; i < n_kv * HD; i += kThreads) {
        const int g = i / HD, e = i % HD;
        vc[((size_t)p * n_kv + g) * HD + e] = row[(size_t)n_q * qhs + (size_t)(n_kv + g) * HD + e];
    }
}

// ---- prefill attention, head_dim 128, fp32 cache, on the fp32 matrix cores ----
//
// One launch per prefill pass, causal, no per-chunk records and no merge: a
// workgroup owns 16 consecutive prompt rows and one kv head, wave w the query
// head g G + w, and walks the keys 0 .. (its last row's position) in tiles of
// 16 with an online softmax per row (attention.cpp:54-82 per row: the scores
// q . k / sqrt(hd), softmax, the weighted sum of V). Both products run on
// v_mfma_f32_16x16x4f32 (A lane l: row l % 16, k l / 16; B lane l: k l / 16,
// column l % 16; D lane l: rows 4 (l / 16) .. +3, column l % 16):
//   S^T = K Q^T: A = 16 keys, B = Q^T of the wave's 16 rows, the head's 128
//     elements split as 32 k-steps of element 32 (l / 16) + s, so a lane
//     loads 32 contiguous floats of its key (and of its query row, once);
//     lane (qd, n) then holds the scores of row n for keys 4 qd .. 4 qd + 3;
//   O^T += V^T P^T: k-step j takes keys 4 qd + j, which is where those
//     scores already are, so the probabilities feed the B operand from the
//     registers that computed them; A lane (qd, n) reads V[key][16 c + n].
// Lane (qd, n) ends with row n's outputs 16 c + 4 qd .. + 3 for c = 0..7.
// Key rows past the tile's last position are clamped to it (their
// probabilities are 0 and the cache beyond is not written yet).
typedef float f32x4 __attribute__((ext_vector_type(4)));

// maximum / sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lane groups of
// a 16-lane column), on lane swaps instead of LDS permutes
__device__ __forceinline__ float cols_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float cols_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int G>
__global__ __launch_bounds__(G * QLM_WAVE) void k_attn_pf(const float* __restrict__ qkv, int ldq,
                                                          int qhs, const float* __restrict__ kc,
                                                          const float* __restrict__ vc, int n_kv,
                                                          int p0, int T, int gated,
                                                          float* __restrict__ out, int ldo,
                                                          float scale) {
    constexpr int HD = 128;
    const int t0 = (gridDim.x - 1 - blockIdx.x) * 16;  // longest tiles first
    const int g = blockIdx.y;
    const int lane = threadIdx.x & (QLM_WAVE - 1), w = threadIdx.x / QLM_WAVE;
    const int h = g * G + w;
    const int qd = lane >> 4, n = lane & 15;
    const int tq = min(t0 + n, T - 1);  // this lane's row (clamped past the pass)
    const int qpos = p0 + tq;
    const int last = p0 + min(t0 + 15, T - 1);  // the tile's last position
    const int ntiles = last / 16 + 1;

    float qv[32];
    {
        const float4* qr =
            reinterpret_cast<const float4*>(qkv + (size_t)tq * ldq + (size_t)h * qhs + 32 * qd);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 x = qr[j];
            qv[4 * j] = x.x;
            qv[4 * j + 1] = x.y;
            qv[4 * j + 2] = x.z;
            qv[4 * j + 3] = x.w;
        }
    }
    f32x4 o[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;
    const size_t kstride = (size_t)n_kv * HD;

    // The workgroup stages each 16-key tile of K and V once in LDS (rows
    // padded to 132 floats: the 16 lanes of a row read distinct banks), two
    // buffers: tile kt + 1 goes from registers to the other buffer while tile
    // kt is multiplied, and tile kt + 2 is requested; one barrier a tile.
    constexpr int NTH = G * QLM_WAVE, RS = 132, NL = 512 / NTH;
    __shared__ __align__(16) float kvs[2][2][16 * RS];
    const int tid = threadIdx.x;
    f32x4 sk[NL], sv[NL];  // vector types: an aggregate copy to LDS would keep them in scratch
    auto fetch = [&](int k0) {
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int i = tid + NTH * u, key = min(k0 + (i >> 5), last), c4 = i & 31;
            const size_t off = (size_t)key * kstride + (size_t)g * HD + 4 * c4;
            sk[u] = *reinterpret_cast<const f32x4*>(kc + off);
            sv[u] = *reinterpret_cast<const f32x4*>(vc + off);
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int u = 0; u < NL; ++u) {
            const int i = tid + NTH * u, r = i >> 5, c4 = i & 31;
            *reinterpret_cast<f32x4*>(&kvs[buf][0][r * RS + 4 * c4]) = sk[u];
            *reinterpret_cast<f32x4*>(&kvs[buf][1][r * RS + 4 * c4]) = sv[u];
        }
    };
    fetch(0);
    stage(0);
    fetch(min(16, 16 * (ntiles - 1)));
    __syncthreads();
    for (int kt = 0; kt < ntiles; ++kt) {
        const int k0 = kt * 16, buf = kt & 1;
        // K row n of the tile, elements 32 qd .. + 31; V[key 4 qd + j][16 c + n]
        float kd[32], vd[4][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 x = *reinterpret_cast<const float4*>(&kvs[buf][0][n * RS + 32 * qd + 4 * j]);
            kd[4 * j] = x.x;
            kd[4 * j + 1] = x.y;
            kd[4 * j + 2] = x.z;
            kd[4 * j + 3] = x.w;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int c = 0; c < 8; ++c) vd[j][c] = kvs[buf][1][(4 * qd + j) * RS + 16 * c + n];
        // S^T: two independent chains over the 32 k-steps
        f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 32; s += 2) {
            s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kd[s], qv[s], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kd[s + 1], qv[s + 1], s1, 0, 0, 0);
        }
        float sc[4], tm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = k0 + 4 * qd + i;
            sc[i] = key <= qpos ? (s0[i] + s1[i]) * scale : -INFINITY;
            tm = fmaxf(tm, sc[i]);
        }
        // the row's maximum over the 16 keys (lanes n, n+16, n+32, n+48)
        tm = cols_max(tm);
        const float mn = fmaxf(m, tm);
        const float alpha = expf(m - mn);  // 0 on the first tile
        float p[4], ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            p[i] = expf(sc[i] - mn);
            ps += p[i];
        }
        ps = cols_sum(ps);
        l = fmaf(l, alpha, ps);
        m = mn;
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[c][i] *= alpha;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int c = 0; c < 8; ++c)
                o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vd[j][c], p[j], o[c], 0, 0, 0);
        stage(buf ^ 1);  // past the end: a copy of the last tile nobody reads
        fetch(min(k0 + 32, 16 * (ntiles - 1)));
        __syncthreads();
    }

    if (t0 + n >= T) return;
    const float* grow = qkv + (size_t)tq * ldq + (size_t)h * qhs + HD;
    float* dst = out + (size_t)tq * ldo + (size_t)h * HD;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int e = 16 * c + 4 * qd;
        float r[4] = {o[c][0] / l, o[c][1] / l, o[c][2] / l, o[c][3] / l};
        if (gated) {
            const float4 gg = *reinterpret_cast<const float4*>(grow + e);
            r[0] *= 1.0f / (1.0f + expf(-gg.x));
            r[1] *= 1.0f / (1.0f + expf(-gg.y));
            r[2] *= 1.0f / (1.0f + expf(-gg.z));
            r[3] *= 1.0f / (1.0f + expf(-gg.w));
        }
        *reinterpret_cast<float4*>(dst + e) = make_float4(r[0], r[1], r[2], r[3]);
    }
}

// ---- bf16 K/V on the matrix cores (the isolated attention, kv_dtype 1) ----
//
// One wave per workgroup owns a chunk of 32 * spw positions of one (kv head
// g, sequence b) and walks it in steps of 16 positions, with its own online
// softmax; the chunk leaves k_attn's record [m, l, -, -, o[HD]] per query
// head, merged by k_attn_combine. Both products run on
// v_mfma_f32_16x16x32_bf16 (lane l = 16 qd + n; A lane: row n, k-slice qd;
// B lane: k-slice qd, column n; D lane: rows 4 qd .. +3, column n):
//   scores  A = the group's query heads, rows 0..7 their bf16 hi parts and
//           rows 8..15 their lo parts (q = hi + lo to 2^-18 |q|; rows of
//           heads >= G zero), B = 16 K rows as stored (bf16 is exact), so
//           one product gives both halves and s = D[h] + D[h + 8] (one lane
//           swap between the wave halves);
//   P.V     on v_mfma_f32_16x16x16_bf16: A = the probabilities, hi rows
//           0..7 and lo rows 8..15 again (through a 512-byte LDS
//           transpose), B = 16 V rows x 16 columns, read
//           column-wise from an LDS copy of the step's V rows (the
//           reduction runs over positions, which lie 512 bytes apart in the
//           cache). The accumulator rows are the heads' hi and lo halves,
//           added once at the end.
// The next step's K rows are requested as soon as the scores have consumed
// the current ones, its V rows once the current ones are in LDS (the last
// step requests nothing: a wave cannot end before its loads return);
// positions past the chunk are clamped onto its last row (their scores are
// -inf).
// Arithmetic intensity is n_q / n_kv flops per cache byte (8 at the 16 / 2
// heads of the long-context workload): on the vector ALUs the dot products
// and their reductions bound the old kernel at ~2.3 TB/s; here the matrix
// cores take them and the loop is HBM-bound.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned bf16_bits(float x) {
    return (unsigned)__builtin_bit_cast(unsigned short, (__bf16)x);
}

// eight floats as the bf16 hi (lo = false) or lo (lo = true) parts
__device__ __forceinline__ bf16x8_t split_part8(const float (&v)[8], bool lo) {
    unsigned w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __bf16 a = (__bf16)v[2 * i], c = (__bf16)v[2 * i + 1];
        float ea = (float)a, ec = (float)c;
        const unsigned ha = (unsigned)__builtin_bit_cast(unsigned short, a);
        const unsigned hc = (unsigned)__builtin_bit_cast(unsigned short, c);
        const unsigned la = bf16_bits(v[2 * i] - ea), lc = bf16_bits(v[2 * i + 1] - ec);
        w[i] = lo ? (la | (lc << 16)) : (ha | (hc << 16));
    }
    return __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
}

// maximum over each row of 16 lanes; every lane of the row gets it
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<kDppXor1>(v));
    v = fmaxf(v, dpp_mov<kDppXor2>(v));
    v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
    return fmaxf(v, dpp_mov<kDppMirror>(v));
}

// D[r] + D[r + 8] of a 16 x 16 tile whose rows 8..15 (lanes 32..63) hold the
// lo halves of rows 0..7: every lane gets the sum for its (qd & 1, n)
__device__ __forceinline__ float add_halves(float d) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(d), __float_as_uint(d), false,
                                                    false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

template <int HD, int G>
__global__ __launch_bounds__(QLM_WAVE, 2) void k_attn_mx(
    const float* __restrict__ q, int ldq, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int max_seq, int n_kv, int ctx, float* __restrict__ work,
    int nchunks, int n_q, float scale, int spw) {
    static_assert(G >= 1 && G <= 8, "query heads per kv head");
    constexpr int KS = HD / 32;          // k-steps of a score product
    constexpr int DB = HD / 16;          // 16-column blocks of the output
    constexpr int VST = HD + 8;          // LDS row stride of the V copy (bf16): +16 bytes
    constexpr int LPR = HD / 8;          // lanes per V row (16 bytes each)
    constexpr int RPI = QLM_WAVE / LPR;  // V rows per load instruction
    constexpr int NVI = 16 / RPI;        // V loads per lane per step
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) uint16_t vs[16 * VST];
    __shared__ __align__(16) float ps[8][16];

    const int lane = threadIdx.x, qd = lane >> 4, n = lane & 15;
    const int chunk = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int start = chunk * 32 * spw;
    const int cnt = min(32 * spw, ctx - start);
    if (cnt <= 0) return;
    const int steps = (cnt + 15) / 16;
    // cache row (b, position start, head g); position p of the chunk adds p * n_kv rows
    const uint16_t* kbase = kc + (((size_t)b * max_seq + start) * n_kv + g) * HD;
    const uint16_t* vbase = vc + (((size_t)b * max_seq + start) * n_kv + g) * HD;
    const size_t pstride = (size_t)n_kv * HD;

    // (vector types, not the uint4 struct: an aggregate copy into LDS keeps
    // the array in scratch memory)
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    u32x4 kr[KS], vr[NVI];
    auto load_k = [&](int p0) {
        const int p = min(p0 + n, cnt - 1);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
            kr[kk] = *reinterpret_cast<const u32x4*>(kbase + p * pstride + 32 * kk + 8 * qd);
    };
    auto load_v = [&](int p0) {
#pragma unroll
        for (int i = 0; i < NVI; ++i) {
            const int p = min(p0 + i * RPI + lane / LPR, cnt - 1);
            vr[i] = *reinterpret_cast<const u32x4*>(vbase + p * pstride + (lane % LPR) * 8);
        }
    };
    // ---- the query operand's rows, then the first step's K and V rows, all
    // requested before any is used (left to itself the compiler waits for
    // each query load in turn, ahead of the K/V requests) ----
    const int hq = n & 7;
    const bool lo_row = n >= 8, real_row = hq < G;
    const float* qrow = q + (size_t)b * ldq + (size_t)(g * G + min(hq, G - 1)) * HD;
    float4 qraw[KS][2];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        qraw[kk][0] = reinterpret_cast<const float4*>(qrow + 32 * kk + 8 * qd)[0];
        qraw[kk][1] = reinterpret_cast<const float4*>(qrow + 32 * kk + 8 * qd)[1];
    }
    load_k(0);
    load_v(0);
    __builtin_amdgcn_sched_barrier(0);
    bf16x8_t qa[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        const float4 a = qraw[kk][0], c = qraw[kk][1];
        float e[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = real_row ? e[i] : 0.0f;
        qa[kk] = split_part8(e, lo_row);
    }

    // online softmax state of heads 4 (qd & 1) + i (the same in all 16 lanes of a row)
    float m_run[4], l_run[4];
    f32x4_t acc[DB];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.0f;
    }
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int s = 0; s < steps; ++s) {
        const int p0 = 16 * s;
        const bool more = s + 1 < steps;  // wave-uniform
        // ---- scores of positions p0 + n ----
        f32x4_t d = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[kk], __builtin_bit_cast(bf16x8_t, kr[kk]),
                                                        d, 0, 0, 0);
        if (more) load_k(p0 + 16);  // the next step's rows
        float pv[4], f[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float sc = add_halves(d[i]) * scale;
            if (p0 + n >= cnt) sc = -INFINITY;
            const float mn = fmaxf(m_run[i], row16_max(sc));
            f[i] = expf(m_run[i] - mn);  // 0 on the first step
            pv[i] = expf(sc - mn);
            l_run[i] = fmaf(l_run[i], f[i], group_sum<16>(pv[i]));
            m_run[i] = mn;
        }
        // ---- P and V into LDS (the same wave reads them back) ----
        if (qd < 2) {
#pragma unroll
            for (int i = 0; i < 4; ++i) ps[4 * qd + i][n] = pv[i];
        }
#pragma unroll
        for (int i = 0; i < NVI; ++i)
            *reinterpret_cast<u32x4*>(vs + (i * RPI + lane / LPR) * VST + (lane % LPR) * 8) = vr[i];
        if (more) load_v(p0 + 16);
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the LDS stores are done
        __builtin_amdgcn_wave_barrier();
        // ---- P.V on v_mfma_f32_16x16x16_bf16 (lane: row / column n, k = 4 qd .. +3) ----
        const float4 pq = reinterpret_cast<const float4*>(&ps[hq][4 * qd])[0];
        float pr[4] = {pq.x, pq.y, pq.z, pq.w};
        unsigned pw[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float a = real_row ? pr[2 * i] : 0.0f, c = real_row ? pr[2 * i + 1] : 0.0f;
            const __bf16 ha = (__bf16)a, hc = (__bf16)c;
            pw[i] = lo_row ? (bf16_bits(a - (float)ha) | (bf16_bits(c - (float)hc) << 16))
                           : ((unsigned)__builtin_bit_cast(unsigned short, ha) |
                              ((unsigned)__builtin_bit_cast(unsigned short, hc) << 16));
        }
        const s16x4 pa = __builtin_bit_cast(s16x4, make_uint2(pw[0], pw[1]));
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const unsigned w0 = (unsigned)vs[(4 * qd) * VST + 16 * db + n] |
                                ((unsigned)vs[(4 * qd + 1) * VST + 16 * db + n] << 16);
            const unsigned w1 = (unsigned)vs[(4 * qd + 2) * VST + 16 * db + n] |
                                ((unsigned)vs[(4 * qd + 3) * VST + 16 * db + n] << 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[db][i] *= f[i];
            acc[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                pa, __builtin_bit_cast(s16x4, make_uint2(w0, w1)), acc[db], 0, 0, 0);
        }
        // the next step rewrites ps and vs only after these reads have returned
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
    }

    // ---- chunk record [m, l, -, -, o[HD]] of heads 4 qd + i (lanes qd < 2) ----
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int h = 4 * qd + i;
        float* rec = work + (((size_t)b * n_q + g * G + min(h, G - 1)) * nchunks + chunk) * (HD + 4);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const float o = add_halves(acc[db][i]);
            if (qd < 2 && h < G) rec[4 + 16 * db + n] = o;
        }
        if (qd < 2 && h < G && n == 0) {
            rec[0] = m_run[i];
            rec[1] = l_run[i];
        }
    }
}

// Sub-tile of positions held in registers per workgroup: 64 rows at hd 128,
// 32 at hd 256 (the K and V rows of a sub-tile are requested together).
template <int HD>
constexpr int tile_for() { return HD == 128 ? 64 : 32; }
constexpr int kNtModel = 1;  // decode step: one sub-tile per chunk (many short chunks)
constexpr int kNtLong = 4;   // isolated API: contexts up to 32k

constexpr int kPrefillSlice = 256;  // query rows per prefill attention launch

int chunk_len(int hd, int nt) { return (hd == 128 ? 64 : 32) * nt; }
int nchunks_for(int max_seq, int ch) { return (max_seq + ch - 1) / ch; }

// Sub-tiles per chunk of the isolated attention over ctx positions: the
// fewest that keep the records of one head at most 256 (the merge reads
// them all), then doubled while B * chunks stays >= 1024 (with one
// workgroup per (chunk, kv head, sequence), >= 4 per compute unit).
int isolated_nt(int B, int hd, int ctx) {
    int nt = 1;
    while (nt < 8 && nchunks_for(ctx, chunk_len(hd, nt)) > 256) nt *= 2;
    while (nt < 8 && (long long)B * nchunks_for(ctx, chunk_len(hd, 2 * nt)) >= 1024) nt *= 2;
    return nt;
}


size_t records_bytes(int B, int n_q, int hd, int max_seq, int nt) {
    return (size_t)B * n_q * nchunks_for(max_seq, chunk_len(hd, nt)) * (hd + 4) * sizeof(float);
}

// nch: chunks per (sequence, head) in the record layout and the grid; the
// positions a launch may attend to (pos[b] + 1, or ctx + pstep * b) must fit
// in nch chunks of tile_for<HD>() * NT.
template <int HD, int NT, typename KV, bool PREP>
int launch_g(int G, const float* q, int ldq, int qhs, const float* qn, const float* kn,
             const float* ct, const float* st, int rot, KV* kc, KV* vc, int max_seq, int n_kv,
             const int* pos, int ctx, int pstep, size_t kvb, float* work, int nch, int n_q,
             int B, hipStream_t s) {
    constexpr int T = tile_for<HD>();
    const dim3 grid(nch, n_kv, B);
    const float scale = 1.0f / sqrtf((float)HD);
#define QLM_ATTN_G(GG)                                                                          \
    if (G == GG) {                                                                              \
        hipLaunchKernelGGL((k_attn<HD, GG, T, NT, KV, PREP>), grid, dim3(kThreads), 0, s, q,    \
                           ldq, qhs, qn, kn, ct, st, rot, kc, vc, max_seq, n_kv, pos, ctx,      \
                           pstep, kvb, work, nch, n_q, scale);                                  \
        return qlm_launch_status();                                                             \
    }
    QLM_ATTN_G(1)
    QLM_ATTN_G(2)
    QLM_ATTN_G(4)
    QLM_ATTN_G(8)
#undef QLM_ATTN_G
    return QLM_ERR_SHAPE;
}

// k_attn_mx over bf16 caches: nch chunks of 32 * spw positions per
// (sequence, kv head), one wave each.
template <int HD>
int launch_mx(int G, const float* q, int ldq, const uint16_t* kc, const uint16_t* vc, int max_seq,
              int n_kv, int ctx, float* work, int nch, int n_q, int B, int spw, hipStream_t s) {
    const dim3 grid(nch, n_kv, B);
    const float scale = 1.0f / sqrtf((float)HD);
#define QLM_ATTN_MX(GG)                                                                         \
    if (G == GG) {                                                                              \
        hipLaunchKernelGGL((k_attn_mx<HD, GG>), grid, dim3(QLM_WAVE), 0, s, q, ldq, kc, vc,     \
                           max_seq, n_kv, ctx, work, nch, n_q, scale, spw);                     \
        return qlm_launch_status();                                                             \
    }
    QLM_ATTN_MX(1)
    QLM_ATTN_MX(2)
    QLM_ATTN_MX(4)
    QLM_ATTN_MX(8)
#undef QLM_ATTN_MX
    return QLM_ERR_SHAPE;
}

// cs: workgroups per (head, sequence), each merging HD / cs columns (1, 2, 4,
// 8 or 16)
template <int HD>
int launch_combine(const float* work, int nch, int ch, int max_seq, const int* pos, int ctx,
                   int pstep, const float* gate, int ldg, int ghs, float* out, int ldo, int n_q,
                   int B, hipStream_t s, int cs = 1) {
#define QLM_COMBINE(CSV)                                                                        \
    if (cs == CSV) {                                                                            \
        hipLaunchKernelGGL((k_attn_combine<HD, CSV>), dim3(n_q, B, CSV), dim3(kCombineThreads), \
                           0, s, work, nch, ch, max_seq, pos, ctx, pstep, gate, ldg, ghs, out,  \
                           ldo, n_q);                                                           \
        return qlm_launch_status();                                                             \
    }
    QLM_COMBINE(1)
    QLM_COMBINE(2)
    QLM_COMBINE(4)
    QLM_COMBINE(8)
    QLM_COMBINE(16)
#undef QLM_COMBINE
    return QLM_ERR_ARG;
}

// column split of the isolated attention's merge: ~256 workgroups or more
// (at 16 splits a workgroup holds 4 columns at hd 256, 2 at hd 128, and
// takes 512 or 1024 records in its first request batch)
int combine_splits(int n_q, int B) {
    const int pairs = n_q * B;
    int cs = 1;
    while (cs < 16 && pairs * cs < 256) cs *= 2;
    return cs;
}

}  // namespace

extern "C" size_t qlm_gqa_workspace_bytes(int B, int n_q, int hd, int max_seq) {
    if (B <= 0 || n_q <= 0 || hd <= 0 || max_seq <= 0) return 0;
    const size_t a = records_bytes(B, n_q, hd, max_seq, kNtModel);
    const size_t b = records_bytes(B, n_q, hd, max_seq, kNtLong);
    return a > b ? a : b;
}

extern "C" int qlm_gqa_decode(float* qkv, int ldqkv, const float* q_norm, const float* k_norm,
                              const float* cos_tab, const float* sin_tab, int rot_dim,
                              float* k_cache, float* v_cache, int max_seq, const int* pos,
                              float* out, int ldo, int B, int n_q, int n_kv, int hd, int gated,
                              void* work, void* stream) {
    if (!qkv || !cos_tab || !sin_tab || !k_cache || !v_cache || !pos || !out || !work)
        return QLM_ERR_ARG;
    if (B <= 0 || n_q <= 0 || n_kv <= 0 || max_seq <= 0) return QLM_ERR_ARG;
    if (n_q % n_kv != 0 || (hd != 128 && hd != 256)) return QLM_ERR_SHAPE;
    if (rot_dim < 0 || rot_dim > hd || rot_dim % 2 != 0) return QLM_ERR_SHAPE;
    const int G = n_q / n_kv;
    if (G != 1 && G != 2 && G != 4 && G != 8) return QLM_ERR_SHAPE;
    const int qstride = gated ? 2 * hd : hd;
    if (ldqkv < n_q * qstride + 2 * n_kv * hd || ldo < n_q * hd) return QLM_ERR_SHAPE;
    hipStream_t st = as_stream(stream);
    float* w = reinterpret_cast<float*>(work);
    const int ch = chunk_len(hd, kNtModel);
    const int nch = nchunks_for(max_seq, ch);
    const float* gate = gated ? qkv : nullptr;
    int rc;
    if (hd == 128) {
        rc = launch_g<128, kNtModel, float, true>(G, qkv, ldqkv, qstride, q_norm, k_norm, cos_tab,
                                                  sin_tab, rot_dim, k_cache, v_cache, max_seq,
                                                  n_kv, pos, 0, 0, (size_t)max_seq, w, nch, n_q, B,
                                                  st);
        if (rc != QLM_OK) return rc;
        return launch_combine<128>(w, nch, ch, max_seq, pos, 0, 0, gate, ldqkv, qstride, out,
                                   ldo, n_q, B, st);
    }
    rc = launch_g<256, kNtModel, float, true>(G, qkv, ldqkv, qstride, q_norm, k_norm, cos_tab,
                                              sin_tab, rot_dim, k_cache, v_cache, max_seq, n_kv,
                                              pos, 0, 0, (size_t)max_seq, w, nch, n_q, B, st);
    if (rc != QLM_OK) return rc;
    return launch_combine<256>(w, nch, ch, max_seq, pos, 0, 0, gate, ldqkv, qstride, out, ldo,
                               n_q, B, st);
}

namespace {

int check_attention_args(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                         int max_seq, int ctx, const float* out, int B, int n_q, int n_kv,
                         int hd) {
    if (!q || !k_cache || !v_cache || !out) return QLM_ERR_ARG;
    if (B <= 0 || n_q <= 0 || n_kv <= 0 || ctx <= 0 || ctx > max_seq) return QLM_ERR_ARG;
    if (n_q % n_kv != 0 || (hd != 128 && hd != 256)) return QLM_ERR_SHAPE;
    if (kv_dtype != 0 && kv_dtype != 1) return QLM_ERR_ARG;
    const int G = n_q / n_kv;
    if (G != 1 && G != 2 && G != 4 && G != 8) return QLM_ERR_SHAPE;
    return QLM_OK;
}

template <int HDV, int NT>
int attention_launch_nt(const float* q, const float* k_cache, const float* v_cache, int max_seq,
                        int ctx, float* out, int B, int n_q, int n_kv, float* w, int nch,
                        hipStream_t st) {
    const int G = n_q / n_kv;
    const int ldq = n_q * HDV;
    const int rc = launch_g<HDV, NT, float, false>(
        G, q, ldq, HDV, nullptr, nullptr, nullptr, nullptr, 0, const_cast<float*>(k_cache),
        const_cast<float*>(v_cache), max_seq, n_kv, nullptr, ctx, 0, (size_t)max_seq, w, nch, n_q,
        B, st);
    if (rc != QLM_OK) return rc;
    return launch_combine<HDV>(w, nch, chunk_len(HDV, NT), max_seq, nullptr, ctx, 0, nullptr, 0,
                               0, out, ldq, n_q, B, st, combine_splits(n_q, B));
}

// 32-position units per wave of the bf16 matrix-core attention: the largest
// power of two up to 32 that keeps >= 1024 waves, then raised until a head
// has <= 256 chunk records (the merge's cost grows with them); >= 2 at hd
// 128. Measured on MI355X at 16 q / 2 kv heads, hd 256 (graph replays):
// 16 x 32768 positions 215 us at 8 units, 193 us at 32; 16 x 8192 54 us at
// 4, 49 us at 8; 1 x 32768 27 us at 2 (512 records), 23 us at 4.
int mx_spw(int B, int n_kv, int hd, int ctx) {
    int spw = hd == 128 ? 2 : 1;
    while (spw < 32 && (long long)B * n_kv * nchunks_for(ctx, 64 * spw) >= 1024) spw *= 2;
    while (spw < (1 << 20) && nchunks_for(ctx, 32 * spw) > 256) spw *= 2;
    return spw;
}

// Chunking of one isolated attention call: chunk length and records per
// (sequence, query head). fp32 caches take k_attn (nt sub-tiles a chunk),
// bf16 caches k_attn_mx (32 * spw positions a wave). Either fits the
// workspace of qlm_gqa_workspace_bytes(B, n_q, hd, max_seq) for ctx <=
// max_seq: at most ceil(ctx / 32) records at hd 256 and ceil(ctx / 64) at
// hd 128.
struct IsoPlan {
    int unit;  // nt (fp32) or spw (bf16)
    int ch, nch;
};
IsoPlan iso_plan(int kv_dtype, int B, int n_kv, int hd, int ctx) {
    IsoPlan p;
    if (kv_dtype == 0) {
        p.unit = isolated_nt(B, hd, ctx);
        p.ch = chunk_len(hd, p.unit);
    } else {
        p.unit = mx_spw(B, n_kv, hd, ctx);
        p.ch = 32 * p.unit;
    }
    p.nch = nchunks_for(ctx, p.ch);
    return p;
}

// The two launches of the isolated attention under plan p, records in w.
int attention_launch(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                     int max_seq, int ctx, float* out, int B, int n_q, int n_kv, int hd,
                     float* w, const IsoPlan& p, hipStream_t st) {
    const int G = n_q / n_kv;
    if (kv_dtype == 1) {
        const uint16_t* kc = static_cast<const uint16_t*>(k_cache);
        const uint16_t* vc = static_cast<const uint16_t*>(v_cache);
        int rc = hd == 128 ? launch_mx<128>(G, q, n_q * hd, kc, vc, max_seq, n_kv, ctx, w, p.nch,
                                            n_q, B, p.unit, st)
                           : launch_mx<256>(G, q, n_q * hd, kc, vc, max_seq, n_kv, ctx, w, p.nch,
                                            n_q, B, p.unit, st);
        if (rc != QLM_OK) return rc;
        return hd == 128 ? launch_combine<128>(w, p.nch, p.ch, max_seq, nullptr, ctx, 0, nullptr,
                                               0, 0, out, n_q * hd, n_q, B, st,
                                               combine_splits(n_q, B))
                         : launch_combine<256>(w, p.nch, p.ch, max_seq, nullptr, ctx, 0, nullptr,
                                               0, 0, out, n_q * hd, n_q, B, st,
                                               combine_splits(n_q, B));
    }
    const float* kc = static_cast<const float*>(k_cache);
    const float* vc = static_cast<const float*>(v_cache);
#define QLM_ISO(HDV, NTV)                                                                       \
    if (hd == HDV && p.unit == NTV)                                                             \
        return attention_launch_nt<HDV, NTV>(q, kc, vc, max_seq, ctx, out, B, n_q, n_kv, w, p.nch, \
                                             st);
    QLM_ISO(128, 1) QLM_ISO(128, 2) QLM_ISO(128, 4) QLM_ISO(128, 8)
    QLM_ISO(256, 1) QLM_ISO(256, 2) QLM_ISO(256, 4) QLM_ISO(256, 8)
#undef QLM_ISO
    return QLM_ERR_SHAPE;
}

}  // namespace

// Device scratch of qlm_attention_decode_noalloc: the chunk records live in
// this array instead of a caller workspace. Each GPU that runs the library
// holds its own copy until the process ends; its device address is looked
// up once per device (hipGetSymbolAddress, with that device current) and
// only that address is ever handed to a kernel or a copy.
static constexpr size_t kScratchBytes = (size_t)QLM_ATTENTION_NOALLOC_MAX_BYTES;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (resolved on its first call).
int scratch_ptr(float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return qlm_status(e);
    if (dev < 0 || dev >= kMaxDevices) return QLM_ERR_ARG;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return qlm_status(e);
        if (!p) return QLM_ERR_NO_DEVICE;
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<float*>(g_scratch_ptr[dev]);
    return QLM_OK;
}

}  // namespace

extern "C" int qlm_attention_decode(const float* q, const void* k_cache, const void* v_cache,
                                    int kv_dtype, int max_seq, int ctx, float* out, int B, int n_q,
                                    int n_kv, int hd, void* work, void* stream) {
    if (!work) return QLM_ERR_ARG;
    const int rc = check_attention_args(q, k_cache, v_cache, kv_dtype, max_seq, ctx, out, B, n_q,
                                        n_kv, hd);
    if (rc != QLM_OK) return rc;
    // records laid out for the positions the launch attends to (ctx): at
    // most qlm_gqa_workspace_bytes(B, n_q, hd, max_seq), the one-sub-tile
    // layout over max_seq
    return attention_launch(q, k_cache, v_cache, kv_dtype, max_seq, ctx, out, B, n_q, n_kv, hd,
                            reinterpret_cast<float*>(work), iso_plan(kv_dtype, B, n_kv, hd, ctx),
                            as_stream(stream));
}

extern "C" size_t qlm_attention_decode_noalloc_bytes(int B, int n_q, int hd, int ctx) {
    if (B <= 0 || n_q <= 0 || (hd != 128 && hd != 256) || ctx <= 0) return 0;
    // the larger of the two caches' layouts; the bf16 one depends on n_kv
    // only through a count of waves, and has at most min(256, ceil(ctx /
    // 32 * spw)) records with spw >= 1 (2 at hd 128)
    const int nf = nchunks_for(ctx, chunk_len(hd, isolated_nt(B, hd, ctx)));
    const int nb0 = nchunks_for(ctx, hd == 128 ? 64 : 32);
    const int nb = nb0 < 256 ? nb0 : 256;
    const int n = nf > nb ? nf : nb;
    return (size_t)B * n_q * n * (hd + 4) * sizeof(float);
}

extern "C" int qlm_attention_decode_noalloc(const float* q, const void* k_cache,
                                            const void* v_cache, int kv_dtype, int max_seq,
                                            int ctx, float* out, int B, int n_q, int n_kv, int hd,
                                            void* stream) {
    int rc = check_attention_args(q, k_cache, v_cache, kv_dtype, max_seq, ctx, out, B, n_q, n_kv,
                                  hd);
    if (rc != QLM_OK) return rc;
    // records for the chunks that cover ctx positions only (the grid stops there)
    const IsoPlan p = iso_plan(kv_dtype, B, n_kv, hd, ctx);
    if ((size_t)B * n_q * p.nch * (hd + 4) * sizeof(float) > kScratchBytes) return QLM_ERR_SCRATCH;
    float* w = nullptr;
    rc = scratch_ptr(&w);
    if (rc != QLM_OK) return rc;
    return attention_launch(q, k_cache, v_cache, kv_dtype, max_seq, ctx, out, B, n_q, n_kv, hd,
                            w, p, as_stream(stream));
}

extern "C" size_t qlm_gqa_prefill_workspace_bytes(int n_q, int hd, int max_seq) {
    if (n_q <= 0 || hd <= 0 || max_seq <= 0) return 0;
    return records_bytes(kPrefillSlice, n_q, hd, max_seq, kNtLong);
}

extern "C" int qlm_gqa_prefill(float* qkv, int ldqkv, const float* q_norm, const float* k_norm,
                               const float* cos_tab, const float* sin_tab, int rot_dim,
                               float* k_cache, float* v_cache, int max_seq, int p0, int T,
                               float* out, int ldo, int n_q, int n_kv, int hd, int gated,
                               void* work, void* stream) {
    if (!qkv || !cos_tab || !sin_tab || !k_cache || !v_cache || !out || !work) return QLM_ERR_ARG;
    if (T <= 0 || p0 < 0 || n_q <= 0 || n_kv <= 0 || max_seq <= 0) return QLM_ERR_ARG;
    if (p0 + T > max_seq) return QLM_ERR_SHAPE;
    if (n_q % n_kv != 0 || (hd != 128 && hd != 256)) return QLM_ERR_SHAPE;
    if (rot_dim < 0 || rot_dim > hd || rot_dim % 2 != 0) return QLM_ERR_SHAPE;
    const int G = n_q / n_kv;
    if (G != 1 && G != 2 && G != 4 && G != 8) return QLM_ERR_SHAPE;
    const int qstride = gated ? 2 * hd : hd;
    if (ldqkv < n_q * qstride + 2 * n_kv * hd || ldo < n_q * hd) return QLM_ERR_SHAPE;
    const size_t lds = (size_t)(n_q + n_kv) * hd * sizeof(float);
    if (lds > 64 * 1024) return QLM_ERR_SHAPE;
    hipStream_t st = as_stream(stream);
    float* w = reinterpret_cast<float*>(work);
    const int ch = chunk_len(hd, kNtLong);
    const int nch = nchunks_for(max_seq, ch);
    if (hd == 128)
        hipLaunchKernelGGL(k_gqa_prep_rows<128>, dim3(T), dim3(kThreads), lds, st, qkv, ldqkv,
                           qstride, q_norm, k_norm, cos_tab, sin_tab, rot_dim, k_cache, v_cache,
                           n_q, n_kv, p0);
    else
        hipLaunchKernelGGL(k_gqa_prep_rows<256>, dim3(T), dim3(kThreads), lds, st, qkv, ldqkv,
                           qstride, q_norm, k_norm, cos_tab, sin_tab, rot_dim, k_cache, v_cache,
                           n_q, n_kv, p0);
    int rc = qlm_launch_status();
    if (rc != QLM_OK) return rc;
    if (hd == 128 && (ldqkv % 4) == 0 && (ldo % 4) == 0 && (qstride % 4) == 0) {
        const dim3 grid((T + 15) / 16, n_kv);
        const float scale = 1.0f / sqrtf(128.0f);
#define QLM_ATTN_PF(GG)                                                                         \
        if (G == GG) {                                                                          \
            hipLaunchKernelGGL((k_attn_pf<GG>), grid, dim3(GG * QLM_WAVE), 0, st, qkv, ldqkv,   \
                               qstride, k_cache, v_cache, n_kv, p0, T, gated, out, ldo, scale); \
            return qlm_launch_status();                                                         \
        }
        QLM_ATTN_PF(1)
        QLM_ATTN_PF(2)
        QLM_ATTN_PF(4)
        QLM_ATTN_PF(8)
#undef QLM_ATTN_PF
    }
    for (int s0 = 0; s0 < T; s0 += kPrefillSlice) {
        const int rows = T - s0 < kPrefillSlice ? T - s0 : kPrefillSlice;
        float* q = qkv + (size_t)s0 * ldqkv;
        const int ctx = p0 + s0 + 1;  // row s0 sits at position p0 + s0
        if (hd == 128) {
            rc = launch_g<128, kNtLong, float, false>(G, q, ldqkv, qstride, nullptr, nullptr,
                                                      nullptr, nullptr, 0, k_cache, v_cache,
                                                      max_seq, n_kv, nullptr, ctx, 1, 0, w, nch,
                                                      n_q, rows, st);
            if (rc != QLM_OK) return rc;
            rc = launch_combine<128>(w, nch, ch, max_seq, nullptr, ctx, 1, gated ? q : nullptr,
                                     ldqkv, qstride, out + (size_t)s0 * ldo, ldo, n_q, rows, st);
        } else {
            rc = launch_g<256, kNtLong, float, false>(G, q, ldqkv, qstride, nullptr, nullptr,
                                                      nullptr, nullptr, 0, k_cache, v_cache,
                                                      max_seq, n_kv, nullptr, ctx, 1, 0, w, nch,
                                                      n_q, rows, st);
            if (rc != QLM_OK) return rc;
            rc = launch_combine<256>(w, nch, ch, max_seq, nullptr, ctx, 1, gated ? q : nullptr,
                                     ldqkv, qstride, out + (size_t)s0 * ldo, ldo, n_q, rows, st);
        }
        if (rc != QLM_OK) return rc;
    }
    return QLM_OK;
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_attention() {
    hipFuncAttributes a;
    hipError_t e = hipFuncGetAttributes(&a, reinterpret_cast<const void*>((k_attn_combine<128, 1>)));
    if (e != hipSuccess) return e;
    // the no-allocation entry point's scratch address on this device, so
    // that its first call (possibly under graph capture) makes no runtime
    // query
    float* w = nullptr;
    const int rc = scratch_ptr(&w);
    return rc == QLM_OK ? hipSuccess : (rc > 0 ? (hipError_t)rc : hipErrorInvalidValue);
}
