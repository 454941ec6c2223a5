// GQA decode attention over a contiguous, position-major KV cache
// [B, max_seq, n_kv, hd] (reference: Qwen3_5Attention::forward,
// attention.cpp:138-232; gqa_attend_head :54-82).
//
// One kernel, k_attn, one workgroup per (chunk of CH positions, kv head g,
// sequence b); the G = n_q/n_kv query heads of the group share every K/V row
// read. Inside a workgroup:
//   PREP          QK-norm (zero-centred gain, eps 1e-6) and partial NeoX RoPE
//                 of the group's query heads from the projection row; the
//                 workgroup whose chunk holds position p = pos[b] also
//                 normalises/rotates k_p and writes k_p, v_p into the cache
//                 (attention.cpp:166-199). Other chunks never read row p.
//   scores        s = q.k * 1/sqrt(hd); the K rows of a chunk are loaded in
//                 batches of 8 per lane before use (latency, not a serial
//                 chain); kept in LDS.
//   softmax/PV    exp against the chunk max, P.V with float4 V rows.
//   COMBINE_LAST  the last workgroup of (b, g) to finish (atomic counter,
//                 release/acquire fences, counter reset to 0 for the next
//                 launch) merges all chunk records and applies the sigmoid
//                 output gate (attention.cpp:216-227). Without it, a separate
//                 combine kernel does the merge (long contexts: hundreds of
//                 chunks would serialise on one workgroup).
// The graph-captured decode step launches the grid for max_seq; chunks past
// pos[b] exit at once and are not counted.

#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kNW = kThreads / QLM_WAVE;
constexpr int kBatch = 8;  // loads in flight per lane in the score and PV loops

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

// Merge the chunk records [m, l, -, -, o[HD]] of one head; returns o/l.
template <int HD>
__device__ __forceinline__ float merge_chunks(const float* base, int nc, int e) {
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, base[(size_t)c * (HD + 4)]);
    float l = 0.0f, o = 0.0f;
    for (int c = 0; c < nc; ++c) {
        const float* pc = base + (size_t)c * (HD + 4);
        const float f = expf(pc[0] - M);
        l = fmaf(f, pc[1], l);
        o = fmaf(f, pc[4 + e], o);
    }
    return o / l;
}

template <int HD, int G, int CH, typename KV, bool PREP, bool COMBINE_LAST>
__global__ __launch_bounds__(kThreads) void k_attn(
    const float* __restrict__ qsrc, int ldq, int qhs, const float* __restrict__ qn_w,
    const float* __restrict__ kn_w, const float* __restrict__ cos_tab,
    const float* __restrict__ sin_tab, int rot, KV* __restrict__ kc, KV* __restrict__ vc,
    int max_seq, int n_kv, const int* __restrict__ pos, int ctx, float* __restrict__ work,
    unsigned* __restrict__ counters, int nchunks, int n_q, int gated, float* __restrict__ out,
    int ldo, float scale) {
    static_assert(!PREP || sizeof(KV) == 4, "the fused prologue writes an fp32 cache");
    constexpr int LPP = HD / 8;            // lanes per position in the score phase
    constexpr int PPW = QLM_WAVE / LPP;    // positions per wave per score step
    constexpr int SPS = kNW * PPW;         // positions per workgroup per score step
    constexpr int C4 = HD / 4;             // float4 columns of a row
    constexpr int NPG = kThreads / C4;     // position groups in the PV phase
    __shared__ float qs[G][HD];
    __shared__ float sc[G][CH];
    __shared__ float4 red[NPG][G][C4];
    __shared__ float kvp[2][HD];
    __shared__ float mstat[G], lstat[G];
    __shared__ int is_last;

    const int chunk = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int p = pos ? pos[b] : ctx - 1;
    const int L = min(p + 1, max_seq);
    const int nc = (L + CH - 1) / CH;
    if (chunk >= nc || p < 0) return;
    const int start = chunk * CH;
    const int n = min(CH, L - start);
    const float* qrow = qsrc + (size_t)b * ldq;
    const bool own_p = PREP && (p / CH == chunk);

    for (int i = tid; i < G * HD; i += kThreads)
        qs[i / HD][i % HD] = qrow[(size_t)(g * G + i / HD) * qhs + i % HD];
    if (own_p) {
        for (int i = tid; i < HD; i += kThreads) {
            kvp[0][i] = qrow[(size_t)n_q * qhs + (size_t)g * HD + i];
            kvp[1][i] = qrow[(size_t)n_q * qhs + (size_t)(n_kv + g) * HD + i];
        }
    }
    __syncthreads();
    if constexpr (PREP) {
        const int nrows = G + (own_p ? 1 : 0);
        for (int r = wave; r < nrows; r += kNW) {
            float* v = r < G ? qs[r] : kvp[0];
            const float* w = r < G ? qn_w : kn_w;
            if (w) {
                float ss = 0.0f;
                for (int e = lane; e < HD; e += QLM_WAVE) ss = fmaf(v[e], v[e], ss);
                ss = wave_sum(ss);
                const float s = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
                for (int e = lane; e < HD; e += QLM_WAVE) v[e] = (v[e] * s) * (1.0f + w[e]);
            }
        }
        __syncthreads();
        const int half = rot / 2;
        const float* ct = cos_tab + (size_t)p * half;
        const float* st = sin_tab + (size_t)p * half;
        for (int i = tid; i < nrows * half; i += kThreads) {
            const int r = i / half, j = i % half;
            float* v = r < G ? qs[r] : kvp[0];
            const float x1 = v[j], x2 = v[j + half];
            v[j] = nc_mul_sub(x1, ct[j], x2, st[j]);
            v[j + half] = nc_mul_add2(x2, ct[j], x1, st[j]);
        }
        __syncthreads();
        if (own_p) {
            const size_t off = (((size_t)b * max_seq + p) * n_kv + g) * HD;
            for (int i = tid; i < HD; i += kThreads) {
                kc[off + i] = kvp[0][i];
                vc[off + i] = kvp[1][i];
            }
        }
        __syncthreads();  // the cache rows written above are read below by other waves
    }

    // ---- scores ----
    {
        const int sub = lane % LPP, pw = lane / LPP;
        float qr[G][8];
#pragma unroll
        for (int gh = 0; gh < G; ++gh)
#pragma unroll
            for (int e = 0; e < 8; ++e) qr[gh][e] = qs[gh][sub * 8 + e];
        const size_t row0 = ((size_t)b * max_seq + start) * n_kv + g;
        for (int it0 = 0; it0 * SPS < n; it0 += kBatch) {
            float kr[kBatch][8];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int pl = (it0 + u) * SPS + wave * PPW + pw;
                if (pl < n) load8<KV>(kc + (row0 + (size_t)pl * n_kv) * HD + sub * 8, kr[u]);
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int pl = (it0 + u) * SPS + wave * PPW + pw;
#pragma unroll
                for (int gh = 0; gh < G; ++gh) {
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d = fmaf(qr[gh][e], kr[u][e], d);
                    d = group_sum<LPP>(d);
                    if (sub == 0 && pl < n) sc[gh][pl] = d * scale;
                }
            }
        }
    }
    __syncthreads();

    // ---- per-head chunk max, exponentials, sum ----
    for (int gh = wave; gh < G; gh += kNW) {
        float m = -INFINITY;
        for (int pl = lane; pl < n; pl += QLM_WAVE) m = fmaxf(m, sc[gh][pl]);
        m = wave_max(m);
        float l = 0.0f;
        for (int pl = lane; pl < n; pl += QLM_WAVE) {
            const float e = expf(sc[gh][pl] - m);
            sc[gh][pl] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            mstat[gh] = m;
            lstat[gh] = l;
        }
    }
    __syncthreads();

    // ---- P.V ----
    {
        const int c4 = tid % C4, pg = tid / C4;
        float4 acc[G];
#pragma unroll
        for (int gh = 0; gh < G; ++gh) acc[gh] = make_float4(0.f, 0.f, 0.f, 0.f);
        const size_t row0 = ((size_t)b * max_seq + start) * n_kv + g;
        for (int it0 = 0; it0 * NPG < n; it0 += kBatch) {
            float4 vv[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int pl = (it0 + u) * NPG + pg;
                if (pl < n) vv[u] = load4<KV>(vc + (row0 + (size_t)pl * n_kv) * HD + c4 * 4);
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int pl = (it0 + u) * NPG + pg;
                if (pl < n) {
#pragma unroll
                    for (int gh = 0; gh < G; ++gh) {
                        const float e = sc[gh][pl];
                        acc[gh].x = fmaf(e, vv[u].x, acc[gh].x);
                        acc[gh].y = fmaf(e, vv[u].y, acc[gh].y);
                        acc[gh].z = fmaf(e, vv[u].z, acc[gh].z);
                        acc[gh].w = fmaf(e, vv[u].w, acc[gh].w);
                    }
                }
            }
        }
#pragma unroll
        for (int gh = 0; gh < G; ++gh) red[pg][gh][c4] = acc[gh];
    }
    __syncthreads();
    for (int i = tid; i < G * C4; i += kThreads) {
        const int gh = i / C4, c4 = i % C4;
        float4 t = red[0][gh][c4];
#pragma unroll
        for (int p2 = 1; p2 < NPG; ++p2) {
            const float4 u = red[p2][gh][c4];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
        float* dst = work + (((size_t)b * n_q + g * G + gh) * nchunks + chunk) * (HD + 4);
        reinterpret_cast<float4*>(dst + 4)[c4] = t;
        if (c4 == 0) {
            dst[0] = mstat[gh];
            dst[1] = lstat[gh];
        }
    }

    if constexpr (COMBINE_LAST) {
        __syncthreads();
        if (tid == 0) {
            __threadfence();  // release this chunk's records
            const unsigned old = atomicAdd(&counters[b * n_kv + g], 1u);
            is_last = (old == (unsigned)nc - 1);
        }
        __syncthreads();
        if (!is_last) return;
        __threadfence();  // acquire the other chunks' records
        for (int i = tid; i < G * HD; i += kThreads) {
            const int gh = i / HD, e = i % HD;
            const int h = g * G + gh;
            const float* base = work + ((size_t)b * n_q + h) * nchunks * (HD + 4);
            float r = merge_chunks<HD>(base, nc, e);
            if (gated) r *= 1.0f / (1.0f + expf(-qrow[(size_t)h * qhs + HD + e]));
            out[(size_t)b * ldo + (size_t)h * HD + e] = r;
        }
        if (tid == 0) atomicExch(&counters[b * n_kv + g], 0u);
    }
}

// Separate merge for long contexts: one workgroup per (query head, sequence).
template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(const float* __restrict__ work, int nchunks,
                                                     int CH, int max_seq, const int* __restrict__ pos,
                                                     int ctx, float* __restrict__ out, int ldo,
                                                     int n_q) {
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const int L = min(pos ? pos[b] + 1 : ctx, max_seq);
    const int nc = min(nchunks, (L + CH - 1) / CH);
    const float* base = work + ((size_t)b * n_q + h) * nchunks * (HD + 4);
    out[(size_t)b * ldo + (size_t)h * HD + i] = merge_chunks<HD>(base, nc, i);
}

constexpr int kChModel = 128;   // decode step: contexts up to a few thousand
constexpr int kChLong = 256;    // isolated API: contexts up to 32k

int nchunks_for(int max_seq, int ch) { return (max_seq + ch - 1) / ch; }

size_t counter_offset(int B, int n_q, int hd, int max_seq) {
    const size_t rec = (size_t)B * n_q * nchunks_for(max_seq, kChModel) * (hd + 4) * sizeof(float);
    const size_t rec_long = (size_t)B * n_q * nchunks_for(max_seq, kChLong) * (hd + 4) * sizeof(float);
    const size_t r = rec > rec_long ? rec : rec_long;
    return (r + 255) & ~(size_t)255;
}

template <int HD, int CH, typename KV, bool PREP, bool LAST>
int launch_g(int G, const float* q, int ldq, int qhs, const float* qn, const float* kn,
             const float* ct, const float* st, int rot, KV* kc, KV* vc, int max_seq, int n_kv,
             const int* pos, int ctx, float* work, unsigned* counters, int n_q, int gated,
             float* out, int ldo, int B, hipStream_t s) {
    const int nch = nchunks_for(max_seq, CH);
    const dim3 grid(nch, n_kv, B);
    const float scale = 1.0f / sqrtf((float)HD);
#define QLM_ATTN_G(GG)                                                                           \
    if (G == GG) {                                                                               \
        hipLaunchKernelGGL((k_attn<HD, GG, CH, KV, PREP, LAST>), grid, dim3(kThreads), 0, s, q,  \
                           ldq, qhs, qn, kn, ct, st, rot, kc, vc, max_seq, n_kv, pos, ctx, work, \
                           counters, nch, n_q, gated, out, ldo, scale);                          \
        return qlm_launch_status();                                                              \
    }
    QLM_ATTN_G(1)
    QLM_ATTN_G(2)
    QLM_ATTN_G(4)
    QLM_ATTN_G(8)
#undef QLM_ATTN_G
    return QLM_ERR_SHAPE;
}

}  // namespace

extern "C" size_t qlm_gqa_workspace_bytes(int B, int n_q, int hd, int max_seq) {
    return counter_offset(B, n_q, hd, max_seq) + (size_t)B * 64 * sizeof(unsigned);
}

extern "C" int qlm_gqa_decode(float* qkv, int ldqkv, const float* q_norm, const float* k_norm,
                              const float* cos_tab, const float* sin_tab, int rot_dim,
                              float* k_cache, float* v_cache, int max_seq, const int* pos,
                              float* out, int ldo, int B, int n_q, int n_kv, int hd, int gated,
                              void* work, void* stream) {
    if (!qkv || !cos_tab || !sin_tab || !k_cache || !v_cache || !pos || !out || !work)
        return QLM_ERR_ARG;
    if (B <= 0 || n_q <= 0 || n_kv <= 0 || max_seq <= 0) return QLM_ERR_ARG;
    if (n_q % n_kv != 0 || (hd != 128 && hd != 256) || n_kv > 64) return QLM_ERR_SHAPE;
    if (rot_dim < 0 || rot_dim > hd || rot_dim % 2 != 0) return QLM_ERR_SHAPE;
    const int G = n_q / n_kv;
    if (G != 1 && G != 2 && G != 4 && G != 8) return QLM_ERR_SHAPE;
    const int qstride = gated ? 2 * hd : hd;
    if (ldqkv < n_q * qstride + 2 * n_kv * hd || ldo < n_q * hd) return QLM_ERR_SHAPE;
    hipStream_t st = as_stream(stream);
    float* w = reinterpret_cast<float*>(work);
    unsigned* cnt = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(work) +
                                                counter_offset(B, n_q, hd, max_seq));
    if (hd == 128)
        return launch_g<128, kChModel, float, true, true>(
            G, qkv, ldqkv, qstride, q_norm, k_norm, cos_tab, sin_tab, rot_dim, k_cache, v_cache,
            max_seq, n_kv, pos, 0, w, cnt, n_q, gated, out, ldo, B, st);
    return launch_g<256, kChModel, float, true, true>(
        G, qkv, ldqkv, qstride, q_norm, k_norm, cos_tab, sin_tab, rot_dim, k_cache, v_cache,
        max_seq, n_kv, pos, 0, w, cnt, n_q, gated, out, ldo, B, st);
}

extern "C" int qlm_attention_decode(const float* q, const void* k_cache, const void* v_cache,
                                    int kv_dtype, int max_seq, int ctx, float* out, int B, int n_q,
                                    int n_kv, int hd, void* work, void* stream) {
    if (!q || !k_cache || !v_cache || !out || !work) return QLM_ERR_ARG;
    if (B <= 0 || n_q <= 0 || n_kv <= 0 || ctx <= 0 || ctx > max_seq) return QLM_ERR_ARG;
    if (n_q % n_kv != 0 || (hd != 128 && hd != 256)) return QLM_ERR_SHAPE;
    if (kv_dtype != 0 && kv_dtype != 1) return QLM_ERR_ARG;
    const int G = n_q / n_kv;
    hipStream_t st = as_stream(stream);
    const int nch = nchunks_for(max_seq, kChLong);
    float* w = reinterpret_cast<float*>(work);
    const int ldq = n_q * hd;
    int rc;
#define QLM_ISO(HDV)                                                                              \
    rc = kv_dtype == 0                                                                            \
             ? launch_g<HDV, kChLong, float, false, false>(                                       \
                   G, q, ldq, hd, nullptr, nullptr, nullptr, nullptr, 0,                          \
                   (float*)const_cast<void*>(k_cache), (float*)const_cast<void*>(v_cache),        \
                   max_seq, n_kv, nullptr, ctx, w, nullptr, n_q, 0, out, ldq, B, st)              \
             : launch_g<HDV, kChLong, uint16_t, false, false>(                                    \
                   G, q, ldq, hd, nullptr, nullptr, nullptr, nullptr, 0,                          \
                   (uint16_t*)const_cast<void*>(k_cache), (uint16_t*)const_cast<void*>(v_cache),  \
                   max_seq, n_kv, nullptr, ctx, w, nullptr, n_q, 0, out, ldq, B, st);             \
    if (rc != QLM_OK) return rc;                                                                  \
    hipLaunchKernelGGL(k_attn_combine<HDV>, dim3(n_q, B), dim3(HDV), 0, st, w, nch, kChLong,      \
                       max_seq, nullptr, ctx, out, ldq, n_q);
    if (hd == 128) {
        QLM_ISO(128)
    } else {
        QLM_ISO(256)
    }
#undef QLM_ISO
    return qlm_launch_status();
}
