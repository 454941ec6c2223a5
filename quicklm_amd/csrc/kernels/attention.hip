// GQA decode attention over a contiguous, position-major KV cache
// [B, max_seq, n_kv, hd] (reference: Qwen3_5Attention::forward,
// attention.cpp:138-232; gqa_attend_head :54-82).
//
//   prep     one wave per (head, sequence): QK-norm (zero-centred gain,
//            eps 1e-6), partial NeoX RoPE from the host-built cos/sin table,
//            K/V written at pos[b]. (attention.cpp:160-199)
//   partial  split-K flash-decoding: one workgroup per (chunk of 256
//            positions, kv head, sequence); all G = n_q/n_kv query heads of
//            the group share each K/V row read. Scores are kept in LDS,
//            exponentiated against the chunk max, and P.V is accumulated.
//   combine  one workgroup per (query head, sequence): merges the chunk
//            partials with the usual max/rescale and applies the sigmoid
//            output gate (attention.cpp:216-227).
//
// The graph-captured decode step launches the grid for max_seq; chunks past
// pos[b] exit at once.

#include "common.hpp"

namespace {

constexpr int kCH = 256;  // positions per chunk
constexpr int kThreads = 256;

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

// ---- prep: QK-norm + RoPE + cache write; one wave per head ----
template <int HD>
__global__ __launch_bounds__(QLM_WAVE) void k_attn_prep(
    float* __restrict__ qkv, int ldqkv, const float* __restrict__ qn_w,
    const float* __restrict__ kn_w, const float* __restrict__ cos_tab,
    const float* __restrict__ sin_tab, int rot, float* __restrict__ kc, float* __restrict__ vc,
    int max_seq, const int* __restrict__ pos, int n_q, int n_kv, int gated) {
    constexpr int E = HD / QLM_WAVE;
    __shared__ float sh[HD];
    const int head = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int p = pos[b];
    if (p < 0 || p >= max_seq) return;
    const int qstride = gated ? 2 * HD : HD;
    float* row = qkv + (size_t)b * ldqkv;
    const bool isq = head < n_q;
    const int kvh = head - n_q;
    float* src = isq ? row + (size_t)head * qstride : row + (size_t)n_q * qstride + (size_t)kvh * HD;
    const float* w = isq ? qn_w : kn_w;

    float x[E];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        x[e] = src[e * QLM_WAVE + lane];
        ss = fmaf(x[e], x[e], ss);
    }
    if (w) {
        ss = wave_sum(ss);
        const float s = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = (x[e] * s) * (1.0f + w[e * QLM_WAVE + lane]);
    }
#pragma unroll
    for (int e = 0; e < E; ++e) sh[e * QLM_WAVE + lane] = x[e];
    __syncthreads();
    const int half = rot / 2;
    const float* ct = cos_tab + (size_t)p * half;
    const float* st = sin_tab + (size_t)p * half;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = e * QLM_WAVE + lane;
        if (i < half) {
            x[e] = nc_mul_sub(sh[i], ct[i], sh[i + half], st[i]);
        } else if (i < rot) {
            const int i2 = i - half;
            x[e] = nc_mul_add2(sh[i], ct[i2], sh[i2], st[i2]);
        }
    }
    if (isq) {
#pragma unroll
        for (int e = 0; e < E; ++e) src[e * QLM_WAVE + lane] = x[e];
    } else {
        const size_t off = (((size_t)b * max_seq + p) * n_kv + kvh) * HD;
        const float* vsrc = row + (size_t)n_q * qstride + (size_t)(n_kv + kvh) * HD;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            kc[off + e * QLM_WAVE + lane] = x[e];
            vc[off + e * QLM_WAVE + lane] = vsrc[e * QLM_WAVE + lane];
        }
    }
}

// ---- partial: one chunk of positions for one kv head and its G q heads ----
template <int HD, int G, typename KV>
__global__ __launch_bounds__(kThreads) void k_attn_partial(
    const float* __restrict__ q, int ldq, int qhs, const KV* __restrict__ kc,
    const KV* __restrict__ vc, int max_seq, int n_kv, const int* __restrict__ pos, int ctx,
    float* __restrict__ work, int nchunks, int n_q, float scale) {
    constexpr int LPP = HD / 8;              // lanes per position in the score phase
    constexpr int PPW = QLM_WAVE / LPP;      // positions per wave step
    constexpr int NW = kThreads / QLM_WAVE;  // 4
    constexpr int C4 = HD / 4;               // float4 columns per row
    constexpr int NPG = kThreads / C4;       // position groups in the PV phase
    __shared__ float qs[G][HD];
    __shared__ float sc[G][kCH];
    __shared__ float4 red[NPG][G][C4];

    const int chunk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = min(pos ? pos[b] + 1 : ctx, max_seq);
    const int start = chunk * kCH;
    if (start >= L) return;
    const int n = min(kCH, L - start);

    for (int i = tid; i < G * HD; i += kThreads) {
        const int g = i / HD, e = i % HD;
        qs[g][e] = q[(size_t)b * ldq + (size_t)(kvh * G + g) * qhs + e];
    }
    __syncthreads();

    // scores
    {
        const int sub = lane % LPP, pw = lane / LPP;
        float qr[G][8];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) qr[g][e] = qs[g][sub * 8 + e];
        for (int pl = wave * PPW + pw; pl < n; pl += NW * PPW) {
            const size_t off = (((size_t)b * max_seq + start + pl) * n_kv + kvh) * HD + sub * 8;
            float kr[8];
            load8<KV>(kc + off, kr);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d = fmaf(qr[g][e], kr[e], d);
                d = group_sum<LPP>(d);
                if (sub == 0) sc[g][pl] = d * scale;
            }
        }
    }
    __syncthreads();

    // per-head chunk max, exponentials and sum
    __shared__ float mstat[G], lstat[G];
    for (int g = wave; g < G; g += NW) {
        float m = -INFINITY;
        for (int pl = lane; pl < n; pl += QLM_WAVE) m = fmaxf(m, sc[g][pl]);
        m = wave_max(m);
        float l = 0.0f;
        for (int pl = lane; pl < n; pl += QLM_WAVE) {
            const float e = expf(sc[g][pl] - m);
            sc[g][pl] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            mstat[g] = m;
            lstat[g] = l;
        }
    }
    __syncthreads();

    // P.V
    {
        const int c4 = tid % C4, pg = tid / C4;
        float4 acc[G];
#pragma unroll
        for (int g = 0; g < G; ++g) acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int pl = pg; pl < n; pl += NPG) {
            const size_t off = (((size_t)b * max_seq + start + pl) * n_kv + kvh) * HD + c4 * 4;
            const float4 v = load4<KV>(vc + off);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float e = sc[g][pl];
                acc[g].x = fmaf(e, v.x, acc[g].x);
                acc[g].y = fmaf(e, v.y, acc[g].y);
                acc[g].z = fmaf(e, v.z, acc[g].z);
                acc[g].w = fmaf(e, v.w, acc[g].w);
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) red[pg][g][c4] = acc[g];
    }
    __syncthreads();
    for (int i = tid; i < G * C4; i += kThreads) {
        const int g = i / C4, c4 = i % C4;
        float4 t = red[0][g][c4];
#pragma unroll
        for (int p2 = 1; p2 < NPG; ++p2) {
            const float4 u = red[p2][g][c4];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
        float* dst = work + (((size_t)b * n_q + kvh * G + g) * nchunks + chunk) * (HD + 4);
        reinterpret_cast<float4*>(dst + 4)[c4] = t;
        if (c4 == 0) {
            dst[0] = mstat[g];
            dst[1] = lstat[g];
        }
    }
}

// ---- combine: merge chunk partials, optional sigmoid output gate ----
template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(const float* __restrict__ work, int nchunks,
                                                     int max_seq, const int* __restrict__ pos,
                                                     int ctx,
                                                     const float* __restrict__ gate, int ldg,
                                                     int ghs, float* __restrict__ out, int ldo,
                                                     int n_q) {
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const int L = min(pos ? pos[b] + 1 : ctx, max_seq);
    const int nc = min(nchunks, (L + kCH - 1) / kCH);
    const float* base = work + ((size_t)b * n_q + h) * nchunks * (HD + 4);
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, base[(size_t)c * (HD + 4)]);
    float l = 0.0f, o = 0.0f;
    for (int c = 0; c < nc; ++c) {
        const float* pc = base + (size_t)c * (HD + 4);
        const float f = expf(pc[0] - M);
        l = fmaf(f, pc[1], l);
        o = fmaf(f, pc[4 + i], o);
    }
    float r = o / l;
    if (gate) {
        const float g = gate[(size_t)b * ldg + (size_t)h * ghs + i];
        r *= 1.0f / (1.0f + expf(-g));
    }
    out[(size_t)b * ldo + (size_t)h * HD + i] = r;
}

int nchunks_for(int max_seq) { return (max_seq + kCH - 1) / kCH; }

template <int HD, typename KV>
int launch_partial_g(int G, const float* q, int ldq, int qhs, const KV* kc, const KV* vc,
                     int max_seq, int n_kv, const int* pos, int ctx, float* work, int nchunks,
                     int n_q, int B, hipStream_t st) {
    const dim3 grid(nchunks, n_kv, B);
    const float scale = 1.0f / sqrtf((float)HD);
#define QLM_ATTN_G(GG)                                                                         \
    if (G == GG) {                                                                             \
        hipLaunchKernelGGL((k_attn_partial<HD, GG, KV>), grid, dim3(kThreads), 0, st, q, ldq,  \
                           qhs, kc, vc, max_seq, n_kv, pos, ctx, work, nchunks, n_q, scale);   \
        return qlm_launch_status();                                                            \
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
    return (size_t)B * n_q * nchunks_for(max_seq) * (hd + 4) * sizeof(float);
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
    const int nch = nchunks_for(max_seq);
    float* w = reinterpret_cast<float*>(work);
    int rc;
    if (hd == 128) {
        hipLaunchKernelGGL(k_attn_prep<128>, dim3(n_q + n_kv, B), dim3(QLM_WAVE), 0, st, qkv,
                           ldqkv, q_norm, k_norm, cos_tab, sin_tab, rot_dim, k_cache, v_cache,
                           max_seq, pos, n_q, n_kv, gated);
        rc = launch_partial_g<128, float>(G, qkv, ldqkv, qstride, k_cache, v_cache, max_seq, n_kv,
                                          pos, 0, w, nch, n_q, B, st);
        if (rc != QLM_OK) return rc;
        hipLaunchKernelGGL(k_attn_combine<128>, dim3(n_q, B), dim3(128), 0, st, w, nch, max_seq, pos, 0,
                           gated ? qkv + hd : nullptr, ldqkv, qstride, out, ldo, n_q);
    } else {
        hipLaunchKernelGGL(k_attn_prep<256>, dim3(n_q + n_kv, B), dim3(QLM_WAVE), 0, st, qkv,
                           ldqkv, q_norm, k_norm, cos_tab, sin_tab, rot_dim, k_cache, v_cache,
                           max_seq, pos, n_q, n_kv, gated);
        rc = launch_partial_g<256, float>(G, qkv, ldqkv, qstride, k_cache, v_cache, max_seq, n_kv,
                                          pos, 0, w, nch, n_q, B, st);
        if (rc != QLM_OK) return rc;
        hipLaunchKernelGGL(k_attn_combine<256>, dim3(n_q, B), dim3(256), 0, st, w, nch, max_seq, pos, 0,
                           gated ? qkv + hd : nullptr, ldqkv, qstride, out, ldo, n_q);
    }
    return qlm_launch_status();
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
    const int nch = nchunks_for(max_seq);
    float* w = reinterpret_cast<float*>(work);
    const int ldq = n_q * hd;
    int rc;
    if (hd == 128) {
        rc = kv_dtype == 0
                 ? launch_partial_g<128, float>(G, q, ldq, hd, (const float*)k_cache,
                                                (const float*)v_cache, max_seq, n_kv, nullptr,
                                                ctx, w, nch, n_q, B, st)
                 : launch_partial_g<128, uint16_t>(G, q, ldq, hd, (const uint16_t*)k_cache,
                                                   (const uint16_t*)v_cache, max_seq, n_kv,
                                                   nullptr, ctx, w, nch, n_q, B, st);
        if (rc != QLM_OK) return rc;
        hipLaunchKernelGGL(k_attn_combine<128>, dim3(n_q, B), dim3(128), 0, st, w, nch, max_seq,
                           nullptr, ctx, nullptr, 0, 0, out, ldq, n_q);
    } else {
        rc = kv_dtype == 0
                 ? launch_partial_g<256, float>(G, q, ldq, hd, (const float*)k_cache,
                                                (const float*)v_cache, max_seq, n_kv, nullptr,
                                                ctx, w, nch, n_q, B, st)
                 : launch_partial_g<256, uint16_t>(G, q, ldq, hd, (const uint16_t*)k_cache,
                                                   (const uint16_t*)v_cache, max_seq, n_kv,
                                                   nullptr, ctx, w, nch, n_q, B, st);
        if (rc != QLM_OK) return rc;
        hipLaunchKernelGGL(k_attn_combine<256>, dim3(n_q, B), dim3(256), 0, st, w, nch, max_seq,
                           nullptr, ctx, nullptr, 0, 0, out, ldq, n_q);
    }
    return qlm_launch_status();
}
