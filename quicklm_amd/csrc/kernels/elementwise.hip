// Small elementwise / per-row kernels: RMSNorm, residual-add RMSNorm, SiLU*mul,
// partial NeoX RoPE, tap-major causal conv1d step, byte fill, embedding
// gather, greedy argmax. All HBM-trivial; they exist as separate entry points
// for operator-level parity and for callers outside the fused decode step.

#include "common.hpp"

namespace {

constexpr int kRowThreads = 256;

// math::rms_norm (math_ops.cpp:1055-1072): s = 1/sqrt(sum(x^2)/n + eps);
// y = (x*s)*(1+w).
__global__ __launch_bounds__(kRowThreads) void k_rms_norm(const float* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          float* __restrict__ y, int n,
                                                          float eps) {
    __shared__ float red[kRowThreads / QLM_WAVE];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(xr[i], xr[i], ss);
    ss = block_sum(ss, red);
    const float s = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) yr[i] = (xr[i] * s) * (1.0f + w[i]);
}

// math::add_rms_norm (math_ops.cpp:1133-1172).
__global__ __launch_bounds__(kRowThreads) void k_add_rms_norm(float* __restrict__ res,
                                                              const float* __restrict__ d,
                                                              const float* __restrict__ w,
                                                              float* __restrict__ y, int n,
                                                              float eps) {
    __shared__ float red[kRowThreads / QLM_WAVE];
    float* rr = res + (size_t)blockIdx.x * n;
    const float* dr = d + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = rr[i] + dr[i];
        rr[i] = v;
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, red);
    const float s = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) yr[i] = (rr[i] * s) * (1.0f + w[i]);
}

__global__ void k_silu_mul(float* __restrict__ a, const float* __restrict__ b, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) a[i] = silu_f(a[i]) * b[i];
}

// math::apply_rope_neox (math_ops.cpp:1237-1289), cos/sin from the table row
// of position pos[0]. One thread per (head, pair).
__global__ void k_rope_neox(float* __restrict__ t, int num_heads, int head_stride, int rot,
                            const float* __restrict__ cos_tab, const float* __restrict__ sin_tab,
                            const int* __restrict__ pos) {
    const int half = rot / 2;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= num_heads * half) return;
    const int h = idx / half, i = idx % half;
    const int p = pos[0];
    const float c = cos_tab[(size_t)p * half + i];
    const float s = sin_tab[(size_t)p * half + i];
    float* hd = t + (size_t)h * head_stride;
    const float x1 = hd[i], x2 = hd[i + half];
    hd[i] = nc_mul_sub(x1, c, x2, s);
    hd[i + half] = nc_mul_add2(x2, c, x1, s);
}

// math::causal_conv1d_update_tapmajor (math_ops.cpp:1321-1364): separate
// multiply and add, chronological taps, then the oldest row takes the input.
__global__ void k_conv1d_update(const float* __restrict__ in, float* __restrict__ state,
                                int oldest, const float* __restrict__ wt,
                                float* __restrict__ out, int C, int ks) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    const int ntaps = ks - 1;
    float acc = 0.0f;
    for (int j = 0; j < ntaps; ++j) {
        const int row = (oldest + j) % ntaps;
        acc = nc_add_mul(acc, state[(size_t)row * C + c], wt[(size_t)j * C + c]);
    }
    const float x = in[c];
    acc = nc_add_mul(acc, x, wt[(size_t)ntaps * C + c]);
    out[c] = acc;
    state[(size_t)oldest * C + c] = x;
}

__global__ void k_fill_u8(uint8_t* __restrict__ p, uint8_t v, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const uint32_t v4 = (uint32_t)v * 0x01010101u;
    const size_t n4 = n / 4;
    uint32_t* p4 = reinterpret_cast<uint32_t*>(p);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) p4[i] = v4;
    for (size_t i = n4 * 4 + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        p[i] = v;
}

// Argmax, stage 1: each workgroup scans a slice of one row. First maximum
// wins (strict >), matching DecoderModel::sample (model.cpp:263-274).
constexpr int kArgThreads = 256;
constexpr int kArgSlice = 4096;
constexpr int kArgPer = kArgSlice / kArgThreads;  // logits per thread

__device__ __forceinline__ void arg_better(float& bv, int& bi, float v, int i) {
    const bool better = v > bv || (v == bv && i < bi);  // selects, no branch
    bv = better ? v : bv;
    bi = better ? i : bi;
}

__global__ __launch_bounds__(kArgThreads) void k_argmax_partial(const float* __restrict__ lg,
                                                                int ldl, int n,
                                                                float* __restrict__ pv,
                                                                int* __restrict__ pi, int nslice) {
    const int b = blockIdx.y;
    const int s = blockIdx.x;
    const float* row = lg + (size_t)b * ldl;
    const int lo = s * kArgSlice;
    const int hi = min(n, lo + kArgSlice);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    // the slice's logits are all requested before the first comparison (a
    // strided loop with a runtime bound would wait for each load in turn);
    // indices past the row are clamped and left out
    float v[kArgPer];
#pragma unroll
    for (int j = 0; j < kArgPer; ++j)
        v[j] = row[min(lo + (int)threadIdx.x + j * kArgThreads, hi - 1)];
#pragma unroll
    for (int j = 0; j < kArgPer; ++j) {
        const int i = lo + (int)threadIdx.x + j * kArgThreads;
        if (i < hi) arg_better(bv, bi, v[j], i);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(bv, m, QLM_WAVE);
        const int oi = __shfl_xor(bi, m, QLM_WAVE);
        arg_better(bv, bi, ov, oi);
    }
    __shared__ float sv[kArgThreads / QLM_WAVE];
    __shared__ int si[kArgThreads / QLM_WAVE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgThreads / QLM_WAVE; ++w) arg_better(bv, bi, sv[w], si[w]);
        pv[(size_t)b * nslice + s] = bv;
        pi[(size_t)b * nslice + s] = bi;
    }
}

// Argmax, stage 2: one wave per row over the slice winners. Optionally
// advances a generation: writes the winner as the token at pos[b]+1 unless
// that position still belongs to the prompt, then pos[b] += 1.
__global__ void k_argmax_final(const float* __restrict__ pv, const int* __restrict__ pi,
                               int nslice, int* __restrict__ idx, int* __restrict__ tokens,
                               int ld_tokens, int* __restrict__ pos,
                               const int* __restrict__ prompt_len) {
    // every argument read in one batch (otherwise the compiler reads some,
    // waits, branches and reads the rest: a second round trip)
    asm volatile("" ::"s"(pv), "s"(pi), "s"(nslice), "s"(idx), "s"(tokens), "s"(ld_tokens),
                 "s"(pos), "s"(prompt_len));
    const int b = blockIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int s = threadIdx.x; s < nslice; s += QLM_WAVE)
        arg_better(bv, bi, pv[(size_t)b * nslice + s], pi[(size_t)b * nslice + s]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(bv, m, QLM_WAVE);
        const int oi = __shfl_xor(bi, m, QLM_WAVE);
        arg_better(bv, bi, ov, oi);
    }
    if (threadIdx.x == 0) {
        // all -inf or NaN rows: the reference returns index 0
        if (bi == 0x7fffffff) bi = 0;
        if (idx) idx[b] = bi;
        if (tokens) {
            const int p = pos[b];
            if (p + 1 < ld_tokens && p + 1 >= prompt_len[b]) tokens[(size_t)b * ld_tokens + p + 1] = bi;
            pos[b] = p + 1;
        }
    }
}

// Embedding row gather for the token at each sequence's current position.
__global__ void k_embed(const float* __restrict__ table, int H, const int* __restrict__ tokens,
                        int ld_tokens, const int* __restrict__ pos, float* __restrict__ out,
                        int ldo, int vocab) {
    asm volatile("" ::"s"(table), "s"(H), "s"(tokens), "s"(ld_tokens), "s"(pos), "s"(out),
                 "s"(ldo), "s"(vocab));
    const int b = blockIdx.y;
    const int p = pos ? pos[b] : 0;
    int tok = tokens[(size_t)b * ld_tokens + p];
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
    const float4* src = reinterpret_cast<const float4*>(table + (size_t)tok * H);
    float4* dst = reinterpret_cast<float4*>(out + (size_t)b * ldo);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < H / 4; i += gridDim.x * blockDim.x)
        dst[i] = src[i];
}

}  // namespace

extern "C" int qlm_rms_norm(const float* x, const float* w, float* y, int rows, int n, float eps,
                            void* stream) {
    if (!x || !w || !y || rows <= 0 || n <= 0) return QLM_ERR_ARG;
    hipLaunchKernelGGL(k_rms_norm, dim3(rows), dim3(kRowThreads), 0, as_stream(stream), x, w, y, n,
                       eps);
    return qlm_launch_status();
}

extern "C" int qlm_add_rms_norm(float* res, const float* delta, const float* w, float* y, int rows,
                                int n, float eps, void* stream) {
    if (!res || !delta || !w || !y || rows <= 0 || n <= 0) return QLM_ERR_ARG;
    hipLaunchKernelGGL(k_add_rms_norm, dim3(rows), dim3(kRowThreads), 0, as_stream(stream), res,
                       delta, w, y, n, eps);
    return qlm_launch_status();
}

extern "C" int qlm_silu_mul(float* a, const float* b, int n, void* stream) {
    if (!a || !b || n <= 0) return QLM_ERR_ARG;
    hipLaunchKernelGGL(k_silu_mul, dim3((n + 255) / 256), dim3(256), 0, as_stream(stream), a, b, n);
    return qlm_launch_status();
}

extern "C" int qlm_rope_neox(float* t, int num_heads, int head_stride, int rot_dim,
                             const float* cos_tab, const float* sin_tab, const int* pos,
                             void* stream) {
    if (!t || !cos_tab || !sin_tab || !pos || num_heads <= 0 || rot_dim <= 0) return QLM_ERR_ARG;
    if (rot_dim % 2 != 0 || rot_dim > head_stride) return QLM_ERR_SHAPE;
    const int n = num_heads * (rot_dim / 2);
    hipLaunchKernelGGL(k_rope_neox, dim3((n + 255) / 256), dim3(256), 0, as_stream(stream), t,
                       num_heads, head_stride, rot_dim, cos_tab, sin_tab, pos);
    return qlm_launch_status();
}

extern "C" int qlm_conv1d_update(const float* in, float* state, int oldest_tap,
                                 const float* weight_t, float* out, int conv_dim, int kernel_size,
                                 void* stream) {
    if (!in || !state || !weight_t || !out || conv_dim <= 0 || kernel_size < 2) return QLM_ERR_ARG;
    if (oldest_tap < 0 || oldest_tap >= kernel_size - 1) return QLM_ERR_ARG;
    hipLaunchKernelGGL(k_conv1d_update, dim3((conv_dim + 255) / 256), dim3(256), 0,
                       as_stream(stream), in, state, oldest_tap, weight_t, out, conv_dim,
                       kernel_size);
    return qlm_launch_status();
}

extern "C" int qlm_fill_u8(void* dst, uint8_t value, size_t bytes, void* stream) {
    if (!dst) return QLM_ERR_ARG;
    if (bytes == 0) return QLM_OK;
    size_t blocks = (bytes / 4 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(k_fill_u8, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       reinterpret_cast<uint8_t*>(dst), value, bytes);
    return qlm_launch_status();
}

static int argmax_slices(int n) { return (n + kArgSlice - 1) / kArgSlice; }

extern "C" size_t qlm_argmax_workspace_bytes(int B, int n) {
    return (size_t)B * argmax_slices(n) * (sizeof(float) + sizeof(int)) + 256;
}

static int argmax_launch(const float* logits, int ldl, int n, int B, int* idx, void* work,
                         int* tokens, int ld_tokens, int* pos, const int* prompt_len,
                         void* stream) {
    if (!logits || !work || n <= 0 || B <= 0 || ldl < n) return QLM_ERR_ARG;
    const int ns = argmax_slices(n);
    float* pv = reinterpret_cast<float*>(work);
    int* pi = reinterpret_cast<int*>(pv + (size_t)B * ns);
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(k_argmax_partial, dim3(ns, B), dim3(kArgThreads), 0, st, logits, ldl, n, pv,
                       pi, ns);
    hipLaunchKernelGGL(k_argmax_final, dim3(B), dim3(QLM_WAVE), 0, st, pv, pi, ns, idx, tokens,
                       ld_tokens, pos, prompt_len);
    return qlm_launch_status();
}

extern "C" int qlm_argmax(const float* logits, int ldl, int n, int B, int* idx, void* work,
                          void* stream) {
    if (!idx) return QLM_ERR_ARG;
    return argmax_launch(logits, ldl, n, B, idx, work, nullptr, 0, nullptr, nullptr, stream);
}

extern "C" int qlm_greedy_advance(const float* logits, int ldl, int n, int B, void* work,
                                  int* tokens, int ld_tokens, int* pos, const int* prompt_len,
                                  void* stream) {
    if (!tokens || !pos || !prompt_len || ld_tokens <= 0) return QLM_ERR_ARG;
    return argmax_launch(logits, ldl, n, B, nullptr, work, tokens, ld_tokens, pos, prompt_len,
                         stream);
}

extern "C" int qlm_embed_tokens(const float* table, int vocab, int H, const int* tokens,
                                int ld_tokens, const int* pos, float* out, int ldo, int B,
                                void* stream) {
    if (!table || !tokens || !out || H <= 0 || B <= 0 || vocab <= 0) return QLM_ERR_ARG;
    if (H % 4 != 0 || ldo % 4 != 0) return QLM_ERR_SHAPE;
    const int blocks = (H / 4 + 255) / 256;
    hipLaunchKernelGGL(k_embed, dim3(blocks, B), dim3(256), 0, as_stream(stream), table, H, tokens,
                       ld_tokens, pos, out, ldo, vocab);
    return qlm_launch_status();
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_elementwise() {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(k_fill_u8));
}
