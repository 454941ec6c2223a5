// Shared device helpers for the gfx950 kernels (wave64, CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qlm_hip.h"

#define QLM_WAVE 64

// Map a HIP status to the C ABI's return convention (positive HIP code).
static inline int qlm_status(hipError_t e) { return e == hipSuccess ? QLM_OK : (int)e; }

static inline int qlm_launch_status() { return qlm_status(hipGetLastError()); }

static inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Butterfly sum over the full wave (64 lanes); every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, QLM_WAVE);
    return v;
}

// Butterfly sum over aligned groups of `width` lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int m = width / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, QLM_WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, QLM_WAVE));
    return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `red` is LDS
// scratch of at least blockDim.x/64 floats. Result valid in every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & (QLM_WAVE - 1);
    const int wave = threadIdx.x / QLM_WAVE;
    const int nw = blockDim.x / QLM_WAVE;
    __syncthreads();  // red may still be read by a previous call
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// Expressions evaluated with one IEEE rounding per operation and no FMA
// contraction (the library is built with -ffp-contract=fast-honor-pragmas, so
// the pragma is binding). Used where the reference computes a separate
// multiply and add and the result must match it bit for bit.
__device__ __forceinline__ float nc_mul_sub(float a, float b, float c, float d) {
#pragma clang fp contract(off)
    return a * b - c * d;  // (a*b) - (c*d)
}
__device__ __forceinline__ float nc_mul_add2(float a, float b, float c, float d) {
#pragma clang fp contract(off)
    return a * b + c * d;  // (a*b) + (c*d)
}
__device__ __forceinline__ float nc_add_mul(float acc, float a, float b) {
#pragma clang fp contract(off)
    return acc + a * b;  // acc + (a*b)
}

// Signed bytes of a 32-bit word as floats (exact).
__device__ __forceinline__ void i8x4_to_f32(int w, float& f0, float& f1, float& f2, float& f3) {
    f0 = (float)((w << 24) >> 24);
    f1 = (float)((w << 16) >> 24);
    f2 = (float)((w << 8) >> 24);
    f3 = (float)(w >> 24);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
