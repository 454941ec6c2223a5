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

// Cross-lane reductions. Within a row of 16 lanes they run on DPP (a VALU
// operand modifier, no LDS round trip): xor 1 and xor 2 as quad permutes;
// once every lane of a quad holds the same value, the row half-mirror
// (lane i <-> 7-i) and mirror (i <-> 15-i) pair quads and half-rows exactly
// as xor 4 and xor 8 would. Across rows, xor 16 and 32 are lane swaps.
// Callers keep every lane of the wave active (the reductions read all of
// them).
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Across rows: v(l) op v(l ^ 16) and v(l) op v(l ^ 32) on every lane, by
// v_permlane16_swap / v_permlane32_swap (VALU lane swaps, no LDS permute).
// With both operands v, the swap's two results hold, on every lane, the
// values of the lane pair in either order; op is commutative.
__device__ __forceinline__ float xor16_add(float v) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float xor32_add(float v) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// Sum over aligned groups of `width` lanes (a power of two, 2..64); every
// lane of a group gets the group total.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(width >= 2 && width <= QLM_WAVE && (width & (width - 1)) == 0, "group width");
    v += dpp_mov<kDppXor1>(v);
    if constexpr (width >= 4) v += dpp_mov<kDppXor2>(v);
    if constexpr (width >= 8) v += dpp_mov<kDppHalfMirror>(v);
    if constexpr (width >= 16) v += dpp_mov<kDppMirror>(v);
    if constexpr (width >= 32) v = xor16_add(v);
    if constexpr (width >= 64) v = xor32_add(v);
    return v;
}

// Sum over the full wave (64 lanes); every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) { return group_sum<QLM_WAVE>(v); }

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<kDppXor1>(v));
    v = fmaxf(v, dpp_mov<kDppXor2>(v));
    v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_mov<kDppMirror>(v));
    return xor32_max(xor16_max(v));
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
