// Load-time symmetric int8 quantiser (Q8_0 layout), bit-exact with the
// reference's IEEE semantics (st_quantize_row_f32 / _bf16,
// safetensors.cpp:296-391): per group m = max|x|, s = m > 0 ? m/127 : 1,
// inv = 1/s, q = clamp(rne(x*inv), -127, 127). Division and sqrt are IEEE in
// HIP by default; the product x*inv is a single rounded multiply (nothing to
// contract); rintf rounds half to even like _mm256_round_ps(NEAREST_INT).

#include "common.hpp"

namespace {

template <typename T>
__device__ __forceinline__ float load_val(const T* p);
template <>
__device__ __forceinline__ float load_val<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_val<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

__device__ __forceinline__ int8_t quant_one(float v, float inv) {
    float r = rintf(__fmul_rn(v, inv));
    int qv = (int)r;
    qv = qv < -127 ? -127 : (qv > 127 ? 127 : qv);
    return (int8_t)qv;
}

// G = 32: one thread per group of 32 contiguous values.
template <typename T>
__global__ __launch_bounds__(256) void k_quant_g32(const T* __restrict__ w, long long ngroups,
                                                   int8_t* __restrict__ q, float* __restrict__ s) {
    const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= ngroups) return;
    const T* src = w + g * 32;
    float v[32];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        v[i] = load_val<T>(src + i);
        m = fmaxf(m, fabsf(v[i]));
    }
    const float scale = (m > 0.0f) ? (m / 127.0f) : 1.0f;
    const float inv = 1.0f / scale;
    s[g] = scale;
    int packed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t b0 = (uint8_t)quant_one(v[4 * i + 0], inv);
        uint32_t b1 = (uint8_t)quant_one(v[4 * i + 1], inv);
        uint32_t b2 = (uint8_t)quant_one(v[4 * i + 2], inv);
        uint32_t b3 = (uint8_t)quant_one(v[4 * i + 3], inv);
        packed[i] = (int)(b0 | (b1 << 8) | (b2 << 16) | (b3 << 24));
    }
    int4* dst = reinterpret_cast<int4*>(q + g * 32);
    dst[0] = make_int4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_int4(packed[4], packed[5], packed[6], packed[7]);
}

// G = K: one workgroup per row.
template <typename T>
__global__ __launch_bounds__(256) void k_quant_row(const T* __restrict__ w, int K,
                                                   int8_t* __restrict__ q, float* __restrict__ s) {
    __shared__ float red[4];
    const long long row = blockIdx.x;
    const T* src = w + row * K;
    float m = 0.0f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) m = fmaxf(m, fabsf(load_val<T>(src + k)));
    m = wave_max(m);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float scale = (m > 0.0f) ? (m / 127.0f) : 1.0f;
    const float inv = 1.0f / scale;
    if (threadIdx.x == 0) s[row] = scale;
    for (int k = threadIdx.x; k < K; k += blockDim.x) q[row * K + k] = quant_one(load_val<T>(src + k), inv);
}

// int4 (Q4_0, st_quantize_row_f32_int4 / _bf16_int4, safetensors.cpp:393-515),
// G = 32: per group m = max|x|, s = m > 0 ? m/8 : 1, inv = 1/s,
// q = clamp(rne(x*inv), -8, 7), packed two per byte as the nibble q + 8 (low
// nibble = even column). One thread per group; with q8 set it also writes
// the signed values as int8, the operand of the int8 kernels (an int4
// matmul is the int8 one over these values, math_ops.cpp:604-700).
template <typename T>
__global__ __launch_bounds__(256) void k_quant4_g32(const T* __restrict__ w, long long ngroups,
                                                    uint8_t* __restrict__ q4,
                                                    float* __restrict__ s,
                                                    int8_t* __restrict__ q8) {
    const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= ngroups) return;
    const T* src = w + g * 32;
    float v[32];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        v[i] = load_val<T>(src + i);
        m = fmaxf(m, fabsf(v[i]));
    }
    const float scale = (m > 0.0f) ? (m / 8.0f) : 1.0f;
    const float inv = 1.0f / scale;
    s[g] = scale;
    int qi[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int r = (int)rintf(__fmul_rn(v[i], inv));
        qi[i] = r < -8 ? -8 : (r > 7 ? 7 : r);
    }
    unsigned pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 16; ++j)
        pk[j / 4] |= ((unsigned)(((qi[2 * j + 1] + 8) << 4) | (qi[2 * j] + 8))) << (8 * (j % 4));
    reinterpret_cast<int4*>(q4 + g * 16)[0] = make_int4(pk[0], pk[1], pk[2], pk[3]);
    if (q8) {
        unsigned b[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            b[i] = (unsigned)(uint8_t)qi[4 * i] | ((unsigned)(uint8_t)qi[4 * i + 1] << 8) |
                   ((unsigned)(uint8_t)qi[4 * i + 2] << 16) | ((unsigned)(uint8_t)qi[4 * i + 3] << 24);
        int4* d = reinterpret_cast<int4*>(q8 + g * 32);
        d[0] = make_int4(b[0], b[1], b[2], b[3]);
        d[1] = make_int4(b[4], b[5], b[6], b[7]);
    }
}

template <typename T>
int quant4_dispatch(const T* w, int rows, int K, uint8_t* q4, float* s, int8_t* q8,
                    void* stream) {
    if (!w || !q4 || !s || rows <= 0 || K <= 0) return QLM_ERR_ARG;
    if (K % 32 != 0 || (((uintptr_t)q4 | (uintptr_t)q8) & 15u)) return QLM_ERR_SHAPE;
    const long long ng = (long long)rows * (K / 32);
    const long long grid = (ng + 255) / 256;
    hipLaunchKernelGGL(k_quant4_g32<T>, dim3((unsigned)grid), dim3(256), 0, as_stream(stream), w,
                       ng, q4, s, q8);
    return qlm_launch_status();
}

template <typename T>
int quant_dispatch(const T* w, int rows, int K, int group, int8_t* q, float* s, void* stream) {
    if (!w || !q || !s || rows <= 0 || K <= 0) return QLM_ERR_ARG;
    hipStream_t st = as_stream(stream);
    if (group == 32) {
        if (K % 32 != 0 || ((uintptr_t)q & 15u)) return QLM_ERR_SHAPE;
        const long long ng = (long long)rows * (K / 32);
        const long long grid = (ng + 255) / 256;
        hipLaunchKernelGGL(k_quant_g32<T>, dim3((unsigned)grid), dim3(256), 0, st, w, ng, q, s);
    } else if (group == K) {
        hipLaunchKernelGGL(k_quant_row<T>, dim3(rows), dim3(256), 0, st, w, K, q, s);
    } else {
        return QLM_ERR_SHAPE;
    }
    return qlm_launch_status();
}

}  // namespace

extern "C" int qlm_quantize_q8_f32(const float* w, int rows, int K, int group, int8_t* q,
                                   float* scales, void* stream) {
    return quant_dispatch<float>(w, rows, K, group, q, scales, stream);
}

extern "C" int qlm_quantize_q8_bf16(const uint16_t* w, int rows, int K, int group, int8_t* q,
                                    float* scales, void* stream) {
    return quant_dispatch<uint16_t>(w, rows, K, group, q, scales, stream);
}

extern "C" int qlm_quantize_q4_f32(const float* w, int rows, int K, uint8_t* q4, float* scales,
                                   int8_t* q8, void* stream) {
    return quant4_dispatch<float>(w, rows, K, q4, scales, q8, stream);
}

extern "C" int qlm_quantize_q4_bf16(const uint16_t* w, int rows, int K, uint8_t* q4,
                                    float* scales, int8_t* q8, void* stream) {
    return quant4_dispatch<uint16_t>(w, rows, K, q4, scales, q8, stream);
}

// Loads this file's code object on the current device now; the runtime
// otherwise loads it at the first launch of one of its kernels (4-20 ms,
// measured inside a first prefill or decode step).
hipError_t qlm_load_quant() {
    hipFuncAttributes a;
    return hipFuncGetAttributes(&a, reinterpret_cast<const void*>((k_quant_g32<float>)));
}
