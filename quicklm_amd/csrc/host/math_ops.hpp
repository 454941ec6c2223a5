// Device operator layer with the reference's `math::` interface
// (src/ops/math_ops.hpp:89-192). Each function validates shapes on the host
// and enqueues gfx950 kernels through the C ABI (include/qlm_hip.h) on the
// current stream; nothing synchronises, so a sequence of calls can be
// captured into a hipGraph. Errors throw std::runtime_error (the reference's
// error convention); unsupported operand kinds throw instead of falling back.
#pragma once

#include <cstddef>

#include "tensor.hpp"

namespace qlm {
namespace math {

// Stream every op enqueues on (hipStream_t as void*; nullptr = null stream).
void set_stream(void* stream);
void* stream();

// C = A * B^T with B an int8 (Q8_0) weight operand; A [M, K] fp32, C [M, N]
// with row stride C.row_stride() (math_ops.hpp:92; math_ops.cpp:820-900).
void matmul(const Tensor& A, const Tensor& B, Tensor& C, bool transpose_B = true);
// Device workspace for the matrix-core forms (M > 1): at least
// qlm_matmul_i8_workspace_bytes() and qlm_matmul_i8_mx_workspace_bytes() of
// every call that follows.
void set_matmul_workspace(void* p, size_t bytes);
// Whether M activation rows against an [N, K] weight with a tile-major copy
// take the int8 matrix-core batched form, and the kernel launches one
// matmul call makes (for launch counts).
bool use_tiles_batched(int64_t M, int64_t N, int64_t K);
int matmul_launches(int64_t M, int64_t N, int64_t K, bool norm, bool native = false);

// math_ops.hpp:102 / :139-140 / :132.
void rms_norm(const Tensor& input, const Tensor& weight, Tensor& output, float eps);
void add_rms_norm(Tensor& residual, const Tensor& delta, const Tensor& weight, Tensor& output,
                  float eps);
void silu_mul(Tensor& A, const Tensor& B);

// math_ops.hpp:152: partial NeoX RoPE on t [num_heads, head_stride]; the
// reference recomputes cos/sin per position, here they come from a table
// built on the host with the same float arithmetic (rope_table()).
void apply_rope_neox(Tensor& t, const int* d_pos, const float* cos_tab, const float* sin_tab,
                     int rotary_dim);
void rope_table(float theta, int rotary_dim, int n_pos, float* cos_tab, float* sin_tab);

// math_ops.hpp:169-171 (device pointers).
void causal_conv1d_update_tapmajor(const float* input, float* state, int oldest_tap,
                                   const float* weight_t, float* output, int conv_dim,
                                   int kernel_size);

// ---- fused decode-step operators (no single reference function) ----
// matmul with RMSNorm(A) folded in (RMSNorm::forward + matmul).
void matmul_rmsnorm(const Tensor& A, const Tensor& norm_w, float eps, const Tensor& B, Tensor& C);
// residual[m, n] += (A * B^T)[m, n] (matmul + elementwise_add).
void matmul_residual(const Tensor& A, const Tensor& B, Tensor& residual);
// One row of the column-split DeltaNet mixer (qlm_deltanet_decode_cols)
// through its out-projection: residual += (U scaled per 128-column head by
// 1/sqrt(sum of ss[head][0..7] / 128 + eps)) * B^T, the head RMSNorm of
// attention.cpp:574-578 applied in the GEMV prologue. headnorm_supported()
// says whether B has the tile-major copy and launch shape this needs.
bool headnorm_supported(const Tensor& B);
void matmul_headnorm_residual(const Tensor& U, const float* ss, float eps, const Tensor& B,
                              Tensor& residual);
// SwiGLU: B holds [gate; up] rows; C = silu(norm(A) gate^T) * (norm(A) up^T).
void matmul_swiglu_rmsnorm(const Tensor& A, const Tensor& norm_w, float eps, const Tensor& B,
                           Tensor& C);

}  // namespace math
}  // namespace qlm
