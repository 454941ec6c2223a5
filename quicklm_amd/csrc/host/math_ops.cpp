#include "math_ops.hpp"

#include <cmath>
#include <stdexcept>
#include <string>

#include "device.hpp"

namespace qlm {
namespace math {

namespace {
void* g_stream = nullptr;
void* g_mm_work = nullptr;
size_t g_mm_work_bytes = 0;

// Rows from which the matrix-core paths replace the row-major GEMV (which
// re-reads the weights once per 4 activation rows).
constexpr int64_t kMfmaMinRows = 2;

void need(bool ok, const char* what) {
    if (!ok) throw std::runtime_error(std::string("math: ") + what);
}

void check_int8(const Tensor& B) {
    need(B.is_int8(), "weight operand must be int8 (or int4 unpacked) on the device");
    need(B.shape.size() == 2, "int8 weight must be [N, K]");
}

// Native (fp32 / bf16) weights: qlm_matmul_w for every M and epilogue.
void matmul_native(const Tensor& A, const float* norm_w, float eps, const Tensor& B, float* C,
                   int64_t ldc, int64_t N, int epilogue) {
    check(qlm_matmul_w(A.data, (int)A.row_stride(), norm_w, eps, B.native_data,
                       B.native_bf16 ? 1 : 0, C, (int)ldc, (int)A.rows(), (int)N, (int)A.cols(),
                       epilogue, g_mm_work, g_mm_work_bytes, g_stream),
          "qlm_matmul_w");
}
}  // namespace

bool use_tiles_batched(int64_t M, int64_t N, int64_t K) {
    (void)N;
    return M >= 2 && M <= 16 && K % 64 == 0;
}

int matmul_launches(int64_t M, int64_t N, int64_t K, bool norm, bool native) {
    if (native) return (int)((M + 15) / 16) * (norm ? 2 : 1);  // row prep + matmul per 16 rows
    if (M == 1) return 1;
    if (use_tiles_batched(M, N, K)) return 2;  // matmul + ordered reduction
    if (M < kMfmaMinRows) return (int)((M + 3) / 4);
    (void)norm;  // row norms are folded into the reduction (or precede a direct store)
    return 2;    // split-K matmul + ordered reduction
}

void set_stream(void* s) { g_stream = s; }
void* stream() { return g_stream; }
void set_matmul_workspace(void* p, size_t bytes) {
    g_mm_work = p;
    g_mm_work_bytes = bytes;
}

namespace {
// One activation row on the matrix cores over the tile-major copy of the
// weight (qlm_gemv_i8_mx); false when the weight has no such copy or no
// launch shape fits K, and the row-major GEMV takes the row.
bool gemv_tiles(const Tensor& A, const float* norm_w, float eps, const Tensor& B, float* C,
                int64_t N, int epilogue) {
    if (A.rows() != 1 || !B.int8_tiles) return false;
    const int rc =
        B.int4_tiles
            ? qlm_gemv_i4_mx(A.data, norm_w, eps, B.int4_tiles, B.int8_tile_scales, C, (int)N,
                             (int)A.cols(), epilogue, g_stream)
            : qlm_gemv_i8_mx(A.data, norm_w, eps, B.int8_tiles, B.int8_tile_scales,
                             B.int8_group, C, (int)N, (int)A.cols(), epilogue, g_stream);
    if (rc == QLM_ERR_SHAPE) return false;
    check(rc, "qlm_gemv_i8_mx");
    return true;
}

// 2..8 activation rows on the int8 matrix cores over the tile-major copy
// (qlm_matmul_i8_mx): measured faster than the split-K bf16 form for wide
// matrices (N >= 4096) and short K (<= 2048); the 2560-row, 9728-column down
// projection keeps the split-K form, which spreads its few 16-row tiles over
// more workgroups. false when not taken.
bool gemm_tiles(const Tensor& A, const float* norm_w, float eps, const Tensor& B, float* C,
                int64_t ldc, int64_t N, int epilogue) {
    const int64_t M = A.rows(), K = A.cols();
    if (!use_tiles_batched(M, N, K) || !B.int8_tiles) return false;
    if (B.int8_group == 32) {  // weights streamed from registers on the bf16 matrix cores
        const size_t need_t = qlm_matmul_i8_t_workspace_bytes((int)M, (int)N, (int)K, epilogue);
        need(g_mm_work && g_mm_work_bytes >= need_t,
             "matmul: batched rows need set_matmul_workspace() of qlm_matmul_i8_t_workspace_bytes()");
        const int rt = qlm_matmul_i8_t(A.data, (int)A.row_stride(), norm_w, eps, B.int8_tiles,
                                       B.int8_tile_scales, B.int8_group, C, (int)ldc, (int)M,
                                       (int)N, (int)K, epilogue, g_mm_work, g_mm_work_bytes,
                                       g_stream);
        if (rt != QLM_ERR_SHAPE) {
            check(rt, "qlm_matmul_i8_t");
            return true;
        }
    }
    // per-row scales: the int8 digit form, up to 8 rows
    if (M > 8 || (N < 4096 && K > 2048)) return false;
    const size_t need_b = qlm_matmul_i8_mx_workspace_bytes((int)M, (int)K);
    need(g_mm_work && g_mm_work_bytes >= need_b,
         "matmul: batched rows need set_matmul_workspace() of qlm_matmul_i8_mx_workspace_bytes()");
    const int rc = qlm_matmul_i8_mx(A.data, (int)A.row_stride(), norm_w, eps, B.int8_tiles,
                                    B.int8_tile_scales, B.int8_group, C, (int)ldc, (int)M, (int)N,
                                    (int)K, epilogue, g_mm_work, g_mm_work_bytes, g_stream);
    if (rc == QLM_ERR_SHAPE) return false;
    check(rc, "qlm_matmul_i8_mx");
    return true;
}

// The split-K bf16 matrix-core matmul for M > 1 rows (norm_w null: no
// RMSNorm prologue), over the tile-major copy when the model has one (then
// the only copy), else the row-major weights; any M.
void matmul_mfma(const Tensor& A, const float* norm_w, float eps, const Tensor& B, float* C,
                 int64_t ldc, int64_t N, int epilogue) {
    const int64_t M = A.rows(), K = A.cols();
    const size_t need_b = qlm_matmul_i8_workspace_bytes((int)M, (int)N, (int)K, epilogue);
    need(g_mm_work && g_mm_work_bytes >= need_b,
         "matmul: M > 1 needs set_matmul_workspace() of qlm_matmul_i8_workspace_bytes()");
    if (B.int8_tiles) {
        check(qlm_matmul_i8_tm(A.data, (int)A.row_stride(), norm_w, eps, B.int8_tiles,
                               B.int8_tile_scales, B.int8_group, C, (int)ldc, (int)M, (int)N,
                               (int)K, epilogue, g_mm_work, g_mm_work_bytes, g_stream),
              "qlm_matmul_i8_tm");
        return;
    }
    check(qlm_matmul_i8(A.data, (int)A.row_stride(), norm_w, eps, B.int8_data, B.int8_scales,
                        B.int8_group, C, (int)ldc, (int)M, (int)N, (int)K, epilogue, g_mm_work,
                        g_mm_work_bytes, g_stream),
          "qlm_matmul_i8");
}
}  // namespace

void matmul(const Tensor& A, const Tensor& B, Tensor& C, bool transpose_B) {
    need(transpose_B, "only the x * W^T form exists on the device");
    const int64_t K = A.cols(), M = A.rows(), N = B.shape[0];
    need(B.shape[1] == K, "matmul: K mismatch");
    need(C.cols() >= N || C.row_stride() >= N, "matmul: output too small");
    if (B.is_native()) return matmul_native(A, nullptr, 0.0f, B, C.data, C.row_stride(), N, 0);
    check_int8(B);
    if (gemm_tiles(A, nullptr, 0.0f, B, C.data, C.row_stride(), N, 0)) return;
    if (M >= kMfmaMinRows) {
        matmul_mfma(A, nullptr, 0.0f, B, C.data, C.row_stride(), N, 0);
        return;
    }
    if (gemv_tiles(A, nullptr, 0.0f, B, C.data, N, 0)) return;
    if (!B.int8_data) return matmul_mfma(A, nullptr, 0.0f, B, C.data, C.row_stride(), N, 0);
    check(qlm_gemv_i8(A.data, (int)A.row_stride(), B.int8_data, B.int8_scales, B.int8_group, C.data,
                      (int)C.row_stride(), (int)M, (int)N, (int)K, g_stream),
          "qlm_gemv_i8");
}

void matmul_rmsnorm(const Tensor& A, const Tensor& norm_w, float eps, const Tensor& B, Tensor& C) {
    const int64_t K = A.cols(), M = A.rows(), N = B.shape[0];
    need(B.shape[1] == K && norm_w.size() == K, "matmul_rmsnorm: K mismatch");
    if (B.is_native()) return matmul_native(A, norm_w.data, eps, B, C.data, C.row_stride(), N, 0);
    check_int8(B);
    if (gemm_tiles(A, norm_w.data, eps, B, C.data, C.row_stride(), N, 0)) return;
    if (M >= kMfmaMinRows) {
        matmul_mfma(A, norm_w.data, eps, B, C.data, C.row_stride(), N, 0);
        return;
    }
    if (gemv_tiles(A, norm_w.data, eps, B, C.data, N, 0)) return;
    if (!B.int8_data) return matmul_mfma(A, norm_w.data, eps, B, C.data, C.row_stride(), N, 0);
    check(qlm_gemv_i8_rmsnorm(A.data, (int)A.row_stride(), norm_w.data, eps, B.int8_data,
                              B.int8_scales, B.int8_group, C.data, (int)C.row_stride(), (int)M,
                              (int)N, (int)K, g_stream),
          "qlm_gemv_i8_rmsnorm");
}

void matmul_residual(const Tensor& A, const Tensor& B, Tensor& residual) {
    const int64_t K = A.cols(), M = A.rows(), N = B.shape[0];
    need(B.shape[1] == K && residual.cols() == N, "matmul_residual: shape mismatch");
    if (B.is_native())
        return matmul_native(A, nullptr, 0.0f, B, residual.data, residual.row_stride(), N, 1);
    check_int8(B);
    if (gemm_tiles(A, nullptr, 0.0f, B, residual.data, residual.row_stride(), N, 1)) return;
    if (M >= kMfmaMinRows) {
        matmul_mfma(A, nullptr, 0.0f, B, residual.data, residual.row_stride(), N, 1);
        return;
    }
    if (gemv_tiles(A, nullptr, 0.0f, B, residual.data, N, 1)) return;
    if (!B.int8_data)
        return matmul_mfma(A, nullptr, 0.0f, B, residual.data, residual.row_stride(), N, 1);
    check(qlm_gemv_i8_residual(A.data, (int)A.row_stride(), B.int8_data, B.int8_scales,
                               B.int8_group, residual.data, (int)residual.row_stride(), (int)M,
                               (int)N, (int)K, g_stream),
          "qlm_gemv_i8_residual");
}

bool headnorm_supported(const Tensor& B) {
    if (B.is_native() || !B.is_int8() || !B.int8_tiles || B.shape.size() != 2) return false;
    const int64_t N = B.shape[0], K = B.shape[1];
    int waves = 0, ring = 0, grid = 0;
    return K % 128 == 0 && qlm_gemv_i8_mx_shape((int)N, (int)K, 1, &waves, &ring, &grid) == QLM_OK;
}

void matmul_headnorm_residual(const Tensor& U, const float* ss, float eps, const Tensor& B,
                              Tensor& residual) {
    const int64_t K = U.cols(), N = B.shape[0];
    need(U.rows() == 1 && B.shape[1] == K && residual.cols() == N,
         "matmul_headnorm_residual: shape mismatch");
    need(headnorm_supported(B), "matmul_headnorm_residual: weight has no tile-major copy");
    const int rc = B.int4_tiles
                       ? qlm_gemv_i4_mx_headnorm(U.data, ss, eps, B.int4_tiles, B.int8_tile_scales,
                                                 residual.data, (int)N, (int)K, 1, g_stream)
                       : qlm_gemv_i8_mx_headnorm(U.data, ss, eps, B.int8_tiles, B.int8_tile_scales,
                                                 B.int8_group, residual.data, (int)N, (int)K, 1,
                                                 g_stream);
    check(rc, "qlm_gemv_i8_mx_headnorm");
}

void matmul_swiglu_rmsnorm(const Tensor& A, const Tensor& norm_w, float eps, const Tensor& B,
                           Tensor& C) {
    const int64_t K = A.cols(), M = A.rows(), F = B.shape[0] / 2;
    need(B.shape[0] % 2 == 0 && B.shape[1] == K && C.cols() == F, "matmul_swiglu: shape mismatch");
    if (B.is_native()) return matmul_native(A, norm_w.data, eps, B, C.data, C.row_stride(), F, 2);
    check_int8(B);
    if (gemm_tiles(A, norm_w.data, eps, B, C.data, C.row_stride(), F, 2)) return;
    if (M >= kMfmaMinRows) {
        matmul_mfma(A, norm_w.data, eps, B, C.data, C.row_stride(), F, 2);
        return;
    }
    if (gemv_tiles(A, norm_w.data, eps, B, C.data, F, 2)) return;
    if (!B.int8_data) return matmul_mfma(A, norm_w.data, eps, B, C.data, C.row_stride(), F, 2);
    check(qlm_gemv_i8_swiglu_rmsnorm(A.data, (int)A.row_stride(), norm_w.data, eps, B.int8_data,
                                     B.int8_scales, B.int8_group, C.data, (int)C.row_stride(),
                                     (int)M, (int)F, (int)K, g_stream),
          "qlm_gemv_i8_swiglu_rmsnorm");
}

void rms_norm(const Tensor& input, const Tensor& weight, Tensor& output, float eps) {
    const int64_t n = weight.size();
    check(qlm_rms_norm(input.data, weight.data, output.data, (int)(input.size() / n), (int)n, eps,
                       g_stream),
          "qlm_rms_norm");
}

void add_rms_norm(Tensor& residual, const Tensor& delta, const Tensor& weight, Tensor& output,
                  float eps) {
    const int64_t n = weight.size();
    check(qlm_add_rms_norm(residual.data, delta.data, weight.data, output.data,
                           (int)(residual.size() / n), (int)n, eps, g_stream),
          "qlm_add_rms_norm");
}

void silu_mul(Tensor& A, const Tensor& B) {
    check(qlm_silu_mul(A.data, B.data, (int)A.size(), g_stream), "qlm_silu_mul");
}

void apply_rope_neox(Tensor& t, const int* d_pos, const float* cos_tab, const float* sin_tab,
                     int rotary_dim) {
    check(qlm_rope_neox(t.data, (int)t.rows(), (int)t.row_stride(), rotary_dim, cos_tab, sin_tab,
                        d_pos, g_stream),
          "qlm_rope_neox");
}

// Same float arithmetic as the reference's cached tables (math_ops.cpp:
// 1255-1272): inv[i] = 1/powf(theta, 2i/rot); angle = (float)pos * inv[i].
void rope_table(float theta, int rotary_dim, int n_pos, float* cos_tab, float* sin_tab) {
    const int half = rotary_dim / 2;
    std::vector<float> inv(half);
    for (int i = 0; i < half; ++i)
        inv[i] = 1.0f / std::pow(theta, (2.0f * i) / rotary_dim);
    for (int p = 0; p < n_pos; ++p)
        for (int i = 0; i < half; ++i) {
            const float ang = p * inv[i];
            cos_tab[(size_t)p * half + i] = std::cos(ang);
            sin_tab[(size_t)p * half + i] = std::sin(ang);
        }
}

void causal_conv1d_update_tapmajor(const float* input, float* state, int oldest_tap,
                                   const float* weight_t, float* output, int conv_dim,
                                   int kernel_size) {
    check(qlm_conv1d_update(input, state, oldest_tap, weight_t, output, conv_dim, kernel_size,
                            g_stream),
          "qlm_conv1d_update");
}

}  // namespace math
}  // namespace qlm
