/*
 * qlm_oracle.h - CPU oracle (TEST INFRASTRUCTURE ONLY).
 *
 * A plain-C restatement of the reference QuickLM CPU arithmetic for the
 * hybrid decode path, written from the reference's source (each function
 * cites the file:line it follows). Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the oracle
 * the results are compared with.
 * The product path never links it.
 *
 * Every reduction keeps the reference's operation order (its 8-lane AVX2
 * accumulators, fused multiply-adds where it uses _mm256_fmadd_ps, separate
 * multiply and add elsewhere), so with -ffp-contract=off this library is
 * bit-identical to the reference sources compiled with the same IEEE flags
 * (oracle/_ref/libqlm_ref_ieee.so); tests/test_oracle.py pins that.
 */
#ifndef QLM_ORACLE_H
#define QLM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A2 quantiser (safetensors.cpp:296-391); group 32 or K. */
void orc_quantize_rows_f32(const float* w, int rows, int K, int group, int8_t* q, float* s);
void orc_quantize_rows_bf16(const uint16_t* w, int rows, int K, int group, int8_t* q, float* s);

/* int4 (Q4_0) quantiser (safetensors.cpp:393-515): packed rows of (K+1)/2
 * bytes (low nibble = even column), one scale per 32 columns; unpacking to
 * the signed values; int4 matmul (math_ops.cpp:581-818). C is [M, ldc]. */
void orc_quantize_rows_q4_f32(const float* w, int rows, int K, uint8_t* q, float* s);
void orc_quantize_rows_q4_bf16(const uint16_t* w, int rows, int K, uint8_t* q, float* s);
void orc_unpack_q4(const uint8_t* p, int rows, int K, int8_t* q);
void orc_matmul_i4(const float* A, int M, int K, const uint8_t* p, const float* s, int N,
                   float* C, int ldc);

/* Native (unquantised) weights, the reference's --precision bf16: fp32 rows
 * (dot_avx2, math_ops.cpp:209-240) or bf16 rows (dot_avx2_bf16, :245-400).
 * W is [N, K]; bf16 = 1 for bf16 bits. C is [M, ldc]. */
void orc_matmul_w(const float* A, int M, int K, const void* W, int bf16, int N, float* C,
                  int ldc);

/* A3/A4 int8 matmul (math_ops.cpp:405-579, :820-900). C is [M, ldc]. */
void orc_matmul_i8(const float* A, int M, int K, const int8_t* q, const float* s, int group,
                   int N, float* C, int ldc);

/* A5/A6 (math_ops.cpp:990-1072, :1133-1172). */
float orc_sumsq(const float* x, int n);
void orc_rms_norm(const float* x, const float* w, float* y, int rows, int n, float eps);
void orc_add_rms_norm(float* res, const float* d, const float* w, float* y, int rows, int n,
                      float eps);

/* A7 (math_ops.cpp:1076-1129). */
void orc_silu_mul(float* a, const float* b, int n);

/* A8 (math_ops.cpp:1237-1289): t is [num_heads, head_stride]. Also returns
 * the cos/sin table rows the reference would use for positions [0, n_pos). */
void orc_rope_neox(float* t, int num_heads, int head_stride, int pos, float theta, int rot);
void orc_rope_table(float theta, int rot, int n_pos, float* cos_tab, float* sin_tab);

/* A10 (math_ops.cpp:1321-1364). */
void orc_conv1d_tapmajor(const float* in, float* state, int oldest, const float* w_t,
                         float* out, int conv_dim, int kernel_size);

/* A12 recurrence, isolated (attention.cpp:498-571), per (b, h). */
void orc_gated_delta_step(const float* q, const float* k, const float* v, const float* decay,
                          const float* beta, float* state, float* out, int B, int H, int d);

/* A10-A12 mixer core of one decode step for one sequence (attention.cpp:
 * 439-585): proj = [qkv | z | b | a]; conv_state [3, 3*H*d] with oldest row
 * `oldest`; writes the gated head output [H*d]. */
void orc_deltanet_core(const float* proj, float* conv_state, int oldest, const float* conv_w_t,
                       const float* A_log, const float* dt_bias, const float* norm_w,
                       float* state, float* out, int H, int d);

/* A8/A9 mixer core of one decode step for one sequence (attention.cpp:160-227):
 * qkv = [q (n_q * qstride) | k | v]; cache [max_seq, n_kv, hd]. */
void orc_gqa_core(float* qkv, const float* q_norm, const float* k_norm, float theta, int rot,
                  float* k_cache, float* v_cache, int max_seq, int pos, float* out, int n_q,
                  int n_kv, int hd, int gated);

/* Isolated attention (gqa_attend_head, attention.cpp:54-82) over the first
 * ctx positions; q, out [n_q, hd]; cache [ctx_stride rows, n_kv, hd]. */
void orc_attention(const float* q, const float* k_cache, const float* v_cache, int ctx, float* out,
                   int n_q, int n_kv, int hd);

/* A14 greedy sampling (model.cpp:263-274). */
int orc_argmax(const float* x, int n);

/* Thread count for orc_matmul_i8 row parallelism (results do not depend on it). */
void orc_set_threads(int n);

#ifdef __cplusplus
}
#endif

#endif
