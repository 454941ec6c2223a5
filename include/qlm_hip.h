/*
 * qlm_hip.h - C ABI of the MI355X (gfx950) decode kernels.
 *
 * Every compute entry point replaces one operator of the reference CPU path
 * (treesoft-ai/quicklm); the comment above each one names the reference
 * interface it stands in for (file:line in the reference tree).
 *
 * Conventions
 *   - All tensor arguments are DEVICE pointers, row-major, fp32 unless noted.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - Every call is asynchronous, allocates nothing, never synchronises the
 *     host and reads no device memory back, so a sequence of calls can be
 *     captured into a hipGraph.
 *   - Return value: QLM_OK (0) or a negative QLM_ERR_* code; on a HIP error
 *     the HIP error code is returned as a positive number. Shape checks are
 *     done here, on the host, before any launch: kernels trust their shapes.
 *   - int8 weights use the reference's Q8_0 layout (tensor.hpp:30-41):
 *     q[n*K + k] int8, scale[n*ceil(K/G) + k/G] fp32, with the group size G
 *     either 32 (reference block size) or K (one scale per output row).
 */
#ifndef QLM_HIP_H
#define QLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QLM_OK 0
#define QLM_ERR_ARG (-1)      /* null pointer or non-positive size */
#define QLM_ERR_SHAPE (-2)    /* shape the kernels do not support */
#define QLM_ERR_NO_DEVICE (-3)
#define QLM_ERR_SCRATCH (-4)  /* work exceeds a no-allocation entry point's static scratch */

/* ---- runtime plumbing (no reference counterpart: the reference is host-only) ---- */

const char* qlm_error_string(int status);
int qlm_device_count(int* count);
/* Makes `device` current and loads every kernel code object of the library
 * on it (otherwise each kernel file's code object loads at its first launch,
 * 4-20 ms each, e.g. inside a first prefill). */
int qlm_set_device(int device);
int qlm_device_name(char* buf, int len);
/* Free and total device memory of the current device (hipMemGetInfo). */
int qlm_mem_info(size_t* free_bytes, size_t* total_bytes);
int qlm_malloc(void** ptr, size_t bytes);
int qlm_free(void* ptr);
int qlm_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int qlm_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int qlm_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* Fill with a byte value by a kernel (capturable; no hipMemset node). */
int qlm_fill_u8(void* dst, uint8_t value, size_t bytes, void* stream);
int qlm_stream_create(void** stream);
int qlm_stream_destroy(void* stream);
int qlm_stream_sync(void* stream);
int qlm_device_sync(void);
int qlm_event_create(void** event);
int qlm_event_destroy(void* event);
int qlm_event_record(void* event, void* stream);
int qlm_event_elapsed_ms(float* ms, void* start, void* stop);
int qlm_graph_begin(void* stream);
int qlm_graph_end(void* stream, void** graph_exec);
int qlm_graph_launch(void* graph_exec, void* stream);
int qlm_graph_destroy(void* graph_exec);

/* ---- A2: load-time int8 quantiser --------------------------------------
 * Replaces st_quantize_row_f32 / st_quantize_row_bf16 driven by
 * SafetensorsLoader::get_tensor_keep_int8 (safetensors.cpp:296-391, :517-585).
 * Per group of G elements: m = max|x|; s = m > 0 ? m/127 : 1; inv = 1/s;
 * q = clamp(round-half-even(x*inv), -127, 127). IEEE division, no FMA: the
 * bytes and scales are bit-identical to the reference's IEEE semantics.
 * K must be a multiple of G; G is 32 or K. */
int qlm_quantize_q8_f32(const float* w, int rows, int K, int group, int8_t* q, float* scales,
                        void* stream);
int qlm_quantize_q8_bf16(const uint16_t* w, int rows, int K, int group, int8_t* q,
                         float* scales, void* stream);

/* ---- A3/A4: int8 weight-only matmul  y = x . (q*s)^T ----------------------
 * Replaces math::matmul's int8 branch (math_ops.hpp:92, math_ops.cpp:820-900,
 * int8_gemv_range :558-579). x is [M, ldx], y is [M, ldy], weights [N, K].
 * fp32 accumulation. M <= 64; K a multiple of 16 (of 32 when G = 32). */
int qlm_gemv_i8(const float* x, int ldx, const int8_t* q, const float* scales, int group,
                float* y, int ldy, int M, int N, int K, void* stream);

/* M = 1 with an explicit launch shape, for tuning sweeps (the M = 1 forms of
 * qlm_gemv_i8 and the fused entry points below pick these from N and K).
 * norm_w NULL: plain x; else the RMSNorm prologue of qlm_gemv_i8_rmsnorm.
 * epilogue 0: y = result; 1: y += result (qlm_gemv_i8_residual); 2: SwiGLU
 * as qlm_gemv_i8_swiglu_rmsnorm (N = F outputs, weights [2F, K]).
 * lanes_per_row in {16,...,256} (power of two, at most 6 16-byte chunks per
 * lane), rows in {1,2} output rows per lane group and block, grid =
 * workgroups (grid-stride over row blocks, launched as given). */
int qlm_gemv_i8_config(const float* x, const float* norm_w, float eps, const int8_t* q,
                       const float* scales, int group, float* y, int N, int K, int epilogue,
                       int lanes_per_row, int rows, int grid, void* stream);

/* Tile-major weight layout of the matrix-core M = 1 GEMV below: each half of
 * the rows (halves = 2 for the [gate; up] SwiGLU matrix; rows = rows per
 * half) is padded with zero rows to 16-row tiles, and every 16-row x
 * 64-column block is stored as one contiguous 1 KB matrix-core operand in
 * lane order, so a wave streams HBM linearly. Group-32 scales are reordered
 * alike (32 floats per block); per-row scales (group = K) keep their layout
 * and s_bytes is 0. No counterpart in the reference (its weights stay
 * row-major in host memory). K a multiple of 64. */
int qlm_mx_layout_bytes(int rows, int K, int group, int halves, size_t* q_bytes,
                        size_t* s_bytes);
int qlm_mx_swizzle(const int8_t* q, const float* scales, int group, int rows, int K, int halves,
                   int8_t* q_out, float* s_out, void* stream);

/* M = 1 on the int8 matrix cores with tile-major weights (q and scales from
 * qlm_mx_swizzle; per-row scales as quantised), explicit launch shape.
 * x (after the RMSNorm prologue when norm_w is given) is written as four
 * int8 digit vectors with a power-of-two scale per wave (over the K blocks
 * that wave multiplies), x = 2^E (d0 + d1/2^7 + d2/2^14 + d3/2^21) to within
 * 2^-27 max|x|, and every weight group's dot products with the digits are
 * exact int32 sums (v_mfma_i32_16x16x64_i8); results match the fp32 path to
 * ~1e-7 normwise. norm_w and epilogue as qlm_gemv_i8_config. waves in
 * {4, 8, 16} per workgroup and ring = ceil(K / 64 / waves) blocks per wave,
 * one of the instantiated pairs (4,1) (4,2) (4,4) (4,8) (4,10) (8,4) (8,5)
 * (8,8) (16,2) (16,4) (16,10) (16,12); K a multiple of 64; grid =
 * workgroups (grid-stride over 16-row tiles). */
int qlm_gemv_i8_mx_config(const float* x, const float* norm_w, float eps, const int8_t* q,
                          const float* scales, int group, float* y, int N, int K, int epilogue,
                          int waves, int ring, int grid, void* stream);

/* The same with the launch shape picked from N, K and the epilogue (the
 * batch-1 decode projections: math::matmul / matmul_rmsnorm /
 * matmul_residual / SwiGLU with M = 1, math_ops.cpp:820-900). Returns
 * QLM_ERR_SHAPE when no instantiated shape fits K; the row-major GEMV
 * serves such weights. */
int qlm_gemv_i8_mx(const float* x, const float* norm_w, float eps, const int8_t* q_tiles,
                   const float* s_tiles, int group, float* y, int N, int K, int epilogue,
                   void* stream);
/* qlm_gemv_i8_mx over the output of qlm_deltanet_decode_cols: x[j] =
 * u[j] / sqrt(sum_s ss[j / 128][s] / 128 + eps) for each 128-column head
 * (ss [K / 128][8]), the head RMSNorm of Qwen3_5GatedDeltaNet::forward
 * (attention.cpp:574-578) applied before the out-projection; epilogue 0
 * store or 1 residual add. K a multiple of 128; u and ss 16-byte aligned.
 * The int4 form takes qlm_mx4_swizzle tiles (group 32). */
int qlm_gemv_i8_mx_headnorm(const float* u, const float* ss, float eps, const int8_t* q_tiles,
                            const float* s_tiles, int group, float* y, int N, int K, int epilogue,
                            void* stream);
int qlm_gemv_i4_mx_headnorm(const float* u, const float* ss, float eps, const uint8_t* q_tiles,
                            const float* s_tiles, float* y, int N, int K, int epilogue,
                            void* stream);
/* The launch shape qlm_gemv_i8_mx picks (waves per workgroup, blocks per
 * wave, workgroups), or QLM_ERR_SHAPE. Host only. */
int qlm_gemv_i8_mx_shape(int N, int K, int epilogue, int* waves, int* ring, int* grid);

/* ---- L2 prefetch plans (no reference counterpart: an MI355X scheduling aid) ----
 * MI355X runs workgroup i of a launch on XCD i % 8, and each XCD's 4 MB L2
 * keeps what one kernel read for the kernels after it. A plan lists a later
 * kernel's operands by tile: segment s of tile t is bytes[s] bytes at
 * base[s] + t * stride[s], read later by a workgroup on XCD t % 8, for
 * t < tiles[s]. The entry points that take a plan (qlm_deltanet_decode_cols_pf)
 * append workgroups that load every tile into the L2 of its XCD while their
 * own latency-bound work runs. A plan changes no result, only where the later
 * kernel finds its operands. Zero-initialise, then append. */
#define QLM_L2_PLAN_SEGMENTS 8
typedef struct qlm_l2_plan {
    const void* base[QLM_L2_PLAN_SEGMENTS];
    long long stride[QLM_L2_PLAN_SEGMENTS];
    int bytes[QLM_L2_PLAN_SEGMENTS]; /* a multiple of 16, > 0 (bases and strides too) */
    int tiles[QLM_L2_PLAN_SEGMENTS];
    int nseg;
} qlm_l2_plan;

/* Appends the tiles that the workgroups of the tile-major M = 1 GEMV
 * (qlm_gemv_i8_mx and its headnorm form with epilogue 0-2; the int4 forms
 * when int4 != 0) over q_tiles / s_tiles read first: 16-row tile t (of each
 * half, for SwiGLU) is read by workgroup t for t < that launch's grid, and
 * tiles 0 .. min(max_tiles, grid) - 1 are appended, weights and group-32
 * scales (per-row scales, 64 bytes a tile, are left out). QLM_ERR_SHAPE when
 * no launch shape fits or the plan has no room for the segments. Host only. */
int qlm_gemv_mx_l2_plan(const void* q_tiles, const float* s_tiles, int group, int int4, int N,
                        int K, int epilogue, int max_tiles, qlm_l2_plan* plan);

/* A4: the same matmul for M > 1 on the matrix cores (batched decode, prefill;
 * math_ops.cpp:845-871). Weights stay exact (int8 in bf16); each activation
 * is split into bf16 hi + lo and the per-group products are scaled in fp32,
 * so results match the fp32 path to ~1e-6 normwise (bit-exact when x holds
 * small integers). norm_w NULL: plain x; else each row of x is first
 * replaced by rms_norm(x, norm_w, eps) (as qlm_gemv_i8_rmsnorm). epilogue
 * 0: y = x.W^T; 1: y += x.W^T; 2: SwiGLU with weights [2F, K] and N = F
 * outputs. Any M >= 1; K a multiple of 32; G = 32 or K. work: device
 * scratch of qlm_matmul_i8_workspace_bytes(M, N, K, epilogue) bytes (row
 * scales and K-split partial sums; no initial contents needed; calls that
 * share it must be ordered on one stream). */
size_t qlm_matmul_i8_workspace_bytes(int M, int N, int K, int epilogue);

int qlm_matmul_i8(const float* x, int ldx, const float* norm_w, float eps, const int8_t* q,
                  const float* scales, int group, float* y, int ldy, int M, int N, int K,
                  int epilogue, void* work, size_t work_bytes, void* stream);
/* qlm_matmul_i8 over the tile-major copy of the weights (qlm_mx_swizzle:
 * halves 2 for SwiGLU; group-32 scales as swizzled, per-row scales in their
 * [rows] layout), so a model needs no row-major copy for its M > 1 rows.
 * Same arithmetic, bit-identical to qlm_matmul_i8 on the same weights,
 * except 2..64 rows with per-row scales (no SwiGLU; N >= 8192, or more than
 * 16 rows and K > 4096), which take qlm_matmul_i8_rows64
 * (within 1e-5 normwise, exact int32 sums); K a multiple of 64; the same
 * workspace. */
int qlm_matmul_i8_tm(const float* x, int ldx, const float* norm_w, float eps,
                     const int8_t* q_tiles, const float* s_tiles, int group, float* y, int ldy,
                     int M, int N, int K, int epilogue, void* work, size_t work_bytes,
                     void* stream);

/* math::matmul's int8 branch (math_ops.cpp:845-871) for 2 <= M <= 64
 * activation rows and one scale per weight row (group = K): tile-major
 * weights (qlm_mx_swizzle) and their scales s_rows [N] as quantised. The
 * rows are written as int8 digit planes, x = 2^E (d0 + d1/2^7 + d2/2^14 +
 * d3/2^21) per row (the RMSNorm folded in when norm_w is given), and
 * multiplied on v_mfma_i32_16x16x64_i8 with exact int32 sums over K,
 * combined and scaled once in fp32: all four digits at 2..8 rows (x to
 * within 2^-27 max|x|, ~1e-7 normwise from the fp32 product), the first
 * three at 9..64 rows (x to within 2^-20 max|x|, ~1.3e-6 normwise on N(0,1)
 * rows). epilogue 0 (store) or 1 (y += result); K a multiple of
 * 64, at most 2^18; QLM_ERR_SHAPE otherwise, for SwiGLU and for M outside
 * 2..64. qlm_matmul_i8_tm takes this form for such calls where measured
 * faster (N >= 8192, or more than 16 rows and K > 4096; its work 256-byte
 * aligned). work: device scratch of
 * qlm_matmul_i8_rows64_workspace_bytes(M, N, K, epilogue) bytes (at most
 * qlm_matmul_i8_workspace_bytes of the same arguments), 256-byte aligned, no
 * initial contents needed. */
size_t qlm_matmul_i8_rows64_workspace_bytes(int M, int N, int K, int epilogue);
int qlm_matmul_i8_rows64(const float* x, int ldx, const float* norm_w, float eps,
                         const int8_t* q_tiles, const float* s_rows, float* y, int ldy, int M,
                         int N, int K, int epilogue, void* work, size_t work_bytes, void* stream);

/* Batched decode (2 <= M <= 16 activation rows) on the int8 matrix cores
 * over the tile-major weights of qlm_mx_swizzle (per-row scales as
 * quantised): a first launch writes each row's (optionally RMSNormed)
 * int8 digit vectors into `work`, the second streams the weights once with
 * one v_mfma_i32_16x16x64_i8 per pair of rows and 64-column block, the
 * whole K inside each workgroup (no partial sums). Same semantics, epilogues
 * and accuracy (~1e-7 normwise) as qlm_matmul_i8. K a multiple of 64, at
 * most 3584 or from 8256 to 10240; QLM_ERR_SHAPE otherwise (and for
 * M > 16), where qlm_matmul_i8 serves. work: device scratch of
 * qlm_matmul_i8_mx_workspace_bytes(M, K), 256-byte aligned, no initial
 * contents needed; calls sharing it must be ordered on one stream. */
size_t qlm_matmul_i8_mx_workspace_bytes(int M, int K);
/* The launch shape qlm_matmul_i8_mx picks (waves per workgroup, blocks per
 * wave and tile, ring slots, workgroups), or QLM_ERR_SHAPE. Host only. */
int qlm_matmul_i8_mx_shape(int M, int N, int K, int epilogue, int* waves, int* blocks, int* ring,
                           int* grid);
int qlm_matmul_i8_mx(const float* x, int ldx, const float* norm_w, float eps,
                     const int8_t* q_tiles, const float* s_tiles, int group, float* y, int ldy,
                     int M, int N, int K, int epilogue, void* work, size_t work_bytes,
                     void* stream);

/* Batched decode (2 <= M <= 16 rows) on the bf16 matrix cores over the same
 * tile-major weights (qlm_mx_swizzle, group 32), weights streamed from
 * registers: each 64-column fragment regrouped by lane swaps into its two
 * scale groups, bf16-exact, against the activation split into bf16 hi + lo
 * (loaded with the weights, times 1 + norm_w for the RMSNorm prologue); K split into slices whose partial sums are then added in order
 * with the epilogue applied (a second launch). Same semantics and epilogues
 * as qlm_matmul_i8 (~1e-6 normwise); K a multiple of 64; QLM_ERR_SHAPE for
 * other groups, K or M > 16. work: qlm_matmul_i8_t_workspace_bytes(M, N,
 * K, epilogue) bytes (slice partial sums of the launch shape it picks), no
 * initial contents needed; calls sharing it must be ordered on one stream.
 * _config takes the launch shape (waves, tiles per workgroup, ring slots, K
 * slices; work then holds slices x M x N (x 2 for SwiGLU) floats); built shapes
 * (4,4,2) (4,2,3) (8,2,2) (8,4,2) (4,8,1) (4,8,2) (8,8,1), others QLM_ERR_ARG;
 * slices of
 * more than 64 blocks QLM_ERR_SHAPE. */
size_t qlm_matmul_i8_t_workspace_bytes(int M, int N, int K, int epilogue);
int qlm_matmul_i8_t(const float* x, int ldx, const float* norm_w, float eps,
                    const int8_t* q_tiles, const float* s_tiles, int group, float* y, int ldy,
                    int M, int N, int K, int epilogue, void* work, size_t work_bytes,
                    void* stream);
int qlm_matmul_i8_t_config(const float* x, int ldx, const float* norm_w, float eps,
                           const int8_t* q_tiles, const float* s_tiles, int group, float* y,
                           int ldy, int M, int N, int K, int epilogue, int waves, int tiles,
                           int ring, int k_slices, void* work, size_t work_bytes, void* stream);
/* Whole-K form of qlm_matmul_i8_t: the waves of a workgroup split K and
 * keep their activation columns split in registers for every tile group;
 * the partial tiles meet in LDS and the epilogue is applied in the same
 * launch (no partial sums, no workspace). Where the activation does not fit
 * a wave's registers, K is cut into k_slices slices, each launched the same
 * way, whose raw sums go to work and are added in slice order by a second
 * launch (RMSNorm, residual and SwiGLU applied there). qlm_matmul_i8_t takes
 * it where it measured faster (the 4B gate/up, DeltaNet in-projection,
 * output projections and lm_head, whole; not the attention q/k/v nor the
 * 9728-column down projection) and reports the workspace of the form it
 * takes. _whole_config takes (waves, tiles per half per tile group, grid,
 * K slices); work: qlm_matmul_i8_t_whole_workspace_bytes(M, N, K,
 * epilogue, k_slices) bytes (0 for one slice; work may then be NULL).
 * Built: waves 8 with 2, 4, 5 or 7 blocks of 64 columns a wave in a slice
 * (blocks per wave = ceil(blocks per slice / waves)) and waves 16 with 2,
 * 1 or 2 tiles per half; QLM_ERR_SHAPE for other K, for the shapes whose
 * registers spill (7 blocks a wave with RMSNorm; SwiGLU with 2 tiles per
 * half at 5 blocks or 16 waves) and for RMSNorm with K > 4096; QLM_ERR_ARG
 * for other waves or tiles, k_slices < 1, or a missing or short workspace.
 * Same semantics, epilogues and tolerance as qlm_matmul_i8_t. */
size_t qlm_matmul_i8_t_whole_workspace_bytes(int M, int N, int K, int epilogue, int k_slices);
int qlm_matmul_i8_t_whole_config(const float* x, int ldx, const float* norm_w, float eps,
                                 const int8_t* q_tiles, const float* s_tiles, int group, float* y,
                                 int ldy, int M, int N, int K, int epilogue, int waves,
                                 int tiles, int grid, int k_slices, void* work,
                                 size_t work_bytes, void* stream);

/* Fused forms used by the decode step (same arithmetic as the unfused
 * reference sequence, one launch instead of two or three):
 *   _rmsnorm: x is first replaced by rms_norm(x, norm_w, eps) (zero-centred
 *             gain, math_ops.cpp:1055-1072) -- RMSNorm::forward + matmul.
 *   _residual: y[m,n] += result  -- matmul + elementwise_add into the
 *             residual stream (modules.hpp:225-240).
 *   _swiglu:  weights hold 2F rows, gate rows [0,F) then up rows [F,2F);
 *             y[m,n] = silu(gate_n) * up_n for n < F -- SwiGLU_MLP::forward
 *             (modules.hpp:139-167). N here is F. */
int qlm_gemv_i8_rmsnorm(const float* x, int ldx, const float* norm_w, float eps,
                        const int8_t* q, const float* scales, int group, float* y, int ldy,
                        int M, int N, int K, void* stream);
int qlm_gemv_i8_residual(const float* x, int ldx, const int8_t* q, const float* scales,
                         int group, float* y, int ldy, int M, int N, int K, void* stream);
int qlm_gemv_i8_swiglu_rmsnorm(const float* x, int ldx, const float* norm_w, float eps,
                               const int8_t* q, const float* scales, int group, float* y,
                               int ldy, int M, int F, int K, void* stream);

/* ---- A5/A6/A7: elementwise ------------------------------------------------ */
/* math::rms_norm (math_ops.cpp:1055-1072): y = x*rsqrt(mean(x^2)+eps)*(1+w). */
int qlm_rms_norm(const float* x, const float* w, float* y, int rows, int n, float eps,
                 void* stream);
/* math::add_rms_norm (math_ops.cpp:1133-1172): res += delta; y = rms_norm(res). */
int qlm_add_rms_norm(float* res, const float* delta, const float* w, float* y, int rows, int n,
                     float eps, void* stream);
/* math::silu_mul (math_ops.cpp:1122-1129): a = a/(1+exp(-a)) * b. */
int qlm_silu_mul(float* a, const float* b, int n, void* stream);

/* ---- A8: partial NeoX RoPE --------------------------------------------------
 * math::apply_rope_neox (math_ops.cpp:1237-1289) on t[num_heads, head_stride]
 * (the first head_dim values of each head row are the head). cos/sin come
 * from a host-built table [n_pos, rot/2] (qlm_rope_table layout); the
 * position is read from pos[0] on the device. */
int qlm_rope_neox(float* t, int num_heads, int head_stride, int rot_dim, const float* cos_tab,
                  const float* sin_tab, const int* pos, void* stream);

/* ---- A10: causal depthwise conv1d step, tap-major ring ---------------------
 * math::causal_conv1d_update_tapmajor (math_ops.cpp:1321-1364). state is
 * [kernel_size-1, conv_dim], weight_t is [kernel_size, conv_dim]. */
int qlm_conv1d_update(const float* in, float* state, int oldest_tap, const float* weight_t,
                      float* out, int conv_dim, int kernel_size, void* stream);

/* ---- A11/A12: Gated DeltaNet recurrent step (isolated) ----------------------
 * The recurrence inlined in Qwen3_5GatedDeltaNet::forward (attention.cpp:
 * 498-571), per sequence b and head h, state S[b,h] is [d, d] (key i, value j):
 *   S <- decay*S; kv = k.S; S += beta*k (v - kv)^T; o = (q.S)/sqrt(d).
 * q,k,v,o are [B, H, d]; decay, beta are [B, H]. d = 128. */
int qlm_gated_delta_step(const float* q, const float* k, const float* v, const float* decay,
                         const float* beta, float* state, float* out, int B, int H, int d,
                         void* stream);

/* ---- A10-A12 fused: the whole DeltaNet mixer core of one decode step -------
 * Qwen3_5GatedDeltaNet::forward (attention.cpp:414-590) from the projection
 * output to the gated head output, for B sequences:
 *   proj[b] = [qkv (3*H*d) | z (H*d) | b (H) | a (H)] (row stride ldp);
 *   conv1d on qkv with the tap-major ring state conv_state[b] [3, 3*H*d]
 *   (oldest tap row = pos[b] % 3), SiLU, per-head L2 norm of q and k,
 *   decay = exp(-exp(A_log)*softplus(a+dt_bias)), beta = sigmoid(b),
 *   recurrence on state[b] [H, d, d], head RMSNorm (gain norm_w, eps 1e-6),
 *   SiLU(z) gate. Output out[b] is [H*d] (row stride ldo). d = 128,
 *   conv kernel 4. pos may be NULL (then the ring index is 0 for all b). */
int qlm_deltanet_decode(const float* proj, int ldp, float* conv_state, const float* conv_w_t,
                        const float* A_log, const float* dt_bias, const float* norm_w,
                        float* state, const int* pos, float* out, int ldo, int B, int H, int d,
                        void* stream);

/* The same mixer with each head's 128 value columns split over 8
 * workgroups (16 columns each), for small batches: H * 8 workgroups per
 * sequence instead of H. The recurrence, conv ring and state updates are
 * qlm_deltanet_decode's; the head RMSNorm, which needs all 128 outputs of a
 * head, is left to the consumer: u[b] [H*d] (row stride ldu) holds
 * o[j] * norm_w[j] * silu(z[j]) and ss [B, H, 8] the sums of o[j]^2 over
 * each 16-column slice, so the mixer output is
 * u[j] / sqrt(sum_s ss[b, h, s] / d + 1e-6) (qlm_gemv_i8_mx_headnorm applies
 * it in its prologue). ticket: B*H*QLM_DN_TICKET_STRIDE unsigned (the
 * ticket of (b, h) at index (b*H + h) * QLM_DN_TICKET_STRIDE), zero before
 * the first call, left at multiples of 8 by every call (the workgroups of a
 * head take one ticket each; the last one overwrites the head's q/k
 * conv-ring row, which all of them read). Calls sharing a ticket array must
 * be ordered on one stream. d = 128. */
#define QLM_DN_TICKET_STRIDE 32
int qlm_deltanet_decode_cols(const float* proj, int ldp, float* conv_state,
                             const float* conv_w_t, const float* A_log, const float* dt_bias,
                             const float* norm_w, float* state, const int* pos, float* u, int ldu,
                             float* ss, unsigned* ticket, int B, int H, int d, void* stream);
/* The same, carrying out an L2 prefetch plan (see qlm_l2_plan; NULL or empty:
 * none) in workgroups of its own beside the mixer's. A non-empty plan needs
 * B = 1. Same results as qlm_deltanet_decode_cols. */
int qlm_deltanet_decode_cols_pf(const float* proj, int ldp, float* conv_state,
                                const float* conv_w_t, const float* A_log, const float* dt_bias,
                                const float* norm_w, float* state, const int* pos, float* u,
                                int ldu, float* ss, unsigned* ticket, int B, int H, int d,
                                const qlm_l2_plan* plan, void* stream);

/* ---- A13: DeltaNet prefill of one sequence -----------------------------------
 * Qwen3_5GatedDeltaNet::forward_chunk (attention.cpp:600-758): the mixer of
 * qlm_deltanet_decode applied to T consecutive projection rows (row t at
 * position p0 + t) in order, as the reference does, carrying the conv ring
 * and the state [H, d, d] of that sequence from row to row; both are left as
 * a decode step at position p0 + T expects them. Bit-identical to T
 * qlm_deltanet_decode calls. out[t] is [H*d] (row stride ldo). */
int qlm_deltanet_prefill(const float* proj, int ldp, int T, float* conv_state,
                         const float* conv_w_t, const float* A_log, const float* dt_bias,
                         const float* norm_w, float* state, int p0, float* out, int ldo, int H,
                         int d, void* stream);

/* The same prefill in the chunked (WY) form: chunks of 64 rows, the
 * intra-chunk products (K K^T, Q K^T, T V, T K) and the chunk-to-chunk
 * state products (W = U - Wk S, Q S, K^T W) on the fp32 matrix cores, the
 * rows of a chunk solved together instead of one after another. Same inputs
 * and outputs as qlm_deltanet_prefill, within 1e-4 of it (reassociated fp32).
 * work: device scratch of qlm_deltanet_chunk_workspace_bytes(T, H, d) bytes,
 * 256-byte aligned, no initial contents needed. */
size_t qlm_deltanet_chunk_workspace_bytes(int T, int H, int d);
int qlm_deltanet_prefill_chunked(const float* proj, int ldp, int T, float* conv_state,
                                 const float* conv_w_t, const float* A_log, const float* dt_bias,
                                 const float* norm_w, float* state, int p0, float* out, int ldo,
                                 int H, int d, void* work, size_t work_bytes, void* stream);

/* ---- A8/A9: GQA decode attention over a contiguous KV cache -----------------
 * Qwen3_5Attention::forward steps 2-6 (attention.cpp:160-227) for B
 * sequences at positions pos[b]:
 *   qkv[b] = [q+gate (n_q * 2*hd if gated else n_q*hd) | k (n_kv*hd) | v (n_kv*hd)]
 *   QK-norm (zero-centred, eps 1e-6), partial NeoX RoPE from the table,
 *   k/v written to the cache at pos[b], softmax(q.K^T/sqrt(hd)) . V over
 *   positions 0..pos[b], sigmoid(gate) output gate when gated.
 * Cache layout [B, max_seq, n_kv, hd] fp32 (position-major, as the reference,
 * attention.cpp:134-135). out[b] is [n_q*hd]. work is a device workspace of
 * qlm_gqa_workspace_bytes(...) bytes (no initial contents needed; also large
 * enough for qlm_attention_decode with the same B, n_q, hd, max_seq). */
size_t qlm_gqa_workspace_bytes(int B, int n_q, int hd, int max_seq);
int qlm_gqa_decode(float* qkv, int ldqkv, const float* q_norm, const float* k_norm,
                   const float* cos_tab, const float* sin_tab, int rot_dim, float* k_cache,
                   float* v_cache, int max_seq, const int* pos, float* out, int ldo, int B,
                   int n_q, int n_kv, int hd, int gated, void* work, void* stream);

/* Prefill of one sequence: the same attention for T consecutive rows of the
 * projection (row t at position p0 + t, causal over 0..p0+t), as the
 * reference's batched forward (attention.cpp:138-232 per row). q rows are
 * normalised and rotated in place; k/v rows go to the cache of that sequence
 * (k_cache, v_cache point at its [max_seq, n_kv, hd] block) before any row
 * attends. out[t] is [n_q*hd] (row stride ldo). work is
 * qlm_gqa_prefill_workspace_bytes(n_q, hd, max_seq) bytes. */
size_t qlm_gqa_prefill_workspace_bytes(int n_q, int hd, int max_seq);
int qlm_gqa_prefill(float* qkv, int ldqkv, const float* q_norm, const float* k_norm,
                    const float* cos_tab, const float* sin_tab, int rot_dim, float* k_cache,
                    float* v_cache, int max_seq, int p0, int T, float* out, int ldo, int n_q,
                    int n_kv, int hd, int gated, void* work, void* stream);

/* Isolated attention core (no norm/RoPE/write): out[b, h] = softmax(q.K^T *
 * scale) . V over the first ctx positions of a [B, max_seq, n_kv, hd] cache,
 * kv_dtype 0 = fp32, 1 = bf16. q, out are [B, n_q, hd] fp32. A bf16 cache
 * runs on the bf16 matrix cores (q and the probabilities split into bf16
 * hi + lo, to 2^-18 of each; products and sums in fp32), an fp32 cache on
 * the vector ALUs. */
int qlm_attention_decode(const float* q, const void* k_cache, const void* v_cache,
                         int kv_dtype, int max_seq, int ctx, float* out, int B, int n_q,
                         int n_kv, int hd, void* work, void* stream);

/* No counterpart in the reference: qlm_attention_decode for callers that
 * cannot allocate device memory (code under hipGraph capture, serving loops
 * that forbid hipMalloc). Same arguments, kernels and results (bit for bit)
 * as qlm_attention_decode, without `work`: the chunk records live in a
 * static device array of QLM_ATTENTION_NOALLOC_MAX_BYTES (32 MiB) that every
 * GPU running the library holds until the process ends. A call needs
 * qlm_attention_decode_noalloc_bytes(B, n_q, hd, ctx) bytes of it (B * n_q
 * * R * (hd + 4) * 4 with R chunk records a head: ceil(ctx / C) for the
 * chunk length C qlm_attention_decode picks for an fp32 cache, 64 to 512
 * positions at hd 128 and 32 to 256 at hd 256, or at most min(256,
 * ceil(ctx / 64)) at hd 128 and min(256, ceil(ctx / 32)) at hd 256 for a
 * bf16 cache; the larger of the two) and returns QLM_ERR_SCRATCH, launching
 * nothing, when the call's records exceed the maximum. The call allocates
 * nothing. qlm_set_device looks the array's address up on that device, so a
 * first call after it (under graph capture included) makes no runtime
 * query; without it, the first call on a device does the lookup (a
 * hipGetSymbolAddress, which should then run outside any capture). Every
 * call on one GPU shares
 * that GPU's array: calls that may overlap on one GPU (different streams,
 * different host threads) race, so order them on one stream. Nothing in the
 * array needs clearing between calls. */
#define QLM_ATTENTION_NOALLOC_MAX_BYTES (32u << 20)
size_t qlm_attention_decode_noalloc_bytes(int B, int n_q, int hd, int ctx);
int qlm_attention_decode_noalloc(const float* q, const void* k_cache, const void* v_cache,
                                 int kv_dtype, int max_seq, int ctx, float* out, int B, int n_q,
                                 int n_kv, int hd, void* stream);

/* ---- A14: greedy sampling ---------------------------------------------------
 * DecoderModel::sample with temperature <= 0 (model.cpp:263-274): index of
 * the first maximum (strict >, lowest index wins ties) of each of the B rows
 * of logits [B, ldl] over n entries. idx is [B] int32. */
int qlm_argmax(const float* logits, int ldl, int n, int B, int* idx, void* work, void* stream);
size_t qlm_argmax_workspace_bytes(int B, int n);

/* ---- A14/A15: device-resident greedy loop ------------------------------------
 * The CLI's decode loop (main.cpp:659-676) with the token stream kept on the
 * device: argmax as qlm_argmax, then for each b with p = pos[b]: if p+1 is
 * past the prompt (p+1 >= prompt_len[b]) the winner is stored as
 * tokens[b, p+1]; then pos[b] = p+1. tokens is [B, ld_tokens] int32. */
int qlm_greedy_advance(const float* logits, int ldl, int n, int B, void* work, int* tokens,
                       int ld_tokens, int* pos, const int* prompt_len, void* stream);

/* The whole tail of a batch-1 decode step in two launches: final RMSNorm +
 * lm_head GEMV (logits [V] stored) with a per-workgroup argmax, then one
 * workgroup that finishes the argmax, does the advance of qlm_greedy_advance
 * and gathers the embedding of the token now at pos[0] into h_next [H]
 * (model.cpp:193-199 and :263-274, main.cpp:659-663, then model.cpp:157-164
 * for the next step). work is qlm_lm_head_greedy_workspace_bytes() bytes
 * (16-byte aligned, no initial contents needed); calls that share a work
 * buffer must be ordered on one stream. */
size_t qlm_lm_head_greedy_workspace_bytes(void);
int qlm_lm_head_greedy(const float* x, const float* norm_w, float eps, const int8_t* q,
                       const float* scales, int group, float* logits, int V, int K, void* work,
                       int* tokens, int ld_tokens, int* pos, const int* prompt_len,
                       const float* embed, int H, float* h_next, void* stream);
/* qlm_lm_head_greedy with the lm_head in the tile-major layout (q_tiles,
 * s_tiles from qlm_mx_swizzle; per-row scales as quantised), on the matrix
 * cores; same workspace and semantics. */
int qlm_lm_head_greedy_mx(const float* x, const float* norm_w, float eps, const int8_t* q_tiles,
                          const float* s_tiles, int group, float* logits, int V, int K,
                          void* work, int* tokens, int ld_tokens, int* pos,
                          const int* prompt_len, const float* embed, int H, float* h_next,
                          void* stream);

/* Embedding gather (model.cpp:157-164, F32 table): out[b] = table[tokens[b,
 * pos[b]]] for a [vocab, H] fp32 table (pos NULL: tokens[b, 0]). */
int qlm_embed_tokens(const float* table, int vocab, int H, const int* tokens, int ld_tokens,
                     const int* pos, float* out, int ldo, int B, void* stream);

/* ---- int4 (Q4_0) weights (reference --precision int4) ----------------------
 * Replaces SafetensorsLoader::get_tensor_keep_int4 (safetensors.cpp:587-656,
 * st_quantize_row_f32_int4 / _bf16_int4 :393-515) and the int4 branch of
 * math::matmul (math_ops.cpp:820-900, int4_gemv_range :768-800). */

/* Load-time quantiser, bit-exact with the reference's IEEE semantics: per
 * 32 columns m = max|x|, s = m > 0 ? m/8 : 1, q = clamp(rne(x * (1/s)),
 * -8, 7); q4 is [rows, K/2] bytes holding the nibble q + 8 (low
 * nibble = even column), scales [rows, K/32]. q8 (optional, may be NULL)
 * receives the signed values as int8 [rows, K]: with the same scales they
 * are an int8 weight for every qlm_*_i8 entry point, whose results then
 * equal the int4 matmul's (the reference's int4 dot is its int8 dot over
 * the unpacked values, math_ops.cpp:604-700). K a multiple of 32; q4, q8
 * 16-byte aligned. */
int qlm_quantize_q4_f32(const float* w, int rows, int K, uint8_t* q4, float* scales, int8_t* q8,
                        void* stream);
int qlm_quantize_q4_bf16(const uint16_t* w, int rows, int K, uint8_t* q4, float* scales,
                         int8_t* q8, void* stream);

/* int4 tile-major copy for the one-row GEMV: the fragments of the int8
 * tile-major layout at 8 bytes a lane (512 B a fragment), nibbles value + 8
 * (padded rows value 0); scales as qlm_mx_swizzle's. K a multiple of 64. */
int qlm_mx4_layout_bytes(int rows, int K, int halves, size_t* q_bytes, size_t* s_bytes);
int qlm_mx4_swizzle(const uint8_t* q4, const float* scales, int rows, int K, int halves,
                    uint8_t* q_out, float* s_out, void* stream);

/* qlm_gemv_i8_mx / _config / qlm_lm_head_greedy_mx over int4 tile-major
 * weights (group 32): each lane widens its 16 nibbles to int8 in registers
 * and the matrix-core arithmetic is the int8 path's, at half the weight
 * bytes. Same arguments, launch shapes and semantics. */
int qlm_gemv_i4_mx_config(const float* x, const float* norm_w, float eps, const uint8_t* q_tiles,
                          const float* s_tiles, float* y, int N, int K, int epilogue, int waves,
                          int ring, int grid, void* stream);
int qlm_gemv_i4_mx(const float* x, const float* norm_w, float eps, const uint8_t* q_tiles,
                   const float* s_tiles, float* y, int N, int K, int epilogue, void* stream);
int qlm_lm_head_greedy_mx4(const float* x, const float* norm_w, float eps,
                           const uint8_t* q_tiles, const float* s_tiles, float* logits, int V,
                           int K, void* work, int* tokens, int ld_tokens, int* pos,
                           const int* prompt_len, const float* embed, int H, float* h_next,
                           void* stream);

/* ---- native (unquantised) weights (reference --precision bf16) -------------
 * The reference keeps each weight in its checkpoint dtype under its default
 * precision (get_tensor_keep_bf16, safetensors.cpp:248-273): bf16 rows for
 * BF16 tensors, fp32 rows for F32 ones, and math::matmul takes fp32 dot
 * products against them (dot_avx2 / bf16_gemv_range, math_ops.cpp:209-400,
 * :820-900). Replaces those branches: y = x . W^T on the fp32 matrix cores
 * (bf16 widened exactly), fp32 accumulation. W [N, K] row-major fp32
 * (w_bf16 = 0) or bf16 bits (w_bf16 = 1); x [M, ldx], y [M, ldy], any M (16
 * rows per launch; bf16 rows with M > 16 go to qlm_matmul_bf16, whose
 * workspace must then fit as well). norm_w / epilogue as qlm_matmul_i8
 * (RMSNorm prologue:
 * the row scale multiplies the finished sums; SwiGLU: W is [2N, K], gate
 * rows then up rows; it needs norm_w); work holds
 * qlm_matmul_w_workspace_bytes(K) bytes when norm_w is given. K a multiple
 * of 16; x, W, norm_w 16-byte aligned. */
/* bf16 weight rows (no scales) with many activation rows, the prefill form:
 * 128 x 64 output tiles on the bf16 matrix cores, the weights staged through
 * LDS as they are, the activation split into bf16 hi + lo (2^-17 of x), the
 * MFMAs chained over K in fp32. Same arguments and epilogues as
 * qlm_matmul_w (which calls it for bf16 weights and M > 16). work: with
 * qlm_matmul_bf16_workspace_bytes(M, K) bytes the activation is split once
 * (RMSNorm applied) into bf16 planes there; with less, each workgroup
 * splits its chunks itself, and then norm_w still needs the first M floats
 * (row scales). K a multiple of 32. */
size_t qlm_matmul_bf16_workspace_bytes(int M, int K);
int qlm_matmul_bf16(const float* x, int ldx, const float* norm_w, float eps, const uint16_t* w,
                    float* y, int ldy, int M, int N, int K, int epilogue, void* work,
                    size_t work_bytes, void* stream);
size_t qlm_matmul_w_workspace_bytes(int K);
int qlm_matmul_w(const float* x, int ldx, const float* norm_w, float eps, const void* w,
                 int w_bf16, float* y, int ldy, int M, int N, int K, int epilogue, void* work,
                 size_t work_bytes, void* stream);
/* One activation row (M = 1) on the vector ALUs, which qlm_matmul_w uses for
 * M = 1: x staged once per workgroup in LDS (times 1 + norm_w, with 1/rms,
 * when norm_w is given; no workspace), each wave streaming 16-byte loads of
 * rows_per_wave rows (both halves for SwiGLU) through a ring of `ring`
 * items, the columns split over k_phases waves. Built shapes (waves,
 * rows_per_wave, k_phases, ring): (4,1,1,4) (8,1,1,4) (4,2,1,3) (8,2,1,3)
 * (4,4,1,2) (8,2,4,3) (8,1,4,4) (16,1,8,4); others return QLM_ERR_ARG.
 * grid <= 0: one workgroup per tile. QLM_ERR_SHAPE when K is too long for
 * the staged x (more than 20 columns per thread or 64 KiB of LDS). */
int qlm_gemv_w_config(const float* x, const float* norm_w, float eps, const void* w, int w_bf16,
                      float* y, int N, int K, int epilogue, int waves, int rows_per_wave,
                      int k_phases, int ring, int grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QLM_HIP_H */
