// Test infrastructure only: an extern "C" face over the reference QuickLM CPU
// engine, compiled from the reference's own sources where they lie (see
// oracle/Makefile). Nothing in the product links or loads this; tests, golden
// generation and bench.py's cpu_baseline leg use it as oracle and baseline.
//
// The reference keeps its int8 quantiser in file-static functions
// (src/io/safetensors.cpp:296-391), so this TU includes that .cpp directly to
// reach them; every other reference .cpp is compiled as its own object.

#include "safetensors.cpp"  // st_quantize_row_f32 / st_quantize_row_bf16 (static)

#include "attention.hpp"
#include "math_ops.hpp"
#include "model.hpp"
#include "modules.hpp"

#include <chrono>
#include <cstdint>
#include <cstring>
#include <iostream>
#include <memory>
#include <sstream>
#include <vector>

namespace {

// The reference logs progress on std::cout (model.cpp:39-130, :177-209);
// keep the caller's stdout clean while reference code runs.
struct QuietCout {
    std::streambuf* saved;
    std::ostringstream sink;
    QuietCout() : saved(std::cout.rdbuf(sink.rdbuf())) {}
    ~QuietCout() { std::cout.rdbuf(saved); }
};

Tensor int8_weight(const int8_t* q, const float* s, int N, int K) {
    Tensor t;
    t.shape = {N, K};
    t.compute_strides();
    int nb = (K + Tensor::INT8_BLOCK_SIZE - 1) / Tensor::INT8_BLOCK_SIZE;
    t.int8_owner = std::make_shared<std::vector<int8_t>>(q, q + (size_t)N * K);
    t.int8_scales = std::make_shared<std::vector<float>>(s, s + (size_t)N * nb);
    t.int8_data = t.int8_owner->data();
    return t;
}

Tensor int4_weight(const uint8_t* q, const float* s, int N, int K) {
    Tensor t;
    t.shape = {N, K};
    t.compute_strides();
    int nb = (K + Tensor::INT4_BLOCK_SIZE - 1) / Tensor::INT4_BLOCK_SIZE;
    int pb = (K + 1) / 2;
    t.int4_owner = std::make_shared<std::vector<uint8_t>>(q, q + (size_t)N * pb);
    t.int4_scales = std::make_shared<std::vector<float>>(s, s + (size_t)N * nb);
    t.int4_data = t.int4_owner->data();
    return t;
}

Tensor owned_f32(const float* p, std::vector<int> shape) {
    Tensor t(shape);
    std::memcpy(t.data, p, (size_t)t.size() * sizeof(float));
    return t;
}

}  // namespace

extern "C" {

void qref_init_threads(int n) { math::init_thread_pool((size_t)n); }

// A2: one row of the load-time Q8_0 quantiser (safetensors.cpp:348-391).
void qref_quantize_rows_f32(const float* w, int rows, int K, int8_t* q, float* s) {
    int nb = (K + Tensor::INT8_BLOCK_SIZE - 1) / Tensor::INT8_BLOCK_SIZE;
    for (int r = 0; r < rows; ++r)
        st_quantize_row_f32(w + (size_t)r * K, K, q + (size_t)r * K, s + (size_t)r * nb);
}

// A2, bf16 input (safetensors.cpp:296-345).
void qref_quantize_rows_bf16(const uint16_t* w, int rows, int K, int8_t* q, float* s) {
    int nb = (K + Tensor::INT8_BLOCK_SIZE - 1) / Tensor::INT8_BLOCK_SIZE;
    for (int r = 0; r < rows; ++r)
        st_quantize_row_bf16(w + (size_t)r * K, K, q + (size_t)r * K, s + (size_t)r * nb);
}

// int4 (Q4_0) load-time quantiser (safetensors.cpp:393-515): packed rows of
// (K+1)/2 bytes, one scale per 32 columns.
void qref_quantize_rows_f32_int4(const float* w, int rows, int K, uint8_t* q, float* s) {
    int nb = (K + Tensor::INT4_BLOCK_SIZE - 1) / Tensor::INT4_BLOCK_SIZE, pb = (K + 1) / 2;
    for (int r = 0; r < rows; ++r)
        st_quantize_row_f32_int4(w + (size_t)r * K, K, q + (size_t)r * pb, s + (size_t)r * nb);
}

void qref_quantize_rows_bf16_int4(const uint16_t* w, int rows, int K, uint8_t* q, float* s) {
    int nb = (K + Tensor::INT4_BLOCK_SIZE - 1) / Tensor::INT4_BLOCK_SIZE, pb = (K + 1) / 2;
    for (int r = 0; r < rows; ++r)
        st_quantize_row_bf16_int4(w + (size_t)r * K, K, q + (size_t)r * pb, s + (size_t)r * nb);
}

// math::matmul int4 branch (math_ops.cpp:820-900 via int4_gemv_range :768-800).
void qref_matmul_i4(const float* A, int M, int K, const uint8_t* q, const float* s, int N,
                    float* C, int ldc) {
    Tensor a({M, K}, const_cast<float*>(A));
    Tensor b = int4_weight(q, s, N, K);
    Tensor c({M, N}, C);
    c.strides = {ldc, 1};
    math::matmul(a, b, c, true);
}

// math::matmul over native weights (math_ops.cpp:820-900): fp32 rows
// (dot_avx2) or bf16 rows (bf16_gemv_range). C is [M, ldc].
void qref_matmul_w(const float* A, int M, int K, const void* W, int bf16, int N, float* C,
                   int ldc) {
    Tensor a({M, K}, const_cast<float*>(A));
    Tensor b;
    b.shape = {N, K};
    b.compute_strides();
    if (bf16)
        b.bf16_data = static_cast<const uint16_t*>(W);
    else
        b.data = const_cast<float*>(static_cast<const float*>(W));
    Tensor c({M, N}, C);
    c.strides = {ldc, 1};
    math::matmul(a, b, c, true);
}

// A3/A4: math::matmul int8 branch (math_ops.cpp:820-900). C is [M, ldc].
void qref_matmul_i8(const float* A, int M, int K, const int8_t* q, const float* s, int N,
                    float* C, int ldc) {
    Tensor a({M, K}, const_cast<float*>(A));
    Tensor b = int8_weight(q, s, N, K);
    Tensor c({M, N}, C);
    c.strides = {ldc, 1};
    math::matmul(a, b, c, true);
}

// A5: math::rms_norm (math_ops.cpp:1055-1072).
void qref_rms_norm(const float* x, const float* w, float* y, int rows, int n, float eps) {
    Tensor in({rows, n}, const_cast<float*>(x));
    Tensor wt({n}, const_cast<float*>(w));
    Tensor out({rows, n}, y);
    math::rms_norm(in, wt, out, eps);
}

// A6: math::add_rms_norm (math_ops.cpp:1133-1172).
void qref_add_rms_norm(float* res, const float* delta, const float* w, float* y, int rows,
                       int n, float eps) {
    Tensor r({rows, n}, res);
    Tensor d({rows, n}, const_cast<float*>(delta));
    Tensor wt({n}, const_cast<float*>(w));
    Tensor out({rows, n}, y);
    math::add_rms_norm(r, d, wt, out, eps);
}

float qref_sumsq(const float* x, int n) { return math::sumsq(x, n); }

// A7: math::silu_mul (math_ops.cpp:1122-1129).
void qref_silu_mul(float* a, const float* b, int n) {
    Tensor ta({n}, a);
    Tensor tb({n}, const_cast<float*>(b));
    math::silu_mul(ta, tb);
}

// A8: math::apply_rope_neox (math_ops.cpp:1237-1289) on [num_heads, head_dim].
void qref_rope_neox(float* t, int num_heads, int head_dim, int pos, float theta, int rot) {
    Tensor tt({num_heads, head_dim}, t);
    math::apply_rope_neox(tt, pos, theta, head_dim, rot);
}

// A10: math::causal_conv1d_update_tapmajor (math_ops.cpp:1321-1364).
void qref_conv1d_tapmajor(const float* in, float* state, int oldest, const float* w_t,
                          float* out, int conv_dim, int kernel_size) {
    math::causal_conv1d_update_tapmajor(in, state, oldest, w_t, out, conv_dim, kernel_size);
}

// A10-A12: one Qwen3_5GatedDeltaNet module (attention.cpp:384-590), int8 weights.
void* qref_deltanet_create(const int8_t* qkv_q, const float* qkv_s, const int8_t* z_q,
                           const float* z_s, const int8_t* b_q, const float* b_s,
                           const int8_t* a_q, const float* a_s, const float* conv_w,
                           const float* norm_w, const float* A_log, const float* dt_bias,
                           const int8_t* out_q, const float* out_s, int hidden, int n_heads,
                           int head_dim, int conv_kernel) {
    int hd = n_heads * head_dim;
    auto* m = new Qwen3_5GatedDeltaNet();
    m->init(int8_weight(qkv_q, qkv_s, 3 * hd, hidden), int8_weight(z_q, z_s, hd, hidden),
            int8_weight(b_q, b_s, n_heads, hidden), int8_weight(a_q, a_s, n_heads, hidden),
            owned_f32(conv_w, {3 * hd, 1, conv_kernel}), owned_f32(norm_w, {head_dim}),
            owned_f32(A_log, {n_heads}), owned_f32(dt_bias, {n_heads}),
            int8_weight(out_q, out_s, hidden, hd), n_heads, head_dim, 0);
    m->reset_states();
    return m;
}

// rows > 1 goes through forward_chunk (attention.cpp:600-758).
void qref_deltanet_forward(void* h, const float* in, int rows, int hidden, float* out, int pos) {
    auto* m = static_cast<Qwen3_5GatedDeltaNet*>(h);
    Context ctx;
    ctx.pos = pos;
    ctx.seq_len = rows;
    Tensor ti = rows > 1 ? Tensor({rows, hidden}, const_cast<float*>(in))
                         : Tensor({hidden}, const_cast<float*>(in));
    Tensor to = rows > 1 ? Tensor({rows, hidden}, out) : Tensor({hidden}, out);
    m->forward(ti, to, ctx);
}

void qref_deltanet_destroy(void* h) { delete static_cast<Qwen3_5GatedDeltaNet*>(h); }

// A8-A9: one Qwen3_5Attention module (attention.cpp:107-369), int8 weights,
// QK-norm on, no biases, output gate on iff q rows == 2*n_heads*head_dim.
void* qref_gqa_create(const int8_t* q_q, const float* q_s, int q_rows, const int8_t* k_q,
                      const float* k_s, const int8_t* v_q, const float* v_s, const int8_t* o_q,
                      const float* o_s, const float* q_norm, const float* k_norm, int hidden,
                      int n_heads, int n_kv, int head_dim, int rot_dim, float theta,
                      int max_seq) {
    auto* m = new Qwen3_5Attention();
    Tensor none;
    m->init(int8_weight(q_q, q_s, q_rows, hidden), int8_weight(k_q, k_s, n_kv * head_dim, hidden),
            int8_weight(v_q, v_s, n_kv * head_dim, hidden),
            int8_weight(o_q, o_s, hidden, n_heads * head_dim), none, none, none,
            owned_f32(q_norm, {head_dim}), owned_f32(k_norm, {head_dim}), n_heads, n_kv,
            head_dim, rot_dim, theta, max_seq);
    m->reset_states();
    return m;
}

void qref_gqa_forward(void* h, const float* in, int rows, int hidden, float* out, int pos) {
    auto* m = static_cast<Qwen3_5Attention*>(h);
    Context ctx;
    ctx.pos = pos;
    ctx.seq_len = rows;
    Tensor ti = rows > 1 ? Tensor({rows, hidden}, const_cast<float*>(in))
                         : Tensor({hidden}, const_cast<float*>(in));
    Tensor to = rows > 1 ? Tensor({rows, hidden}, out) : Tensor({hidden}, out);
    m->forward(ti, to, ctx);
}

void qref_gqa_destroy(void* h) { delete static_cast<Qwen3_5Attention*>(h); }

// A14: DecoderModel (model.cpp:34-274), loaded from a model directory.
void* qref_model_load(const char* dir, int max_seq_len, const char* precision) {
    QuietCout quiet;
    auto* m = new DecoderModel();
    if (!m->load(dir, max_seq_len, precision)) {
        delete m;
        return nullptr;
    }
    return m;
}

int qref_model_vocab(void* h) { return static_cast<DecoderModel*>(h)->get_config().vocab_size; }

void qref_model_reset(void* h) { static_cast<DecoderModel*>(h)->reset_states(); }

void qref_model_forward(void* h, int token, int pos, float* logits) {
    QuietCout quiet;
    auto* m = static_cast<DecoderModel*>(h);
    Context ctx;
    ctx.pos = pos;
    Tensor lg({m->get_config().vocab_size}, logits);
    m->forward(token, lg, ctx);
}

void qref_model_forward_batch(void* h, const int* tokens, int n, int pos, float* logits) {
    QuietCout quiet;
    auto* m = static_cast<DecoderModel*>(h);
    Context ctx;
    ctx.pos = pos;
    std::vector<int> ids(tokens, tokens + n);
    Tensor lg({n, m->get_config().vocab_size}, logits);
    m->forward_batch(ids, lg, ctx);
}

int qref_model_sample_greedy(void* h, const float* logits) {
    auto* m = static_cast<DecoderModel*>(h);
    Tensor lg({m->get_config().vocab_size}, const_cast<float*>(logits));
    return m->sample(lg, 0.0f, 0);
}

// A15: the CLI's single-turn greedy loop (main.cpp:574-690) without tokenizer
// or EOS stop: batched prefill of prompt[0..n-2], then n_new steps of
// forward(next) + greedy sample. Returns decode wall seconds (prefill
// excluded) in *decode_s and prefill seconds in *prefill_s. If logits_out is
// non-null, the logits of every decode step are written there [n_new, V].
int qref_model_generate(void* h, const int* prompt, int n, int n_new, int* out,
                        double* prefill_s, double* decode_s, float* logits_out) {
    QuietCout quiet;
    auto* m = static_cast<DecoderModel*>(h);
    int V = m->get_config().vocab_size;
    m->reset_states();
    Context ctx;
    auto t0 = std::chrono::steady_clock::now();
    int prefill_count = n - 1;
    if (prefill_count > 0) {
        std::vector<int> ids(prompt, prompt + prefill_count);
        Tensor pl({prefill_count, V});
        ctx.pos = 0;
        m->forward_batch(ids, pl, ctx);
    }
    auto t1 = std::chrono::steady_clock::now();
    Tensor logits({V});
    int next = prompt[n - 1];
    int pos = prefill_count;
    for (int i = 0; i < n_new; ++i) {
        ctx.pos = pos++;
        m->forward(next, logits, ctx);
        if (logits_out) std::memcpy(logits_out + (size_t)i * V, logits.data, (size_t)V * 4);
        next = m->sample(logits, 0.0f, 0);
        out[i] = next;
    }
    auto t2 = std::chrono::steady_clock::now();
    if (prefill_s) *prefill_s = std::chrono::duration<double>(t1 - t0).count();
    if (decode_s) *decode_s = std::chrono::duration<double>(t2 - t1).count();
    return n_new;
}

void qref_model_free(void* h) { delete static_cast<DecoderModel*>(h); }

}  // extern "C"
