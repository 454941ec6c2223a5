/*
 * qlm_engine.h - C ABI of the C++17 host engine (quicklm_amd/libqlm_engine.so).
 *
 * The engine is the MI355X counterpart of the reference's DecoderModel
 * (src/model/model.hpp:16-91): it loads a Qwen3.5-hybrid checkpoint from a
 * directory of safetensors + config.json, keeps every weight and state on
 * the GPU, and runs the decode loop as a replayed hipGraph. It reaches the
 * GPU only through libqlm_hip.so (qlm_hip.h).
 *
 * All functions return 0 on success or a nonzero code; qlm_engine_last_error()
 * then holds the message (the reference throws std::runtime_error with the
 * same texts, e.g. "context length exceeded max_seq_len (...)").
 */
#ifndef QLM_ENGINE_H
#define QLM_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* qlm_engine_last_error(void);

/* DecoderModel::load(dir, max_seq_len, precision) (model.cpp:34-131) plus a
 * batch capacity. precision "int8" = Q8_0 group-32 scales (reference
 * parity), "int8_row" = one scale per output row. */
int qlm_engine_load(const char* dir, int max_seq_len, int max_batch, const char* precision,
                    void** handle);
int qlm_engine_free(void* handle);

/* vocab, hidden, layers, group size (0 = per row), max_seq, max_batch. */
int qlm_engine_info(void* handle, int* vocab, int* hidden, int* layers, int* group,
                    int* max_seq, int* max_batch, size_t* weight_bytes);

/* DecoderModel::reset_states (model.cpp:133-137). */
int qlm_engine_reset(void* handle);

/* DecoderModel::forward(token, logits, ctx) with ctx.pos = pos
 * (model.cpp:151-211), sequence 0; logits copied to a host array [vocab]. */
int qlm_engine_forward(void* handle, int token, int pos, float* logits);

/* Greedy generation with the CLI convention (main.cpp:574-690): prompts
 * [B, n] host int32; out [B, n_new]; timings in seconds (prefill = the n-1
 * prompt forwards, decode = the n_new steps). use_graph 0 launches eagerly.
 * prefill_mode 1: positions 0..n-2 of each sequence go through the batched
 * prefill (the reference's forward_batch, model.cpp:213-258: every layer
 * over all prompt rows) with the DeltaNet recurrence in its chunked form on
 * the matrix cores; 2: the same with the recurrence row by row (bit-identical
 * to mode 0's DeltaNet arithmetic); 0: each position is forwarded by its own
 * decode step. */
int qlm_engine_generate(void* handle, const int* prompts, int B, int n, int n_new, int* out,
                        double* prefill_s, double* decode_s, int use_graph, int prefill_mode);

/* Stepwise generation for benchmarks: start() resets and installs B prompts
 * of length n (prefill_mode 1 or 2 also prefills positions 0..n-2, wall time
 * in *prefill_s, so the first step forwards position n-1); steps() runs k
 * decode steps (with prefill_mode 0 the prompt forwards come first) as graph
 * replays and reports their GPU time in ms (HIP events on the engine's
 * stream); tokens() copies count tokens of sequence b from position first. */
int qlm_engine_start(void* handle, const int* prompts, int B, int n, int prefill_mode,
                     double* prefill_s);
int qlm_engine_steps(void* handle, int k, int use_graph, double* gpu_ms);
int qlm_engine_tokens(void* handle, int b, int first, int count, int* out);

/* Logits of sequence b after the last step, host array [vocab]. */
int qlm_engine_last_logits(void* handle, int b, float* logits);

/* Kernel launches in one captured decode step of batch B (after a step ran). */
int qlm_engine_kernels_per_step(void* handle);

/* ---- speculative decoding and sessions (sequence 0) --------------------------
 * DecoderModel::snapshot_states / restore_states (model.cpp:139-149,
 * attention.cpp:766-790): one device slot holding every DeltaNet recurrence
 * and conv ring; restore before any snapshot is an error. */
int qlm_engine_snapshot(void* handle);
int qlm_engine_restore(void* handle);

/* DecoderModel::forward(token) at pos followed by the greedy pick
 * (model.cpp:151-211, :263-274): one replayed decode step; *next = argmax. */
int qlm_engine_forward_greedy(void* handle, int token, int pos, int* next);

/* DecoderModel::forward_batch (model.cpp:213-258): tokens[0..n) at positions
 * pos..pos+n-1 through every layer at once (n == 1: one decode step). argmax
 * [n] (host, may be NULL): the greedy pick of each row; logits [n, vocab]
 * (host, may be NULL): the rows' logits. With both NULL the lm_head is not
 * run (a replay or a prompt prefill). */
int qlm_engine_forward_batch(void* handle, const int* tokens, int n, int pos, int* argmax,
                             float* logits);

/* The CLI's turn loop (main.cpp:455-690) over token ids, with
 * SpeculativeDecoder (speculative.cpp:1-222) when draft is non-NULL: target
 * and draft are engine handles (kept alive by the caller; the draft is
 * usually the same checkpoint at "int4", main.cpp:366-394). draft_tokens is
 * K (>= 1); eos_id / im_end_id end a turn (never emitted); kv_reuse keeps the
 * live state for a turn whose ids extend the ids already consumed. */
int qlm_session_create(void* target, void* draft, int draft_tokens, int eos_id, int im_end_id,
                       int kv_reuse, void** session);
int qlm_session_free(void* session);
int qlm_session_reset(void* session);
/* One turn: ids [n] = the turn's whole prompt; up to max_tokens tokens to
 * out [cap], count in *n_out; info [7] (may be NULL) = reused prompt
 * positions, recomputed positions, speculative rounds, drafted, accepted,
 * emitted, rejections; prefill and decode wall times in seconds. */
int qlm_session_turn(void* session, const int* ids, int n, int max_tokens, int* out, int cap,
                     int* n_out, int* info, double* prefill_s, double* decode_s);
/* The ids whose state both models hold (*n of them; out [cap] may be NULL). */
int qlm_session_cached(void* session, int* out, int cap, int* n);

/* ---- synthetic checkpoints (no reference counterpart) ----
 * Deterministic counter-based generators used to write random-init weights
 * of a given architecture: element i of a tensor with seed s depends only on
 * (s, i), so a tensor can be filled in parallel and identically on any host.
 * normal: mean + std * N(0,1) (Box-Muller over splitmix64 uniforms, double
 * precision, rounded to the output type); uniform: lo + (hi-lo)*U[0,1). */
int qlm_synth_normal_f32(float* out, size_t n, uint64_t seed, float mean, float std_dev);
int qlm_synth_normal_bf16(uint16_t* out, size_t n, uint64_t seed, float mean, float std_dev);
int qlm_synth_uniform_f32(float* out, size_t n, uint64_t seed, float lo, float hi);
uint64_t qlm_synth_tensor_seed(uint64_t base, const char* name);

#ifdef __cplusplus
}
#endif

#endif /* QLM_ENGINE_H */
