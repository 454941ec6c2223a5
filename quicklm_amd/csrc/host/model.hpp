// Device-resident decoder for the Qwen3.5 hybrid (Gated DeltaNet + GQA)
// family: the MI355X counterpart of the reference's DecoderModel
// (src/model/model.hpp:16-91, model.cpp:34-274) and its module tree
// (DecoderLayer / Qwen3_5GatedDeltaNet / Qwen3_5Attention / SwiGLU_MLP,
// modules.hpp:100-282, attention.cpp).
//
// Differences in shape, not in arithmetic:
//   - weights live in HBM as int8 + fp32 group scales (quantised on the
//     device at load, bit-identical to the reference quantiser); the
//     projections that share an input are stacked into one matrix
//     (DeltaNet qkv|z|b|a, attention q|k|v, MLP gate|up);
//   - every sequence of a batch has its own position, token stream, KV cache
//     and DeltaNet state (the reference holds one sequence);
//   - one decode step is a fixed launch sequence captured once into a
//     hipGraph per batch size and replayed; positions and tokens stay on the
//     device, the argmax runs on the device.
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "config.hpp"
#include "device.hpp"
#include "safetensors.hpp"
#include "speculative.hpp"
#include "tensor.hpp"

namespace qlm {

struct LinearI8 {
    DeviceBuffer q, s;
    int N = 0, K = 0, group = 32;
    // tile-major copy for the one-row GEMV (halves = 2: [gate; up] rows);
    // sz stays empty with per-row scales, which keep their layout
    DeviceBuffer qz, sz;
    int halves = 1;
    // int4 models: packed rows [N, K/2] as quantised (q then holds their
    // unpacked values) and the int4 tile-major copy (scales: sz)
    DeviceBuffer q4, qz4;
    // native-precision models: the rows as stored (fp32 or bf16), no int8
    DeviceBuffer w;
    int wdtype = 0;  // 0 int8 forms, 1 fp32, 2 bf16
    Tensor view() const {
        if (wdtype) {
            Tensor t;
            t.shape = {N, K};
            t.compute_strides();
            t.native_data = w.get();
            t.native_bf16 = wdtype == 2;
            return t;
        }
        Tensor t = Tensor::int8(q.get<int8_t>(), s.get<float>(), N, K, group);
        if (qz.bytes()) {
            t.int8_tiles = qz.get<int8_t>();
            t.int8_tile_scales = sz.bytes() ? sz.get<float>() : s.get<float>();
        }
        if (qz4.bytes()) t.int4_tiles = qz4.get<uint8_t>();
        return t;
    }
    int blocks_per_row() const { return group >= K ? 1 : K / group; }
};

struct LayerWeights {
    bool linear = true;
    DeviceBuffer in_ln, post_ln;   // zero-centred RMSNorm gains [H]
    // Gated DeltaNet
    LinearI8 dn_in;                // [3HD + HD + nh + nh, H]: qkv | z | b | a
    LinearI8 dn_out;               // [H, HD]
    DeviceBuffer conv_wt;          // [4, 3HD] (tap-major, reference attention.cpp:397-408)
    DeviceBuffer A_log, dt_bias;   // [nh]
    DeviceBuffer dn_norm;          // [d] plain gain
    // GQA
    LinearI8 at_qkv;               // [q_rows + 2 n_kv hd, H]
    LinearI8 at_o;                 // [H, n_q hd]
    DeviceBuffer q_norm, k_norm;   // [hd] zero-centred (may be empty)
    bool gated = true;
    // MLP
    LinearI8 gate_up;              // [2F, H]
    LinearI8 down;                 // [H, F]
};

struct GenStats {
    double prefill_s = 0.0;
    double decode_s = 0.0;
    int steps = 0;
};

class DecoderModel : public GreedyModel {
   public:
    DecoderModel() = default;
    ~DecoderModel() override;

    // precision: "int8" (reference Q8_0, group 32) or "int8_row" (one scale
    // per output row). max_batch sequences of up to max_seq_len positions.
    void load(const std::string& dir, int max_seq_len, const std::string& precision,
              int max_batch);

    void reset_states() override;

    // GreedyModel on sequence 0, for speculative decoding and sessions.
    // snapshot_states / restore_states (model.cpp:139-149,
    // attention.cpp:766-790): device copies of every DeltaNet recurrence and
    // conv ring (one slot, allocated on first use).
    void snapshot_states() override;
    void restore_states() override;
    int vocab_size() const override { return cfg_.vocab_size; }
    int max_seq_len() const override { return max_seq_; }
    // forward(token) at pos (one decode step, the replayed graph); returns
    // the greedy pick, which the step also stores as token pos + 1.
    int forward_greedy(int token, int pos) override;
    // forward_batch (model.cpp:213-258): tokens[0..n) at positions
    // pos..pos+n-1 through every layer at once; with argmax / logits (host
    // arrays [n] / [n, vocab]) the final norm and lm_head run over every row.
    // n == 1 is a decode step, as in the reference.
    void forward_batch(const int* tokens, int n, int pos, int* argmax, float* logits);
    void forward_batch_greedy(const int* tokens, int n, int pos, int* argmax) override {
        forward_batch(tokens, n, pos, argmax, nullptr);
    }

    // Reference-shaped single-sequence step (model.cpp:151-211) on sequence 0:
    // forwards `token` at position `pos` and copies the logits to the host.
    void forward(int token, int pos, float* logits_host);

    // Greedy generation, main.cpp:574-690 convention: for each of B
    // sequences, positions 0..n-2 of the prompt are forwarded as prefill,
    // then n_new steps each forward the newest token and append the argmax.
    // prompts [B, n], out [B, n_new]. use_graph = false launches eagerly.
    // Prefill of prompt positions 0..n-2: kPrefillSteps forwards each by its
    // own decode step; the batched modes run every layer over all prompt rows
    // at once (the reference's forward_batch), with the DeltaNet recurrence
    // in the chunked matrix-core form or row by row (bit-identical to steps).
    enum PrefillMode { kPrefillSteps = 0, kPrefillChunked = 1, kPrefillRows = 2 };
    // prefill_mode (PrefillMode) selects how positions 0..n-2 are forwarded.
    void generate(const int* prompts, int B, int n, int n_new, int* out, GenStats* st,
                  bool use_graph = true, int prefill_mode = kPrefillChunked);

    // Stepwise form of generate() for benchmarking: start() resets the state
    // and installs B prompts of length n (with batched_prefill it also runs
    // the prefill of positions 0..n-2 and returns its wall time, so the next
    // step forwards position n-1); steps(k) replays k decode steps of batch B
    // (without batched_prefill the first n-1 are prompt forwards) and returns
    // the GPU time in milliseconds measured with events on the engine stream;
    // tokens() reads back count tokens of sequence b from position first.
    double start(const int* prompts, int B, int n, int prefill_mode = kPrefillSteps);
    double steps(int k, bool use_graph = true);
    void tokens(int b, int first, int count, int* out) const;

    // Logits of sequence b from the most recent step (host copy).
    void last_logits(int b, float* host) const;

    const ModelConfig& config() const { return cfg_; }
    size_t weight_bytes() const { return weight_bytes_; }
    int max_batch() const { return max_batch_; }
    int max_seq() const { return max_seq_; }
    int group() const { return group_; }
    int kernels_per_step() const { return kernels_per_step_; }

   private:
    void enqueue_step(int B);
    void prefill(int b, int n, bool chunked_deltanet);
    // rows first..first+count-1 of sequence b's tokens through every layer;
    // with lm_rows, each pass's rows also get the final norm, lm_head and a
    // greedy pick (stored at lm_idx[row - first], device) and, with
    // logits_host, their logits copied out
    void run_rows(int b, int first, int count, bool chunked_deltanet, int* lm_idx = nullptr,
                  float* logits_host = nullptr);
    void ensure_prefill_buffers(int rows);
    size_t matmul_workspace(int M) const;
    void embed_current(int B);
    // the decode step of batch B captured n times in a row as one graph
    // (cached per (B, n))
    void* graph_for(int B, int n = 1);
    void quantize_into(LinearI8& lin, int row_off, const std::string& name);
    void upload_f32(DeviceBuffer& dst, const std::string& name, int64_t expect);
    void alloc_linear(LinearI8& lin, int N, int K);
    void tile_linear(LinearI8& lin, int halves);

    ModelConfig cfg_;
    std::unique_ptr<WeightStore> ws_;
    int max_seq_ = 0, max_batch_ = 0, group_ = 32;
    bool int4_ = false;  // --precision int4: Q4_0 weights (lm_head included)
    bool native_ = false;  // --precision bf16: weights kept in the checkpoint dtype
    // whether the batch-1 DeltaNet mixer brings the out-projection's int8
    // tiles into L2 (env QLM_L2_PREFETCH=0 turns it off)
    bool l2_plan_ = true;
    int HD_ = 0, PD_ = 0, QR_ = 0, PQ_ = 0, CORE_ = 0;
    size_t weight_bytes_ = 0;
    int kernels_per_step_ = 0;
    void* stream_ = nullptr;

    std::vector<LayerWeights> layers_;
    DeviceBuffer final_norm_, embed_;
    LinearI8 lm_head_;
    DeviceBuffer rope_cos_, rope_sin_;

    // per-sequence state
    std::vector<DeviceBuffer> conv_state_, dn_state_;   // per DeltaNet layer
    std::vector<DeviceBuffer> k_cache_, v_cache_;       // per attention layer
    DeviceBuffer tokens_, pos_, prompt_len_;
    int ld_tokens_ = 0;
    // activations
    DeviceBuffer h_, proj_, core_, act_, logits_, argmax_work_, attn_work_, tail_work_;
    DeviceBuffer mm_work_;  // workspace of the matrix-core matmuls (M > 1)
    // batch-1 column-split DeltaNet mixer: per-head partial sums of squares
    // [nh, 8] (consumed by the out-projection) and tickets [nh]
    DeviceBuffer dn_ss_, dn_ticket_;
    // prefill activations for up to pf_rows_ prompt rows per chunk
    DeviceBuffer hx_pf_, proj_pf_, core_pf_, act_pf_, gqa_pf_work_, dn_pf_work_;
    int pf_rows_ = 0;
    DeviceBuffer staging_;

    // speculative decoding: the state snapshot slot, per-row lm_head logits
    // and greedy picks of a batched forward
    std::vector<DeviceBuffer> conv_snap_, dn_snap_;
    bool have_snapshot_ = false;
    DeviceBuffer lm_pf_, lm_pf_idx_, lm_pf_work_;

    std::map<std::pair<int, int>, void*> graphs_;
    int run_B_ = 0, run_n_ = 0, run_steps_ = 0;
};

}  // namespace qlm
