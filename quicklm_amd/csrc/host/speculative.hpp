// Greedy self-speculative decoding and the multi-turn session caller, over an
// abstract greedy model so that the same round logic drives the GPU engine
// and, in the host-logic tests, a deterministic stand-in.
//
// Reference: SpeculativeDecoder (src/model/speculative.{hpp,cpp}:1-222) and
// the turn loop of main.cpp:455-690 (kv-reuse, batched prefill, the
// speculative or plain greedy decode of one turn).
#pragma once

#include <functional>
#include <vector>

namespace qlm {

// What the round loop and the session need of a model: the reference
// DecoderModel's forward / forward_batch / reset_states / snapshot_states /
// restore_states (model.hpp:28-66), used greedily, with the argmax taken
// where the logits live (on the device for the GPU engine).
class GreedyModel {
   public:
    virtual ~GreedyModel() = default;
    virtual int vocab_size() const = 0;
    virtual int max_seq_len() const = 0;
    virtual void reset_states() = 0;
    // One snapshot slot of every recurrent state (DeltaNet recurrence and
    // conv ring); attention K/V is position-indexed and needs none
    // (attention.cpp:766-790, model.cpp:139-149).
    virtual void snapshot_states() = 0;
    virtual void restore_states() = 0;
    // forward(token) at position pos; returns the argmax of its logits.
    virtual int forward_greedy(int token, int pos) = 0;
    // forward_batch over tokens[0..n) at positions pos..pos+n-1; when argmax
    // is non-null, argmax[r] is the greedy pick of row r's logits.
    virtual void forward_batch_greedy(const int* tokens, int n, int pos, int* argmax) = 0;
};

// Per-turn instrumentation (speculative.hpp:7-18).
struct SpeculativeStats {
    int rounds = 0;          // draft/verify rounds
    int drafted = 0;         // tokens proposed by the draft model
    int draft_accepted = 0;  // of those, the ones the target agreed with
    int emitted = 0;         // tokens handed to the caller (terminators excluded)
    int rejections = 0;      // rounds that restored and replayed
};

// Greedy speculative decoding (speculative.hpp:20-81): the draft proposes K
// tokens one at a time, the target checks all K in one batched pass, the
// agreed prefix plus the target's own next token is committed. The committed
// stream is the target's plain greedy stream.
class SpeculativeDecoder {
   public:
    SpeculativeDecoder(GreedyModel& target, GreedyModel& draft, int draft_tokens,
                       int max_seq_len, int eos_id, int im_end_id);

    // Entry: both models have consumed exactly cached_ids, and `pending` (the
    // prompt's final token) has not been forwarded. Exit: cached_ids is again
    // exactly what both models' states hold. At most max_tokens tokens go to
    // on_token, in order; a terminator ends the turn and is not emitted.
    SpeculativeStats generate_turn(std::vector<int>& cached_ids, int pending, int max_tokens,
                                   const std::function<void(int)>& on_token);

   private:
    bool terminator(int t) const { return t == eos_ || t == im_end_; }
    void replay(const int* toks, int n, int pos);

    GreedyModel& target_;
    GreedyModel& draft_;
    int k_, max_seq_, eos_, im_end_;
};

struct TurnResult {
    std::vector<int> tokens;  // emitted tokens of the turn
    int reused = 0;           // prompt positions whose state was kept from the last turn
    int recomputed = 0;       // prompt positions prefilled this turn
    SpeculativeStats spec;    // zero without a draft model
    double prefill_s = 0.0, decode_s = 0.0;
};

// The CLI's turn loop over token ids (main.cpp:455-690 without the tokenizer
// and chat template, which stay with the caller): with kv-reuse, a turn whose
// ids extend the ids already consumed only prefills the new suffix;
// otherwise both models are reset and the whole prompt is prefilled. Then
// the decode runs speculatively when a draft model is given, else as plain
// greedy steps.
class Session {
   public:
    // Resets both models: the session starts from an empty cache.
    Session(GreedyModel& target, GreedyModel* draft, int draft_tokens, int eos_id,
            int im_end_id, bool kv_reuse);

    TurnResult turn(const std::vector<int>& ids, int max_tokens);
    void reset();
    const std::vector<int>& cached_ids() const { return cached_; }

   private:
    GreedyModel& target_;
    GreedyModel* draft_;
    int eos_, im_end_;
    bool kv_reuse_;
    int max_seq_;
    std::vector<int> cached_;  // tokens whose state both models hold
    std::vector<SpeculativeDecoder> spec_;
};

}  // namespace qlm
