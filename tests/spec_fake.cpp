// Host-logic test double for the speculative round loop and the session:
// a deterministic "model" whose state is the list of tokens it consumed and
// whose greedy pick is a hash of that list. The draft variant disagrees with
// the target wherever a second hash says so. Every forward must come at
// exactly the next position (pos == tokens consumed), so a protocol slip
// (a lost restore, a replay at the wrong position, a double forward) throws.
// Built by tests/test_speculative.py with g++ together with
// quicklm_amd/csrc/host/speculative.cpp; no GPU involved.

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "speculative.hpp"

namespace {

uint64_t mix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

class FakeModel : public qlm::GreedyModel {
   public:
    FakeModel(int vocab, int max_seq, int disagree_mod)
        : vocab_(vocab), max_seq_(max_seq), disagree_(disagree_mod) {}
    int vocab_size() const override { return vocab_; }
    int max_seq_len() const override { return max_seq_; }
    void reset_states() override { hist_.clear(); }
    void snapshot_states() override {
        snap_ = hist_;
        have_ = true;
        ++snapshots;
    }
    void restore_states() override {
        if (!have_) throw std::runtime_error("restore before snapshot");
        hist_ = snap_;
        ++restores;
    }
    int forward_greedy(int token, int pos) override {
        consume(token, pos);
        ++singles;
        return pick();
    }
    void forward_batch_greedy(const int* t, int n, int pos, int* argmax) override {
        ++batches;
        for (int r = 0; r < n; ++r) {
            consume(t[r], pos + r);
            if (argmax) argmax[r] = pick();
        }
    }
    const std::vector<int>& history() const { return hist_; }
    int singles = 0, batches = 0, snapshots = 0, restores = 0;

   private:
    void consume(int token, int pos) {
        if (pos != (int)hist_.size())
            throw std::runtime_error("forward at position " + std::to_string(pos) + " with " +
                                     std::to_string(hist_.size()) + " tokens consumed");
        if (pos >= max_seq_) throw std::runtime_error("fake: past max_seq");
        if (token < 0 || token >= vocab_) throw std::runtime_error("fake: bad token");
        hist_.push_back(token);
    }
    // the target's pick depends on the last three tokens and the length; the
    // draft's differs from it where a second hash of the same falls on 0
    int pick() const {
        uint64_t h = hist_.size();
        for (size_t i = hist_.size() >= 3 ? hist_.size() - 3 : 0; i < hist_.size(); ++i)
            h = mix(h * 31 + (uint64_t)hist_[i]);
        const int t = (int)(mix(h) % (uint64_t)vocab_);
        if (disagree_ > 0 && mix(h ^ 0xD1B54A32D192ED03ull) % (uint64_t)disagree_ == 0)
            return (t + 1) % vocab_;
        return t;
    }
    int vocab_, max_seq_, disagree_;
    std::vector<int> hist_, snap_;
    bool have_ = false;
};

thread_local std::string g_err;

}  // namespace

extern "C" const char* fake_last_error() { return g_err.c_str(); }

// Runs `turns` session turns; turn t's ids are ids[off[t] .. off[t+1]).
// draft_mod < 0: no draft model (plain greedy). Outputs of all turns are
// concatenated into out (count per turn in n_out[t]); info[t*7 ..] as
// qlm_session_turn; the final consumed ids of target and draft and the
// session's cached ids go to hist (3 rows of max_seq, lengths in hlen[3]);
// calls[8] = target singles, batches, snapshots, restores, then the draft's.
extern "C" int fake_session(int vocab, int max_seq, int draft_tokens, int eos, int im_end,
                            int draft_mod, int kv_reuse, int turns, const int* ids,
                            const int* off, int max_tokens, int* out, int* n_out, int* info,
                            int* hist, int* hlen, int* calls) {
    try {
        FakeModel target(vocab, max_seq, 0);
        FakeModel draft(vocab, max_seq, draft_mod > 0 ? draft_mod : 0);
        qlm::Session s(target, draft_mod >= 0 ? &draft : nullptr, draft_tokens, eos, im_end,
                       kv_reuse != 0);
        int w = 0;
        for (int t = 0; t < turns; ++t) {
            std::vector<int> v(ids + off[t], ids + off[t + 1]);
            const qlm::TurnResult r = s.turn(v, max_tokens);
            for (int x : r.tokens) out[w++] = x;
            n_out[t] = (int)r.tokens.size();
            const int iv[7] = {r.reused,       r.recomputed,         r.spec.rounds,
                               r.spec.drafted, r.spec.draft_accepted, r.spec.emitted,
                               r.spec.rejections};
            std::memcpy(info + 7 * t, iv, sizeof(iv));
        }
        const std::vector<int>* hs[3] = {&target.history(), &draft.history(), &s.cached_ids()};
        for (int i = 0; i < 3; ++i) {
            hlen[i] = (int)hs[i]->size();
            std::memcpy(hist + (size_t)i * max_seq, hs[i]->data(), hs[i]->size() * sizeof(int));
        }
        const int c[8] = {target.singles, target.batches, target.snapshots, target.restores,
                          draft.singles,  draft.batches,  draft.snapshots,  draft.restores};
        std::memcpy(calls, c, sizeof(c));
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}
