// Greedy speculative decoding and the session turn loop (see speculative.hpp).
//
// Round invariant (speculative.cpp:6-19): between rounds both models have
// consumed exactly cached_ids, and t_next / d_next hold each model's greedy
// pick for the next position. t_next checks the round's first drafted token;
// verify row i checks drafted token i + 1, and the last row gives the bonus
// token when every drafted token is accepted. Each round therefore closes
// with one single-token forward per model (of the bonus or the correction),
// which both advances the states and yields the next round's picks.

#include "speculative.hpp"

#include <algorithm>
#include <chrono>
#include <stdexcept>
#include <string>

namespace qlm {
namespace {

[[noreturn]] void context_exceeded(int max_seq) {
    throw std::runtime_error("context length exceeded max_seq_len (" + std::to_string(max_seq) +
                             ")");
}

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

}  // namespace

SpeculativeDecoder::SpeculativeDecoder(GreedyModel& target, GreedyModel& draft,
                                       int draft_tokens, int max_seq_len, int eos_id,
                                       int im_end_id)
    : target_(target), draft_(draft), k_(draft_tokens), max_seq_(max_seq_len), eos_(eos_id),
      im_end_(im_end_id) {
    // speculative.cpp:28-45: both checks are hard errors
    if (k_ < 1)
        throw std::runtime_error("--draft-tokens must be >= 1, got " + std::to_string(k_));
    if (draft.vocab_size() != target.vocab_size())
        throw std::runtime_error("speculative: draft model vocab_size (" +
                                 std::to_string(draft.vocab_size()) + ") differs from target's (" +
                                 std::to_string(target.vocab_size()) + ")");
}

void SpeculativeDecoder::replay(const int* toks, int n, int pos) {
    if (n <= 0) return;
    target_.forward_batch_greedy(toks, n, pos, nullptr);
    draft_.forward_batch_greedy(toks, n, pos, nullptr);
}

SpeculativeStats SpeculativeDecoder::generate_turn(std::vector<int>& cached, int pending,
                                                   int max_tokens,
                                                   const std::function<void(int)>& on_token) {
    SpeculativeStats st;
    if (max_tokens <= 0) return st;

    // the prompt's last token starts the decode on both models
    int base = (int)cached.size();
    if (base >= max_seq_) context_exceeded(max_seq_);
    int t_next = target_.forward_greedy(pending, base);
    int d_next = draft_.forward_greedy(pending, base);
    cached.push_back(pending);

    std::vector<int> drafted, picks, commit;
    while (st.emitted < max_tokens) {
        base = (int)cached.size();
        // K drafted positions base..base+K-1 plus the closing forward at
        // base+K must fit (speculative.cpp:104-114)
        const int K = std::min(k_, max_seq_ - base - 1);
        if (K < 1) context_exceeded(max_seq_);

        target_.snapshot_states();
        draft_.snapshot_states();

        // draft K tokens greedily; the draft model consumes every one of them
        drafted.assign(K, 0);
        drafted[0] = d_next;
        for (int i = 0; i < K; ++i) {
            const int nx = draft_.forward_greedy(drafted[i], base + i);
            if (i + 1 < K) drafted[i + 1] = nx;
        }
        st.drafted += K;

        // one batched target pass over the drafted tokens: picks[i] is the
        // target's greedy token at drafted[i]'s position, picks[K] the bonus
        picks.assign(K + 1, 0);
        picks[0] = t_next;
        target_.forward_batch_greedy(drafted.data(), K, base, picks.data() + 1);

        int acc = 0;
        while (acc < K && picks[acc] == drafted[acc]) ++acc;
        ++st.rounds;
        st.draft_accepted += acc;

        const int last = picks[acc];  // bonus (acc == K) or the target's correction
        commit.assign(drafted.begin(), drafted.begin() + acc);
        commit.push_back(last);
        if (acc < K) {
            // both models ran past the agreed prefix and a recurrent state
            // cannot be truncated: back to the round start, replay the prefix
            ++st.rejections;
            target_.restore_states();
            draft_.restore_states();
            replay(drafted.data(), acc, base);
        }
        t_next = target_.forward_greedy(last, base + acc);
        d_next = draft_.forward_greedy(last, base + acc);

        // cut at a terminator or at the token budget; if fewer tokens are
        // kept than were consumed, restore and replay exactly the kept ones
        // (speculative.cpp:180-210)
        size_t keep = commit.size();
        bool stop = false;
        for (size_t i = 0; i < commit.size(); ++i)
            if (terminator(commit[i])) {
                keep = i;
                stop = true;
                break;
            }
        const size_t budget = (size_t)(max_tokens - st.emitted);
        if (keep > budget) {
            keep = budget;
            stop = true;
        }
        if (stop && keep < commit.size()) {
            target_.restore_states();
            draft_.restore_states();
            replay(commit.data(), (int)keep, base);
        }
        for (size_t i = 0; i < keep; ++i) {
            cached.push_back(commit[i]);
            on_token(commit[i]);
            ++st.emitted;
        }
        if (stop) break;
    }
    return st;
}

Session::Session(GreedyModel& target, GreedyModel* draft, int draft_tokens, int eos_id,
                 int im_end_id, bool kv_reuse)
    : target_(target), draft_(draft), eos_(eos_id), im_end_(im_end_id), kv_reuse_(kv_reuse) {
    max_seq_ = target.max_seq_len();
    if (draft) {
        max_seq_ = std::min(max_seq_, draft->max_seq_len());
        spec_.emplace_back(target, *draft, draft_tokens, max_seq_, eos_id, im_end_id);
    }
    reset();  // an empty cached_ids stands for freshly reset models
}

void Session::reset() {
    target_.reset_states();
    if (draft_) draft_->reset_states();
    cached_.clear();
}

TurnResult Session::turn(const std::vector<int>& ids, int max_tokens) {
    if (ids.empty()) throw std::runtime_error("Tokenized turn is empty");
    for (int t : ids)
        if (t < 0 || t >= target_.vocab_size())
            throw std::runtime_error("turn: token id out of range");
    TurnResult r;
    const double t0 = now_s();

    // kv-reuse (main.cpp:536-566): keep the live state when this turn's ids
    // extend the consumed ones (the reference compares the decoded text;
    // token ids are the caller's side of the tokenizer here), else start over
    int reused = 0;
    if (kv_reuse_ && !cached_.empty() && ids.size() > cached_.size() &&
        std::equal(cached_.begin(), cached_.end(), ids.begin()))
        reused = (int)cached_.size();
    else if (!cached_.empty())
        reset();

    // prefill ids[reused .. n-2] in one batched pass per model (main.cpp:587-622)
    const int prefill_end = (int)ids.size() - 2;
    const int count = prefill_end - reused + 1;
    if (count > 0) {
        const int pos = (int)cached_.size();
        if (pos + count > max_seq_) context_exceeded(max_seq_);
        target_.forward_batch_greedy(ids.data() + reused, count, pos, nullptr);
        if (draft_) draft_->forward_batch_greedy(ids.data() + reused, count, pos, nullptr);
        cached_.insert(cached_.end(), ids.begin() + reused, ids.begin() + prefill_end + 1);
    }
    r.reused = reused;
    r.recomputed = std::max(0, count);
    const double t1 = now_s();

    auto emit = [&](int t) { r.tokens.push_back(t); };
    if (!spec_.empty()) {
        r.spec = spec_[0].generate_turn(cached_, ids.back(), max_tokens, emit);
    } else {
        // plain greedy loop (main.cpp:659-676): forward, pick, stop at a
        // terminator; the last emitted token is not forwarded
        int next = ids.back();
        for (int i = 0; i < max_tokens; ++i) {
            const int pos = (int)cached_.size();
            if (pos >= max_seq_) context_exceeded(max_seq_);
            const int pick = target_.forward_greedy(next, pos);
            cached_.push_back(next);
            next = pick;
            if (next == eos_ || next == im_end_) break;
            emit(next);
        }
    }
    r.prefill_s = t1 - t0;
    r.decode_s = now_s() - t1;
    return r;
}

}  // namespace qlm
