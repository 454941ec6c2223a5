// extern "C" face of the host engine (include/qlm_engine.h). Exceptions never
// cross the ABI: they become a nonzero return plus qlm_engine_last_error().

#include <algorithm>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "model.hpp"
#include "speculative.hpp"
#include "qlm_engine.h"

namespace {
thread_local std::string g_err;

template <typename F>
int guarded(F&& f) {
    try {
        f();
        g_err.clear();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
    } catch (...) {
        g_err = "unknown error";
    }
    return 1;
}

qlm::DecoderModel* M(void* h) {
    if (!h) throw std::runtime_error("null engine handle");
    return static_cast<qlm::DecoderModel*>(h);
}

qlm::Session* S(void* h) {
    if (!h) throw std::runtime_error("null session handle");
    return static_cast<qlm::Session*>(h);
}
}  // namespace

extern "C" {

const char* qlm_engine_last_error(void) { return g_err.c_str(); }

int qlm_engine_load(const char* dir, int max_seq_len, int max_batch, const char* precision,
                    void** handle) {
    return guarded([&] {
        if (!dir || !precision || !handle) throw std::runtime_error("null argument");
        *handle = nullptr;
        auto* m = new qlm::DecoderModel();
        try {
            m->load(dir, max_seq_len, precision, max_batch);
        } catch (...) {
            delete m;
            throw;
        }
        *handle = m;
    });
}

int qlm_engine_free(void* handle) {
    return guarded([&] { delete static_cast<qlm::DecoderModel*>(handle); });
}

int qlm_engine_info(void* handle, int* vocab, int* hidden, int* layers, int* group, int* max_seq,
                    int* max_batch, size_t* weight_bytes) {
    return guarded([&] {
        auto* m = M(handle);
        const auto& c = m->config();
        if (vocab) *vocab = c.vocab_size;
        if (hidden) *hidden = c.hidden_size;
        if (layers) *layers = c.num_hidden_layers;
        if (group) *group = m->group();
        if (max_seq) *max_seq = m->max_seq();
        if (max_batch) *max_batch = m->max_batch();
        if (weight_bytes) *weight_bytes = m->weight_bytes();
    });
}

int qlm_engine_reset(void* handle) { return guarded([&] { M(handle)->reset_states(); }); }

int qlm_engine_forward(void* handle, int token, int pos, float* logits) {
    return guarded([&] {
        if (!logits) throw std::runtime_error("null logits");
        M(handle)->forward(token, pos, logits);
    });
}

int qlm_engine_generate(void* handle, const int* prompts, int B, int n, int n_new, int* out,
                        double* prefill_s, double* decode_s, int use_graph, int prefill_mode) {
    return guarded([&] {
        if (!prompts || !out) throw std::runtime_error("null argument");
        qlm::GenStats st;
        if (prefill_mode < 0 || prefill_mode > 2) throw std::runtime_error("bad prefill_mode");
        M(handle)->generate(prompts, B, n, n_new, out, &st, use_graph != 0, prefill_mode);
        if (prefill_s) *prefill_s = st.prefill_s;
        if (decode_s) *decode_s = st.decode_s;
    });
}

int qlm_engine_start(void* handle, const int* prompts, int B, int n, int prefill_mode,
                     double* prefill_s) {
    return guarded([&] {
        if (!prompts) throw std::runtime_error("null prompts");
        if (prefill_mode < 0 || prefill_mode > 2) throw std::runtime_error("bad prefill_mode");
        const double s = M(handle)->start(prompts, B, n, prefill_mode);
        if (prefill_s) *prefill_s = s;
    });
}

int qlm_engine_steps(void* handle, int k, int use_graph, double* gpu_ms) {
    return guarded([&] {
        const double ms = M(handle)->steps(k, use_graph != 0);
        if (gpu_ms) *gpu_ms = ms;
    });
}

int qlm_engine_tokens(void* handle, int b, int first, int count, int* out) {
    return guarded([&] {
        if (!out) throw std::runtime_error("null output");
        M(handle)->tokens(b, first, count, out);
    });
}

int qlm_engine_snapshot(void* handle) { return guarded([&] { M(handle)->snapshot_states(); }); }

int qlm_engine_restore(void* handle) { return guarded([&] { M(handle)->restore_states(); }); }

int qlm_engine_forward_greedy(void* handle, int token, int pos, int* next) {
    return guarded([&] {
        const int t = M(handle)->forward_greedy(token, pos);
        if (next) *next = t;
    });
}

int qlm_engine_forward_batch(void* handle, const int* tokens, int n, int pos, int* argmax,
                             float* logits) {
    return guarded([&] { M(handle)->forward_batch(tokens, n, pos, argmax, logits); });
}

int qlm_session_create(void* target, void* draft, int draft_tokens, int eos_id, int im_end_id,
                       int kv_reuse, void** session) {
    return guarded([&] {
        if (!session) throw std::runtime_error("null argument");
        *session = nullptr;
        *session = new qlm::Session(*M(target), draft ? M(draft) : nullptr, draft_tokens, eos_id,
                                    im_end_id, kv_reuse != 0);
    });
}

int qlm_session_free(void* session) {
    return guarded([&] { delete static_cast<qlm::Session*>(session); });
}

int qlm_session_reset(void* session) {
    return guarded([&] { S(session)->reset(); });
}

int qlm_session_turn(void* session, const int* ids, int n, int max_tokens, int* out, int cap,
                     int* n_out, int* info, double* prefill_s, double* decode_s) {
    return guarded([&] {
        if (!ids || n < 0 || !out || !n_out) throw std::runtime_error("null argument");
        const qlm::TurnResult r = S(session)->turn(std::vector<int>(ids, ids + n), max_tokens);
        if ((int)r.tokens.size() > cap) throw std::runtime_error("session: output too small");
        std::copy(r.tokens.begin(), r.tokens.end(), out);
        *n_out = (int)r.tokens.size();
        if (info) {
            const int v[7] = {r.reused,          r.recomputed,     r.spec.rounds,
                              r.spec.drafted,    r.spec.draft_accepted, r.spec.emitted,
                              r.spec.rejections};
            std::copy(v, v + 7, info);
        }
        if (prefill_s) *prefill_s = r.prefill_s;
        if (decode_s) *decode_s = r.decode_s;
    });
}

int qlm_session_cached(void* session, int* out, int cap, int* n) {
    return guarded([&] {
        const auto& c = S(session)->cached_ids();
        if (n) *n = (int)c.size();
        if (out) {
            if ((int)c.size() > cap) throw std::runtime_error("session: output too small");
            std::copy(c.begin(), c.end(), out);
        }
    });
}

int qlm_engine_last_logits(void* handle, int b, float* logits) {
    return guarded([&] { M(handle)->last_logits(b, logits); });
}

int qlm_engine_kernels_per_step(void* handle) {
    try {
        return M(handle)->kernels_per_step();
    } catch (...) {
        return -1;
    }
}

}  // extern "C"
