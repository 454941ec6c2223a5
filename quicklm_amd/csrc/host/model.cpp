#include "model.hpp"

#include <algorithm>
#include <chrono>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <stdexcept>

#include "math_ops.hpp"
#include "safetensors.hpp"

namespace qlm {

namespace {

std::string lp(int i) { return "model.layers." + std::to_string(i) + "."; }

std::vector<float> to_f32(const TensorView& t) {
    std::vector<float> out((size_t)t.numel());
    if (t.dtype == "F32") {
        std::memcpy(out.data(), t.data, out.size() * sizeof(float));
    } else if (t.dtype == "BF16") {
        const uint16_t* src = reinterpret_cast<const uint16_t*>(t.data);
        for (size_t i = 0; i < out.size(); ++i) {
            uint32_t bits = (uint32_t)src[i] << 16;
            std::memcpy(&out[i], &bits, 4);
        }
    } else {
        throw std::runtime_error("Unsupported tensor datatype: " + t.dtype +
                                 " (only F32 and BF16 supported)");
    }
    return out;
}

constexpr int kPrefillChunk = 2048;  // prompt rows per pass through the layers
constexpr int kLmRows = 64;          // rows per lm_head pass of a batched forward
constexpr int kRowsMax = 64;         // batched forwards up to this many rows run the
                                     // DeltaNet recurrence row by row
// Decode steps per replayed graph: consecutive graph launches leave a gap of
// a few us between the last kernel of one and the first of the next (4B at
// batch 1: 1.373 ms a step with one step a graph, 1.370 with 4 or 16)
constexpr int kStepsPerGraph = 8;

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

DecoderModel::~DecoderModel() {
    for (auto& kv : graphs_) qlm_graph_destroy(kv.second);
    if (stream_) qlm_stream_destroy(stream_);
}

void DecoderModel::alloc_linear(LinearI8& lin, int N, int K) {
    lin.N = N;
    lin.K = K;
    lin.group = (group_ == 0) ? K : group_;
    if (native_) return;  // sized by the first tensor's dtype (quantize_into)
    lin.q.alloc((size_t)N * K);
    lin.s.alloc((size_t)N * lin.blocks_per_row() * sizeof(float));
    // bytes a one-row step streams: int8 values, or the int4 copy
    const size_t scale_bytes = (size_t)N * lin.blocks_per_row() * sizeof(float);
    if (int4_) {
        lin.q4.alloc((size_t)N * K / 2);
        weight_bytes_ += (size_t)N * K / 2 + scale_bytes;
    } else {
        weight_bytes_ += (size_t)N * K + scale_bytes;
    }
}

// Device-side equivalent of get_weight -> get_tensor_keep_int8
// (weights.cpp:54-70, safetensors.cpp:517-585): the raw F32/BF16 rows are
// uploaded and quantised on the GPU straight into rows [row_off, row_off+N).
void DecoderModel::quantize_into(LinearI8& lin, int row_off, const std::string& name) {
    TensorView t = ws_->get(name);
    if (t.shape.size() != 2 || t.shape[1] != lin.K || row_off + t.shape[0] > lin.N)
        throw std::runtime_error("weight '" + name + "' has an unexpected shape");
    if (t.dtype != "F32" && t.dtype != "BF16")
        throw std::runtime_error("Unsupported tensor datatype for '" + name + "': " + t.dtype +
                                 " (only F32 and BF16 supported for int8 quantization)");
    if (native_) {  // get_tensor_keep_bf16 / get_tensor (safetensors.cpp:248-273): dtype kept
        const int dt = t.dtype == "BF16" ? 2 : 1;
        const size_t elt = dt == 2 ? 2 : 4;
        if (!lin.wdtype) {
            lin.wdtype = dt;
            lin.w.alloc((size_t)lin.N * lin.K * elt);
            weight_bytes_ += (size_t)lin.N * lin.K * elt;
        } else if (lin.wdtype != dt) {
            throw std::runtime_error("weight '" + name + "' mixes F32 and BF16 with the rows it "
                                     "is stacked with");
        }
        check(qlm_memcpy_h2d(static_cast<char*>(lin.w.get()) + (size_t)row_off * lin.K * elt,
                             t.data, t.nbytes, stream_),
              "upload");
        check(qlm_stream_sync(stream_), "sync");  // the mapped source may be unmapped later
        return;
    }
    if (staging_.bytes() < t.nbytes) {
        check(qlm_stream_sync(stream_), "sync");
        staging_.alloc(t.nbytes);
    }
    check(qlm_memcpy_h2d(staging_.get(), t.data, t.nbytes, stream_), "upload");
    const int rows = (int)t.shape[0];
    int8_t* q = lin.q.get<int8_t>() + (size_t)row_off * lin.K;
    float* s = lin.s.get<float>() + (size_t)row_off * lin.blocks_per_row();
    if (int4_) {  // get_tensor_keep_int4 (safetensors.cpp:587-656)
        uint8_t* q4 = lin.q4.get<uint8_t>() + (size_t)row_off * lin.K / 2;
        if (t.dtype == "F32")
            check(qlm_quantize_q4_f32(staging_.get<float>(), rows, lin.K, q4, s, q, stream_),
                  "quantize");
        else
            check(qlm_quantize_q4_bf16(staging_.get<uint16_t>(), rows, lin.K, q4, s, q, stream_),
                  "quantize");
        return;
    }
    if (t.dtype == "F32")
        check(qlm_quantize_q8_f32(staging_.get<float>(), rows, lin.K, lin.group, q, s, stream_),
              "quantize");
    else
        check(qlm_quantize_q8_bf16(staging_.get<uint16_t>(), rows, lin.K, lin.group, q, s, stream_),
              "quantize");
}

// The tile-major copy the one-row GEMV streams (qlm_mx_swizzle); skipped
// where K is not a multiple of 64 (the row-major GEMV serves those).
void DecoderModel::tile_linear(LinearI8& lin, int halves) {
    size_t qb = 0, sb = 0;
    if (native_) return;
    if (lin.K % 64 != 0 || lin.N % halves != 0) return;
    const int rows = lin.N / halves;
    check(qlm_mx_layout_bytes(rows, lin.K, lin.group, halves, &qb, &sb), "tile layout");
    lin.halves = halves;
    lin.qz.alloc(qb);
    if (sb) lin.sz.alloc(sb);
    check(qlm_mx_swizzle(lin.q.get<int8_t>(), lin.s.get<float>(), lin.group, rows, lin.K, halves,
                         lin.qz.get<int8_t>(), sb ? lin.sz.get<float>() : nullptr, stream_),
          "tile swizzle");
    if (int4_) {  // the int4 copy; its scales are the ones just written to sz
        check(qlm_mx4_layout_bytes(rows, lin.K, halves, &qb, &sb), "int4 tile layout");
        lin.qz4.alloc(qb);
        check(qlm_mx4_swizzle(lin.q4.get<uint8_t>(), lin.s.get<float>(), rows, lin.K, halves,
                              lin.qz4.get<uint8_t>(), lin.sz.get<float>(), stream_),
              "int4 tile swizzle");
    }
    // Every device matmul reads the tile-major copy, so the row-major one
    // (and the packed int4 rows) go; per-row scales are the tile scales.
    check(qlm_stream_sync(stream_), "sync");
    lin.q.release();
    lin.q4.release();
    if (lin.sz.bytes()) lin.s.release();
}

void DecoderModel::upload_f32(DeviceBuffer& dst, const std::string& name, int64_t expect) {
    TensorView t = ws_->get(name);
    if (expect >= 0 && t.numel() != expect)
        throw std::runtime_error("tensor '" + name + "' has " + std::to_string(t.numel()) +
                                 " elements, expected " + std::to_string(expect));
    std::vector<float> v = to_f32(t);
    dst.alloc(v.size() * sizeof(float));
    check(qlm_memcpy_h2d(dst.get(), v.data(), v.size() * sizeof(float), stream_), "upload");
    check(qlm_stream_sync(stream_), "sync");  // v is freed on return
}

void DecoderModel::load(const std::string& dir, int max_seq_len, const std::string& precision,
                        int max_batch) {
    if (max_seq_len <= 0 || max_batch <= 0) throw std::runtime_error("load: bad sizes");
    int4_ = precision == "int4";
    native_ = precision == "bf16";  // the reference's default: weights as stored
    if (precision == "int8" || int4_ || native_) group_ = 32;
    else if (precision == "int8_row") group_ = 0;  // resolved per matrix to K
    else
        throw std::runtime_error("load: precision must be int8, int8_row, int4 or bf16, got " +
                                 precision);
    cfg_ = parse_model_config(dir);
    ws_ = std::make_unique<WeightStore>(dir);
    max_seq_ = max_seq_len;
    max_batch_ = max_batch;
    if (const char* e = std::getenv("QLM_L2_PREFETCH")) l2_plan_ = std::atoi(e) != 0;
    check(qlm_stream_create(&stream_), "stream");
    math::set_stream(stream_);

    const int H = cfg_.hidden_size, F = cfg_.intermediate_size, L = cfg_.num_hidden_layers;
    const int nh = cfg_.linear_num_heads, d = cfg_.linear_head_dim;
    const int nq = cfg_.num_attention_heads, nkv = cfg_.num_key_value_heads, hd = cfg_.head_dim;
    HD_ = nh * d;
    PD_ = 4 * HD_ + 2 * nh;
    QR_ = 0;
    for (int i = 0; i < L; ++i)
        if (!cfg_.is_linear(i)) {
            QR_ = (int)ws_->get(lp(i) + "self_attn.q_proj.weight").shape[0];
            break;
        }
    PQ_ = QR_ + 2 * nkv * hd;
    CORE_ = std::max(HD_, nq * hd);

    layers_.resize(L);
    for (int i = 0; i < L; ++i) {
        LayerWeights& w = layers_[i];
        const std::string p = lp(i);
        w.linear = cfg_.is_linear(i);
        upload_f32(w.in_ln, p + "input_layernorm.weight", H);
        upload_f32(w.post_ln, p + "post_attention_layernorm.weight", H);
        if (w.linear) {
            if (d != 128) throw std::runtime_error("DeltaNet head_dim must be 128");
            alloc_linear(w.dn_in, PD_, H);
            quantize_into(w.dn_in, 0, p + "linear_attn.in_proj_qkv.weight");
            quantize_into(w.dn_in, 3 * HD_, p + "linear_attn.in_proj_z.weight");
            quantize_into(w.dn_in, 4 * HD_, p + "linear_attn.in_proj_b.weight");
            quantize_into(w.dn_in, 4 * HD_ + nh, p + "linear_attn.in_proj_a.weight");
            tile_linear(w.dn_in, 1);
            alloc_linear(w.dn_out, H, HD_);
            quantize_into(w.dn_out, 0, p + "linear_attn.out_proj.weight");
            tile_linear(w.dn_out, 1);
            // conv1d.weight [3HD, 1, ks] -> tap-major [ks, 3HD]
            TensorView cw = ws_->get(p + "linear_attn.conv1d.weight");
            const int C = 3 * HD_;
            const int ks = (int)cw.shape.back();
            if (ks != 4 || cw.numel() != (int64_t)C * ks)
                throw std::runtime_error("conv1d weight must be [3*H*d, 1, 4]");
            std::vector<float> cv = to_f32(cw), ct((size_t)C * ks);
            for (int c = 0; c < C; ++c)
                for (int k = 0; k < ks; ++k) ct[(size_t)k * C + c] = cv[(size_t)c * ks + k];
            w.conv_wt.alloc(ct.size() * sizeof(float));
            check(qlm_memcpy_h2d(w.conv_wt.get(), ct.data(), ct.size() * 4, stream_), "upload");
            check(qlm_stream_sync(stream_), "sync");
            upload_f32(w.A_log, p + "linear_attn.A_log", nh);
            upload_f32(w.dt_bias, p + "linear_attn.dt_bias", nh);
            upload_f32(w.dn_norm, p + "linear_attn.norm.weight", d);
        } else {
            if (ws_->has(p + "self_attn.q_proj.bias"))
                throw std::runtime_error("attention projection biases are not supported");
            const int qr = (int)ws_->get(p + "self_attn.q_proj.weight").shape[0];
            if (qr != QR_) throw std::runtime_error("q_proj rows differ between layers");
            w.gated = (qr == 2 * nq * hd);
            if (!w.gated && qr != nq * hd) throw std::runtime_error("q_proj has unexpected rows");
            alloc_linear(w.at_qkv, PQ_, H);
            quantize_into(w.at_qkv, 0, p + "self_attn.q_proj.weight");
            quantize_into(w.at_qkv, qr, p + "self_attn.k_proj.weight");
            quantize_into(w.at_qkv, qr + nkv * hd, p + "self_attn.v_proj.weight");
            tile_linear(w.at_qkv, 1);
            alloc_linear(w.at_o, H, nq * hd);
            quantize_into(w.at_o, 0, p + "self_attn.o_proj.weight");
            tile_linear(w.at_o, 1);
            if (ws_->has(p + "self_attn.q_norm.weight")) {
                upload_f32(w.q_norm, p + "self_attn.q_norm.weight", hd);
                upload_f32(w.k_norm, p + "self_attn.k_norm.weight", hd);
            }
        }
        alloc_linear(w.gate_up, 2 * F, H);
        quantize_into(w.gate_up, 0, p + "mlp.gate_proj.weight");
        quantize_into(w.gate_up, F, p + "mlp.up_proj.weight");
        tile_linear(w.gate_up, 2);
        alloc_linear(w.down, H, F);
        quantize_into(w.down, 0, p + "mlp.down_proj.weight");
        tile_linear(w.down, 1);
    }
    upload_f32(final_norm_, "model.norm.weight", H);
    // Embedding gathered as fp32 (model.cpp:157-164); tied lm_head is the
    // int8-quantised embedding (model.cpp:116-120).
    TensorView et = ws_->get("model.embed_tokens.weight");
    if (et.shape.size() != 2 || et.shape[1] != H) throw std::runtime_error("embed_tokens shape");
    const int V = (int)et.shape[0];
    upload_f32(embed_, "model.embed_tokens.weight", (int64_t)V * H);
    if (ws_->has("lm_head.weight")) {
        const int Vh = (int)ws_->get("lm_head.weight").shape[0];
        alloc_linear(lm_head_, Vh, H);
        quantize_into(lm_head_, 0, "lm_head.weight");
    } else {
        alloc_linear(lm_head_, V, H);
        if (native_)  // tied: the embedding table itself, in its stored dtype
            quantize_into(lm_head_, 0, "model.embed_tokens.weight");
        else if (int4_)
            check(qlm_quantize_q4_f32(embed_.get<float>(), V, H, lm_head_.q4.get<uint8_t>(),
                                      lm_head_.s.get<float>(), lm_head_.q.get<int8_t>(), stream_),
                  "quantize lm_head");
        else
            check(qlm_quantize_q8_f32(embed_.get<float>(), V, H, lm_head_.group,
                                      lm_head_.q.get<int8_t>(), lm_head_.s.get<float>(), stream_),
                  "quantize lm_head");
    }
    tile_linear(lm_head_, 1);
    cfg_.vocab_size = lm_head_.N;  // model.cpp:123
    check(qlm_stream_sync(stream_), "sync");
    staging_.release();

    // RoPE table for every position the cache can hold.
    const int rot = cfg_.rotary_dim();
    if (QR_ > 0) {
        std::vector<float> ct((size_t)max_seq_ * (rot / 2)), st(ct.size());
        math::rope_table(cfg_.rope_theta, rot, max_seq_, ct.data(), st.data());
        rope_cos_.alloc(ct.size() * 4);
        rope_sin_.alloc(st.size() * 4);
        check(qlm_memcpy_h2d(rope_cos_.get(), ct.data(), ct.size() * 4, stream_), "upload");
        check(qlm_memcpy_h2d(rope_sin_.get(), st.data(), st.size() * 4, stream_), "upload");
        check(qlm_stream_sync(stream_), "sync");
    }

    // Per-sequence state and activations for max_batch sequences.
    const size_t B = (size_t)max_batch_;
    for (int i = 0; i < L; ++i) {
        if (cfg_.is_linear(i)) {
            conv_state_.emplace_back(B * 3 * 3 * HD_ * sizeof(float));
            dn_state_.emplace_back(B * nh * d * d * sizeof(float));
        } else {
            k_cache_.emplace_back(B * max_seq_ * nkv * hd * sizeof(float));
            v_cache_.emplace_back(B * max_seq_ * nkv * hd * sizeof(float));
        }
    }
    ld_tokens_ = max_seq_ + 1;
    tokens_.alloc(B * ld_tokens_ * sizeof(int));
    pos_.alloc(B * sizeof(int));
    prompt_len_.alloc(B * sizeof(int));
    const int Pmax = std::max(PD_, PQ_);
    h_.alloc(B * H * sizeof(float));
    proj_.alloc(B * Pmax * sizeof(float));
    core_.alloc(B * CORE_ * sizeof(float));
    act_.alloc(B * F * sizeof(float));
    // one allocation for the whole life of the model: captured decode graphs
    // hold its address. Batched decode rows and prefill chunks both fit; the
    // K-split partials of the M <= 64 form grow with M, so M = 64 bounds
    // every shorter prefill chunk.
    mm_work_.alloc(std::max({matmul_workspace((int)B), matmul_workspace(64),
                             matmul_workspace(std::min(kPrefillChunk, max_seq_))}));
    logits_.alloc(B * cfg_.vocab_size * sizeof(float));
    argmax_work_.alloc(qlm_argmax_workspace_bytes((int)B, cfg_.vocab_size));
    tail_work_.alloc(qlm_lm_head_greedy_workspace_bytes());
    check(qlm_fill_u8(tail_work_.get(), 0, tail_work_.bytes(), stream_), "fill");
    if (nh > 0) {  // the column-split mixer's partial sums and tickets (batch 1)
        dn_ss_.alloc((size_t)nh * 8 * sizeof(float));
        dn_ticket_.alloc((size_t)nh * QLM_DN_TICKET_STRIDE * sizeof(unsigned));
        check(qlm_fill_u8(dn_ticket_.get(), 0, dn_ticket_.bytes(), stream_), "fill");
    }
    if (QR_ > 0) {
        attn_work_.alloc(qlm_gqa_workspace_bytes((int)B, nq, hd, max_seq_));
        check(qlm_fill_u8(attn_work_.get(), 0, attn_work_.bytes(), stream_), "fill");
    }
    reset_states();
}

void DecoderModel::reset_states() {
    for (auto& b : conv_state_) check(qlm_fill_u8(b.get(), 0, b.bytes(), stream_), "fill");
    for (auto& b : dn_state_) check(qlm_fill_u8(b.get(), 0, b.bytes(), stream_), "fill");
    for (auto& b : k_cache_) check(qlm_fill_u8(b.get(), 0, b.bytes(), stream_), "fill");
    for (auto& b : v_cache_) check(qlm_fill_u8(b.get(), 0, b.bytes(), stream_), "fill");
    check(qlm_fill_u8(tokens_.get(), 0, tokens_.bytes(), stream_), "fill");
    check(qlm_fill_u8(pos_.get(), 0, pos_.bytes(), stream_), "fill");
    check(qlm_stream_sync(stream_), "sync");
}

// Appends to `plan` the tiles that the one-row GEMV over weight B (N outputs,
// K inputs, epilogue as qlm_gemv_i8_mx) reads first, where B has a
// tile-major copy; nothing where no launch shape fits.
static void plan_gemv_tiles(const Tensor& B, int N, int K, int epi, int max_tiles,
                            qlm_l2_plan& plan) {
    const void* q = B.int4_tiles ? static_cast<const void*>(B.int4_tiles)
                                 : static_cast<const void*>(B.int8_tiles);
    if (!q || B.is_native()) return;
    const int rc = qlm_gemv_mx_l2_plan(q, B.int8_tile_scales, B.int8_group, B.int4_tiles ? 1 : 0,
                                       N, K, epi, max_tiles, &plan);
    if (rc != QLM_OK && rc != QLM_ERR_SHAPE) check(rc, "qlm_gemv_mx_l2_plan");
}

// One decode step for sequences [0, B): the forward of DecoderModel::forward
// (model.cpp:151-199) with every layer's elementwise work fused into the
// projections, followed by greedy sampling and the position advance.

void DecoderModel::enqueue_step(int B) {
    math::set_stream(stream_);
    math::set_matmul_workspace(mm_work_.get(), mm_work_.bytes());
    const int H = cfg_.hidden_size, F = cfg_.intermediate_size, V = cfg_.vocab_size;
    const int nh = cfg_.linear_num_heads, d = cfg_.linear_head_dim;
    const int nq = cfg_.num_attention_heads, nkv = cfg_.num_key_value_heads, hd = cfg_.head_dim;
    const float eps = cfg_.rms_norm_eps;
    const int Pmax = std::max(PD_, PQ_);
    int n = 0;
    Tensor hx({B, H}, h_.get<float>());
    int dn_i = 0, at_i = 0;
    for (auto& w : layers_) {
        Tensor in_ln({H}, w.in_ln.get<float>()), post_ln({H}, w.post_ln.get<float>());
        // the column-split mixer reads proj rows as float4 (stride % 4 == 0)
        if (w.linear && B == 1 && Pmax % 4 == 0 && math::headnorm_supported(w.dn_out.view())) {
            // one sequence: the mixer over H x 8 workgroups, its head RMSNorm
            // applied by the out-projection's prologue
            Tensor proj({B, PD_}, proj_.get<float>());
            proj.strides = {Pmax, 1};
            math::matmul_rmsnorm(hx, in_ln, eps, w.dn_in.view(), proj);
            // the mixer leaves HBM mostly idle: its extra workgroups bring the
            // out-projection's tiles into the L2 of the XCDs that will read them
            // (int8: +0.7% a step; int4 tiles, half the bytes, lost 0.3%)
            qlm_l2_plan plan{};
            if (l2_plan_ && !int4_) plan_gemv_tiles(w.dn_out.view(), H, HD_, 1, 1 << 30, plan);
            check(qlm_deltanet_decode_cols_pf(proj_.get<float>(), Pmax,
                                              conv_state_[dn_i].get<float>(),
                                              w.conv_wt.get<float>(), w.A_log.get<float>(),
                                              w.dt_bias.get<float>(), w.dn_norm.get<float>(),
                                              dn_state_[dn_i].get<float>(), pos_.get<int>(),
                                              core_.get<float>(), CORE_, dn_ss_.get<float>(),
                                              dn_ticket_.get<unsigned>(), 1, nh, d, &plan,
                                              stream_),
                  "deltanet");
            Tensor core({B, HD_}, core_.get<float>());
            core.strides = {CORE_, 1};
            math::matmul_headnorm_residual(core, dn_ss_.get<float>(), 1e-6f, w.dn_out.view(), hx);
            ++dn_i;
            n += math::matmul_launches(B, PD_, H, true, native_) + 2;
        } else if (w.linear) {
            Tensor proj({B, PD_}, proj_.get<float>());
            proj.strides = {Pmax, 1};
            math::matmul_rmsnorm(hx, in_ln, eps, w.dn_in.view(), proj);
            check(qlm_deltanet_decode(proj_.get<float>(), Pmax, conv_state_[dn_i].get<float>(),
                                      w.conv_wt.get<float>(), w.A_log.get<float>(),
                                      w.dt_bias.get<float>(), w.dn_norm.get<float>(),
                                      dn_state_[dn_i].get<float>(), pos_.get<int>(),
                                      core_.get<float>(), CORE_, B, nh, d, stream_),
                  "deltanet");
            Tensor core({B, HD_}, core_.get<float>());
            core.strides = {CORE_, 1};
            math::matmul_residual(core, w.dn_out.view(), hx);
            ++dn_i;
            n += math::matmul_launches(B, PD_, H, true, native_) + 1 +
                 math::matmul_launches(B, H, HD_, false, native_);
        } else {
            Tensor proj({B, PQ_}, proj_.get<float>());
            proj.strides = {Pmax, 1};
            math::matmul_rmsnorm(hx, in_ln, eps, w.at_qkv.view(), proj);
            check(qlm_gqa_decode(proj_.get<float>(), Pmax, w.q_norm.get<float>(),
                                 w.k_norm.get<float>(), rope_cos_.get<float>(),
                                 rope_sin_.get<float>(), cfg_.rotary_dim(),
                                 k_cache_[at_i].get<float>(), v_cache_[at_i].get<float>(), max_seq_,
                                 pos_.get<int>(), core_.get<float>(), CORE_, B, nq, nkv, hd,
                                 w.gated ? 1 : 0, attn_work_.get(), stream_),
                  "gqa");
            Tensor core({B, nq * hd}, core_.get<float>());
            core.strides = {CORE_, 1};
            math::matmul_residual(core, w.at_o.view(), hx);
            ++at_i;
            n += math::matmul_launches(B, PQ_, H, true, native_) + 2 +  // + attention, combine
                 math::matmul_launches(B, H, nq * hd, false, native_);
        }
        Tensor act({B, F}, act_.get<float>());
        math::matmul_swiglu_rmsnorm(hx, post_ln, eps, w.gate_up.view(), act);
        math::matmul_residual(act, w.down.view(), hx);
        n += math::matmul_launches(B, F, H, true, native_) +
             math::matmul_launches(B, H, F, false, native_);
    }
    // Step tail: final norm + lm_head + greedy sample + advance, then the
    // embedding of the token now at pos (the next step's input, or the next
    // prompt token) -- model.cpp:193-199, :263-274, :157-164.
    const Tensor lm = lm_head_.view();
    // the fused greedy tail needs a one-row GEMV shape for the lm_head (the
    // tile-major mx forms, or the row-major GEMV when the model kept rows)
    int tail_waves = 0, tail_ring = 0, tail_grid = 0;
    const bool fused_tail =
        B == 1 && !native_ &&
        (lm.int8_data ||
         qlm_gemv_i8_mx_shape(V, H, 0, &tail_waves, &tail_ring, &tail_grid) == QLM_OK);
    if (fused_tail) {
        int rc = QLM_ERR_SHAPE;
        if (lm.int4_tiles)
            rc = qlm_lm_head_greedy_mx4(h_.get<float>(), final_norm_.get<float>(), eps,
                                        lm.int4_tiles, lm.int8_tile_scales, logits_.get<float>(),
                                        V, H, tail_work_.get(), tokens_.get<int>(), ld_tokens_,
                                        pos_.get<int>(), prompt_len_.get<int>(),
                                        embed_.get<float>(), H, h_.get<float>(), stream_);
        else if (lm.int8_tiles)
            rc = qlm_lm_head_greedy_mx(h_.get<float>(), final_norm_.get<float>(), eps, lm.int8_tiles,
                                       lm.int8_tile_scales, lm_head_.group, logits_.get<float>(), V,
                                       H, tail_work_.get(), tokens_.get<int>(), ld_tokens_,
                                       pos_.get<int>(), prompt_len_.get<int>(), embed_.get<float>(),
                                       H, h_.get<float>(), stream_);
        if (rc == QLM_ERR_SHAPE && lm.int8_data)
            rc = qlm_lm_head_greedy(h_.get<float>(), final_norm_.get<float>(), eps,
                                    lm_head_.q.get<int8_t>(), lm_head_.s.get<float>(),
                                    lm_head_.group, logits_.get<float>(), V, H, tail_work_.get(),
                                    tokens_.get<int>(), ld_tokens_, pos_.get<int>(),
                                    prompt_len_.get<int>(), embed_.get<float>(), H, h_.get<float>(),
                                    stream_);
        check(rc, "lm_head");
        n += 2;
    } else {
        Tensor fn({H}, final_norm_.get<float>());
        Tensor lg({B, V}, logits_.get<float>());
        math::matmul_rmsnorm(hx, fn, eps, lm_head_.view(), lg);
        check(qlm_greedy_advance(logits_.get<float>(), V, V, B, argmax_work_.get(),
                                 tokens_.get<int>(), ld_tokens_, pos_.get<int>(),
                                 prompt_len_.get<int>(), stream_),
              "argmax");
        embed_current(B);
        n += math::matmul_launches(B, V, H, true, native_) + 3;  // + argmax (two passes), embedding
    }
    kernels_per_step_ = n;
}

void DecoderModel::embed_current(int B) {
    check(qlm_embed_tokens(embed_.get<float>(), cfg_.vocab_size, cfg_.hidden_size,
                           tokens_.get<int>(), ld_tokens_, pos_.get<int>(), h_.get<float>(),
                           cfg_.hidden_size, B, stream_),
          "embed");
}

void* DecoderModel::graph_for(int B, int n) {
    auto it = graphs_.find({B, n});
    if (it != graphs_.end()) return it->second;
    check(qlm_graph_begin(stream_), "graph begin");
    try {
        for (int i = 0; i < n; ++i) enqueue_step(B);
    } catch (...) {
        void* g = nullptr;
        qlm_graph_end(stream_, &g);
        if (g) qlm_graph_destroy(g);
        throw;
    }
    void* g = nullptr;
    check(qlm_graph_end(stream_, &g), "graph end");
    graphs_[{B, n}] = g;
    return g;
}

void DecoderModel::forward(int token, int pos, float* logits_host) {
    if (pos < 0 || pos >= max_seq_)
        throw std::runtime_error("KV cache index out of bounds: pos = " + std::to_string(pos) +
                                 ", max_seq_len = " + std::to_string(max_seq_));
    if (token < 0 || token >= cfg_.vocab_size)
        throw std::runtime_error("forward: token id out of range");
    const int big = INT_MAX;
    check(qlm_memcpy_h2d(tokens_.get<int>() + pos, &token, sizeof(int), stream_), "upload");
    check(qlm_memcpy_h2d(pos_.get<int>(), &pos, sizeof(int), stream_), "upload");
    check(qlm_memcpy_h2d(prompt_len_.get<int>(), &big, sizeof(int), stream_), "upload");
    embed_current(1);
    check(qlm_graph_launch(graph_for(1), stream_), "graph launch");
    check(qlm_memcpy_d2h(logits_host, logits_.get(), (size_t)cfg_.vocab_size * sizeof(float),
                         stream_),
          "download");
    check(qlm_stream_sync(stream_), "sync");
}

void DecoderModel::last_logits(int b, float* host) const {
    check(qlm_memcpy_d2h(host, logits_.get<float>() + (size_t)b * cfg_.vocab_size,
                         (size_t)cfg_.vocab_size * sizeof(float), stream_),
          "download");
    check(qlm_stream_sync(stream_), "sync");
}

double DecoderModel::start(const int* prompts, int B, int n, int prefill_mode) {
    const bool batched_prefill = prefill_mode != kPrefillSteps;
    if (B <= 0 || B > max_batch_) throw std::runtime_error("generate: batch exceeds max_batch");
    if (n <= 0) throw std::runtime_error("generate: empty prompt");
    if (n > max_seq_)
        throw std::runtime_error("context length exceeded max_seq_len (" + std::to_string(max_seq_) +
                                 ")");
    for (int i = 0; i < B * n; ++i)
        if (prompts[i] < 0 || prompts[i] >= cfg_.vocab_size)
            throw std::runtime_error("generate: token id out of range");
    reset_states();
    std::vector<int> tok((size_t)B * ld_tokens_, 0), pl(B, n), p(B, 0);
    for (int b = 0; b < B; ++b) std::memcpy(&tok[(size_t)b * ld_tokens_], prompts + (size_t)b * n, n * 4);
    check(qlm_memcpy_h2d(tokens_.get(), tok.data(), tok.size() * 4, stream_), "upload");
    check(qlm_memcpy_h2d(prompt_len_.get(), pl.data(), B * 4, stream_), "upload");
    double prefill_s = 0.0;
    run_steps_ = 0;
    if (batched_prefill && n > 1) {
        check(qlm_stream_sync(stream_), "sync");
        const double t0 = now_s();
        for (int b = 0; b < B; ++b) prefill(b, n, prefill_mode == kPrefillChunked);
        check(qlm_stream_sync(stream_), "sync");
        prefill_s = now_s() - t0;
        std::fill(p.begin(), p.end(), n - 1);
        run_steps_ = n - 1;
    }
    check(qlm_memcpy_h2d(pos_.get(), p.data(), B * 4, stream_), "upload");
    embed_current(B);
    check(qlm_stream_sync(stream_), "sync");
    run_B_ = B;
    run_n_ = n;
    return prefill_s;
}

// Largest workspace any matrix-core matmul of the model needs at M rows.
size_t DecoderModel::matmul_workspace(int M) const {
    const int H = cfg_.hidden_size, F = cfg_.intermediate_size, V = cfg_.vocab_size;
    const int nq = cfg_.num_attention_heads, hd = cfg_.head_dim;
    size_t b = 256;
    auto upd = [&](int N, int K, int epi) {
        b = std::max(b, qlm_matmul_i8_workspace_bytes(M, N, K, epi));
        if (M <= 16) b = std::max(b, qlm_matmul_i8_mx_workspace_bytes(M, K));
        if (M >= 2) b = std::max(b, qlm_matmul_i8_t_workspace_bytes(std::min(M, 16), N, K, epi));
        b = std::max(b, qlm_matmul_w_workspace_bytes(K));
        b = std::max(b, qlm_matmul_bf16_workspace_bytes(M, K));
    };
    if (PD_ > 0) {
        upd(PD_, H, 0);
        upd(H, HD_, 1);
    }
    if (PQ_ > 0) {
        upd(PQ_, H, 0);
        upd(H, nq * hd, 1);
    }
    upd(F, H, 2);
    upd(H, F, 1);
    upd(V, H, 0);
    return b;
}

void DecoderModel::ensure_prefill_buffers(int rows) {
    if (rows <= pf_rows_) return;
    const size_t H = cfg_.hidden_size, F = cfg_.intermediate_size;
    const size_t Pmax = (size_t)std::max(PD_, PQ_);
    hx_pf_.alloc(rows * H * sizeof(float));
    proj_pf_.alloc(rows * Pmax * sizeof(float));
    core_pf_.alloc(rows * (size_t)CORE_ * sizeof(float));
    act_pf_.alloc(rows * F * sizeof(float));
    if (matmul_workspace(rows) > mm_work_.bytes())
        throw std::runtime_error("prefill: matmul workspace smaller than a prefill chunk needs");
    if (QR_ > 0 && gqa_pf_work_.bytes() == 0)
        gqa_pf_work_.alloc(qlm_gqa_prefill_workspace_bytes(cfg_.num_attention_heads,
                                                           cfg_.head_dim, max_seq_));
    if (HD_ > 0)
        dn_pf_work_.alloc(qlm_deltanet_chunk_workspace_bytes(rows, cfg_.linear_num_heads,
                                                             cfg_.linear_head_dim));
    pf_rows_ = rows;
}

// Prefill of sequence b: prompt positions 0..n-2 through every layer, in
// chunks of up to kPrefillChunk rows (the reference's forward_batch,
// model.cpp:213-258, with main.cpp:590-622's convention that the last prompt
// token is forwarded by the first decode step). Fills the conv rings,
// DeltaNet states and KV caches of sequence b; no logits are needed.
void DecoderModel::prefill(int b, int n, bool chunked_deltanet) {
    run_rows(b, 0, n - 1, chunked_deltanet);
}

void DecoderModel::run_rows(int b, int first, int count, bool chunked_deltanet, int* lm_idx,
                            float* logits_host) {
    if (count <= 0) return;
    const int chunk = std::min(count, kPrefillChunk);
    ensure_prefill_buffers(chunk);
    math::set_stream(stream_);
    math::set_matmul_workspace(mm_work_.get(), mm_work_.bytes());
    const int H = cfg_.hidden_size, F = cfg_.intermediate_size, V = cfg_.vocab_size;
    const int nh = cfg_.linear_num_heads, d = cfg_.linear_head_dim;
    const int nq = cfg_.num_attention_heads, nkv = cfg_.num_key_value_heads, hd = cfg_.head_dim;
    const float eps = cfg_.rms_norm_eps;
    const int Pmax = std::max(PD_, PQ_);
    const int C = 3 * HD_;
    for (int p0 = first; p0 < first + count; p0 += chunk) {
        const int rows = std::min(chunk, first + count - p0);
        check(qlm_embed_tokens(embed_.get<float>(), V, H,
                               tokens_.get<int>() + (size_t)b * ld_tokens_ + p0, 1, nullptr,
                               hx_pf_.get<float>(), H, rows, stream_),
              "embed");
        Tensor hx({rows, H}, hx_pf_.get<float>());
        int dn_i = 0, at_i = 0;
        for (auto& w : layers_) {
            Tensor in_ln({H}, w.in_ln.get<float>()), post_ln({H}, w.post_ln.get<float>());
            if (w.linear) {
                Tensor proj({rows, PD_}, proj_pf_.get<float>());
                proj.strides = {Pmax, 1};
                math::matmul_rmsnorm(hx, in_ln, eps, w.dn_in.view(), proj);
                float* cs = conv_state_[dn_i].get<float>() + (size_t)b * 3 * C;
                float* S = dn_state_[dn_i].get<float>() + (size_t)b * nh * d * d;
                if (chunked_deltanet)
                    check(qlm_deltanet_prefill_chunked(
                              proj_pf_.get<float>(), Pmax, rows, cs, w.conv_wt.get<float>(),
                              w.A_log.get<float>(), w.dt_bias.get<float>(),
                              w.dn_norm.get<float>(), S, p0, core_pf_.get<float>(), CORE_, nh, d,
                              dn_pf_work_.get(), dn_pf_work_.bytes(), stream_),
                          "deltanet prefill");
                else
                    check(qlm_deltanet_prefill(proj_pf_.get<float>(), Pmax, rows, cs,
                                               w.conv_wt.get<float>(), w.A_log.get<float>(),
                                               w.dt_bias.get<float>(), w.dn_norm.get<float>(), S,
                                               p0, core_pf_.get<float>(), CORE_, nh, d, stream_),
                          "deltanet prefill");
                Tensor core({rows, HD_}, core_pf_.get<float>());
                core.strides = {CORE_, 1};
                math::matmul_residual(core, w.dn_out.view(), hx);
                ++dn_i;
            } else {
                Tensor proj({rows, PQ_}, proj_pf_.get<float>());
                proj.strides = {Pmax, 1};
                math::matmul_rmsnorm(hx, in_ln, eps, w.at_qkv.view(), proj);
                const size_t cache_off = (size_t)b * max_seq_ * nkv * hd;
                check(qlm_gqa_prefill(proj_pf_.get<float>(), Pmax, w.q_norm.get<float>(),
                                      w.k_norm.get<float>(), rope_cos_.get<float>(),
                                      rope_sin_.get<float>(), cfg_.rotary_dim(),
                                      k_cache_[at_i].get<float>() + cache_off,
                                      v_cache_[at_i].get<float>() + cache_off, max_seq_, p0, rows,
                                      core_pf_.get<float>(), CORE_, nq, nkv, hd, w.gated ? 1 : 0,
                                      gqa_pf_work_.get(), stream_),
                      "gqa prefill");
                Tensor core({rows, nq * hd}, core_pf_.get<float>());
                core.strides = {CORE_, 1};
                math::matmul_residual(core, w.at_o.view(), hx);
                ++at_i;
            }
            Tensor act({rows, F}, act_pf_.get<float>());
            math::matmul_swiglu_rmsnorm(hx, post_ln, eps, w.gate_up.view(), act);
            math::matmul_residual(act, w.down.view(), hx);
        }
        if (!lm_idx && !logits_host) continue;
        // final norm + lm_head + greedy pick of these rows (model.cpp:246-255),
        // kLmRows rows at a time
        Tensor fn({H}, final_norm_.get<float>());
        for (int r0 = 0; r0 < rows; r0 += kLmRows) {
            const int m = std::min(kLmRows, rows - r0);
            const size_t row = (size_t)(p0 - first + r0);
            Tensor xs({m, H}, hx_pf_.get<float>() + (size_t)r0 * H);
            Tensor lg({m, V}, lm_pf_.get<float>());
            math::matmul_rmsnorm(xs, fn, eps, lm_head_.view(), lg);
            if (lm_idx)
                check(qlm_argmax(lm_pf_.get<float>(), V, V, m, lm_idx + row, lm_pf_work_.get(),
                                 stream_),
                      "argmax");
            if (logits_host)
                check(qlm_memcpy_d2h(logits_host + row * V, lm_pf_.get(),
                                     (size_t)m * V * sizeof(float), stream_),
                      "download");
        }
    }
}

void DecoderModel::snapshot_states() {
    if (conv_snap_.size() != conv_state_.size()) {
        conv_snap_.clear();
        dn_snap_.clear();
        for (auto& b : conv_state_) conv_snap_.emplace_back(b.bytes());
        for (auto& b : dn_state_) dn_snap_.emplace_back(b.bytes());
    }
    for (size_t i = 0; i < conv_state_.size(); ++i) {
        check(qlm_memcpy_d2d(conv_snap_[i].get(), conv_state_[i].get(), conv_state_[i].bytes(),
                             stream_),
              "snapshot");
        check(qlm_memcpy_d2d(dn_snap_[i].get(), dn_state_[i].get(), dn_state_[i].bytes(), stream_),
              "snapshot");
    }
    have_snapshot_ = true;
}

void DecoderModel::restore_states() {
    if (!have_snapshot_)
        throw std::runtime_error("restore_states() called before any snapshot_states()");
    for (size_t i = 0; i < conv_state_.size(); ++i) {
        check(qlm_memcpy_d2d(conv_state_[i].get(), conv_snap_[i].get(), conv_state_[i].bytes(),
                             stream_),
              "restore");
        check(qlm_memcpy_d2d(dn_state_[i].get(), dn_snap_[i].get(), dn_state_[i].bytes(), stream_),
              "restore");
    }
}

int DecoderModel::forward_greedy(int token, int pos) {
    if (pos < 0 || pos >= max_seq_)
        throw std::runtime_error("context length exceeded max_seq_len (" + std::to_string(max_seq_) +
                                 ")");
    if (token < 0 || token >= cfg_.vocab_size)
        throw std::runtime_error("forward: token id out of range");
    const int zero = 0;
    // the step's tail stores its pick as token pos + 1 (past the "prompt")
    check(qlm_memcpy_h2d(tokens_.get<int>() + pos, &token, sizeof(int), stream_), "upload");
    check(qlm_memcpy_h2d(pos_.get<int>(), &pos, sizeof(int), stream_), "upload");
    check(qlm_memcpy_h2d(prompt_len_.get<int>(), &zero, sizeof(int), stream_), "upload");
    embed_current(1);
    check(qlm_graph_launch(graph_for(1), stream_), "graph launch");
    int next = 0;
    check(qlm_memcpy_d2h(&next, tokens_.get<int>() + pos + 1, sizeof(int), stream_), "download");
    check(qlm_stream_sync(stream_), "sync");
    return next;
}

void DecoderModel::forward_batch(const int* toks, int n, int pos, int* argmax, float* logits) {
    if (n <= 0) return;
    if (!toks) throw std::runtime_error("forward_batch: null tokens");
    if (pos < 0 || pos + n > max_seq_)
        throw std::runtime_error("context length exceeded max_seq_len (" + std::to_string(max_seq_) +
                                 ")");
    for (int i = 0; i < n; ++i)
        if (toks[i] < 0 || toks[i] >= cfg_.vocab_size)
            throw std::runtime_error("forward_batch: token id out of range");
    if (n == 1) {  // model.cpp:215-219: one row is a plain forward
        const int t = forward_greedy(toks[0], pos);
        if (argmax) argmax[0] = t;
        if (logits) last_logits(0, logits);
        return;
    }
    const bool lm = argmax || logits;
    if (lm && !lm_pf_) {
        lm_pf_.alloc((size_t)kLmRows * cfg_.vocab_size * sizeof(float));
        lm_pf_work_.alloc(qlm_argmax_workspace_bytes(kLmRows, cfg_.vocab_size));
    }
    if (argmax && lm_pf_idx_.bytes() < (size_t)n * sizeof(int)) lm_pf_idx_.alloc((size_t)n * 4);
    check(qlm_memcpy_h2d(tokens_.get<int>() + pos, toks, (size_t)n * sizeof(int), stream_),
          "upload");
    // short runs (a verify batch, a replay) take the row-by-row recurrence,
    // the decode step's arithmetic; long prompt suffixes the chunked form
    run_rows(0, pos, n, n > kRowsMax, argmax ? lm_pf_idx_.get<int>() : nullptr, logits);
    if (argmax)
        check(qlm_memcpy_d2h(argmax, lm_pf_idx_.get(), (size_t)n * sizeof(int), stream_),
              "download");
    check(qlm_stream_sync(stream_), "sync");
}

double DecoderModel::steps(int k, bool use_graph) {
    if (run_B_ == 0) throw std::runtime_error("steps: call start() first");
    // positions 0 .. run_steps_+k-1 are forwarded; the last token is written
    // at position run_steps_+k, which the token array must hold
    if (run_steps_ + k > max_seq_)
        throw std::runtime_error("context length exceeded max_seq_len (" + std::to_string(max_seq_) +
                                 ")");
    // whole groups of kStepsPerGraph steps replay one graph each (the
    // device advances the positions, so the steps need no host work in
    // between); the rest replay the one-step graph
    void* g = use_graph ? graph_for(run_B_) : nullptr;
    void* gk = use_graph && k >= kStepsPerGraph ? graph_for(run_B_, kStepsPerGraph) : nullptr;
    void *e0 = nullptr, *e1 = nullptr;
    check(qlm_event_create(&e0), "event");
    check(qlm_event_create(&e1), "event");
    check(qlm_event_record(e0, stream_), "event");
    int s = 0;
    if (gk)
        for (; s + kStepsPerGraph <= k; s += kStepsPerGraph)
            check(qlm_graph_launch(gk, stream_), "graph launch");
    for (; s < k; ++s) {
        if (g) check(qlm_graph_launch(g, stream_), "graph launch");
        else enqueue_step(run_B_);
    }
    check(qlm_event_record(e1, stream_), "event");
    float ms = 0.0f;
    check(qlm_event_elapsed_ms(&ms, e0, e1), "event");
    qlm_event_destroy(e0);
    qlm_event_destroy(e1);
    run_steps_ += k;
    return ms;
}

void DecoderModel::tokens(int b, int first, int count, int* out) const {
    if (b < 0 || b >= run_B_ || first < 0 || first + count > ld_tokens_)
        throw std::runtime_error("tokens: range outside the token stream");
    check(qlm_memcpy_d2h(out, tokens_.get<int>() + (size_t)b * ld_tokens_ + first,
                         (size_t)count * sizeof(int), stream_),
          "download");
    check(qlm_stream_sync(stream_), "sync");
}

void DecoderModel::generate(const int* prompts, int B, int n, int n_new, int* out, GenStats* st,
                            bool use_graph, int prefill_mode) {
    if (n_new < 0) throw std::runtime_error("generate: negative token count");
    if (n + n_new - 1 > max_seq_)
        throw std::runtime_error("context length exceeded max_seq_len (" + std::to_string(max_seq_) +
                                 ")");
    const double t0 = now_s();
    start(prompts, B, n, prefill_mode);
    if (prefill_mode == kPrefillSteps) steps(n - 1, use_graph);
    check(qlm_stream_sync(stream_), "sync");
    const double t1 = now_s();
    steps(n_new, use_graph);
    const double t2 = now_s();
    for (int b = 0; b < B; ++b) tokens(b, n, n_new, out + (size_t)b * n_new);
    if (st) {
        st->prefill_s = t1 - t0;
        st->decode_s = t2 - t1;
        st->steps = n - 1 + n_new;
    }
}

}  // namespace qlm
