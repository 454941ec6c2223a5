// Model configuration for the Qwen3.5 hybrid family (reference:
// ModelConfig, src/model/config.hpp:12-27, filled by
// Qwen3_5Architecture::parse_config, src/arch/qwen3_5.cpp:11-72).
#pragma once

#include <cmath>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "json.hpp"

namespace qlm {

struct ModelConfig {
    std::string model_type;
    int vocab_size = 248320;
    int hidden_size = 1024;
    int intermediate_size = 3584;
    int num_hidden_layers = 24;
    int num_attention_heads = 8;
    int num_key_value_heads = 2;
    int head_dim = 256;
    int linear_num_heads = 16;
    int linear_head_dim = 128;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 1000000.0f;
    float partial_rotary_factor = 1.0f;
    std::vector<std::string> layer_types;

    int rotary_dim() const { return (int)(head_dim * partial_rotary_factor); }
    bool is_linear(int i) const { return layer_types[i] != "full_attention"; }
};

inline bool qwen35_matches(const std::string& t) { return t.rfind("qwen3_5", 0) == 0; }

// Same field names, defaults and 3:1 default layer pattern as the reference.
inline ModelConfig parse_model_config(const std::string& dir) {
    std::ifstream f(dir + "/config.json");
    if (!f) throw std::runtime_error("Failed to open config.json at: " + dir + "/config.json");
    std::stringstream ss;
    ss << f.rdbuf();
    Json root = Json::parse(ss.str());
    const Json& c = root.has("text_config") ? root.at("text_config") : root;
    ModelConfig cfg;
    if (c.has("model_type")) cfg.model_type = c.at("model_type").string();
    else if (root.has("model_type")) cfg.model_type = root.at("model_type").string();
    if (!qwen35_matches(cfg.model_type))
        throw std::runtime_error("Unsupported model architecture: '" + cfg.model_type + "'");
    cfg.vocab_size = (int)c.at("vocab_size").number();
    cfg.hidden_size = (int)c.at("hidden_size").number();
    cfg.intermediate_size = (int)c.at("intermediate_size").number();
    cfg.num_hidden_layers = (int)c.at("num_hidden_layers").number();
    cfg.num_attention_heads = (int)c.at("num_attention_heads").number();
    cfg.num_key_value_heads = (int)c.get("num_key_value_heads", cfg.num_attention_heads);
    cfg.rms_norm_eps = (float)c.get("rms_norm_eps", cfg.rms_norm_eps);
    if (c.has("rope_theta")) {
        cfg.rope_theta = (float)c.at("rope_theta").number();
    } else if (c.has("rope_parameters")) {
        const Json& rp = c.at("rope_parameters");
        cfg.rope_theta = (float)rp.get("rope_theta", cfg.rope_theta);
        cfg.partial_rotary_factor = (float)rp.get("partial_rotary_factor", cfg.partial_rotary_factor);
    }
    cfg.partial_rotary_factor = (float)c.get("partial_rotary_factor", cfg.partial_rotary_factor);
    cfg.head_dim = c.has("head_dim") ? (int)c.at("head_dim").number()
                                     : cfg.hidden_size / cfg.num_attention_heads;
    cfg.linear_num_heads = (int)c.get("linear_num_key_heads", cfg.linear_num_heads);
    cfg.linear_head_dim = (int)c.get("linear_key_head_dim", cfg.linear_head_dim);
    if (c.has("layer_types") && c.at("layer_types").is_array()) {
        for (const auto& t : c.at("layer_types").arr) cfg.layer_types.push_back(t.string());
    } else {
        for (int i = 0; i < cfg.num_hidden_layers; ++i)
            cfg.layer_types.push_back(i % 4 == 3 ? "full_attention" : "linear_attention");
    }
    if ((int)cfg.layer_types.size() < cfg.num_hidden_layers)
        throw std::runtime_error("config: layer_types shorter than num_hidden_layers");
    return cfg;
}

}  // namespace qlm
