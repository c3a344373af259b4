/** @file hf_model.hpp
 *  @brief Hugging Face model configuration (the fields of include/pulsatrix/hf_model.hpp:33-101
 *         the Llama-family causal-LM path reads) and ToAttentionConfig (src/hf_model.cpp:282-313).
 */
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "pulsatrix/multihead_attention_module.hpp"

namespace pulsatrix {

struct HfModelConfig {
    std::string architecture;
    std::string model_type = "llama";
    int64_t hidden_size = 0;
    int64_t intermediate_size = 0;
    int64_t num_hidden_layers = 0;
    int64_t num_attention_heads = 0;
    int64_t num_key_value_heads = 0;
    int64_t head_dim = 0;
    int64_t vocab_size = 0;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 10000.0f;
    bool tie_word_embeddings = true;
    bool qkv_bias = false;
    bool out_bias = false;
    bool mlp_bias = false;
    bool qk_norm = false;
    bool causal = true;
    std::string hidden_act = "silu";
    float embed_scale = 1.0f;
};

/** @brief Rotate-half RoPE at rope_theta, GQA, causal: the Llama attention of the config. */
AttentionConfig ToAttentionConfig(const HfModelConfig& config);

}  // namespace pulsatrix
