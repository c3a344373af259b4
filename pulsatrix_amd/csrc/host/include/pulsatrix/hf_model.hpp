/** @file hf_model.hpp
 *  @brief Hugging Face model configuration (the fields of include/pulsatrix/hf_model.hpp:33-101
 *         the Llama, Qwen and Gemma 3 causal-LM paths read) and ToAttentionConfig
 *         (src/hf_model.cpp:282-313).
 */
#pragma once

#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "pulsatrix/multihead_attention_module.hpp"

namespace pulsatrix {

/** @brief HfRopeScaling (include/pulsatrix/hf_model.hpp:20-31): "linear" or "llama3". */
struct HfRopeScaling {
    std::string type = "default";
    float factor = 1.0f;
    float low_freq_factor = 1.0f;
    float high_freq_factor = 1.0f;
    int64_t original_max_position_embeddings = 0;
};

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
    /** @brief The full-attention layers' RoPE scaling (all layers' when there is one kind). */
    std::optional<HfRopeScaling> rope_scaling;
    /** @brief Sliding-window layers' own RoPE base, unscaled (Gemma 3's rope_local_base_freq). */
    std::optional<float> rope_local_base_freq;
    bool tie_word_embeddings = true;
    bool qkv_bias = false;
    bool out_bias = false;
    bool mlp_bias = false;
    bool qk_norm = false;
    bool causal = true;
    /** @brief "silu", or "gelu_pytorch_tanh" / "gelu_new" (Gemma's GeGLU). */
    std::string hidden_act = "silu";
    int64_t max_position_embeddings = 0;
    std::optional<int64_t> sliding_window;
    std::optional<float> query_pre_attn_scalar;
    /** @brief "sliding_attention" / "full_attention" per layer. */
    std::vector<std::string> layer_types;
    /** @brief RMSNorms scale by offset + w (Gemma 3: 1). */
    float norm_weight_offset = 0.0f;
    /** @brief Token embeddings are multiplied by this (Gemma 3: sqrt(hidden_size)). */
    float embed_scale = 1.0f;
    /** @brief Gemma 3's sandwich norms after the attention and after the MLP. */
    bool post_norms = false;

    /** @brief Whether layer i uses sliding-window attention (hf_model.cpp:249-253). */
    [[nodiscard]] bool is_sliding_layer(int64_t i) const;
};

/** @brief RopeInverseFrequencies (hf_model.cpp:255-287): 1 / theta^(2i/D) with the config's
 *         linear or llama3 scaling. */
std::vector<double> RopeInverseFrequencies(const HfModelConfig& config);
/** @brief The attention every layer shares (hf_model.cpp:289-303): rotate-half RoPE at rope_theta
 *         (scaled), GQA, QK-Norm and score scale as configured. */
AttentionConfig ToAttentionConfig(const HfModelConfig& config);
/** @brief Layer i's attention (hf_model.cpp:305-313): a sliding layer gets the window and, when
 *         given, its own unscaled RoPE base. */
AttentionConfig ToAttentionConfig(const HfModelConfig& config, int64_t layer);

}  // namespace pulsatrix
