/** @file transformer_block.hpp
 *  @brief Pre-norm decoder block x + attn(norm1(x)), then + mlp(norm2(.)) (the surface of
 *         include/pulsatrix/transformer_block.hpp); relevance per transformer_block.cpp:189-227
 *         with both residual adds fused into the sublayers' last GEMM epilogues. With Gemma's
 *         sandwich norms each sublayer output is normalised again before its residual add (the
 *         adds then run after the norms), and relevance passes those norms unchanged.
 */
#pragma once

#include <memory>

#include "pulsatrix/multihead_attention_module.hpp"
#include "pulsatrix/rms_norm_module.hpp"
#include "pulsatrix/swiglu_module.hpp"

namespace pulsatrix {

/** @brief TransformerBlockOptions of include/pulsatrix/transformer_block.hpp:20-32. */
struct TransformerBlockOptions {
    float norm_eps = 1e-6f;
    bool mlp_bias = true;
    GatedActivation mlp_activation = GatedActivation::Silu;
    bool post_norms = false;
    float norm_weight_offset = 0.0f;
};

class TransformerBlock : public Module {
public:
    TransformerBlock(const AttentionConfig& attention, int64_t d_ff, DeviceBackend* backend,
                     const TransformerBlockOptions& options = {});
    TransformerBlock(int64_t d_model, int64_t num_heads, int64_t d_ff, DeviceBackend* backend, bool use_rope = true,
                     bool use_qk_norm = false);

    [[nodiscard]] Tensor propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) override;

    [[nodiscard]] RMSNormModule& norm1() { return norm1_; }
    [[nodiscard]] RMSNormModule& norm2() { return norm2_; }
    [[nodiscard]] MultiHeadAttentionModule& mha() { return mha_; }
    [[nodiscard]] SwiGLUModule& swiglu() { return swiglu_; }
    /** @brief Gemma's sandwich norms (TransformerBlockOptions::post_norms); throw std::logic_error
     *         when the block has none. */
    [[nodiscard]] RMSNormModule& post_attn_norm();
    [[nodiscard]] RMSNormModule& post_mlp_norm();
    [[nodiscard]] bool has_post_norms() const noexcept { return post_attn_norm_ != nullptr; }

    /** @brief Fused-path forward; x must stay valid until the relevance pass. Returns y2. */
    const float* run_forward(const float* x, int64_t n, int64_t l);
    /** @brief After run_forward over n sequences: repeats every activation the relevance pass reads
     *         `copies` times in place, as if the forward had run over copies * n sequences that
     *         repeat the n (storage from an earlier pass at least that large). */
    void replicate_forward(int64_t copies);
    /** @brief Sizes the buffers replicate_forward() repeats into for `n sequences of length l`, without computing. */
    void reserve_forward(int64_t n, int64_t l);
    const float* run_relevance(const float* relevance_out, const LRPRuleConfig& config);
    /** @brief The epsilon split of this block's output y2 = y1 + mlp, for the GEMM that produces the
     *         block's output relevance to perform into this block's buffers. Valid after run_forward.
     *         With `divide_for` (an epsilon rule), the MLP's share is requested divided by the down
     *         projection's denominator: the producer must honour ResidualSplit::b_den. */
    detail::ResidualSplit output_split(const LRPRuleConfig* divide_for = nullptr);
    /** @brief Relevance pass once the producer applied output_split(); `below` is the split the block
     *         underneath asks for (its output is this block's input), or none. Returns the input
     *         relevance when `below` is empty, else nullptr. */
    const float* run_relevance_split(const LRPRuleConfig& config, const detail::ResidualSplit& below);
    /** @brief One KV-cached decode step of n sequences at the device position *pos
     *         (forward_cached, transformer_block.cpp:135-153). Returns y2 (n, d_model). x_normed
     *         (nullable) is norm1(x) when the caller has it. With next_norm and next_normed, a block
     *         with sandwich norms also writes next_norm(y2) and points *next_normed at it (else
     *         nullptr). */
    const float* decode_step(const float* x, const float* x_normed, int64_t n, KVCacheState& cache,
                             const int32_t* pos, RMSNormModule* next_norm = nullptr,
                             const float** next_normed = nullptr);

protected:
    Tensor forward_impl(const Tensor& input) override;

private:
    int64_t d_;
    MI355XBackend* be_;
    RMSNormModule norm1_;
    MultiHeadAttentionModule mha_;
    RMSNormModule norm2_;
    SwiGLUModule swiglu_;
    std::unique_ptr<RMSNormModule> post_attn_norm_, post_mlp_norm_;
    const float* attn_out_ = nullptr;  // the sublayer outputs the residual sums add (after any post norm)
    const float* ffn_out_ = nullptr;
    int64_t N_ = 0, L_ = 0;
    const float* x_ = nullptr;
    Shape last_shape_;
    detail::DevBuf x_copy_, y1_, y2_, r_y1d_, r_ffn_, r_y1_, r_xd_, r_attn_, dec_y1_, dec_y2_, dec_n2_, dec_next_;
    bool r_ffn_divided_ = false;  // the last output_split() asked for the MLP's share pre-divided
};

}  // namespace pulsatrix
