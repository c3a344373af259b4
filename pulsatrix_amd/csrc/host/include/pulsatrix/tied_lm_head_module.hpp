/** @file tied_lm_head_module.hpp
 *  @brief LM head sharing the embedding table: logits = x E^T (the surface of
 *         include/pulsatrix/tied_lm_head_module.hpp). Relevance is the bias-in-denominator
 *         epsilon rule against a zero bias (tied_lm_head_module.cpp:76-111): one split-K MFMA
 *         GEMM with the divide by stab(logits) in its prologue and the multiply by x in its epilogue.
 *         Gamma, AlphaBeta and ZBox run on W = E^T over stacked-weight GEMMs.
 */
#pragma once

#include "pulsatrix/detail/rules.hpp"
#include "pulsatrix/embedding_module.hpp"

namespace pulsatrix {

class TiedLMHeadModule : public Module {
public:
    TiedLMHeadModule(EmbeddingModule& embedding, DeviceBackend* backend);

    [[nodiscard]] Tensor propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) override;

    const float* run_forward(const float* x, int64_t rows);
    const float* run_relevance(const float* relevance_out, const LRPRuleConfig& config,
                               const detail::ResidualSplit& split = {});
    /** @brief The epsilon rule for the seed pxk_lm_seed would form over n sequences of l rows
     *         (one-hot at each last row, at targets_in or the argmax), without forming it: only
     *         the seeded rows are computed, the others are the dense rule's exact zeros
     *         (pxk_lm_seed_head_relevance). Writes the targets to the device array targets_out.
     *         Returns the relevance, or nullptr when it went into `split`. */
    const float* run_seeded_relevance(int64_t n, int64_t l, const int64_t* targets_in, int64_t* targets_out,
                                      bool unit_seed, const LRPRuleConfig& config,
                                      const detail::ResidualSplit& split = {});
    [[nodiscard]] const float* logits() const noexcept { return logits_.data(); }

protected:
    Tensor forward_impl(const Tensor& input) override;

private:
    EmbeddingModule& embedding_;
    MI355XBackend* be_;
    int64_t rows_ = 0;
    const float* x_ = nullptr;
    Shape last_in_shape_, last_out_shape_;
    detail::DevBuf x_copy_, logits_, r_in_;
    detail::AffineRule rule_;
};

}  // namespace pulsatrix
