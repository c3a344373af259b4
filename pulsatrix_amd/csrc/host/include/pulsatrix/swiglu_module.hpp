/** @file swiglu_module.hpp
 *  @brief Gated MLP down(act(gate(x)) * up(x)) (the surface of include/pulsatrix/swiglu_module.hpp).
 *         Fused path: one [gate | up] GEMM, the gate kernel, the down GEMM; relevance is the down
 *         projection's epsilon rule with Eq. 15's split of gate * up and both projection
 *         denominators fused into its epilogue, then one GEMM over [gate | up] (swiglu_module.cpp:139-170).
 */
#pragma once

#include "pulsatrix/detail/fused.hpp"
#include "pulsatrix/linear_module.hpp"
#include "pulsatrix/module.hpp"

namespace pulsatrix {

class RMSNormModule;

enum class GatedActivation { Silu, GeluTanh };

class SwiGLUModule : public Module {
public:
    SwiGLUModule(int64_t d_model, int64_t d_ff, DeviceBackend* backend, bool use_bias = true,
                 GatedActivation activation = GatedActivation::Silu);

    [[nodiscard]] Tensor propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) override;

    [[nodiscard]] LinearModule& gate_proj() { return gate_proj_; }
    [[nodiscard]] LinearModule& up_proj() { return up_proj_; }
    [[nodiscard]] LinearModule& down_proj() { return down_proj_; }

    /** @brief Fused-path forward. With `norm`, x is that RMSNorm's input and the gate/up GEMM
     *         applies the norm itself (RMSNormModule::fold); the relevance pass then reads the norm's
     *         output the same way. */
    const float* run_forward(const float* x, int64_t rows, const float* resid = nullptr, float* resid_out = nullptr,
                             RMSNormModule* norm = nullptr);
    /** @brief After run_forward over n sequences: repeats every activation the relevance pass reads
     *         `copies` times in place, as if the forward had run over copies * n sequences that
     *         repeat the n (storage from an earlier pass at least that large). */
    void replicate_forward(int64_t copies);
    /** @brief Sizes the buffers replicate_forward() repeats into for `rows`, without computing. */
    void reserve_forward(int64_t rows);
    /** @brief Fused-path relevance. `divided`: relevance_out already holds R / stab(z) of the down
     *         projection (a producer honoured relevance_denominator()), so no prologue divides it. */
    const float* run_relevance(const float* relevance_out, const LRPRuleConfig& config, const float* add = nullptr,
                               const detail::ResidualSplit& split = {}, bool divided = false);
    /** @brief The epsilon rule's denominator of the down projection for `config`: its pre-bias
     *         output z and, under the bias-in-denominator rule, its bias (else nullptr). */
    void relevance_denominator(const LRPRuleConfig& config, const float** den, const float** bias) const;
    [[nodiscard]] const float* output() const noexcept;

protected:
    Tensor forward_impl(const Tensor& input) override;

private:
    void pack_weights();
    const float* run_relevance_rule(const float* relevance_out, const LRPRuleConfig& config, const float* add,
                                    const detail::ResidualSplit& split);
    /** @brief The forward applies the gate in the gate/up GEMM's epilogue (no bias, F a multiple of 32). */
    [[nodiscard]] bool fused_gate() const noexcept { return !use_bias_ && F_ % 32 == 0; }

    int64_t d_, F_;
    bool use_bias_;
    MI355XBackend* be_;
    LinearModule gate_proj_, up_proj_, down_proj_;
    int act_;  // the gate: 0 SiLU, 1 GeLU tanh
    uint64_t packed_version_ = ~uint64_t{0};
    detail::DevBuf wgu_, wgu_il_, bgu_;
    int64_t rows_ = 0;
    const float* x_ = nullptr;
    Shape last_shape_;
    detail::DevBuf x_copy_, gu_z_, gu_y_, gate_post_, hidden_, down_z_, down_y_, g_, r_in_;
    RMSNormModule* norm_in_ = nullptr;  // the RMSNorm folded into the gate/up GEMM by the last forward, if any
    detail::DevBuf wgu_g_;              // the gate/up GEMM's weight with the folded norm's gamma on its rows
    const RMSNormModule* wg_norm_ = nullptr;
    uint64_t wg_version_ = ~uint64_t{0}, wg_packed_ = ~uint64_t{0};
    const float* folded_weights(RMSNormModule* norm);
    detail::AffineRule down_rule_, gate_up_rule_;
};

}  // namespace pulsatrix
