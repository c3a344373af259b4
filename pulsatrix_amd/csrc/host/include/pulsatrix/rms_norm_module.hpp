/** @file rms_norm_module.hpp
 *  @brief RMSNorm over the last axis (the surface of include/pulsatrix/rms_norm_module.hpp).
 *         gamma starts at zero, as the reference's does; relevance is the identity
 *         (rms_norm_module.cpp:101-111).
 */
#pragma once

#include <vector>

#include "pulsatrix/detail/fused.hpp"
#include "pulsatrix/module.hpp"

namespace pulsatrix {

class RMSNormModule : public Module {
public:
    RMSNormModule(int64_t num_features, DeviceBackend* backend, DeviceType device = DeviceType::Hip, float eps = 1e-6f);

    [[nodiscard]] Tensor propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) override;

    void set_gamma(const std::vector<float>& values);
    [[nodiscard]] const Tensor& gamma() const noexcept { return gamma_; }
    /** @brief Mutable access counts as a change (the effective scale is rebuilt). */
    [[nodiscard]] Tensor& gamma() noexcept {
        ++version_;
        return gamma_;
    }
    /** @brief Scale by offset + gamma (Gemma's 1 + w; rms_norm_module.cpp:40-49). */
    void set_weight_offset(float offset) noexcept {
        offset_ = offset;
        ++version_;
    }
    [[nodiscard]] float weight_offset() const noexcept { return offset_; }
    /** @brief The scale the forward applies: gamma, or offset + gamma computed on the device. */
    const float* effective_gamma();
    [[nodiscard]] float eps() const noexcept { return eps_; }
    /** @brief Changes whenever the effective scale may have changed. */
    [[nodiscard]] uint64_t version() const noexcept { return version_; }
    [[nodiscard]] int64_t num_features() const noexcept { return d_; }

    /** @brief Fused-path forward into a module-owned buffer. */
    const float* run_forward(const float* x, int64_t rows);
    /** @brief Fused path with the norm folded into the GEMM that reads its output (PXK_PRO_RMS):
     *         that GEMM normalises `rows` rows of its input itself and writes each row's rms into the
     *         buffer returned here; the norm's output is not stored. */
    float* fold(int64_t rows);
    /** @brief After fold(): the norm's output of the input x the GEMM read, computed and stored now
     *         (for the consumers that read it stored: the Gamma / AlphaBeta / ZBox rules). */
    const float* materialize(const float* x);
    /** @brief Each row's rms from the last forward or fold(). */
    [[nodiscard]] const float* rms() const noexcept { return rms_.data(); }
    /** @brief After run_forward over n sequences: repeats every activation the relevance pass reads
     *         `copies` times in place, as if the forward had run over copies * n sequences that
     *         repeat the n (storage from an earlier pass at least that large). */
    void replicate_forward(int64_t copies);
    /** @brief Sizes the buffers replicate_forward() repeats into for `rows`, without computing. */
    void reserve_forward(int64_t rows);
    [[nodiscard]] const float* output() const noexcept { return out_.data(); }

protected:
    Tensor forward_impl(const Tensor& input) override;

private:
    int64_t d_;
    float eps_;
    MI355XBackend* be_;
    Tensor gamma_;
    float offset_ = 0.0f;
    uint64_t version_ = 0, eff_version_ = ~uint64_t{0};
    int64_t rows_ = 0;
    bool folded_ = false;  // the last forward was folded into a GEMM: out_ holds nothing of it
    detail::DevBuf out_, rms_, eff_;
};

}  // namespace pulsatrix
