/** @file linear_module.hpp
 *  @brief Dense layer y = x W + b with W (in, out) (the surface of include/pulsatrix/linear_module.hpp).
 */
#pragma once

#include <cstdint>
#include <vector>

#include "pulsatrix/detail/fused.hpp"
#include "pulsatrix/detail/rules.hpp"
#include "pulsatrix/module.hpp"

namespace pulsatrix {

class LinearModule : public Module {
public:
    LinearModule(int64_t in_features, int64_t out_features, DeviceBackend* backend, bool use_bias = true);

    /** @brief Epsilon rule, pre-bias or bias-in-denominator (linear_module.cpp:333-341,
     *         lrp_rules.cpp:197-220), as one fused MFMA GEMM: x * ((r / stab(z [+ b])) W^T);
     *         Gamma, AlphaBeta and ZBox (lrp_rules.cpp:72-160) over stacked-weight GEMMs. */
    [[nodiscard]] Tensor propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) override;

    void set_weight(const std::vector<float>& values);
    void set_bias(const std::vector<float>& values);
    /** @brief Mutable access counts as a change (packed copies are rebuilt). */
    [[nodiscard]] Tensor& weight() {
        ++version_;
        return weight_;
    }
    [[nodiscard]] const Tensor& weight() const noexcept { return weight_; }
    [[nodiscard]] Tensor& bias() {
        ++version_;
        return bias_;
    }
    [[nodiscard]] const Tensor& bias() const noexcept { return bias_; }
    [[nodiscard]] const float* weight_data() const noexcept { return weight_.data(); }
    [[nodiscard]] const float* bias_data() const noexcept { return bias_.data(); }
    [[nodiscard]] bool use_bias() const noexcept { return use_bias_; }
    [[nodiscard]] int64_t in_features() const noexcept { return in_; }
    [[nodiscard]] int64_t out_features() const noexcept { return out_; }
    [[nodiscard]] uint64_t version() const noexcept { return version_; }

    /** @brief Fused-path forward over `rows` rows of x (kept by pointer until the next call). */
    const float* run_forward(const float* x, int64_t rows);
    /** @brief Fused-path relevance; `add` (nullable) is summed into the result. */
    const float* run_relevance(const float* r, const LRPRuleConfig& config, const float* add = nullptr,
                               const detail::ResidualSplit& split = {});

protected:
    Tensor forward_impl(const Tensor& input) override;

private:
    int64_t in_, out_;
    bool use_bias_;
    MI355XBackend* be_;
    Tensor weight_, bias_;
    uint64_t version_ = 0;
    const float* x_ = nullptr;
    int64_t rows_ = 0;
    detail::DevBuf x_copy_, z_, y_, r_in_;
    detail::AffineRule rule_;
};

}  // namespace pulsatrix
