/** @file module.hpp
 *  @brief Module base class (the surface of include/pulsatrix/module.hpp:93-168): forward() is a
 *         non-virtual wrapper that checks the input, propagate_relevance() is pure virtual.
 */
#pragma once

#include <optional>
#include <stdexcept>

#include "pulsatrix/lrp_rule_config.hpp"
#include "pulsatrix/tensor.hpp"

namespace pulsatrix {

class Module {
public:
    virtual ~Module() = default;

    /** @brief Checks the input is non-empty and on this module's device, then runs forward_impl(). */
    [[nodiscard]] Tensor forward(const Tensor& input) {
        if (input.numel() <= 0) throw std::invalid_argument("Module::forward: input must not be empty");
        if (auto dev = compute_device()) require_device(input, *dev, "Module::forward");
        return forward_impl(input);
    }

    /** @brief Relevance at this module's input from relevance at its output. */
    [[nodiscard]] virtual Tensor propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) = 0;

    /** @brief Gradients are not part of the MI355X forward + AttnLRP path. */
    [[nodiscard]] virtual Tensor backward(const Tensor&) {
        throw std::logic_error("Module::backward: the MI355X path runs forward and relevance only");
    }

    [[nodiscard]] virtual std::optional<DeviceType> compute_device() const { return DeviceType::Hip; }
    virtual void set_training(bool training) { training_ = training; }
    [[nodiscard]] bool is_training() const noexcept { return training_; }

protected:
    virtual Tensor forward_impl(const Tensor& input) = 0;

private:
    bool training_ = false;
};

}  // namespace pulsatrix
