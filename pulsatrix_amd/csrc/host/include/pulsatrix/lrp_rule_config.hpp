/** @file lrp_rule_config.hpp
 *  @brief LRP rule configuration (the surface of include/pulsatrix/lrp_rule_config.hpp:15-115).
 *
 *  The MI355X path runs every rule the reference defines for the causal LM's affine layers:
 *  epsilon in both of Pulsatrix's forms (pre-bias, the default, and bias-in-denominator as LXT and
 *  Zennit use it) on the fused GEMMs, and Zennit's Gamma, AlphaBeta and ZBox (lrp_rules.cpp:72-160)
 *  over stacked-weight GEMMs. The attention, SwiGLU and residual rules read only `epsilon`, as in
 *  the reference.
 */
#pragma once

#include <string>

namespace pulsatrix {

/** @brief The reference's LRPRule, in its declaration order (lrp_rule_config.hpp:21-35). */
enum class LRPRule { Epsilon, Gamma, AlphaBeta, ZBox };

/** @brief Lower-case rule name (lrp_rule_config.hpp:52-64). */
inline std::string lrp_rule_name(LRPRule rule) {
    switch (rule) {
        case LRPRule::Epsilon: return "epsilon";
        case LRPRule::Gamma: return "gamma";
        case LRPRule::AlphaBeta: return "alpha_beta";
        case LRPRule::ZBox: return "zbox";
    }
    return "unknown";
}

struct LRPRuleConfig {
    float epsilon = 1e-6f;
    LRPRule rule = LRPRule::Epsilon;
    float gamma = 0.25f;
    float alpha = 1.0f;
    float beta = 0.0f;
    float low = 0.0f;
    float high = 1.0f;
    bool epsilon_bias_in_denominator = false;
    bool layer_norm_detach_std = false;
};

/** @brief LXT 2.1's AttnLRP settings: epsilon 1e-9, bias in the denominator (attnlrp_parity.cpp:67-72). */
inline LRPRuleConfig LxtAttnLrpConfig() {
    LRPRuleConfig config{1e-9f};
    config.epsilon_bias_in_denominator = true;
    config.layer_norm_detach_std = true;
    return config;
}

}  // namespace pulsatrix
