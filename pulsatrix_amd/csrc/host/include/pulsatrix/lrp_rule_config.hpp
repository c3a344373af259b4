/** @file lrp_rule_config.hpp
 *  @brief LRP rule configuration (the surface of include/pulsatrix/lrp_rule_config.hpp:72-115).
 *
 *  The MI355X path implements the epsilon rule in both of Pulsatrix's forms: the pre-bias rule
 *  (the default) and the bias-in-denominator rule LXT and Zennit use. Other rules throw.
 */
#pragma once

#include <string>

namespace pulsatrix {

enum class LRPRule { Epsilon, AlphaBeta, Gamma, ZBox };

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

/** @brief Throws std::invalid_argument unless the config is an epsilon rule (the one this path runs). */
void require_epsilon_rule(const LRPRuleConfig& config, const char* module_name);

}  // namespace pulsatrix
