/** @file rules.hpp
 *  @brief The Zennit-compatible affine rules (Gamma, AlphaBeta, ZBox; lrp_rules.cpp:72-160) on
 *         the MI355X modules: two MFMA GEMMs over the layer's stacked weights with the sign split,
 *         gated divide and recombination as small kernels around them (include/pxk.h).
 */
#pragma once

#include <cstdint>
#include <vector>

#include "pulsatrix/detail/fused.hpp"
#include "pulsatrix/lrp_rule_config.hpp"

namespace pulsatrix::detail {

/** @brief One column block of a (possibly column-packed) affine layer: W (in x cols) stored with
 *         row stride ld, or transposed (cols x in) when trans; bias (cols) nullable. */
struct RuleBlock {
    const float* w;
    int64_t ld;
    int64_t cols;
    bool trans;
    const float* bias;
};

/** @brief lrp_rules::validate (lrp_rules.cpp:162-175): throws std::invalid_argument naming the
 *         module when AlphaBeta's parameters break alpha, beta >= 0 and alpha - beta == 1. */
void validate_rule(const LRPRuleConfig& config, const char* module_name);

/** @brief Whether config is one of the rules this helper runs (not epsilon). */
inline bool is_affine_rule(const LRPRuleConfig& config) { return config.rule != LRPRule::Epsilon; }

/** @brief A layer's rule state: its stacked weights, rebuilt when the rule, its parameters or the
 *         layer's weights change, and the per-pass scratch. */
class AffineRule {
public:
    struct Pass {
        const float* x;       ///< layer input (rows x in, row stride ldx)
        int64_t ldx;
        int64_t rows, in;
        const float* z;       ///< pre-bias x W (rows x out, row stride ldz)
        int64_t ldz;
        const float* bias;    ///< the layer's bias over out, packed like the blocks (nullable)
        const float* r;       ///< output relevance r[m][j % r_cols] (row stride ldr)
        int64_t ldr, r_cols;
        float* r_in;          ///< input relevance (rows x in, contiguous)
        const float* add;     ///< summed into r_in (nullable)
    };

    /** @brief Runs config's rule over the layer made of `blocks` (their cols sum to out); with a
     *         split request the split shares are written instead of r_in. `version` changes
     *         whenever the blocks' weights do. */
    void run(MI355XBackend* be, const LRPRuleConfig& config, uint64_t version, const std::vector<RuleBlock>& blocks,
             const Pass& p, const ResidualSplit& split = {});
    void release();

private:
    void ensure_weights(MI355XBackend* be, const LRPRuleConfig& config, uint64_t version,
                        const std::vector<RuleBlock>& blocks, int64_t in, int64_t out);

    DevBuf w2_, b2_, xs_, den_, c_;
    bool built_ = false;
    LRPRule rule_ = LRPRule::Epsilon;
    float params_[4] = {0, 0, 0, 0};
    uint64_t version_ = 0;
    const float* first_w_ = nullptr;
    int64_t in_ = 0, out_ = 0;
};

}  // namespace pulsatrix::detail
