// The Zennit-compatible affine rules on MI355XBackend (src/lrp_rules.cpp:72-175).
#include "pulsatrix/detail/rules.hpp"

#include <stdexcept>
#include <string>

namespace pulsatrix::detail {

void validate_rule(const LRPRuleConfig& config, const char* module_name) {
    if (config.rule != LRPRule::AlphaBeta) return;
    if (!(config.alpha >= 0.0f) || !(config.beta >= 0.0f))
        throw std::invalid_argument(std::string(module_name) +
                                    "::propagate_relevance: AlphaBeta rule needs alpha >= 0 and beta >= 0");
    if (config.alpha - config.beta != 1.0f)
        throw std::invalid_argument(std::string(module_name) +
                                    "::propagate_relevance: AlphaBeta rule needs alpha - beta == 1");
}

namespace {

pxk_rule_params params_of(const LRPRuleConfig& c) {
    pxk_rule_params p{};
    p.rule = static_cast<int32_t>(c.rule);  // LRPRule order: Epsilon, Gamma, AlphaBeta, ZBox
    p.eps = c.epsilon;
    p.gamma = c.gamma;
    p.alpha = c.alpha;
    p.beta = c.beta;
    p.low = c.low;
    p.high = c.high;
    return p;
}

// The parameters that shape a rule's stacked weights (the rest only enter the divide).
void shape_params(const LRPRuleConfig& c, float out[4]) {
    out[0] = c.rule == LRPRule::Gamma ? c.gamma : 0.0f;
    out[1] = c.rule == LRPRule::ZBox ? c.low : 0.0f;
    out[2] = c.rule == LRPRule::ZBox ? c.high : 0.0f;
    out[3] = 0.0f;
}

}  // namespace

void AffineRule::ensure_weights(MI355XBackend* be, const LRPRuleConfig& config, uint64_t version,
                                const std::vector<RuleBlock>& blocks, int64_t in, int64_t out) {
    float shape[4];
    shape_params(config, shape);
    const bool same = built_ && rule_ == config.rule && version_ == version && first_w_ == blocks.front().w &&
                      in_ == in && out_ == out && shape[0] == params_[0] && shape[1] == params_[1] &&
                      shape[2] == params_[2];
    if (same) return;
    const bool zbox = config.rule == LRPRule::ZBox;
    float* w2 = w2_.ensure(be, 2 * in * (zbox ? out : 2 * out));
    float* b2 = b2_.ensure(be, 2 * out);
    std::vector<pxk_rule_block> kb;
    for (const RuleBlock& b : blocks) kb.push_back({b.w, b.ld, b.cols, b.trans ? 1 : 0, b.bias});
    const pxk_rule_params p = params_of(config);
    MI355XBackend::check(pxk_lrp_rule_weights(&p, kb.data(), static_cast<int>(kb.size()), in, w2, b2, be->stream()),
                         "lrp rule weights");
    built_ = true;
    rule_ = config.rule;
    version_ = version;
    first_w_ = blocks.front().w;
    in_ = in;
    out_ = out;
    for (int i = 0; i < 4; ++i) params_[i] = shape[i];
}

void AffineRule::run(MI355XBackend* be, const LRPRuleConfig& config, uint64_t version,
                     const std::vector<RuleBlock>& blocks, const Pass& p, const ResidualSplit& split) {
    if (blocks.empty()) throw std::logic_error("AffineRule::run: a layer needs at least one weight block");
    int64_t out = 0;
    for (const RuleBlock& b : blocks) out += b.cols;
    const int64_t rows = p.rows, in = p.in;
    if (rows == 0) return;
    ensure_weights(be, config, version, blocks, in, out);
    const pxk_rule_params rp = params_of(config);
    void* st = be->stream();
    const bool zbox = config.rule == LRPRule::ZBox;
    const int64_t wo = zbox ? out : 2 * out;  // W2's width: the GEMMs' output (den) or reduction (C) extent
    float* g = den_.ensure(be, rows * wo);
    if (!zbox) {
        // den = [x+ | x-] W2: both stabilised denominators of every output in one GEMM.
        float* xs = xs_.ensure(be, rows * 2 * in);
        MI355XBackend::check(pxk_lrp_sign_split(p.x, p.ldx, rows, in, xs, st), "lrp rule sign split");
        pxk_gemm_desc d = gemm_desc(rows, wo, 2 * in);
        d.a = mat(xs, 2 * in);
        d.b = mat(w2_.data(), wo);
        d.c = mat(g, wo);
        be->run_gemm(d);
    }
    MI355XBackend::check(pxk_lrp_rule_divide(&rp, p.r, p.ldr, p.r_cols, g, wo, p.z, p.ldz, p.bias, b2_.data(), rows,
                                             out, g, wo, st),
                         "lrp rule divide");
    // C = g W2^T: every backward product of the rule side by side (2 in wide).
    float* c = c_.ensure(be, rows * 2 * in);
    {
        pxk_gemm_desc d = gemm_desc(rows, 2 * in, wo);
        d.trans_b = 1;
        d.a = mat(g, wo);
        d.b = mat(w2_.data(), wo);
        d.c = mat(c, 2 * in);
        be->run_gemm(d);
    }
    if (split.b_den)
        throw std::logic_error("AffineRule: a rule's residual split cannot divide by the next layer's denominator");
    if (split.requested()) {
        MI355XBackend::check(pxk_lrp_rule_combine(rp.rule, p.x, p.ldx, c, 2 * in, p.add, rows, in, split.r_a, in,
                                                  split.a, split.b, split.s, split.r_b, config.epsilon, st),
                             "lrp rule combine");
    } else {
        MI355XBackend::check(pxk_lrp_rule_combine(rp.rule, p.x, p.ldx, c, 2 * in, p.add, rows, in, p.r_in, in,
                                                  nullptr, nullptr, nullptr, nullptr, config.epsilon, st),
                             "lrp rule combine");
    }
}

void AffineRule::release() {
    w2_.release();
    b2_.release();
    xs_.release();
    den_.release();
    c_.release();
    built_ = false;
}

}  // namespace pulsatrix::detail
