// SwiGLUModule and TransformerBlock on MI355XBackend.
#include <stdexcept>

#include "pulsatrix/rms_norm_module.hpp"
#include "pulsatrix/swiglu_module.hpp"
#include "pulsatrix/transformer_block.hpp"

namespace pulsatrix {

using detail::gemm_desc;
using detail::mat;

// ---- SwiGLUModule (src/swiglu_module.cpp) ----------------------------------------------------------

SwiGLUModule::SwiGLUModule(int64_t d_model, int64_t d_ff, DeviceBackend* backend, bool use_bias,
                           GatedActivation activation)
    : d_(d_model),
      F_(d_ff),
      use_bias_(use_bias),
      be_(detail::require_mi355x(backend, "SwiGLUModule")),
      gate_proj_(d_model, d_ff, backend, use_bias),
      up_proj_(d_model, d_ff, backend, use_bias),
      down_proj_(d_ff, d_model, backend, use_bias),
      act_(activation == GatedActivation::GeluTanh ? 1 : 0) {}

void SwiGLUModule::pack_weights() {
    const uint64_t v = gate_proj_.version() + up_proj_.version();
    if (v == packed_version_ && wgu_.size() > 0) return;
    float* w = wgu_.ensure(be_, d_ * 2 * F_);  // [W_gate | W_up], (d, 2F)
    be_->copy_2d(w, 2 * F_, gate_proj_.weight_data(), F_, d_, F_);
    be_->copy_2d(w + F_, 2 * F_, up_proj_.weight_data(), F_, d_, F_);
    if (use_bias_) {
        float* b = bgu_.ensure(be_, 2 * F_);
        be_->copy_2d(b, 2 * F_, gate_proj_.bias_data(), F_, 1, F_);
        be_->copy_2d(b + F_, 2 * F_, up_proj_.bias_data(), F_, 1, F_);
    }
    if (fused_gate()) {
        // The forward's copy: 32-column blocks alternate gate and up (block 2b = gate features
        // 32b..32b+31, block 2b+1 = the same up features), so one GEMM tile holds both factors of
        // its hidden features and applies the gate in its epilogue (PXK_EPI_SWIGLU_FWD). Seen as
        // d * F / 32 rows of 32 floats, the source blocks are 32 apart and their places 64 apart,
        // so each projection is one strided copy.
        float* wi = wgu_il_.ensure(be_, d_ * 2 * F_);
        be_->copy_2d(wi, 64, gate_proj_.weight_data(), 32, d_ * F_ / 32, 32);
        be_->copy_2d(wi + 32, 64, up_proj_.weight_data(), 32, d_ * F_ / 32, 32);
    }
    packed_version_ = v;
}

// The gate/up GEMM's weight (interleaved for the fused gate, else [Wgate | Wup]) with row k scaled
// by the norm's gamma[k] (PXK_PRO_RMS). Rebuilt when the projections or the norm's scale change.
const float* SwiGLUModule::folded_weights(RMSNormModule* norm) {
    if (wg_norm_ != norm || wg_version_ != norm->version() || wg_packed_ != packed_version_ || wgu_g_.size() == 0) {
        const int64_t f2 = 2 * F_;
        float* w = wgu_g_.ensure(be_, d_ * f2);
        MI355XBackend::check(pxk_scale_rows(fused_gate() ? wgu_il_.data() : wgu_.data(), norm->effective_gamma(), w,
                                            d_, f2, be_->stream()),
                             "SwiGLUModule::forward");
        wg_norm_ = norm;
        wg_version_ = norm->version();
        wg_packed_ = packed_version_;
    }
    return wgu_g_.data();
}

const float* SwiGLUModule::output() const noexcept { return use_bias_ ? down_y_.data() : down_z_.data(); }

const float* SwiGLUModule::run_forward(const float* x, int64_t rows, const float* resid, float* resid_out,
                                       RMSNormModule* norm) {
    pack_weights();
    x_ = x;
    norm_in_ = norm;
    rows_ = rows;
    // the block's pre-norm applied by the gate/up GEMM: gamma in the weights, x / rms per row
    auto fold = [&](pxk_gemm_desc& d) {
        if (!norm) return;
        d.prologue = PXK_PRO_RMS;
        d.b = mat(folded_weights(norm), 2 * F_);
        d.norm_eps = norm->eps();
        d.row_rms = norm->fold(rows);
    };
    const int64_t f2 = 2 * F_;
    float* gz = gu_z_.ensure(be_, rows * f2);
    float* gy = gz;
    float* gp = gate_post_.ensure(be_, rows * F_);
    float* h = hidden_.ensure(be_, rows * F_);
    if (fused_gate()) {  // gate and up projections and the gate itself in one GEMM
        pxk_gemm_desc d = gemm_desc(rows, f2, d_);
        d.a = mat(x, d_);
        d.b = mat(wgu_il_.data(), f2);
        d.c = mat(gz, f2);
        d.c2 = mat(h, F_);
        d.c3 = mat(gp, F_);
        d.epilogue = PXK_EPI_SWIGLU_FWD;
        d.gate_act = act_;
        fold(d);
        be_->run_gemm(d);
    } else {  // gate and up projections in one GEMM, then the gate
        pxk_gemm_desc d = gemm_desc(rows, f2, d_);
        d.a = mat(x, d_);
        d.b = mat(wgu_.data(), f2);
        d.c = mat(gz, f2);
        if (use_bias_) {
            gy = gu_y_.ensure(be_, rows * f2);
            d.epilogue = PXK_EPI_STORE_BIAS;
            d.c2 = mat(gy, f2);
            d.e_bias = mat(bgu_.data(), 0);
        }
        fold(d);
        be_->run_gemm(d);
        MI355XBackend::check(pxk_swiglu_forward(gy, f2, gp, h, rows, F_, act_, be_->stream()), "SwiGLUModule::forward");
    }
    float* dz = down_z_.ensure(be_, rows * d_);
    float* dy = use_bias_ ? down_y_.ensure(be_, rows * d_) : dz;
    {
        pxk_gemm_desc d = gemm_desc(rows, d_, F_);
        d.a = mat(h, F_);
        d.b = mat(down_proj_.weight_data(), d_);
        d.c = mat(dz, d_);
        if (use_bias_) {
            d.c2 = mat(dy, d_);
            d.e_bias = mat(down_proj_.bias_data(), 0);
        }
        if (resid) {
            d.epilogue = PXK_EPI_ADD_RESID;
            d.x = mat(resid, d_);
            d.c3 = mat(resid_out, d_);
        } else {
            d.epilogue = use_bias_ ? PXK_EPI_STORE_BIAS : PXK_EPI_STORE;
        }
        be_->run_gemm(d);
    }
    return dy;
}

void SwiGLUModule::relevance_denominator(const LRPRuleConfig& config, const float** den, const float** bias) const {
    *den = down_z_.data();
    *bias = detail::rule_bias(down_proj_.bias_data(), use_bias_, config.epsilon_bias_in_denominator);
}

const float* SwiGLUModule::run_relevance(const float* relevance_out, const LRPRuleConfig& config, const float* add,
                                         const detail::ResidualSplit& split, bool divided) {
    if (x_ == nullptr) throw std::logic_error("SwiGLUModule::propagate_relevance: called before any forward()");
    detail::validate_rule(config, "LinearModule");  // the projections validate it (linear_module.cpp:342)
    const bool bid = config.epsilon_bias_in_denominator;
    const int64_t rows = rows_, f2 = 2 * F_;
    const float* gz = gu_z_.data();
    const float* gy = use_bias_ ? gu_y_.data() : gz;
    if (detail::is_affine_rule(config)) {
        if (divided) throw std::logic_error("SwiGLUModule::propagate_relevance: a divided relevance under a rule");
        return run_relevance_rule(relevance_out, config, add, split);
    }
    float* g = g_.ensure(be_, rows * f2);
    {  // down projection's rule, Eq. 15's gate * up split and both projections' denominators
        pxk_gemm_desc d = gemm_desc(rows, F_, d_);
        d.trans_b = 1;
        d.epilogue = PXK_EPI_SWIGLU_REL;
        d.eps = config.epsilon;
        d.a = mat(relevance_out, d_);
        if (!divided) {  // else the producer of relevance_out already divided it by stab(z + bias)
            d.prologue = PXK_PRO_DIV_STAB;
            d.z = mat(down_z_.data(), d_);
            if (const float* bd = detail::rule_bias(down_proj_.bias_data(), use_bias_, bid)) d.z_bias = mat(bd, 0);
        }
        d.b = mat(down_proj_.weight_data(), d_);
        d.c = mat(g, f2);
        d.c2 = mat(g + F_, f2);
        d.z2 = mat(gz, f2);
        d.z3 = mat(gz + F_, f2);
        if (use_bias_) {
            d.x = mat(hidden_.data(), F_);
            d.y = mat(gate_post_.data(), F_);
            d.w = mat(gy + F_, f2);
        } else {  // the epilogue recomputes gate_post, up and hidden from the two z
            d.gate_act = act_;
        }
        if (use_bias_ && bid) {
            d.e_bias = mat(gate_proj_.bias_data(), 0);
            d.e_bias2 = mat(up_proj_.bias_data(), 0);
        }
        be_->run_gemm(d);
    }
    float* r_in = r_in_.ensure(be_, rows * d_);
    {  // gate and up projections' input relevance in one GEMM: x * ([g_gate | g_up] [W_gate | W_up]^T)
        pxk_gemm_desc d = gemm_desc(rows, d_, f2);
        d.trans_b = 1;
        d.epilogue = PXK_EPI_MUL_X;
        d.a = mat(g, f2);
        d.b = mat(wgu_.data(), f2);
        d.c = mat(r_in, d_);
        d.x = mat(x_, d_);
        if (norm_in_) {  // x_ is the folded norm's input: the epilogue forms its output from the rms
            d.x_rms = norm_in_->rms();
            d.x_gamma = norm_in_->effective_gamma();
        }
        if (add) d.y = mat(add, d_);
        detail::apply_split(d, split, d_, config.epsilon);
        be_->run_gemm(d);
    }
    return split.requested() ? nullptr : r_in;
}

// Gamma / AlphaBeta / ZBox (swiglu_module.cpp:139-170): the down projection's rule, Eq. 15's
// share of gate * up for both factors, then the rule over the packed gate | up projections with
// that one share as the relevance of both halves.
const float* SwiGLUModule::run_relevance_rule(const float* relevance_out, const LRPRuleConfig& config,
                                              const float* add, const detail::ResidualSplit& split) {
    const int64_t rows = rows_, f2 = 2 * F_;
    const float* gz = gu_z_.data();
    const float* gy = use_bias_ ? gu_y_.data() : gz;
    void* st = be_->stream();
    float* rh = g_.ensure(be_, rows * f2);  // r_hidden, then the product's share
    float* up = rh + rows * F_;             // the up projection's output, contiguous
    const float* bd = use_bias_ ? down_proj_.bias_data() : nullptr;
    down_rule_.run(be_, config, down_proj_.version(), {{down_proj_.weight_data(), d_, d_, false, bd}},
                   {hidden_.data(), F_, rows, F_, down_z_.data(), d_, bd, relevance_out, d_, d_, rh, nullptr});
    be_->copy_2d(up, F_, gy + F_, f2, static_cast<size_t>(rows), static_cast<size_t>(F_));
    MI355XBackend::check(pxk_lrp_bilinear_elementwise(gate_post_.data(), up, rh, rh, rows * F_, config.epsilon, st),
                         "SwiGLUModule::propagate_relevance");
    float* r_in = r_in_.ensure(be_, rows * d_);
    const float* bg = use_bias_ ? gate_proj_.bias_data() : nullptr;
    const float* bu = use_bias_ ? up_proj_.bias_data() : nullptr;
    gate_up_rule_.run(be_, config, gate_proj_.version() + up_proj_.version(),
                      {{gate_proj_.weight_data(), F_, F_, false, bg}, {up_proj_.weight_data(), F_, F_, false, bu}},
                      {norm_in_ ? norm_in_->materialize(x_) : x_, d_, rows, d_, gz, f2, use_bias_ ? bgu_.data() : nullptr,
                       rh, F_, F_, r_in, add},
                      split);
    return split.requested() ? nullptr : r_in;
}

Tensor SwiGLUModule::forward_impl(const Tensor& input) {
    if (input.rank() < 2 || input.shape().dim(static_cast<size_t>(input.rank() - 1)) != d_)
        throw std::invalid_argument("SwiGLUModule::forward: input must be rank >= 2 with final dimension d_model");
    last_shape_ = input.shape();
    const float* out = run_forward(detail::keep_input(be_, x_copy_, input), input.numel() / d_);
    return detail::copy_out(be_, out, last_shape_);
}

Tensor SwiGLUModule::propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) {
    if (x_ == nullptr) throw std::logic_error("SwiGLUModule::propagate_relevance: called before any forward()");
    if (relevance_out.shape() != last_shape_)
        throw std::invalid_argument("SwiGLUModule::propagate_relevance: relevance_out must match the cached forward shape");
    return detail::copy_out(be_, run_relevance(relevance_out.data(), config), last_shape_);
}

// ---- TransformerBlock (src/transformer_block.cpp) ------------------------------------------------

TransformerBlock::TransformerBlock(const AttentionConfig& attention, int64_t d_ff, DeviceBackend* backend,
                                   const TransformerBlockOptions& options)
    : d_(attention.d_model),
      be_(detail::require_mi355x(backend, "TransformerBlock")),
      norm1_(attention.d_model > 0 ? attention.d_model : 1, backend, DeviceType::Hip, options.norm_eps),
      mha_(attention, backend),
      norm2_(attention.d_model > 0 ? attention.d_model : 1, backend, DeviceType::Hip, options.norm_eps),
      swiglu_(attention.d_model, d_ff, backend, options.mlp_bias, options.mlp_activation) {
    norm1_.set_weight_offset(options.norm_weight_offset);
    norm2_.set_weight_offset(options.norm_weight_offset);
    if (options.post_norms) {  // transformer_block.cpp:60-80
        post_attn_norm_ = std::make_unique<RMSNormModule>(d_, backend, DeviceType::Hip, options.norm_eps);
        post_mlp_norm_ = std::make_unique<RMSNormModule>(d_, backend, DeviceType::Hip, options.norm_eps);
        post_attn_norm_->set_weight_offset(options.norm_weight_offset);
        post_mlp_norm_->set_weight_offset(options.norm_weight_offset);
    }
}

RMSNormModule& TransformerBlock::post_attn_norm() {
    if (!post_attn_norm_) throw std::logic_error("TransformerBlock::post_attn_norm: the block has no sandwich norms");
    return *post_attn_norm_;
}

RMSNormModule& TransformerBlock::post_mlp_norm() {
    if (!post_mlp_norm_) throw std::logic_error("TransformerBlock::post_mlp_norm: the block has no sandwich norms");
    return *post_mlp_norm_;
}

TransformerBlock::TransformerBlock(int64_t d_model, int64_t num_heads, int64_t d_ff, DeviceBackend* backend,
                                   bool use_rope, bool use_qk_norm)
    : d_(d_model),
      be_(detail::require_mi355x(backend, "TransformerBlock")),
      norm1_(d_model, backend),
      mha_(d_model, num_heads, backend, use_rope, use_qk_norm),
      norm2_(d_model, backend),
      swiglu_(d_model, d_ff, backend) {}

const float* TransformerBlock::run_forward(const float* x, int64_t n, int64_t l) {
    N_ = n;
    L_ = l;
    x_ = x;
    const int64_t M = n * l;
    float* y1 = y1_.ensure(be_, M * d_);
    float* y2 = y2_.ensure(be_, M * d_);
    // Each pre-norm is applied by the projection GEMM that reads it (RMSNormModule::fold), except
    // for a handful of rows, where the skinny kernels of the unfused path are faster.
    const bool fold = M > 16;
    if (!post_attn_norm_) {
        if (fold) {
            mha_.run_forward(x, n, l, x, y1, &norm1_);          // y1 = x + attn(norm1(x))
            swiglu_.run_forward(y1, M, y1, y2, &norm2_);        // y2 = y1 + mlp(norm2(y1))
        } else {
            mha_.run_forward(norm1_.run_forward(x, M), n, l, x, y1);
            swiglu_.run_forward(norm2_.run_forward(y1, M), M, y1, y2);
        }
        attn_out_ = mha_.output();
        ffn_out_ = swiglu_.output();
        return y2;
    }
    // Sandwich norms: y1 = x + post_attn_norm(attn(norm1(x))), y2 = y1 + post_mlp_norm(mlp(norm2(y1))).
    void* st = be_->stream();
    attn_out_ = post_attn_norm_->run_forward(
        fold ? mha_.run_forward(x, n, l, nullptr, nullptr, &norm1_) : mha_.run_forward(norm1_.run_forward(x, M), n, l), M);
    MI355XBackend::check(pxk_add(x, attn_out_, y1, M * d_, st), "TransformerBlock::forward");
    ffn_out_ = post_mlp_norm_->run_forward(
        fold ? swiglu_.run_forward(y1, M, nullptr, nullptr, &norm2_) : swiglu_.run_forward(norm2_.run_forward(y1, M), M),
        M);
    MI355XBackend::check(pxk_add(y1, ffn_out_, y2, M * d_, st), "TransformerBlock::forward");
    return y2;
}

void SwiGLUModule::reserve_forward(int64_t rows) {
    gu_z_.ensure(be_, rows * 2 * F_);
    if (use_bias_) gu_y_.ensure(be_, rows * 2 * F_);
    gate_post_.ensure(be_, rows * F_);
    hidden_.ensure(be_, rows * F_);
    down_z_.ensure(be_, rows * d_);
    if (use_bias_) down_y_.ensure(be_, rows * d_);
}

void SwiGLUModule::replicate_forward(int64_t copies) {
    const char* who = "SwiGLUModule::replicate_forward";
    gu_z_.repeat(be_, rows_ * 2 * F_, copies, who);
    if (use_bias_) gu_y_.repeat(be_, rows_ * 2 * F_, copies, who);
    gate_post_.repeat(be_, rows_ * F_, copies, who);
    hidden_.repeat(be_, rows_ * F_, copies, who);
    down_z_.repeat(be_, rows_ * d_, copies, who);
    if (use_bias_) down_y_.repeat(be_, rows_ * d_, copies, who);
    rows_ *= copies;
}

void TransformerBlock::reserve_forward(int64_t n, int64_t l) {
    const int64_t M = n * l;
    norm1_.reserve_forward(M);
    mha_.reserve_forward(n, l);
    norm2_.reserve_forward(M);
    swiglu_.reserve_forward(M);
    if (post_attn_norm_) {
        post_attn_norm_->reserve_forward(M);
        post_mlp_norm_->reserve_forward(M);
    }
    y1_.ensure(be_, M * d_);
    y2_.ensure(be_, M * d_);
}

void TransformerBlock::replicate_forward(int64_t copies) {
    const int64_t M = N_ * L_;
    norm1_.replicate_forward(copies);
    mha_.replicate_forward(copies);
    norm2_.replicate_forward(copies);
    swiglu_.replicate_forward(copies);
    if (post_attn_norm_) {
        post_attn_norm_->replicate_forward(copies);
        post_mlp_norm_->replicate_forward(copies);
    }
    y1_.repeat(be_, M * d_, copies, "TransformerBlock::replicate_forward");
    y2_.repeat(be_, M * d_, copies, "TransformerBlock::replicate_forward");
    N_ *= copies;
}

const float* TransformerBlock::decode_step(const float* x, const float* x_normed, int64_t n, KVCacheState& cache,
                                          const int32_t* pos, RMSNormModule* next_norm, const float** next_normed) {
    float* y1 = dec_y1_.ensure(be_, n * d_);
    float* y2 = dec_y2_.ensure(be_, n * d_);
    const float* xn = x_normed ? x_normed : norm1_.run_forward(x, n);
    if (next_normed) *next_normed = nullptr;
    if (!post_attn_norm_) {
        mha_.decode_step(xn, n, cache, pos, x, y1);
        swiglu_.run_forward(norm2_.run_forward(y1, n), n, y1, y2);
        return y2;
    }
    // Each sublayer's post-norm, its residual add and the norm that reads the sum next run as one
    // row kernel: y1 = x + post_attn_norm(attn) with norm2(y1), then y2 = y1 + post_mlp_norm(mlp)
    // with the caller's next norm (the next block's norm1 or the final norm) of y2.
    void* st = be_->stream();
    const float* a = mha_.decode_step(xn, n, cache, pos);
    float* n2 = dec_n2_.ensure(be_, n * d_);
    MI355XBackend::check(pxk_rms_norm_add(x, a, post_attn_norm_->effective_gamma(), post_attn_norm_->eps(), y1,
                                          norm2_.effective_gamma(), norm2_.eps(), n2, n, d_, st),
                         "TransformerBlock::decode_step");
    const float* f = swiglu_.run_forward(n2, n);
    float* nn = next_norm && next_normed ? dec_next_.ensure(be_, n * d_) : nullptr;
    MI355XBackend::check(pxk_rms_norm_add(y1, f, post_mlp_norm_->effective_gamma(), post_mlp_norm_->eps(), y2,
                                          nn ? next_norm->effective_gamma() : nullptr, nn ? next_norm->eps() : 0.0f, nn,
                                          n, d_, st),
                         "TransformerBlock::decode_step");
    if (nn) *next_normed = nn;
    return y2;
}

detail::ResidualSplit TransformerBlock::output_split(const LRPRuleConfig* divide_for) {
    const int64_t n = N_ * L_ * d_;
    detail::ResidualSplit sp{y1_.data(), ffn_out_, y2_.data(), r_y1d_.ensure(be_, n), r_ffn_.ensure(be_, n)};
    r_ffn_divided_ = divide_for != nullptr && !detail::is_affine_rule(*divide_for);
    if (r_ffn_divided_) swiglu_.relevance_denominator(*divide_for, &sp.b_den, &sp.b_den_bias);
    return sp;
}

const float* TransformerBlock::run_relevance_split(const LRPRuleConfig& config, const detail::ResidualSplit& below) {
    if (x_ == nullptr) throw std::logic_error("TransformerBlock::propagate_relevance: called before any forward()");
    const int64_t n = N_ * L_ * d_;
    // The producer of this block's output relevance wrote its two shares (output_split). The MLP's
    // last GEMM writes the split one level up (y1 = x + attn) the same way.
    float* rxd = r_xd_.ensure(be_, n);
    float* rattn = r_attn_.ensure(be_, n);
    // The sandwich norms pass relevance unchanged (PostNormRelevance, transformer_block.cpp:92-95).
    // Under an epsilon rule the MLP's last GEMM writes the attention's share already divided by
    // the output projection's denominator, so that projection's relevance GEMM has no prologue.
    detail::ResidualSplit up{x_, attn_out_, y1_.data(), rxd, rattn};
    const bool divide = !detail::is_affine_rule(config);
    if (divide) mha_.relevance_denominator(config, &up.b_den, &up.b_den_bias);
    swiglu_.run_relevance(r_ffn_.data(), config, r_y1d_.data(), up, r_ffn_divided_);
    return mha_.run_relevance(rattn, config, rxd, below, divide);
}

const float* TransformerBlock::run_relevance(const float* relevance_out, const LRPRuleConfig& config) {
    if (x_ == nullptr) throw std::logic_error("TransformerBlock::propagate_relevance: called before any forward()");
    const int64_t M = N_ * L_, n = M * d_;
    void* st = be_->stream();
    // y2 = y1 + ffn: epsilon split, the MLP's relevance (RMSNorm's rule is the identity), then
    // r_y1 = r_y1_direct + r_from_norm2 fused into the MLP's last GEMM.
    float* ry1d = r_y1d_.ensure(be_, n);
    float* rffn = r_ffn_.ensure(be_, n);
    MI355XBackend::check(pxk_lrp_residual_split(y1_.data(), ffn_out_, relevance_out, ry1d, rffn, n,
                                                config.epsilon, st),
                         "TransformerBlock::propagate_relevance");
    const float* ry1 = swiglu_.run_relevance(rffn, config, ry1d);
    // y1 = x + attn: the same one level up.
    float* rxd = r_xd_.ensure(be_, n);
    float* rattn = r_attn_.ensure(be_, n);
    MI355XBackend::check(pxk_lrp_residual_split(x_, attn_out_, ry1, rxd, rattn, n, config.epsilon, st),
                         "TransformerBlock::propagate_relevance");
    return mha_.run_relevance(rattn, config, rxd);
}

Tensor TransformerBlock::forward_impl(const Tensor& input) {
    if (input.rank() != 3 || input.shape().dim(2) != d_)
        throw std::invalid_argument("TransformerBlock::forward: input must be rank-3 (N, L, d_model)");
    last_shape_ = input.shape();
    const float* out = run_forward(detail::keep_input(be_, x_copy_, input), input.shape().dim(0), input.shape().dim(1));
    return detail::copy_out(be_, out, last_shape_);
}

Tensor TransformerBlock::propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) {
    if (x_ == nullptr) throw std::logic_error("TransformerBlock::propagate_relevance: called before any forward()");
    if (relevance_out.shape() != last_shape_)
        throw std::invalid_argument(
            "TransformerBlock::propagate_relevance: relevance_out must match the cached forward shape");
    return detail::copy_out(be_, run_relevance(relevance_out.data(), config), last_shape_);
}

}  // namespace pulsatrix
