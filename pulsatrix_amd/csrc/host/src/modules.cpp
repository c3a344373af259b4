// LinearModule, RMSNormModule, EmbeddingModule and TiedLMHeadModule on MI355XBackend.
#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

#include "pulsatrix/embedding_module.hpp"
#include "pulsatrix/linear_module.hpp"
#include "pulsatrix/rms_norm_module.hpp"
#include "pulsatrix/tied_lm_head_module.hpp"

namespace pulsatrix {

using detail::gemm_desc;
using detail::mat;

namespace detail {

/** @brief A fresh tensor holding a copy of n device floats (the reference returns new tensors). */
Tensor copy_out(MI355XBackend* be, const float* src, Shape shape) {
    Tensor t = Tensor::uninitialized(std::move(shape), be);
    if (t.numel() > 0) be->copy(t.data(), src, static_cast<size_t>(t.numel()) * sizeof(float), CopyDirection::DeviceToDevice);
    return t;
}

/** @brief Copies a caller's tensor into a module buffer (the module keeps its input for relevance). */
const float* keep_input(MI355XBackend* be, DevBuf& buf, const Tensor& t) {
    float* p = buf.ensure(be, t.numel());
    be->copy(p, t.data(), static_cast<size_t>(t.numel()) * sizeof(float), CopyDirection::DeviceToDevice);
    return p;
}

void DevBuf::repeat(MI355XBackend* be, int64_t count, int64_t copies, const char* who) {
    if (copies <= 1) return;
    if (t_.numel() < count * copies)
        throw std::logic_error(std::string(who) + ": no storage for " + std::to_string(copies) + " copies");
    MI355XBackend::check(pxk_repeat_block(t_.data(), count, copies, be->stream()), who);
    n_ = count * copies;
}

}  // namespace detail

// ---- LinearModule (src/linear_module.cpp) ----------------------------------------------------------

LinearModule::LinearModule(int64_t in_features, int64_t out_features, DeviceBackend* backend, bool use_bias)
    : in_(in_features),
      out_(out_features),
      use_bias_(use_bias),
      be_(detail::require_mi355x(backend, "LinearModule")),
      weight_(Shape({in_features, out_features}), backend),
      bias_(Shape({out_features}), backend) {
    if (in_features <= 0 || out_features <= 0)
        throw std::invalid_argument("LinearModule: in_features and out_features must be positive");
}

void LinearModule::set_weight(const std::vector<float>& values) {
    weight_ = Tensor(weight_.shape(), be_, values);
    ++version_;
}

void LinearModule::set_bias(const std::vector<float>& values) {
    if (!use_bias_) throw std::logic_error("LinearModule::set_bias: this layer was built without a bias");
    bias_ = Tensor(bias_.shape(), be_, values);
    ++version_;
}

const float* LinearModule::run_forward(const float* x, int64_t rows) {
    x_ = x;
    rows_ = rows;
    float* z = z_.ensure(be_, rows * out_);
    pxk_gemm_desc d = gemm_desc(rows, out_, in_);
    d.a = mat(x, in_);
    d.b = mat(weight_.data(), out_);
    d.c = mat(z, out_);
    d.epilogue = PXK_EPI_STORE;
    float* y = z;
    if (use_bias_) {
        y = y_.ensure(be_, rows * out_);
        d.epilogue = PXK_EPI_STORE_BIAS;
        d.c2 = mat(y, out_);
        d.e_bias = mat(bias_.data(), 0);
    }
    be_->run_gemm(d);
    return y;
}

const float* LinearModule::run_relevance(const float* r, const LRPRuleConfig& config, const float* add,
                                         const detail::ResidualSplit& split) {
    if (x_ == nullptr) throw std::logic_error("LinearModule::propagate_relevance: called before any forward()");
    detail::validate_rule(config, "LinearModule");
    float* out = r_in_.ensure(be_, rows_ * in_);
    if (detail::is_affine_rule(config)) {  // lrp_rules::apply (lrp_rules.cpp:177-195)
        const float* b = use_bias_ ? bias_.data() : nullptr;
        rule_.run(be_, config, version_, {{weight_.data(), out_, out_, false, b}},
                  {x_, in_, rows_, in_, z_.data(), out_, b, r, out_, out_, out, add}, split);
        return split.requested() ? nullptr : out;
    }
    pxk_gemm_desc d = gemm_desc(rows_, in_, out_);
    d.trans_b = 1;
    d.prologue = PXK_PRO_DIV_STAB;
    d.epilogue = PXK_EPI_MUL_X;
    d.eps = config.epsilon;
    d.a = mat(r, out_);
    d.z = mat(z_.data(), out_);
    if (const float* b = detail::rule_bias(bias_.data(), use_bias_, config.epsilon_bias_in_denominator))
        d.z_bias = mat(b, 0);
    d.b = mat(weight_.data(), out_);
    d.c = mat(out, in_);
    d.x = mat(x_, in_);
    if (add) d.y = mat(add, in_);
    detail::apply_split(d, split, in_, config.epsilon);
    be_->run_gemm(d);
    return split.requested() ? nullptr : out;
}

Tensor LinearModule::forward_impl(const Tensor& input) {
    if (input.rank() != 2 || input.shape().dim(1) != in_)
        throw std::invalid_argument("LinearModule::forward: input must be rank-2 (N, in_features)");
    const int64_t n = input.shape().dim(0);
    const float* y = run_forward(detail::keep_input(be_, x_copy_, input), n);
    return detail::copy_out(be_, y, Shape({n, out_}));
}

Tensor LinearModule::propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) {
    require_device(relevance_out, DeviceType::Hip, "LinearModule::propagate_relevance");
    if (x_ == nullptr) throw std::logic_error("LinearModule::propagate_relevance: called before any forward()");
    if (relevance_out.rank() != 2 || relevance_out.shape().dim(0) != rows_ || relevance_out.shape().dim(1) != out_)
        throw std::invalid_argument(
            "LinearModule::propagate_relevance: relevance_out must be rank-2 (N, out_features) matching the cached "
            "batch size");
    return detail::copy_out(be_, run_relevance(relevance_out.data(), config), Shape({rows_, in_}));
}

// ---- RMSNormModule (src/rms_norm_module.cpp) -----------------------------------------------------

RMSNormModule::RMSNormModule(int64_t num_features, DeviceBackend* backend, DeviceType, float eps)
    : d_(num_features),
      eps_(eps),
      be_(detail::require_mi355x(backend, "RMSNormModule")),
      gamma_(Shape({num_features > 0 ? num_features : 1}), backend) {
    if (num_features <= 0) throw std::invalid_argument("RMSNormModule: num_features must be positive");
}

void RMSNormModule::set_gamma(const std::vector<float>& values) {
    gamma_ = Tensor(gamma_.shape(), be_, values);
    ++version_;
}

const float* RMSNormModule::effective_gamma() {
    if (offset_ == 0.0f) return gamma_.data();
    if (eff_version_ != version_ || eff_.size() != d_) {
        // EffectiveGamma (rms_norm_module.cpp:40-49): fill(offset), then add gamma, in float.
        float* e = eff_.ensure(be_, d_);
        MI355XBackend::check(pxk_fill(e, offset_, d_, be_->stream()), "RMSNormModule::forward");
        MI355XBackend::check(pxk_add(e, gamma_.data(), e, d_, be_->stream()), "RMSNormModule::forward");
        eff_version_ = version_;
    }
    return eff_.data();
}

const float* RMSNormModule::run_forward(const float* x, int64_t rows) {
    rows_ = rows;
    folded_ = false;
    float* out = out_.ensure(be_, rows * d_);
    float* rms = rms_.ensure(be_, rows);
    const float* gamma = effective_gamma();
    const int64_t d = d_;
    const float eps = eps_;
    // x read, out written (8 B per element), one rms per row
    be_->launch("rms_norm", "rows", 0.0, 8.0 * rows * d + 4.0 * (rows + d), "RMSNormModule::forward",
                [=](void* st) { return pxk_rms_norm_forward(x, gamma, out, rms, rows, d, eps, st); });
    return out;
}

float* RMSNormModule::fold(int64_t rows) {
    rows_ = rows;
    folded_ = true;
    return rms_.ensure(be_, rows);
}

const float* RMSNormModule::materialize(const float* x) {
    if (!folded_) return out_.data();
    float* out = out_.ensure(be_, rows_ * d_);
    const float* gamma = effective_gamma();
    const int64_t rows = rows_, d = d_;
    const float eps = eps_;
    // The rms the folding GEMM wrote stays; the row kernel recomputes its own for the output.
    be_->launch("rms_norm", "rows", 0.0, 8.0 * rows * d + 4.0 * d, "RMSNormModule::forward", [=](void* st) {
        return pxk_rms_norm_forward(x, gamma, out, nullptr, rows, d, eps, st);
    });
    folded_ = false;
    return out;
}

void RMSNormModule::reserve_forward(int64_t rows) {
    out_.ensure(be_, rows * d_);
    rms_.ensure(be_, rows);
}

void RMSNormModule::replicate_forward(int64_t copies) {
    if (!folded_) out_.repeat(be_, rows_ * d_, copies, "RMSNormModule::replicate_forward");
    rms_.repeat(be_, rows_, copies, "RMSNormModule::replicate_forward");
    rows_ *= copies;
}

Tensor RMSNormModule::forward_impl(const Tensor& input) {
    if (input.rank() != 2 || input.shape().dim(1) != d_)
        throw std::invalid_argument("RMSNormModule::forward: input must be rank-2 (N, num_features)");
    const int64_t n = input.shape().dim(0);
    return detail::copy_out(be_, run_forward(input.data(), n), Shape({n, d_}));
}

Tensor RMSNormModule::propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig&) {
    if (rows_ == 0) throw std::logic_error("RMSNormModule::propagate_relevance: called before any forward()");
    if (relevance_out.numel() != rows_ * d_)
        throw std::invalid_argument(
            "RMSNormModule::propagate_relevance: relevance_out size must match the cached forward shape");
    return Tensor(relevance_out);  // the identity rule
}

// ---- EmbeddingModule (src/embedding_module.cpp) ----------------------------------------------------

EmbeddingModule::EmbeddingModule(int64_t num_embeddings, int64_t embedding_dim, DeviceBackend* backend)
    : V_(num_embeddings),
      d_(embedding_dim),
      be_(detail::require_mi355x(backend, "EmbeddingModule")),
      weight_(Shape({num_embeddings, embedding_dim}), backend) {
    if (num_embeddings <= 0 || embedding_dim <= 0)
        throw std::invalid_argument("EmbeddingModule: num_embeddings and embedding_dim must be positive");
}

void EmbeddingModule::set_weight(const std::vector<float>& values) {
    weight_ = Tensor(weight_.shape(), be_, values);
    ++version_;
}

void EmbeddingModule::reserve_forward(int64_t count) { out_.ensure(be_, count * d_); }

void EmbeddingModule::replicate_forward(int64_t copies) {
    const int64_t n = last_shape_.dim(0), l = last_shape_.dim(1);
    out_.repeat(be_, n * l * d_, copies, "EmbeddingModule::replicate_forward");
    last_shape_ = Shape({n * copies, l});
}

const float* EmbeddingModule::run_forward_device(const float* ids, int64_t n, int64_t l) {
    const int64_t count = n * l;
    last_shape_ = Shape({n, l});
    float* out = out_.ensure(be_, count * d_);
    // The ids are validated on the device (rounded, range-checked, out-of-range ones replaced by 0
    // and reported through ids_status()); the host never waits for them.
    float* checked = ids_checked_.ensure(be_, count);
    auto* status = reinterpret_cast<int32_t*>(ids_status_.ensure(be_, 1));
    const int64_t V = num_embeddings(), d = d_;
    const float* table = weight_.data();
    be_->launch("embedding_ids", "rows", 0.0, 8.0 * count, "EmbeddingModule::forward",
                [=](void* st) { return pxk_embedding_ids(ids, count, V, checked, status, st); });
    be_->launch("gather_rows", "rows", 0.0, 8.0 * count * d + 4.0 * count, "EmbeddingModule::forward",
                [=](void* st) { return pxk_gather_rows(table, checked, out, count, d, st); });
    return out;
}

bool EmbeddingModule::device_ids_valid() {
    if (ids_status_.size() == 0) return true;
    int32_t status = 0;
    be_->copy(&status, ids_status_.data(), sizeof(status), CopyDirection::DeviceToHost);
    return status == 0;
}

Tensor EmbeddingModule::forward_impl(const Tensor& input) {
    if (input.rank() != 2) throw std::invalid_argument("EmbeddingModule::forward: input must be rank-2 (N, L)");
    const int64_t n = input.shape().dim(0), l = input.shape().dim(1), count = n * l;
    // Host-side validation, as the reference does it (embedding_module.cpp:48-59).
    std::vector<float> raw = input.to_host_vector();
    for (float& v : raw) {
        const auto idx = static_cast<int64_t>(std::llround(static_cast<double>(v)));
        if (idx < 0 || idx >= V_)
            throw std::invalid_argument("EmbeddingModule::forward: index out of range [0, num_embeddings)");
        v = static_cast<float>(idx);
    }
    float* ids = ids_.ensure(be_, count);
    be_->copy(ids, raw.data(), raw.size() * sizeof(float), CopyDirection::HostToDevice);
    return detail::copy_out(be_, run_forward_device(ids, n, l), Shape({n, l, d_}));
}

void EmbeddingModule::token_relevance(const float* relevance, int64_t count, float* out) {
    const int64_t d = d_;
    be_->launch("row_sums", "rows", 0.0, 4.0 * count * (d + 1), "EmbeddingModule::propagate_relevance",
                [=](void* st) { return pxk_row_sums(relevance, out, count, d, st); });
}

Tensor EmbeddingModule::propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig&) {
    if (last_shape_.rank() != 2) throw std::logic_error("EmbeddingModule::propagate_relevance: called before any forward()");
    const int64_t n = last_shape_.dim(0), l = last_shape_.dim(1);
    if (relevance_out.numel() != n * l * d_)
        throw std::invalid_argument(
            "EmbeddingModule::propagate_relevance: relevance_out must be (N, L, embedding_dim) matching the cached "
            "forward shape");
    Tensor out = Tensor::uninitialized(last_shape_, be_);
    token_relevance(relevance_out.data(), n * l, out.data());
    return out;
}

// ---- TiedLMHeadModule (src/tied_lm_head_module.cpp) -------------------------------------------------

TiedLMHeadModule::TiedLMHeadModule(EmbeddingModule& embedding, DeviceBackend* backend)
    : embedding_(embedding), be_(detail::require_mi355x(backend, "TiedLMHeadModule")) {}

const float* TiedLMHeadModule::run_forward(const float* x, int64_t rows) {
    const int64_t V = embedding_.num_embeddings(), D = embedding_.embedding_dim();
    x_ = x;
    rows_ = rows;
    float* logits = logits_.ensure(be_, rows * V);
    pxk_gemm_desc d = gemm_desc(rows, V, D);
    d.trans_b = 1;  // E (V, D) read transposed in place
    d.a = mat(x, D);
    d.b = mat(embedding_.weight_data(), D);
    d.c = mat(logits, V);
    be_->run_gemm(d);
    return logits;
}

const float* TiedLMHeadModule::run_relevance(const float* relevance_out, const LRPRuleConfig& config,
                                             const detail::ResidualSplit& split) {
    if (x_ == nullptr) throw std::logic_error("TiedLMHeadModule::propagate_relevance: called before any forward()");
    detail::validate_rule(config, "TiedLMHeadModule");
    const int64_t V = embedding_.num_embeddings(), D = embedding_.embedding_dim();
    float* out = r_in_.ensure(be_, rows_ * D);
    if (detail::is_affine_rule(config)) {
        // The rules on W = E^T (read transposed in place) against a zero bias
        // (tied_lm_head_module.cpp:85-111).
        rule_.run(be_, config, embedding_.version(), {{embedding_.weight_data(), D, V, true, nullptr}},
                  {x_, D, rows_, D, logits_.data(), V, nullptr, relevance_out, V, V, out, nullptr}, split);
        return split.requested() ? nullptr : out;
    }
    // z = logits + 0 bias; g = R / stab(z); r_in = x * (g E): K = V, split-K across the chip.
    pxk_gemm_desc d = gemm_desc(rows_, D, V);
    d.prologue = PXK_PRO_DIV_STAB;
    d.epilogue = PXK_EPI_MUL_X;
    d.eps = config.epsilon;
    d.a = mat(relevance_out, V);
    d.z = mat(logits_.data(), V);
    d.b = mat(embedding_.weight_data(), D);
    d.c = mat(out, D);
    d.x = mat(x_, D);
    detail::apply_split(d, split, D, config.epsilon);
    be_->run_gemm(d);
    return split.requested() ? nullptr : out;
}

const float* TiedLMHeadModule::run_seeded_relevance(int64_t n, int64_t l, const int64_t* targets_in,
                                                    int64_t* targets_out, bool unit_seed, const LRPRuleConfig& config,
                                                    const detail::ResidualSplit& split) {
    if (x_ == nullptr) throw std::logic_error("TiedLMHeadModule::propagate_relevance: called before any forward()");
    detail::validate_rule(config, "TiedLMHeadModule");
    if (detail::is_affine_rule(config))
        throw std::invalid_argument("TiedLMHeadModule::run_seeded_relevance: epsilon rules only");
    if (n * l != rows_) throw std::invalid_argument("TiedLMHeadModule::run_seeded_relevance: n * l must match the forward");
    const int64_t V = embedding_.num_embeddings(), D = embedding_.embedding_dim();
    pxk_seed_head_desc d{};
    d.logits = logits_.data();
    d.x = x_;
    d.e = embedding_.weight_data();
    d.n = n;
    d.l = l;
    d.vocab = V;
    d.d = D;
    d.eps = config.epsilon;
    d.unit = unit_seed;
    d.targets_out = targets_out;
    float* out = nullptr;
    if (split.requested()) {
        d.a = split.a;
        d.b = split.b;
        d.s = split.s;
        d.r_a = split.r_a;
        d.r_b = split.r_b;
        d.b_den = split.b_den;
        d.b_den_bias = split.b_den_bias;
    } else {
        out = r_in_.ensure(be_, rows_ * D);
        d.r = out;
    }
    // one scan of each sequence's last logit row, then every row of the relevance written once
    // (the seeded row also reads its logit and E's target row)
    const std::vector<int64_t> given = targets_in ? std::vector<int64_t>(targets_in, targets_in + n) : std::vector<int64_t>();
    const double bytes = 4.0 * (n * V + (split.requested() ? 2 : 1) * rows_ * D + 3 * n * D);
    be_->launch("head_seeded_relevance", "rows", 0.0, bytes, "TiedLMHeadModule::propagate_relevance", [=](void* st) {
        pxk_seed_head_desc dd = d;
        dd.targets_in = given.empty() ? nullptr : given.data();
        return pxk_lm_seed_head_relevance(&dd, st);
    });
    return out;
}

Tensor TiedLMHeadModule::forward_impl(const Tensor& input) {
    const int64_t D = embedding_.embedding_dim(), V = embedding_.num_embeddings();
    if (input.rank() < 2 || input.shape().dim(static_cast<size_t>(input.rank() - 1)) != D)
        throw std::invalid_argument("TiedLMHeadModule::forward: input must be rank >= 2 with shape (..., d_model)");
    const int64_t m = input.numel() / D;
    std::vector<int64_t> dims = input.shape().dims();
    dims.back() = V;
    last_in_shape_ = input.shape();
    last_out_shape_ = Shape(dims);
    return detail::copy_out(be_, run_forward(detail::keep_input(be_, x_copy_, input), m), last_out_shape_);
}

Tensor TiedLMHeadModule::propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) {
    if (x_ == nullptr) throw std::logic_error("TiedLMHeadModule::propagate_relevance: called before any forward()");
    if (relevance_out.shape() != last_out_shape_)
        throw std::invalid_argument("TiedLMHeadModule::propagate_relevance: relevance_out must match the cached output shape");
    return detail::copy_out(be_, run_relevance(relevance_out.data(), config), last_in_shape_);
}

}  // namespace pulsatrix
