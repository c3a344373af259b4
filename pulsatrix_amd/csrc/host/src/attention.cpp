// MultiHeadAttentionModule on MI355XBackend: fused GQA attention forward and its AttnLRP pass.
#include <cmath>
#include <stdexcept>

#include "pulsatrix/rms_norm_module.hpp"
#include "pulsatrix/multihead_attention_module.hpp"

namespace pulsatrix {

using detail::gemm_desc;
using detail::mat;

namespace {

AttentionConfig resolve(AttentionConfig c) {  // multihead_attention_module.cpp:20-51
    if (c.d_model <= 0) throw std::invalid_argument("MultiHeadAttentionModule: d_model must be positive");
    if (c.num_heads <= 0) throw std::invalid_argument("MultiHeadAttentionModule: num_heads must be positive");
    if (c.num_kv_heads < 0 || c.head_dim < 0)
        throw std::invalid_argument("MultiHeadAttentionModule: num_kv_heads and head_dim must not be negative");
    if (c.num_kv_heads == 0) c.num_kv_heads = c.num_heads;
    if (c.num_heads % c.num_kv_heads != 0)
        throw std::invalid_argument("MultiHeadAttentionModule: num_heads must be a multiple of num_kv_heads");
    if (c.head_dim == 0) {
        if (c.d_model % c.num_heads != 0)
            throw std::invalid_argument("MultiHeadAttentionModule: d_model must be divisible by num_heads");
        c.head_dim = c.d_model / c.num_heads;
    }
    if (c.use_rope && c.head_dim % 2 != 0)
        throw std::invalid_argument("MultiHeadAttentionModule: use_rope requires an even head_dim (d_model / num_heads)");
    if (c.sliding_window < 0) throw std::invalid_argument("MultiHeadAttentionModule: sliding_window must not be negative");
    return c;
}

AttentionConfig legacy(int64_t d_model, int64_t num_heads, bool use_rope, bool use_qk_norm) {
    AttentionConfig c;
    c.d_model = d_model;
    c.num_heads = num_heads;
    c.use_rope = use_rope;
    c.use_qk_norm = use_qk_norm;
    return c;
}

}  // namespace

MultiHeadAttentionModule::MultiHeadAttentionModule(int64_t d_model, int64_t num_heads, DeviceBackend* backend,
                                                   bool use_rope, bool use_qk_norm)
    : MultiHeadAttentionModule(legacy(d_model, num_heads, use_rope, use_qk_norm), backend) {}

MultiHeadAttentionModule::MultiHeadAttentionModule(const AttentionConfig& config, DeviceBackend* backend)
    : config_(resolve(config)),
      d_(config_.d_model),
      H_(config_.num_heads),
      Hkv_(config_.num_kv_heads),
      D_(config_.head_dim),
      be_(detail::require_mi355x(backend, "MultiHeadAttentionModule")),
      q_proj_(d_, H_ * D_, backend, config_.qkv_bias),
      k_proj_(d_, Hkv_ * D_, backend, config_.qkv_bias),
      v_proj_(d_, Hkv_ * D_, backend, config_.qkv_bias),
      out_proj_(H_ * D_, d_, backend, config_.out_bias) {
    if (config_.use_qk_norm) {  // multihead_attention_module.cpp:116-121
        q_norm_ = std::make_unique<RMSNormModule>(D_, backend, DeviceType::Hip, config_.qk_norm_eps);
        k_norm_ = std::make_unique<RMSNormModule>(D_, backend, DeviceType::Hip, config_.qk_norm_eps);
        q_norm_->set_weight_offset(config_.qk_norm_weight_offset);
        k_norm_->set_weight_offset(config_.qk_norm_weight_offset);
    }
}

RMSNormModule& MultiHeadAttentionModule::q_norm() {
    if (!q_norm_) throw std::logic_error("MultiHeadAttentionModule::q_norm: the module has no QK-Norm");
    return *q_norm_;
}

RMSNormModule& MultiHeadAttentionModule::k_norm() {
    if (!k_norm_) throw std::logic_error("MultiHeadAttentionModule::k_norm: the module has no QK-Norm");
    return *k_norm_;
}

int64_t MultiHeadAttentionModule::window_for(int64_t l) const {
    // A window no query of this length reaches back past masks nothing.
    return (config_.causal && config_.sliding_window > 0 && config_.sliding_window < l) ? config_.sliding_window : 0;
}

bool MultiHeadAttentionModule::fused_attention(int64_t l) const {
    const int64_t qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd;
    const int64_t ldq = (config_.use_rope || config_.use_qk_norm) ? qd + kvd : w3;
    return window_for(l) == 0 && pxk_attention_supported(D_, l, ldq, ldq, w3);
}

float MultiHeadAttentionModule::score_scale() const {
    return config_.score_scale > 0.0f ? config_.score_scale : 1.0f / std::sqrt(static_cast<float>(D_));
}

void MultiHeadAttentionModule::pack_weights() {
    const uint64_t v = q_proj_.version() + k_proj_.version() + v_proj_.version();
    if (v == packed_version_ && wqkv_.size() > 0) return;
    const int64_t qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd;
    float* w = wqkv_.ensure(be_, d_ * w3);  // [Wq | Wk | Wv], (d, w3)
    be_->copy_2d(w, w3, q_proj_.weight_data(), qd, d_, qd);
    be_->copy_2d(w + qd, w3, k_proj_.weight_data(), kvd, d_, kvd);
    be_->copy_2d(w + qd + kvd, w3, v_proj_.weight_data(), kvd, d_, kvd);
    if (config_.qkv_bias) {
        float* b = bqkv_.ensure(be_, w3);
        be_->copy_2d(b, w3, q_proj_.bias_data(), qd, 1, qd);
        be_->copy_2d(b + qd, w3, k_proj_.bias_data(), kvd, 1, kvd);
        be_->copy_2d(b + qd + kvd, w3, v_proj_.bias_data(), kvd, 1, kvd);
    }
    packed_version_ = v;
}

// [Wq | Wk | Wv] with row k scaled by the norm's gamma[k]: x (Wq' | Wk' | Wv') / rms is the
// projection of the norm's output gamma x / rms (PXK_PRO_RMS). Rebuilt when the projections or the
// norm's scale change.
const float* MultiHeadAttentionModule::folded_weights(RMSNormModule* norm) {
    if (wg_norm_ != norm || wg_version_ != norm->version() || wg_packed_ != packed_version_ || wqkv_g_.size() == 0) {
        const int64_t w3 = H_ * D_ + 2 * Hkv_ * D_;
        float* w = wqkv_g_.ensure(be_, d_ * w3);
        MI355XBackend::check(pxk_scale_rows(wqkv_.data(), norm->effective_gamma(), w, d_, w3, be_->stream()),
                             "MultiHeadAttentionModule::forward");
        wg_norm_ = norm;
        wg_version_ = norm->version();
        wg_packed_ = packed_version_;
    }
    return wqkv_g_.data();
}

void MultiHeadAttentionModule::ensure_tables(int64_t l) {
    // Position-major tables: the first l rows of a longer table are this length's table, so the
    // tables only grow (no host work when the length shrinks, as it does along a decode).
    if (!config_.use_rope || l <= table_len_) return;
    // RoPEModule::ensure_tables (rope_module.cpp:67-69, 83-101): tables in double, rounded to float.
    const int64_t half = D_ / 2;
    std::vector<double> inv(static_cast<size_t>(half));
    for (int64_t i = 0; i < half; ++i)
        inv[static_cast<size_t>(i)] =
            config_.rope_inverse_frequencies.empty()
                ? std::pow(static_cast<double>(config_.rope_base), -2.0 * static_cast<double>(i) / static_cast<double>(D_))
                : config_.rope_inverse_frequencies.at(static_cast<size_t>(i));
    std::vector<float> c(static_cast<size_t>(l * half)), s(c.size());
    for (int64_t pos = 0; pos < l; ++pos)
        for (int64_t i = 0; i < half; ++i) {
            const double theta = static_cast<double>(pos) * inv[static_cast<size_t>(i)];
            c[static_cast<size_t>(pos * half + i)] = static_cast<float>(std::cos(theta));
            s[static_cast<size_t>(pos * half + i)] = static_cast<float>(std::sin(theta));
        }
    be_->copy(cos_.ensure(be_, l * half), c.data(), c.size() * sizeof(float), CopyDirection::HostToDevice);
    be_->copy(sin_.ensure(be_, l * half), s.data(), s.size() * sizeof(float), CopyDirection::HostToDevice);
    table_len_ = l;
}

const float* MultiHeadAttentionModule::output() const noexcept {
    return config_.out_bias ? out_y_.data() : out_z_.data();
}

const float* MultiHeadAttentionModule::run_forward(const float* x, int64_t n, int64_t l, const float* resid,
                                                   float* resid_out, RMSNormModule* norm) {
    pack_weights();
    ensure_tables(l);
    N_ = n;
    L_ = l;
    x_ = x;
    norm_in_ = norm;
    const int64_t M = n * l, qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd, LL = l * l;
    const bool causal = config_.causal;
    void* st = be_->stream();

    // 1-2. q, k, v in one GEMM against [Wq | Wk | Wv], z (pre-bias) kept for the relevance pass;
    //      with RoPE the epilogue also writes the rotated q | k heads (positions from 0: no KV
    //      cache here), one batch entry per sequence so that a row's position is its row.
    float* z = qkv_z_.ensure(be_, M * w3);
    float* y = config_.qkv_bias ? qkv_y_.ensure(be_, M * w3) : z;
    const int64_t rw = qd + kvd;  // row length of the rotated q | k block
    float* rot = config_.use_rope ? qk_rot_.ensure(be_, M * rw) : nullptr;
    // The ROPE_FWD epilogue needs whole heads inside the GEMM's 128-wide tiles and no QK-Norm in
    // between; otherwise the norm and the rotation run as their own launches.
    const bool qkn = config_.use_qk_norm;
    const bool rope_in_gemm = config_.use_rope && !qkn && (w3 <= 128 || 128 % D_ == 0);
    {
        pxk_gemm_desc d = gemm_desc(l, w3, d_);
        d.batch = n;
        d.a = mat(x, d_, l * d_);
        d.b = mat(wqkv_.data(), w3);
        d.c = mat(z, w3, l * w3);
        if (norm) {  // the block's pre-norm applied by this GEMM: gamma in the weights, x / rms per row
            d.prologue = PXK_PRO_RMS;
            d.b = mat(folded_weights(norm), w3);
            d.norm_eps = norm->eps();
            d.row_rms = norm->fold(M);
        }
        if (config_.qkv_bias) {
            d.epilogue = PXK_EPI_STORE_BIAS;
            d.c2 = mat(y, w3, l * w3);
            d.e_bias = mat(bqkv_.data(), 0);
        }
        if (rope_in_gemm) {
            d.epilogue = PXK_EPI_ROPE_FWD;
            d.c3 = mat(rot, rw, l * rw);
            d.cos_t = cos_.data();
            d.sin_t = sin_.data();
            d.head_dim = D_;
            d.rope_half = config_.rope_layout == RoPELayout::RotateHalf;
            d.rope_cols = rw;
        }
        be_->run_gemm(d);
    }
    const float* pre = y;  // q | k before the rotation (the RoPE rule's x), row stride ld_pre
    int64_t ld_pre = w3;
    if (qkn) {  // step 3: QK-Norm over each head's queries and keys
        float* nq = qk_norm_out_.ensure(be_, M * rw);
        MI355XBackend::check(pxk_rms_norm_heads(y, w3, nq, rw, q_norm_->effective_gamma(), M, H_, D_,
                                                q_norm_->eps(), st),
                             "MultiHeadAttentionModule::forward (QK-Norm)");
        MI355XBackend::check(pxk_rms_norm_heads(y + qd, w3, nq + qd, rw, k_norm_->effective_gamma(), M, Hkv_, D_,
                                                k_norm_->eps(), st),
                             "MultiHeadAttentionModule::forward (QK-Norm)");
        pre = nq;
        ld_pre = rw;
    }
    if (config_.use_rope && !rope_in_gemm)
        MI355XBackend::check(pxk_rope_qk(pre, pre + qd, ld_pre, rot, rot + qd, rw, cos_.data(), sin_.data(), M, l, H_,
                                         Hkv_, D_, config_.rope_layout == RoPELayout::RotateHalf, st),
                             "MultiHeadAttentionModule::forward (RoPE)");
    const float* q = config_.use_rope ? rot : pre;
    const float* k = config_.use_rope ? rot + qd : pre + qd;
    const float* v = y + qd + kvd;
    const int64_t ldq = config_.use_rope ? rw : ld_pre, ldk = ldq;
    const bool fused = fused_attention(l);
    float* ctx = ctx_.ensure(be_, M * qd);
    if (fused) {
        // 3-5 fused: scores, mask, softmax and P V in one launch. The relevance pass recomputes the
        // scores and P from q, k and the rows' softmax statistics, which are all that is kept.
        float* stats = stats_.ensure(be_, n * H_ * l * 2);
        const float scale = score_scale();
        const int64_t H = H_, Hkv = Hkv_, D = D_;
        // dense algorithmic work: Q K^T and P V over every (query, key) square, as the reference computes it
        be_->launch("attn_fwd", "attention", 4.0 * n * H * l * l * D, 0.0, "MultiHeadAttentionModule::forward (attention)",
                    [=](void* s) {
                        return pxk_attention_forward_stats(q, ldq, k, ldk, v, w3, nullptr, nullptr, stats, ctx, qd,
                                                           n, l, H, Hkv, D, scale, causal, s);
                    });
    } else {
        raw_.ensure(be_, n * H_ * LL);
        p_.ensure(be_, n * H_ * LL);
        run_attention_unfused(q, ldq, k, ldk, v, n, l);
    }
    // 6. output projection, with the block's residual add fused into the epilogue when asked.
    float* oz = out_z_.ensure(be_, M * d_);
    float* oy = config_.out_bias ? out_y_.ensure(be_, M * d_) : oz;
    {
        pxk_gemm_desc d = gemm_desc(M, d_, qd);
        d.a = mat(ctx, qd);
        d.b = mat(out_proj_.weight_data(), d_);
        d.c = mat(oz, d_);
        if (config_.out_bias) {
            d.c2 = mat(oy, d_);
            d.e_bias = mat(out_proj_.bias_data(), 0);
        }
        if (resid) {
            d.epilogue = PXK_EPI_ADD_RESID;
            d.x = mat(resid, d_);
            d.c3 = mat(resid_out, d_);
        } else {
            d.epilogue = config_.out_bias ? PXK_EPI_STORE_BIAS : PXK_EPI_STORE;
        }
        be_->run_gemm(d);
    }
    return oy;
}

void MultiHeadAttentionModule::reserve_forward(int64_t n, int64_t l) {
    const int64_t M = n * l, qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd, rw = qd + kvd;
    qkv_z_.ensure(be_, M * w3);
    if (config_.qkv_bias) qkv_y_.ensure(be_, M * w3);
    if (config_.use_qk_norm) qk_norm_out_.ensure(be_, M * rw);
    if (config_.use_rope) qk_rot_.ensure(be_, M * rw);
    if (fused_attention(l)) {
        stats_.ensure(be_, n * H_ * l * 2);
    } else {
        raw_.ensure(be_, n * H_ * l * l);
        p_.ensure(be_, n * H_ * l * l);
    }
    ctx_.ensure(be_, M * qd);
    out_z_.ensure(be_, M * d_);
    if (config_.out_bias) out_y_.ensure(be_, M * d_);
}

void MultiHeadAttentionModule::replicate_forward(int64_t copies) {
    const int64_t M = N_ * L_, qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd, rw = qd + kvd;
    const char* who = "MultiHeadAttentionModule::replicate_forward";
    qkv_z_.repeat(be_, M * w3, copies, who);
    if (config_.qkv_bias) qkv_y_.repeat(be_, M * w3, copies, who);
    if (config_.use_qk_norm) qk_norm_out_.repeat(be_, M * rw, copies, who);
    if (config_.use_rope) qk_rot_.repeat(be_, M * rw, copies, who);
    if (fused_attention(L_)) {
        stats_.repeat(be_, N_ * H_ * L_ * 2, copies, who);
    } else {
        raw_.repeat(be_, N_ * H_ * L_ * L_, copies, who);
        p_.repeat(be_, N_ * H_ * L_ * L_, copies, who);
    }
    ctx_.repeat(be_, M * qd, copies, who);
    out_z_.repeat(be_, M * d_, copies, who);
    if (config_.out_bias) out_y_.repeat(be_, M * d_, copies, who);
    N_ *= copies;
}

void MultiHeadAttentionModule::export_kv(KVCacheState& cache, int64_t positions) {
    if (x_ == nullptr) throw std::logic_error("MultiHeadAttentionModule::export_kv: called before any forward()");
    if (positions < L_) throw std::invalid_argument("MultiHeadAttentionModule::export_kv: the cache is shorter than the prompt");
    const int64_t qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd, rw = qd + kvd;
    ensure_tables(positions);
    cache.n = N_;
    cache.positions = positions;
    float* kc = cache.k.ensure(be_, N_ * positions * kvd);
    float* vc = cache.v.ensure(be_, N_ * positions * kvd);
    const float* z = qkv_z_.data();
    const float* y = config_.qkv_bias ? qkv_y_.data() : z;
    // The keys the attention read: rotated, or after QK-Norm alone, or the projection itself.
    const float* k = config_.use_rope ? qk_rot_.data() + qd : (config_.use_qk_norm ? qk_norm_out_.data() + qd : y + qd);
    const int64_t ldk = (config_.use_rope || config_.use_qk_norm) ? rw : w3;
    for (int64_t b = 0; b < N_; ++b) {
        be_->copy_2d(kc + b * positions * kvd, static_cast<size_t>(kvd), k + b * L_ * ldk, static_cast<size_t>(ldk),
                     static_cast<size_t>(L_), static_cast<size_t>(kvd));
        be_->copy_2d(vc + b * positions * kvd, static_cast<size_t>(kvd), y + qd + kvd + b * L_ * w3,
                     static_cast<size_t>(w3), static_cast<size_t>(L_), static_cast<size_t>(kvd));
    }
}

const float* MultiHeadAttentionModule::decode_step(const float* x, int64_t n, KVCacheState& cache, const int32_t* pos,
                                                   const float* resid, float* resid_out) {
    if (cache.positions <= 0 || cache.n != n)
        throw std::logic_error("MultiHeadAttentionModule::decode_step: the cache holds no prompt for this batch");
    pack_weights();
    const int64_t qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd, rw = qd + kvd;
    void* st = be_->stream();
    float* z = dec_z_.ensure(be_, n * w3);
    float* y = config_.qkv_bias ? dec_y_.ensure(be_, n * w3) : z;
    {
        pxk_gemm_desc d = gemm_desc(n, w3, d_);
        d.a = mat(x, d_);
        d.b = mat(wqkv_.data(), w3);
        d.c = mat(z, w3);
        if (config_.qkv_bias) {
            d.epilogue = PXK_EPI_STORE_BIAS;
            d.c2 = mat(y, w3);
            d.e_bias = mat(bqkv_.data(), 0);
        }
        be_->run_gemm(d);
    }
    const float* pre = y;
    int64_t ld_pre = w3;
    // QK-Norm inside the RoPE / cache kernel when both norms share their eps (they do for every
    // checkpoint the loader reads); otherwise its own two launches first.
    const bool fused_norm = config_.use_qk_norm && q_norm_->eps() == k_norm_->eps();
    if (config_.use_qk_norm && !fused_norm) {
        float* nq = dec_qkn_.ensure(be_, n * rw);
        MI355XBackend::check(pxk_rms_norm_heads(y, w3, nq, rw, q_norm_->effective_gamma(), n, H_, D_, q_norm_->eps(), st),
                             "MultiHeadAttentionModule::decode_step (QK-Norm)");
        MI355XBackend::check(pxk_rms_norm_heads(y + qd, w3, nq + qd, rw, k_norm_->effective_gamma(), n, Hkv_, D_,
                                                k_norm_->eps(), st),
                             "MultiHeadAttentionModule::decode_step (QK-Norm)");
        pre = nq;
        ld_pre = rw;
    }
    const int64_t stride = cache.positions * kvd;
    float* q = dec_q_.ensure(be_, n * qd);
    MI355XBackend::check(pxk_decode_rope_append(pre, ld_pre, pre + qd, ld_pre, y + qd + kvd, w3, q, cache.k.data(),
                                                cache.v.data(), stride, cache.positions, cos_.data(), sin_.data(), pos, n,
                                                H_, Hkv_, D_, config_.use_rope,
                                                config_.rope_layout == RoPELayout::RotateHalf,
                                                fused_norm ? q_norm_->effective_gamma() : nullptr,
                                                fused_norm ? k_norm_->effective_gamma() : nullptr,
                                                fused_norm ? q_norm_->eps() : 0.0f, st),
                         "MultiHeadAttentionModule::decode_step (RoPE, cache)");
    float* ctx = dec_ctx_.ensure(be_, n * qd);
    const int64_t window = config_.causal ? config_.sliding_window : 0;
    const size_t ws_bytes = pxk_decode_attention_workspace(n, H_, D_, cache.positions);
    float* ws = dec_ws_.ensure(be_, static_cast<int64_t>(ws_bytes / sizeof(float)));
    MI355XBackend::check(pxk_decode_attention(q, cache.k.data(), cache.v.data(), stride, ctx, pos, n, H_, Hkv_, D_,
                                              window, cache.positions, score_scale(), ws, ws_bytes, st),
                         "MultiHeadAttentionModule::decode_step (attention)");
    float* oz = dec_oz_.ensure(be_, n * d_);
    float* oy = config_.out_bias ? dec_oy_.ensure(be_, n * d_) : oz;
    pxk_gemm_desc d = gemm_desc(n, d_, qd);
    d.a = mat(ctx, qd);
    d.b = mat(out_proj_.weight_data(), d_);
    d.c = mat(oz, d_);
    if (config_.out_bias) {
        d.c2 = mat(oy, d_);
        d.e_bias = mat(out_proj_.bias_data(), 0);
    }
    if (resid) {
        d.epilogue = PXK_EPI_ADD_RESID;
        d.x = mat(resid, d_);
        d.c3 = mat(resid_out, d_);
    } else {
        d.epilogue = config_.out_bias ? PXK_EPI_STORE_BIAS : PXK_EPI_STORE;
    }
    be_->run_gemm(d);
    return oy;
}

// Scores GEMM, softmax and P V as three launches: head_dim outside pxk_attention_supported().
void MultiHeadAttentionModule::run_attention_unfused(const float* q, int64_t ldq, const float* k, int64_t ldk,
                                                     const float* v, int64_t n, int64_t l) {
    const int64_t qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd, grp = H_ / Hkv_, LL = l * l;
    const bool causal = config_.causal;
    void* st = be_->stream();
    float* raw = raw_.data();
    float* p = p_.data();
    float* ctx = ctx_.data();
    // 3. raw scores = Q K^T per query head; K read through the KV-head map.
    {
        pxk_gemm_desc d = gemm_desc(l, l, D_);
        d.batch = n * H_;
        d.inner = H_;
        d.trans_b = 1;
        d.causal = causal ? PXK_CAUSAL_TRI : PXK_CAUSAL_NONE;
        d.a = mat(q, ldq, l * ldq, D_);
        d.b = mat(k, ldk, l * ldk, D_, grp);
        d.c = mat(raw, l, H_ * LL, LL);
        be_->run_gemm(d);
    }
    // 4. P = softmax(scale * raw) over the visible keys.
    MI355XBackend::check(pxk_attention_softmax(raw, p, n * H_, l, score_scale(), causal, window_for(l), st),
                         "MultiHeadAttentionModule::forward (softmax)");
    // 5. context = P V, written head-packed (N*L, H*D): the merge permute is the store layout.
    {
        pxk_gemm_desc d = gemm_desc(l, D_, l);
        d.batch = n * H_;
        d.inner = H_;
        d.causal = causal ? PXK_CAUSAL_K_LE_M : PXK_CAUSAL_NONE;
        d.a = mat(p, l, H_ * LL, LL);
        d.b = mat(v, w3, l * w3, D_, grp);
        d.c = mat(ctx, qd, l * qd, D_);
        be_->run_gemm(d);
    }
}

void MultiHeadAttentionModule::relevance_denominator(const LRPRuleConfig& config, const float** den,
                                                     const float** bias) const {
    *den = out_z_.data();
    *bias = detail::rule_bias(out_proj_.bias_data(), config_.out_bias, config.epsilon_bias_in_denominator);
}

const float* MultiHeadAttentionModule::run_relevance(const float* relevance_out, const LRPRuleConfig& config,
                                                     const float* add, const detail::ResidualSplit& split,
                                                     bool divided) {
    if (x_ == nullptr)
        throw std::logic_error("MultiHeadAttentionModule::propagate_relevance: called before any forward()");
    detail::validate_rule(config, "LinearModule");  // the projections validate it (linear_module.cpp:342)
    // Gamma / AlphaBeta / ZBox reach the four projections; the bilinear, softmax and RoPE rules
    // read only epsilon (multihead_attention_module.cpp:404-485).
    const bool affine = detail::is_affine_rule(config);
    if (affine && divided)
        throw std::logic_error("MultiHeadAttentionModule::propagate_relevance: a divided relevance under a rule");
    const int64_t n = N_, l = L_, M = n * l, qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd, grp = H_ / Hkv_;
    const int64_t LL = l * l;
    const bool causal = config_.causal, bid = config.epsilon_bias_in_denominator;
    const float eps = config.epsilon;
    const float* z = qkv_z_.data();
    const float* y = config_.qkv_bias ? qkv_y_.data() : z;
    // q | k before the rotation (after QK-Norm when there is one): the RoPE rule's x
    const float* pre = config_.use_qk_norm ? qk_norm_out_.data() : y;
    const int64_t ld_pre = config_.use_qk_norm ? qd + kvd : w3;
    const float* q = config_.use_rope ? qk_rot_.data() : pre;
    const float* k = config_.use_rope ? qk_rot_.data() + qd : pre + qd;
    const float* v = y + qd + kvd;
    const int64_t ldq = config_.use_rope ? qd + kvd : ld_pre, ldk = ldq;  // q | k rotated rows, or the packed rows
    const float* bq = detail::rule_bias(bqkv_.data(), config_.qkv_bias, bid);
    void* st = be_->stream();

    // 1. out_proj epsilon rule; its epilogue forms the P V bilinear factor
    //    s_pv = r_ctx / (2 ctx + eps sign ctx) with r_ctx = ctx * (g W_o^T).
    float* spv = spv_.ensure(be_, M * qd);
    if (affine) {
        // r_ctx under the rule, then the P V bilinear factor s_pv = r_ctx / (2 ctx + eps sign ctx).
        float* rctx = rctx_.ensure(be_, M * qd);
        const float* bo = config_.out_bias ? out_proj_.bias_data() : nullptr;
        out_rule_.run(be_, config, out_proj_.version(), {{out_proj_.weight_data(), d_, d_, false, bo}},
                      {ctx_.data(), qd, M, qd, out_z_.data(), d_, bo, relevance_out, d_, d_, rctx, nullptr});
        MI355XBackend::check(pxk_lrp_bilinear_scale(rctx, ctx_.data(), spv, M * qd, eps, st),
                             "MultiHeadAttentionModule::propagate_relevance");
    } else {
        pxk_gemm_desc d = gemm_desc(M, qd, d_);
        d.trans_b = 1;
        d.epilogue = PXK_EPI_SPV;
        d.eps = eps;
        d.a = mat(relevance_out, d_);
        if (!divided) {  // else the producer of relevance_out already divided it by stab(z + bias)
            d.prologue = PXK_PRO_DIV_STAB;
            d.z = mat(out_z_.data(), d_);
            if (const float* bo = detail::rule_bias(out_proj_.bias_data(), config_.out_bias, bid)) d.z_bias = mat(bo, 0);
        }
        d.b = mat(out_proj_.weight_data(), d_);
        d.c = mat(spv, qd);
        d.x = mat(ctx_.data(), qd);
        be_->run_gemm(d);
    }
    float* ra = ra_.ensure(be_, n * H_ * LL);  // r_attn, then the Q K^T factor s
    // P: the forward's on the unfused path; on the fused path the q-side kernel recomputes it and
    // writes it here for the key side.
    float* p = p_.ensure(be_, n * H_ * LL);
    // [g_q | g_k | g_v]: relevance / stab(z) per projection, or the relevances themselves under a rule
    float* g = g_.ensure(be_, M * w3);
    if (!key_rel_.data() || key_rel_.numel() != M * kvd) {
        key_rel_ = Tensor::uninitialized(Shape({M, kvd}), be_);
        value_rel_ = Tensor::uninitialized(Shape({M, kvd}), be_);
    }
    if (fused_attention(l)) {
        // 2-4 fused: r_attn, the softmax rule with the Q K^T denominator (s), and the query share
        // with the RoPE rule and q_proj's denominator, one launch per layer.
        pxk_attn_rel_desc rd{};
        rd.n = n;
        rd.l = l;
        rd.heads = H_;
        rd.kv_heads = Hkv_;
        rd.head_dim = D_;
        rd.scale = score_scale();
        rd.eps = eps;
        rd.causal = causal;
        rd.rope = config_.use_rope;
        rd.rope_half = config_.rope_layout == RoPELayout::RotateHalf;
        rd.spv = spv;
        rd.ld_spv = qd;
        rd.v = v;
        rd.ld_v = w3;
        rd.k = k;
        rd.ld_k = ldk;
        rd.s = ra;
        rd.q = q;
        rd.ld_q = ldq;
        rd.q_pre = pre;
        rd.ld_q_pre = ld_pre;
        rd.z = z;
        rd.ld_z = w3;
        rd.bias = bq;
        rd.cos_t = cos_.data();
        rd.sin_t = sin_.data();
        rd.g = g;
        rd.ld_g = w3;
        rd.relevance_only = affine;
        // The recomputing form: raw and P from q, k and the forward's statistics, the softmax
        // rule's row sums of r_attn as s_pv . ctx.
        rd.ctx = ctx_.data();
        rd.ld_ctx = qd;
        rd.stats = stats_.data();
        rd.p_out = p;
        // r_attn = P * (s_pv V^T) and r_q = Q * (s K): two L x L x D products per head
        be_->launch("attn_rel_q", "attention", 4.0 * n * H_ * l * l * D_, 0.0,
                    "MultiHeadAttentionModule::propagate_relevance", [rd](void* s) { return pxk_attention_relevance_q(&rd, s); });
    } else {
        relevance_scores_unfused(spv, eps, bid, affine);
    }
    // 5-6. key and value shares per KV head, summed over its query heads, fused:
    //      r_k = K * sum_h s_qk_h^T Q_h with the RoPE rule, r_v = V * sum_h P_h^T s_pv_h, and the
    //      k/v projections' denominators into g.
    {
        pxk_attn_rel_kv_desc kd{};
        kd.n = n;
        kd.l = l;
        kd.heads = H_;
        kd.kv_heads = Hkv_;
        kd.head_dim = D_;
        kd.eps = eps;
        kd.causal = causal;
        kd.rope = config_.use_rope;
        kd.rope_half = config_.rope_layout == RoPELayout::RotateHalf;
        kd.s = ra;
        kd.p = p;
        kd.q = q;
        kd.ld_q = ldq;
        kd.spv = spv;
        kd.ld_spv = qd;
        kd.k = k;
        kd.ld_k = ldk;
        kd.k_pre = pre + qd;
        kd.ld_k_pre = ld_pre;
        kd.v = v;
        kd.ld_v = w3;
        kd.z_k = z + qd;
        kd.z_v = z + qd + kvd;
        kd.ld_z = w3;
        kd.bias_k = bq ? bq + qd : nullptr;
        kd.bias_v = bq ? bq + qd + kvd : nullptr;
        kd.cos_t = cos_.data();
        kd.sin_t = sin_.data();
        kd.key_rel = key_rel_.data();
        kd.value_rel = value_rel_.data();
        kd.ld_rel = kvd;
        kd.g_k = g + qd;
        kd.g_v = g + qd + kvd;
        kd.ld_g = w3;
        kd.relevance_only = affine;
        // r_k = K * sum_h s_h^T Q_h and r_v = V * sum_h P_h^T s_pv_h: two L x L x D products per query head
        be_->launch("attn_rel_kv", "attention", 4.0 * n * H_ * l * l * D_, 0.0,
                    "MultiHeadAttentionModule::propagate_relevance (k/v)",
                    [kd](void* s) { return pxk_attention_relevance_kv(&kd, s); });
    }
    // 7. the three projections' input relevance in one GEMM: x * ([g_q | g_k | g_v] [Wq | Wk | Wv]^T).
    float* r_in = r_in_.ensure(be_, M * d_);
    if (affine) {  // the rule over the packed q | k | v projections: the sum of their input relevances
        const bool qb = config_.qkv_bias;
        qkv_rule_.run(be_, config, packed_version_,
                      {{q_proj_.weight_data(), qd, qd, false, qb ? q_proj_.bias_data() : nullptr},
                       {k_proj_.weight_data(), kvd, kvd, false, qb ? k_proj_.bias_data() : nullptr},
                       {v_proj_.weight_data(), kvd, kvd, false, qb ? v_proj_.bias_data() : nullptr}},
                      {norm_in_ ? norm_in_->materialize(x_) : x_, d_, M, d_, z, w3, qb ? bqkv_.data() : nullptr, g,
                       w3, w3, r_in, add},
                      split);
    } else {
        pxk_gemm_desc d = gemm_desc(M, d_, w3);
        d.trans_b = 1;
        d.epilogue = PXK_EPI_MUL_X;
        d.a = mat(g, w3);
        d.b = mat(wqkv_.data(), w3);
        d.c = mat(r_in, d_);
        d.x = mat(x_, d_);
        if (norm_in_) {  // x_ is the folded norm's input: the epilogue forms its output from the rms
            d.x_rms = norm_in_->rms();
            d.x_gamma = norm_in_->effective_gamma();
        }
        if (add) d.y = mat(add, d_);
        detail::apply_split(d, split, d_, eps);
        be_->run_gemm(d);
    }
    has_relevance_ = true;
    return split.requested() ? nullptr : r_in;
}

// Steps 2-4 of run_relevance as GEMM and row-kernel launches: head_dim outside
// pxk_attention_supported().
void MultiHeadAttentionModule::relevance_scores_unfused(const float* spv, float eps, bool bid, bool rel_only) {
    const int64_t n = N_, l = L_, qd = H_ * D_, kvd = Hkv_ * D_, w3 = qd + 2 * kvd, grp = H_ / Hkv_, LL = l * l;
    const bool causal = config_.causal;
    const float* z = qkv_z_.data();
    const float* y = config_.qkv_bias ? qkv_y_.data() : z;
    const float* pre = config_.use_qk_norm ? qk_norm_out_.data() : y;
    const int64_t ld_pre = config_.use_qk_norm ? qd + kvd : w3;
    const float* q = config_.use_rope ? qk_rot_.data() : pre;
    const float* k = config_.use_rope ? qk_rot_.data() + qd : pre + qd;
    const float* v = y + qd + kvd;
    const int64_t ldq = config_.use_rope ? qd + kvd : ld_pre, ldk = ldq;  // q | k rotated rows, or the packed rows
    const float* bq = detail::rule_bias(bqkv_.data(), config_.qkv_bias, bid);
    void* st = be_->stream();
    float* ra = ra_.data();
    const float* p = p_.data();
    float* g = g_.data();
    // 2. r_attn = P * (s_pv V^T) per query head (Eq. 15, A-share of P V).
    {
        pxk_gemm_desc d = gemm_desc(l, l, D_);
        d.batch = n * H_;
        d.inner = H_;
        d.trans_b = 1;
        d.causal = causal ? PXK_CAUSAL_TRI : PXK_CAUSAL_NONE;
        d.epilogue = PXK_EPI_MUL_X;
        d.a = mat(spv, qd, l * qd, D_);
        d.b = mat(v, w3, l * w3, D_, grp);
        d.c = mat(ra, l, H_ * LL, LL);
        d.x = mat(p, l, H_ * LL, LL);
        be_->run_gemm(d);
    }
    // 3. softmax rule on the scaled scores, mask, then the Q K^T factor s_qk (in place).
    MI355XBackend::check(pxk_attention_lrp_scores(ra, p, raw_.data(), ra, n * H_, l, score_scale(), eps, causal,
                                                  window_for(l), st),
                         "MultiHeadAttentionModule::propagate_relevance (scores)");
    if (config_.use_rope && D_ > 128) {
        // 4 with head_dims the ROPE_REL epilogue cannot hold in one tile: acc = s K per query head,
        // then the RoPE rule and q_proj's denominator on the head-packed rows.
        float* acc = rctx_.ensure(be_, n * l * qd);
        pxk_gemm_desc d = gemm_desc(l, D_, l);
        d.batch = n * H_;
        d.inner = H_;
        d.causal = causal ? PXK_CAUSAL_K_LE_M : PXK_CAUSAL_NONE;
        d.a = mat(ra, l, H_ * LL, LL);
        d.b = mat(k, ldk, l * ldk, D_, grp);
        d.c = mat(acc, qd, l * qd, D_);
        be_->run_gemm(d);
        MI355XBackend::check(pxk_lrp_rope_rows(acc, qd, pre, ld_pre, q, ldq, z, w3, bq, cos_.data(), sin_.data(), g, w3,
                                               n * l, l, H_, D_, eps, config_.rope_layout == RoPELayout::RotateHalf,
                                               rel_only, st),
                             "MultiHeadAttentionModule::propagate_relevance (RoPE rule)");
        return;
    }
    // 4. query share: r_q = Q * (s_qk K), then the RoPE rule and q_proj's denominator.
    {
        pxk_gemm_desc d = gemm_desc(l, D_, l);
        d.batch = n * H_;
        d.inner = H_;
        d.causal = causal ? PXK_CAUSAL_K_LE_M : PXK_CAUSAL_NONE;
        d.eps = eps;
        d.a = mat(ra, l, H_ * LL, LL);
        d.b = mat(k, ldk, l * ldk, D_, grp);
        d.c2 = mat(g, w3, l * w3, D_);
        if (rel_only) {  // the relevance itself into g; the divided copy lands in scratch
            d.c = mat(g, w3, l * w3, D_);
            d.c2 = mat(rctx_.ensure(be_, n * l * qd), qd, l * qd, D_);
        }
        d.z = mat(z, w3, l * w3, D_);
        if (bq) d.e_bias = mat(bq, 0, 0, D_);
        if (config_.use_rope) {
            d.epilogue = PXK_EPI_ROPE_REL;
            d.x = mat(pre, ld_pre, l * ld_pre, D_);
            d.y = mat(q, ldq, l * ldq, D_);
            d.cos_t = cos_.data();
            d.sin_t = sin_.data();
            d.head_dim = D_;
            d.rope_half = config_.rope_layout == RoPELayout::RotateHalf;
        } else {
            d.epilogue = PXK_EPI_VALUE_REL;
            d.y = mat(q, ldq, l * ldq, D_);
        }
        be_->run_gemm(d);
    }
}

Tensor MultiHeadAttentionModule::forward_impl(const Tensor& input) {
    if (input.rank() != 3 || input.shape().dim(2) != d_)
        throw std::invalid_argument("MultiHeadAttentionModule::forward: input must be rank-3 (N, L, d_model)");
    const int64_t n = input.shape().dim(0), l = input.shape().dim(1);
    const float* out = run_forward(detail::keep_input(be_, x_copy_, input), n, l);
    return detail::copy_out(be_, out, Shape({n, l, d_}));
}

Tensor MultiHeadAttentionModule::propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) {
    if (x_ == nullptr)
        throw std::logic_error("MultiHeadAttentionModule::propagate_relevance: called before any forward()");
    if (relevance_out.rank() != 3 || relevance_out.shape().dim(0) != N_ || relevance_out.shape().dim(1) != L_ ||
        relevance_out.shape().dim(2) != d_)
        throw std::invalid_argument(
            "MultiHeadAttentionModule::propagate_relevance: relevance_out must be rank-3 (N, L, d_model) matching the "
            "cached forward shape");
    return detail::copy_out(be_, run_relevance(relevance_out.data(), config), Shape({N_, L_, d_}));
}

const Tensor& MultiHeadAttentionModule::key_relevance() const {
    if (!has_relevance_)
        throw std::logic_error("MultiHeadAttentionModule::key_relevance: no propagate_relevance() yet");
    return key_rel_;
}

const Tensor& MultiHeadAttentionModule::value_relevance() const {
    if (!has_relevance_)
        throw std::logic_error("MultiHeadAttentionModule::value_relevance: no propagate_relevance() yet");
    return value_rel_;
}

}  // namespace pulsatrix
