// ref_driver.cpp -- C API over the reference's own TransformerBlock, CausalLM, LinearModule and
// LRP::explain, on one of two backends.
//
// TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile together with the reference's path
// sources, read where they lie under /root/reference (nothing is copied):
//   * oracle/_ref/libpxref.so         on the reference's own CPUBackend: the entry points mirror
//                                     oracle/pxo.h with a pxr_ prefix, so the tests run the oracle
//                                     restatement and the real reference on identical inputs;
//   * oracle/_ref/libpxref_mi355x.so  (PXR_ON_MI355X) the same reference modules on MI355XBackend,
//                                     compiled against the reference's own DeviceBackend header:
//                                     the drop-in, run. It adds pxr_be_*, a shim that calls each
//                                     DeviceBackend virtual on device pointers, for the primitive
//                                     tests; its declarations live only here and in the tests.

#include <algorithm>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "pulsatrix/causal_lm.hpp"
#include "pulsatrix/cpu_backend.hpp"
#include "pulsatrix/explainer_context.hpp"
#include "pulsatrix/generation.hpp"
#include "pulsatrix/hf_model.hpp"
#include "pulsatrix/linear_module.hpp"
#include "pulsatrix/lrp.hpp"
#include "pulsatrix/lrp_rule_config.hpp"
#include "pulsatrix/multihead_attention_module.hpp"
#include "pulsatrix/relu_module.hpp"
#include "pulsatrix/transformer_block.hpp"
#ifdef PXR_ON_MI355X
#include "pulsatrix/mi355x_backend.hpp"
#endif

#include "pxo.h"

using namespace pulsatrix;

namespace {

thread_local std::string g_error;

// The backend every model of this library runs on: the reference's CPUBackend, or one
// process-wide MI355XBackend on device 0 (created on first use, kept until the process ends).
DeviceBackend* driver_backend() {
#ifdef PXR_ON_MI355X
    static MI355XBackend* be = new MI355XBackend(0);
    return be;
#else
    static CPUBackend be;
    return &be;
#endif
}

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

int64_t kv_heads(const px_model_config& c) { return c.num_kv_heads > 0 ? c.num_kv_heads : c.num_heads; }
int64_t head_dim(const px_model_config& c) { return c.head_dim > 0 ? c.head_dim : c.hidden_size / c.num_heads; }

// The reference's HfModelConfig for a px_model_config: its own ToAttentionConfig(config, layer)
// then builds each layer's attention.
HfModelConfig hf_config(const px_model_config& c) {
    HfModelConfig hc;
    hc.model_type = "llama";
    hc.hidden_size = c.hidden_size;
    hc.intermediate_size = c.intermediate_size;
    hc.num_hidden_layers = c.num_layers;
    hc.num_attention_heads = c.num_heads;
    hc.num_key_value_heads = kv_heads(c);
    hc.head_dim = head_dim(c);
    hc.vocab_size = c.vocab_size;
    hc.rms_norm_eps = c.rms_norm_eps;
    hc.rope_theta = c.rope_theta;
    hc.tie_word_embeddings = c.tie_word_embeddings != 0;
    hc.qkv_bias = c.qkv_bias != 0;
    hc.out_bias = c.out_bias != 0;
    hc.mlp_bias = c.mlp_bias != 0;
    hc.causal = c.causal != 0;
    hc.hidden_act = c.hidden_act == 1 ? "gelu_pytorch_tanh" : "silu";
    hc.qk_norm = c.qk_norm != 0;
    hc.post_norms = c.post_norms != 0;
    hc.norm_weight_offset = c.norm_weight_offset;
    if (c.embed_scale != 0.0f) hc.embed_scale = c.embed_scale;
    if (c.query_pre_attn_scalar > 0.0f) hc.query_pre_attn_scalar = c.query_pre_attn_scalar;
    if (c.rope_local_base > 0.0f) hc.rope_local_base_freq = c.rope_local_base;
    if (c.rope_scaling != 0) {
        HfRopeScaling r;
        r.type = c.rope_scaling == 1 ? "linear" : "llama3";
        r.factor = c.rope_factor;
        r.low_freq_factor = c.rope_low_freq_factor;
        r.high_freq_factor = c.rope_high_freq_factor;
        r.original_max_position_embeddings = c.rope_original_max_position;
        hc.rope_scaling = r;
    }
    if (c.sliding_window > 0) {
        hc.sliding_window = c.sliding_window;
        if (c.sliding_layers != 0)
            for (int64_t i = 0; i < c.num_layers; ++i)
                hc.layer_types.push_back(((c.sliding_layers >> i) & 1u) ? "sliding_attention" : "full_attention");
    }
    return hc;
}

AttentionConfig attention_config(const px_model_config& c) {
    if (c.use_rope && c.rope_rotate_half) return ToAttentionConfig(hf_config(c), 0);
    AttentionConfig a;  // the layouts ToAttentionConfig does not produce (no RoPE, adjacent pairs)
    a.d_model = c.hidden_size;
    a.num_heads = c.num_heads;
    a.num_kv_heads = kv_heads(c);
    a.head_dim = head_dim(c);
    a.use_rope = c.use_rope != 0;
    a.rope_layout = c.rope_rotate_half ? RoPELayout::RotateHalf : RoPELayout::AdjacentPairs;
    a.rope_base = c.rope_theta;
    a.qkv_bias = c.qkv_bias != 0;
    a.out_bias = c.out_bias != 0;
    a.causal = c.causal != 0;
    return a;
}

TransformerBlockOptions block_options(const px_model_config& c) {
    TransformerBlockOptions opt;
    opt.norm_eps = c.rms_norm_eps;
    opt.mlp_bias = c.mlp_bias != 0;
    opt.mlp_activation = c.hidden_act == 1 ? GatedActivation::GeluTanh : GatedActivation::Silu;
    opt.post_norms = c.post_norms != 0;
    opt.norm_weight_offset = c.norm_weight_offset;
    return opt;
}

// Names and sizes of one block's parameters in the flat blob's order.
std::vector<std::pair<std::string, int64_t>> block_layout(const px_model_config& c) {
    const int64_t d = c.hidden_size, q = c.num_heads * head_dim(c), kv = kv_heads(c) * head_dim(c),
                  f = c.intermediate_size;
    std::vector<std::pair<std::string, int64_t>> out{{"norm1.weight", d}};
    auto lin = [&](const std::string& name, int64_t in, int64_t o, bool bias) {
        out.push_back({name + ".weight", in * o});
        if (bias) out.push_back({name + ".bias", o});
    };
    lin("mha.q_proj", d, q, c.qkv_bias);
    lin("mha.k_proj", d, kv, c.qkv_bias);
    lin("mha.v_proj", d, kv, c.qkv_bias);
    lin("mha.out_proj", q, d, c.out_bias);
    if (c.qk_norm) {
        out.push_back({"mha.q_norm.weight", head_dim(c)});
        out.push_back({"mha.k_norm.weight", head_dim(c)});
    }
    out.push_back({"norm2.weight", d});
    lin("swiglu.gate_proj", d, f, c.mlp_bias);
    lin("swiglu.up_proj", d, f, c.mlp_bias);
    lin("swiglu.down_proj", f, d, c.mlp_bias);
    if (c.post_norms) {
        out.push_back({"post_attn_norm.weight", d});
        out.push_back({"post_mlp_norm.weight", d});
    }
    return out;
}

void load(Module& m, const std::vector<std::pair<std::string, int64_t>>& layout, const float* params,
          DeviceBackend* be) {
    std::map<std::string, Tensor*> targets;
    for (NamedParamRef& p : m.named_parameters()) targets.emplace(p.name, p.ref.value);
    const float* p = params;
    for (const auto& [name, size] : layout) {
        auto it = targets.find(name);
        if (it == targets.end()) throw std::invalid_argument("ref_driver: the model has no parameter " + name);
        if (it->second->numel() != size) throw std::invalid_argument("ref_driver: size mismatch for " + name);
        *it->second = Tensor(it->second->shape(), be, std::vector<float>(p, p + size));
        p += size;
    }
}

struct RefBlock {
    DeviceBackend* be = driver_backend();
    std::unique_ptr<TransformerBlock> block;
    int64_t n = 0, l = 0, d = 0;
};

struct RefLM {
    DeviceBackend* be = driver_backend();
    std::unique_ptr<CausalLM> lm;
    px_model_config c{};
    int64_t n = 0, l = 0;
    std::vector<std::pair<std::string, int64_t>> layout;  // the parameter blob's order
};

LRPRuleConfig rule(float eps, int bias_in_denominator) {
    LRPRuleConfig r{eps};
    r.epsilon_bias_in_denominator = bias_in_denominator != 0;
    return r;
}

LRPRuleConfig rule_of(const px_lrp_rule& p) {
    LRPRuleConfig r{p.epsilon};
    r.rule = static_cast<LRPRule>(p.rule);
    r.gamma = p.gamma;
    r.alpha = p.alpha;
    r.beta = p.beta;
    r.low = p.low;
    r.high = p.high;
    r.epsilon_bias_in_denominator = p.bias_in_denominator != 0;
    return r;
}

}  // namespace

extern "C" {

const char* pxr_last_error(void) { return g_error.c_str(); }

void* pxr_block_create(const px_model_config* cfg, const float* params) {
    RefBlock* out = nullptr;
    guarded([&] {
        auto b = std::make_unique<RefBlock>();
        b->block = std::make_unique<TransformerBlock>(attention_config(*cfg), cfg->intermediate_size, b->be,
                                                      block_options(*cfg));
        load(*b->block, block_layout(*cfg), params, b->be);
        b->d = cfg->hidden_size;
        out = b.release();
    });
    return out;
}

int pxr_block_forward(void* h, const float* x, int64_t n, int64_t l, float* y) {
    return guarded([&] {
        auto* b = static_cast<RefBlock*>(h);
        b->n = n;
        b->l = l;
        Tensor in(Shape({n, l, b->d}), b->be, std::vector<float>(x, x + n * l * b->d));
        const std::vector<float> out = b->block->forward(in).to_host_vector();
        std::copy(out.begin(), out.end(), y);
    });
}

static int block_relevance(void* h, const float* r_out, const LRPRuleConfig& cfg, float* r_in) {
    return guarded([&] {
        auto* b = static_cast<RefBlock*>(h);
        Tensor r(Shape({b->n, b->l, b->d}), b->be, std::vector<float>(r_out, r_out + b->n * b->l * b->d));
        const std::vector<float> out = b->block->propagate_relevance(r, cfg).to_host_vector();
        std::copy(out.begin(), out.end(), r_in);
    });
}

int pxr_block_relevance(void* h, const float* r_out, float eps, int bias_in_denominator, float* r_in) {
    return block_relevance(h, r_out, rule(eps, bias_in_denominator), r_in);
}

int pxr_block_relevance_rule(void* h, const float* r_out, const px_lrp_rule* r, float* r_in) {
    return block_relevance(h, r_out, rule_of(*r), r_in);
}

void pxr_block_destroy(void* h) { delete static_cast<RefBlock*>(h); }

// One case of the reference's Hugging Face attention tests (tests/attention_reference_test.cpp:
// 105-200), run through the reference's own MultiHeadAttentionModule on this library's backend:
// the AttentionConfig (rotate-half RoPE), the weights and biases ((in, out) layout), the QK-Norm
// gains, the key padding mask (n * l keep flags) and the position offset as given; forward of x
// (n, l, d_model) into out, then the backward of sum(out * g) into grad_in.
struct pxr_mha_spec {
    int64_t d_model, heads, kv_heads, head_dim;
    float rope_base;
    int32_t qkv_bias, qk_norm, causal;
    int64_t position_offset, n, l;
    const float *wq, *bq, *wk, *bk, *wv, *bv, *wo, *q_gamma, *k_gamma, *keep;
};

int pxr_mha_case(const pxr_mha_spec* s, const float* x, const float* g, float* out, float* grad_in) {
    return guarded([&] {
        DeviceBackend* be = driver_backend();
        AttentionConfig c;
        c.d_model = s->d_model;
        c.num_heads = s->heads;
        c.num_kv_heads = s->kv_heads;
        c.head_dim = s->head_dim;
        c.rope_layout = RoPELayout::RotateHalf;
        c.rope_base = s->rope_base;
        c.use_qk_norm = s->qk_norm != 0;
        c.qkv_bias = s->qkv_bias != 0;
        c.out_bias = false;
        c.causal = s->causal != 0;
        MultiHeadAttentionModule attn(c, be);
        const int64_t qd = s->heads * s->head_dim, kvd = s->kv_heads * s->head_dim, d = s->d_model;
        auto vec = [](const float* p, int64_t count) { return std::vector<float>(p, p + count); };
        attn.q_proj().set_weight(vec(s->wq, d * qd));
        attn.k_proj().set_weight(vec(s->wk, d * kvd));
        attn.v_proj().set_weight(vec(s->wv, d * kvd));
        attn.out_proj().set_weight(vec(s->wo, qd * d));
        if (s->qkv_bias) {
            attn.q_proj().set_bias(vec(s->bq, qd));
            attn.k_proj().set_bias(vec(s->bk, kvd));
            attn.v_proj().set_bias(vec(s->bv, kvd));
        }
        if (s->qk_norm) {
            attn.q_norm()->set_gamma(vec(s->q_gamma, s->head_dim));
            attn.k_norm()->set_gamma(vec(s->k_gamma, s->head_dim));
        }
        if (s->position_offset) attn.set_position_offset(s->position_offset);
        const int64_t count = s->n * s->l * d;
        if (s->keep) attn.set_key_padding_mask(Tensor(Shape({s->n, s->l}), be, vec(s->keep, s->n * s->l)));
        const std::vector<float> y = attn.forward(Tensor(Shape({s->n, s->l, d}), be, vec(x, count))).to_host_vector();
        std::copy(y.begin(), y.end(), out);
        const std::vector<float> gi = attn.backward(Tensor(Shape({s->n, s->l, d}), be, vec(g, count))).to_host_vector();
        std::copy(gi.begin(), gi.end(), grad_in);
    });
}

// The reference's independent-AttnLRP block test (tests/transformer_block_test.cpp:262-318): the
// legacy TransformerBlock(d_model, heads, d_ff, backend, use_rope = false, use_qk_norm = false)
// with the given gains and (in, out) weights (norm1, q, k, v, out, norm2, gate, up, down, packed in
// that order), forward of x (1, l, d_model) into y, then propagate_relevance(r_out, LRPRuleConfig{})
// into r_in.
int pxr_legacy_block_case(int64_t d_model, int64_t heads, int64_t d_ff, int64_t l, const float* params, const float* x,
                          const float* r_out, float* y, float* r_in) {
    return guarded([&] {
        DeviceBackend* be = driver_backend();
        TransformerBlock block(d_model, heads, d_ff, be, false, false);
        const float* p = params;
        auto take = [&p](int64_t count) {
            std::vector<float> v(p, p + count);
            p += count;
            return v;
        };
        const int64_t d = d_model;
        block.norm1().set_gamma(take(d));
        block.mha().q_proj().set_weight(take(d * d));
        block.mha().k_proj().set_weight(take(d * d));
        block.mha().v_proj().set_weight(take(d * d));
        block.mha().out_proj().set_weight(take(d * d));
        block.norm2().set_gamma(take(d));
        block.swiglu().gate_proj().set_weight(take(d * d_ff));
        block.swiglu().up_proj().set_weight(take(d * d_ff));
        block.swiglu().down_proj().set_weight(take(d_ff * d));
        const int64_t count = l * d;
        const std::vector<float> out =
            block.forward(Tensor(Shape({1, l, d}), be, std::vector<float>(x, x + count))).to_host_vector();
        std::copy(out.begin(), out.end(), y);
        const std::vector<float> r =
            block.propagate_relevance(Tensor(Shape({1, l, d}), be, std::vector<float>(r_out, r_out + count)),
                                      LRPRuleConfig{})
                .to_host_vector();
        std::copy(r.begin(), r.end(), r_in);
    });
}

void* pxr_lm_create(const px_model_config* cfg, const float* params) {
    RefLM* out = nullptr;
    guarded([&] {
        auto m = std::make_unique<RefLM>();
        m->lm = std::make_unique<CausalLM>(hf_config(*cfg), m->be);
        std::vector<std::pair<std::string, int64_t>> layout{{"embed_tokens.weight", cfg->vocab_size * cfg->hidden_size}};
        for (int64_t i = 0; i < cfg->num_layers; ++i)
            for (const auto& [name, size] : block_layout(*cfg)) layout.push_back({"layers." + std::to_string(i) + "." + name, size});
        layout.push_back({"norm.weight", cfg->hidden_size});
        if (!cfg->tie_word_embeddings) layout.push_back({"lm_head.weight", cfg->hidden_size * cfg->vocab_size});
        load(*m->lm, layout, params, m->be);
        m->c = *cfg;
        m->layout = layout;
        out = m.release();
    });
    return out;
}

int pxr_lm_forward(void* h, const int64_t* ids, int64_t n, int64_t l, float* logits) {
    return guarded([&] {
        auto* m = static_cast<RefLM*>(h);
        m->n = n;
        m->l = l;
        std::vector<float> x(static_cast<size_t>(n * l));
        for (size_t i = 0; i < x.size(); ++i) x[i] = static_cast<float>(ids[i]);
        const std::vector<float> out = m->lm->forward(Tensor(Shape({n, l}), m->be, x)).to_host_vector();
        if (logits) std::copy(out.begin(), out.end(), logits);
    });
}

static int lm_relevance(void* h, const float* seed, const LRPRuleConfig& cfg, float* r_embed, float* r_tokens, float* key_rel,
                 float* value_rel) {
    return guarded([&] {
        auto* m = static_cast<RefLM*>(h);
        const int64_t V = m->c.vocab_size;
        Tensor s(Shape({m->n, m->l, V}), m->be, std::vector<float>(seed, seed + m->n * m->l * V));
        const std::vector<Tensor> bounds = m->lm->propagate_relevance_by_layer(s, cfg);
        if (r_embed) {
            const std::vector<float> e = bounds.front().to_host_vector();
            std::copy(e.begin(), e.end(), r_embed);
        }
        if (r_tokens) {
            const std::vector<float> t = m->lm->embed_tokens().propagate_relevance(bounds.front(), cfg).to_host_vector();
            std::copy(t.begin(), t.end(), r_tokens);
        }
        const size_t kv = static_cast<size_t>(m->n * m->l * kv_heads(m->c) * head_dim(m->c));
        for (int64_t i = 0; i < m->lm->num_layers(); ++i) {
            MultiHeadAttentionModule& mha = m->lm->layer(i).mha();
            if (key_rel) {
                const std::vector<float> k = mha.key_relevance().to_host_vector();
                std::copy(k.begin(), k.end(), key_rel + i * kv);
            }
            if (value_rel) {
                const std::vector<float> v = mha.value_relevance().to_host_vector();
                std::copy(v.begin(), v.end(), value_rel + i * kv);
            }
        }
    });
}

int pxr_lm_relevance(void* h, const float* seed, float eps, int bias_in_denominator, float* r_embed, float* r_tokens,
                     float* key_rel, float* value_rel) {
    return lm_relevance(h, seed, rule(eps, bias_in_denominator), r_embed, r_tokens, key_rel, value_rel);
}

int pxr_lm_relevance_rule(void* h, const float* seed, const px_lrp_rule* r, float* r_embed, float* r_tokens,
                          float* key_rel, float* value_rel) {
    return lm_relevance(h, seed, rule_of(*r), r_embed, r_tokens, key_rel, value_rel);
}

void pxr_lm_destroy(void* h) { delete static_cast<RefLM*>(h); }

// CausalLM::backward (causal_lm.cpp:82-92) of grad_logits (N, L, V) after the last forward; every
// parameter's gradient goes to grads in the parameter blob's layout.
int pxr_lm_backward(void* h, const float* grad_logits, float* grads) {
    return guarded([&] {
        auto* m = static_cast<RefLM*>(h);
        const int64_t V = m->c.vocab_size;
        Tensor g(Shape({m->n, m->l, V}), m->be, std::vector<float>(grad_logits, grad_logits + m->n * m->l * V));
        (void)m->lm->backward(g);
        std::map<std::string, Tensor*> by_name;
        for (NamedParamRef& p : m->lm->named_parameters()) by_name.emplace(p.name, p.ref.grad);
        float* out = grads;
        for (const auto& [name, size] : m->layout) {
            const std::vector<float> v = by_name.at(name)->to_host_vector();
            if (static_cast<int64_t>(v.size()) != size) throw std::runtime_error("pxr_lm_backward: size of " + name);
            std::copy(v.begin(), v.end(), out);
            out += size;
        }
    });
}

// A next-token function behind a C callback (the product's pxa_lm_next_token_logits, or the
// reference CausalLM's own below): the logits after tokens[0 .. n) into logits (vocab floats).
typedef int (*pxr_next_token_cb)(void* ctx, const int64_t* tokens, int64_t n, float* logits, int64_t vocab);

// Generate (generation.hpp:95-135, generation.cpp) over such a callback with a GenerationConfig
// built from the arguments (seed < 0: unset). new_tokens and log_probs hold up to cap entries.
int pxr_generate(pxr_next_token_cb cb, void* ctx, int64_t vocab, const int64_t* prompt, int64_t n_prompt,
                 int64_t max_new_tokens, int64_t min_new_tokens, const int64_t* eos, int64_t n_eos, int do_sample,
                 float temperature, int64_t top_k, float top_p, float min_p, float repetition_penalty, int64_t seed,
                 int64_t* new_tokens, float* log_probs, int64_t cap, int64_t* n_new, int* finish_reason) {
    return guarded([&] {
        NextTokenLogitsFn model = [cb, ctx, vocab](const std::vector<int64_t>& tokens) {
            std::vector<float> out(static_cast<size_t>(vocab));
            if (cb(ctx, tokens.data(), static_cast<int64_t>(tokens.size()), out.data(), vocab) != 0)
                throw std::runtime_error("pxr_generate: the next-token callback failed");
            return out;
        };
        GenerationConfig gc;
        gc.max_new_tokens = max_new_tokens;
        gc.min_new_tokens = min_new_tokens;
        gc.eos_token_ids.assign(eos, eos + n_eos);
        gc.do_sample = do_sample != 0;
        gc.temperature = temperature;
        gc.top_k = top_k;
        gc.top_p = top_p;
        gc.min_p = min_p;
        gc.repetition_penalty = repetition_penalty;
        if (seed >= 0) gc.seed = static_cast<uint64_t>(seed);
        const GenerationResult r = Generate(model, std::vector<int64_t>(prompt, prompt + n_prompt), gc);
        if (static_cast<int64_t>(r.new_tokens.size()) > cap) throw std::runtime_error("pxr_generate: output too small");
        std::copy(r.new_tokens.begin(), r.new_tokens.end(), new_tokens);
        std::copy(r.log_probs.begin(), r.log_probs.end(), log_probs);
        *n_new = static_cast<int64_t>(r.new_tokens.size());
        *finish_reason = r.finish_reason == FinishReason::Eos ? 0 : 1;
    });
}

// CausalLM::next_token_logits (causal_lm.hpp:116) of the reference model, behind the callback.
void* pxr_lm_next_token_logits_create(void* h, int64_t max_length) {
    NextTokenLogitsFn* out = nullptr;
    guarded([&] { out = new NextTokenLogitsFn(static_cast<RefLM*>(h)->lm->next_token_logits(max_length)); });
    return out;
}

int pxr_lm_next_token_logits(void* f, const int64_t* tokens, int64_t n, float* logits, int64_t vocab) {
    return guarded([&] {
        const std::vector<float> v = (*static_cast<NextTokenLogitsFn*>(f))(std::vector<int64_t>(tokens, tokens + n));
        if (static_cast<int64_t>(v.size()) != vocab) throw std::runtime_error("pxr_lm_next_token_logits: vocab");
        std::copy(v.begin(), v.end(), logits);
    });
}

void pxr_lm_next_token_logits_destroy(void* f) { delete static_cast<NextTokenLogitsFn*>(f); }

int pxr_linear_relevance(const float* x, const float* w, const float* bias, const float* r, int64_t n, int64_t in,
                         int64_t out, float eps, int bias_in_denominator, float* r_in) {
    return guarded([&] {
        DeviceBackend* be = driver_backend();
        LinearModule lin(in, out, be, bias != nullptr);
        lin.set_weight(std::vector<float>(w, w + in * out));
        if (bias) lin.set_bias(std::vector<float>(bias, bias + out));
        (void)lin.forward(Tensor(Shape({n, in}), be, std::vector<float>(x, x + n * in)));
        Tensor rr(Shape({n, out}), be, std::vector<float>(r, r + n * out));
        const std::vector<float> res = lin.propagate_relevance(rr, rule(eps, bias_in_denominator)).to_host_vector();
        std::copy(res.begin(), res.end(), r_in);
    });
}

int pxr_linear_relevance_rule(const float* x, const float* w, const float* bias, const float* r, int64_t n, int64_t in,
                              int64_t out, const px_lrp_rule* rl, float* r_in) {
    return guarded([&] {
        DeviceBackend* be = driver_backend();
        LinearModule lin(in, out, be, bias != nullptr);
        lin.set_weight(std::vector<float>(w, w + in * out));
        if (bias) lin.set_bias(std::vector<float>(bias, bias + out));
        (void)lin.forward(Tensor(Shape({n, in}), be, std::vector<float>(x, x + n * in)));
        Tensor rr(Shape({n, out}), be, std::vector<float>(r, r + n * out));
        const std::vector<float> res = lin.propagate_relevance(rr, rule_of(*rl)).to_host_vector();
        std::copy(res.begin(), res.end(), r_in);
    });
}

// LRP::explain (include/pulsatrix/lrp.hpp:218-241) over the reference's Linear -> ReLU -> ... ->
// Linear chain in an ExplainerContext, OneHot seeds at targets[n] (one per input row): the path of
// tests/lrp_reference_test.cpp:285-303. Layer i is (in[i], out[i]) with weights w[i] stored
// (in, out) and biases b[i]; `relevance` receives the (n, in[0]) attribution, and `in_sum` the
// Attribution's relevance_in_sum (DeviceBackend::sum). preset 0 applies `r` to every module; 1, 2
// and 3 are the reference's LRP::epsilon_plus(), epsilon_alpha2_beta1() and
// epsilon_gamma_box(-3, 3) composites (lrp.hpp:186-197).
int pxr_mlp_explain(int layers, const int64_t* in, const int64_t* out, const float* const* w, const float* const* b,
                    const float* x, int64_t n, const int64_t* targets, const px_lrp_rule* r, int preset,
                    float* relevance, float* in_sum) {
    return guarded([&] {
        DeviceBackend* be = driver_backend();
        std::vector<std::unique_ptr<Module>> owned;
        std::vector<Module*> chain;
        for (int i = 0; i < layers; ++i) {
            auto lin = std::make_unique<LinearModule>(in[i], out[i], be, b[i] != nullptr);
            lin->set_weight(std::vector<float>(w[i], w[i] + in[i] * out[i]));
            if (b[i]) lin->set_bias(std::vector<float>(b[i], b[i] + out[i]));
            chain.push_back(lin.get());
            owned.push_back(std::move(lin));
            if (i + 1 < layers) {
                owned.push_back(std::make_unique<ReluModule>(be));
                chain.push_back(owned.back().get());
            }
        }
        ExplainerContext ctx(chain);
        const Tensor input(Shape({n, in[0]}), be, std::vector<float>(x, x + n * in[0]));
        const LRP lrp = preset == 1   ? LRP::epsilon_plus()
                        : preset == 2 ? LRP::epsilon_alpha2_beta1()
                        : preset == 3 ? LRP::epsilon_gamma_box(-3.0f, 3.0f)
                                      : LRP(rule_of(*r));
        Attribution a = lrp.explain(ctx, input, LRPTarget{std::vector<int64_t>(targets, targets + n), {}, LRPSeed::OneHot},
                                    be);
        const std::vector<float> v = a.values.to_host_vector();
        std::copy(v.begin(), v.end(), relevance);
        if (in_sum) *in_sum = std::stof(a.metadata.at("relevance_in_sum"));
    });
}

#ifndef PXR_ON_MI355X
// ---- CPU build only: host-pointer helpers of the oracle tests ----
void pxr_lrp_bilinear_matmul(const float* a, const float* b, const float* o, const float* r_o, float* r_a, float* r_b,
                             size_t slices, size_t m, size_t p, size_t q, float eps, int bt) {
    CPUBackend be;
    be.lrp_bilinear_matmul(a, b, o, r_o, r_a, r_b, slices, m, p, q, eps, bt != 0);
}

void pxr_gemm_ex(const float* a, int ta, const float* b, int tb, float* out, size_t m, size_t k, size_t n, float beta) {
    CPUBackend be;
    be.gemm_ex(a, ta != 0, b, tb != 0, out, m, k, n, beta);
}
#endif

// ---- pxr_be_*: each DeviceBackend virtual of this library's backend: host pointers on the
// reference's CPUBackend, device pointers on MI355XBackend; the tests run both on the same data ----

#define PXR_BE(name, params, call) \
    int pxr_be_##name params { return guarded([&] { driver_backend()->call; }); }

PXR_BE(copy, (void* dst, const void* src, size_t bytes, int dir),
       copy(dst, src, bytes, static_cast<CopyDirection>(dir)))
PXR_BE(fill, (float* p, float value, size_t n), fill(p, value, n))
PXR_BE(gemm, (const float* a, const float* b, float* out, size_t m, size_t k, size_t n), gemm(a, b, out, m, k, n))
PXR_BE(gemm_ex, (const float* a, int ta, const float* b, int tb, float* out, size_t m, size_t k, size_t n, float beta),
       gemm_ex(a, ta != 0, b, tb != 0, out, m, k, n, beta))
PXR_BE(gemm_strided_batched,
       (const float* a, int ta, size_t sa, const float* b, int tb, size_t sb, float* out, size_t so, size_t m, size_t k,
        size_t n, size_t batch, float beta),
       gemm_strided_batched(a, ta != 0, sa, b, tb != 0, sb, out, so, m, k, n, batch, beta))
PXR_BE(elementwise, (int op, const float* in, float* out, size_t n), elementwise(static_cast<ElementwiseOp>(op), in, out, n))
PXR_BE(add, (const float* a, const float* b, float* out, size_t n), add(a, b, out, n))
PXR_BE(mul, (const float* a, const float* b, float* out, size_t n), mul(a, b, out, n))
PXR_BE(axpby, (float alpha, const float* x, float beta, const float* y, float* out, size_t n),
       axpby(alpha, x, beta, y, out, n))
PXR_BE(column_sums, (const float* in, float* out, size_t rows, size_t cols, float beta),
       column_sums(in, out, rows, cols, beta))
PXR_BE(add_row_vector, (const float* in, const float* row, float* out, size_t rows, size_t cols),
       add_row_vector(in, row, out, rows, cols))
PXR_BE(dot_into, (const float* a, const float* b, size_t n, float* out), dot_into(a, b, n, out))
PXR_BE(softmax_rows, (const float* in, float* out, size_t rows, size_t cols), softmax_rows(in, out, rows, cols))
PXR_BE(rms_norm_forward, (const float* in, const float* g, float* out, float* rms, size_t rows, size_t cols, float eps),
       rms_norm_forward(in, g, out, rms, rows, cols, eps))
PXR_BE(rope_rotate,
       (const float* in, const float* c, const float* s, float* out, size_t slices, size_t seq, size_t hd, int inverse,
        int half),
       rope_rotate(in, c, s, out, slices, seq, hd, inverse != 0, half != 0))
PXR_BE(permute_0213, (const float* in, float* out, size_t d0, size_t d1, size_t d2, size_t d3),
       permute_0213(in, out, d0, d1, d2, d3))
PXR_BE(attention_mask_fill,
       (float* scores, const float* keep, size_t batch, size_t heads, size_t q_len, size_t k_len, int causal,
        size_t q_offset, size_t window, float value),
       attention_mask_fill(scores, keep, batch, heads, q_len, k_len, causal != 0, q_offset, window, value))
PXR_BE(gather_rows, (const float* table, const float* idx, float* out, size_t count, size_t dim),
       gather_rows(table, idx, out, count, dim))
PXR_BE(lrp_linear,
       (const float* x, const float* w, const float* z, const float* r, float* r_in, size_t rows, size_t in, size_t out,
        float eps),
       lrp_linear(x, w, z, r, r_in, rows, in, out, eps))
PXR_BE(lrp_residual_split, (const float* a, const float* b, const float* r, float* ra, float* rb, size_t n, float eps),
       lrp_residual_split(a, b, r, ra, rb, n, eps))
PXR_BE(lrp_bilinear_elementwise, (const float* a, const float* b, const float* r, float* out, size_t n, float eps),
       lrp_bilinear_elementwise(a, b, r, out, n, eps))
PXR_BE(lrp_bilinear_matmul,
       (const float* a, const float* b, const float* o, const float* r_o, float* r_a, float* r_b, size_t slices,
        size_t m, size_t p, size_t q, float eps, int bt),
       lrp_bilinear_matmul(a, b, o, r_o, r_a, r_b, slices, m, p, q, eps, bt != 0))
PXR_BE(lrp_softmax_rows, (const float* x, const float* y, const float* r, float* r_in, size_t rows, size_t cols),
       lrp_softmax_rows(x, y, r, r_in, rows, cols))
PXR_BE(lrp_rope,
       (const float* x, const float* y, const float* r, const float* c, const float* s, float* r_in, size_t slices,
        size_t seq, size_t hd, float eps, int half),
       lrp_rope(x, y, r, c, s, r_in, slices, seq, hd, eps, half != 0))
PXR_BE(lrp_stabilized_divide,
       (const float* r, const float* d, const float* gate, float* out, size_t n, float eps, int mode),
       lrp_stabilized_divide(r, d, gate, out, n, eps, static_cast<LrpGate>(mode)))
PXR_BE(copy_2d, (float* dst, size_t ds, const float* src, size_t ss, size_t rows, size_t cols),
       copy_2d(dst, ds, src, ss, rows, cols))
PXR_BE(accumulate_rows, (const float* in, float* out, size_t rows, size_t cols), accumulate_rows(in, out, rows, cols))

PXR_BE(elementwise_backward, (int op, const float* x, const float* g, float* out, size_t n),
       elementwise_backward(static_cast<ElementwiseOp>(op), x, g, out, n))
PXR_BE(softmax_rows_backward, (const float* y, const float* dy, float* dx, size_t rows, size_t cols),
       softmax_rows_backward(y, dy, dx, rows, cols))
PXR_BE(rms_norm_backward,
       (const float* g, const float* gamma, const float* x, const float* rms, float* gx, float* gt, size_t rows,
        size_t cols),
       rms_norm_backward(g, gamma, x, rms, gx, gt, rows, cols))
PXR_BE(layer_norm_forward,
       (const float* x, const float* gamma, const float* beta, float* xhat, float* out, float* sd, size_t rows,
        size_t cols, float eps),
       layer_norm_forward(x, gamma, beta, xhat, out, sd, rows, cols, eps))
PXR_BE(layer_norm_backward,
       (const float* g, const float* gamma, const float* xhat, const float* sd, float* gx, size_t rows, size_t cols),
       layer_norm_backward(g, gamma, xhat, sd, gx, rows, cols))
PXR_BE(logsumexp_rows, (const float* in, float* out, size_t rows, size_t cols), logsumexp_rows(in, out, rows, cols))
PXR_BE(scatter_add_rows, (const float* src, const float* idx, float* table, size_t count, size_t dim),
       scatter_add_rows(src, idx, table, count, dim))
PXR_BE(adam_step,
       (float* p, const float* g, float* m, float* v, size_t n, float lr, float b1, float b2, float eps, float c1,
        float c2),
       adam_step(p, g, m, v, n, lr, b1, b2, eps, c1, c2))
PXR_BE(dropout_forward, (const float* in, float* out, float* mask, size_t n, float p, float scale, uint64_t seed,
                         uint64_t offset),
       dropout_forward(in, out, mask, n, p, scale, seed, offset))
PXR_BE(bce_with_logits, (const float* x, const float* y, float* out, size_t n), bce_with_logits(x, y, out, n))
PXR_BE(bce_with_logits_grad, (const float* x, const float* y, float* out, size_t n, float scale),
       bce_with_logits_grad(x, y, out, n, scale))
PXR_BE(tanh_gaussian_forward,
       (const float* mean, const float* log_std, const float* e, float* action, float* std_cache, float* log_prob,
        size_t rows, size_t cols, float stabilizer, double half_log_two_pi),
       tanh_gaussian_forward(mean, log_std, e, action, std_cache, log_prob, rows, cols, stabilizer, half_log_two_pi))
PXR_BE(tanh_gaussian_backward,
       (const float* action, const float* std_cache, const float* e, const float* ga, const float* glp, float* gm,
        float* gls, size_t n, float stabilizer),
       tanh_gaussian_backward(action, std_cache, e, ga, glp, gm, gls, n, stabilizer))
PXR_BE(top_k_rows, (const float* in, float* values, float* indices, size_t rows, size_t cols, size_t k, int largest),
       top_k_rows(in, values, indices, rows, cols, k, largest != 0))

// The non-LLM modules' virtuals. ConvGeometry goes as six sizes; the slot structs of recurrent_cell,
// ssm_pass and rl_rows as arrays of pointers (10 / 6, 12 / 10 and 5 / 4 entries) and their scalars.
PXR_BE(logic_pointwise,
       (int op, int norm, const float* a, const float* b, const float* g, const float* y, float* oa, float* ob, size_t n,
        float eps),
       logic_pointwise(static_cast<LogicOp>(op), norm, a, b, g, y, oa, ob, n, eps))
PXR_BE(aggregator_forward, (const float* x, float* mp, float* out, size_t n, size_t cols, float p),
       aggregator_forward(x, mp, out, n, cols, p))
PXR_BE(aggregator_backward, (const float* x, const float* mp, const float* go, float* gi, size_t n, size_t cols, float p),
       aggregator_backward(x, mp, go, gi, n, cols, p))
PXR_BE(aggregator_lrp,
       (const float* x, const float* mp, const float* ro, float* ri, size_t n, size_t cols, float p, float eps),
       aggregator_lrp(x, mp, ro, ri, n, cols, p, eps))
PXR_BE(im2col,
       (const float* in, float* col, size_t n, size_t c, size_t h, size_t w, size_t kh, size_t kw, size_t sh, size_t sw,
        size_t ph, size_t pw),
       im2col(in, col, n, c, h, w, ConvGeometry{kh, kw, sh, sw, ph, pw}))
PXR_BE(col2im_add,
       (const float* col, float* out, size_t n, size_t c, size_t h, size_t w, size_t kh, size_t kw, size_t sh, size_t sw,
        size_t ph, size_t pw),
       col2im_add(col, out, n, c, h, w, ConvGeometry{kh, kw, sh, sw, ph, pw}))
PXR_BE(add_channel_vector, (const float* in, const float* vec, float* out, size_t n, size_t c, size_t inner),
       add_channel_vector(in, vec, out, n, c, inner))
PXR_BE(lrp_conv,
       (const float* col, const float* kernel, const float* z, const float* r, float* rc, size_t n, size_t oc, size_t p,
        size_t q, float eps),
       lrp_conv(col, kernel, z, r, rc, n, oc, p, q, eps))
PXR_BE(max_pool_forward,
       (const float* in, float* out, float* am, size_t planes, size_t h, size_t w, size_t kh, size_t kw, size_t sh,
        size_t sw, size_t ph, size_t pw),
       max_pool_forward(in, out, am, planes, h, w, kh, kw, sh, sw, ph, pw))
PXR_BE(max_unpool,
       (const float* src, const float* am, float* dst, size_t planes, size_t h, size_t w, size_t kh, size_t kw, size_t sh,
        size_t sw, size_t ph, size_t pw),
       max_unpool(src, am, dst, planes, h, w, kh, kw, sh, sw, ph, pw))
PXR_BE(avg_pool_forward, (const float* in, float* out, size_t planes, size_t h, size_t w, size_t kh, size_t kw),
       avg_pool_forward(in, out, planes, h, w, kh, kw))
PXR_BE(avg_pool_backward, (const float* go, float* gi, size_t planes, size_t h, size_t w, size_t kh, size_t kw),
       avg_pool_backward(go, gi, planes, h, w, kh, kw))
PXR_BE(lrp_avg_pool,
       (const float* x, const float* r, float* ri, size_t planes, size_t h, size_t w, size_t kh, size_t kw, float eps),
       lrp_avg_pool(x, r, ri, planes, h, w, kh, kw, eps))
PXR_BE(batch_norm_forward,
       (const float* in, const float* gm, const float* bt, float* xh, float* out, float* sd, size_t n, size_t c,
        size_t sp, float eps),
       batch_norm_forward(in, gm, bt, xh, out, sd, n, c, sp, eps))
PXR_BE(batch_norm_backward,
       (const float* go, const float* gm, const float* xh, const float* sd, float* gi, float* gg, float* bg, size_t n,
        size_t c, size_t sp),
       batch_norm_backward(go, gm, xh, sd, gi, gg, bg, n, c, sp))
PXR_BE(batch_norm_update_running,
       (const float* in, float* rm, float* rv, size_t n, size_t c, size_t sp, float momentum),
       batch_norm_update_running(in, rm, rv, n, c, sp, momentum))
PXR_BE(batch_norm_eval_forward,
       (const float* in, const float* gm, const float* bt, const float* rm, const float* rv, float* xh, float* out,
        float* sd, size_t n, size_t c, size_t sp, float eps),
       batch_norm_eval_forward(in, gm, bt, rm, rv, xh, out, sd, n, c, sp, eps))
PXR_BE(batch_norm_eval_backward,
       (const float* go, const float* gm, const float* xh, const float* sd, float* gi, float* gg, float* bg, size_t n,
        size_t c, size_t sp),
       batch_norm_eval_backward(go, gm, xh, sd, gi, gg, bg, n, c, sp))
PXR_BE(group_norm_forward,
       (const float* in, const float* gm, const float* bt, float* xh, float* out, float* sd, size_t n, size_t c,
        size_t sp, size_t groups, float eps),
       group_norm_forward(in, gm, bt, xh, out, sd, n, c, sp, groups, eps))
PXR_BE(group_norm_backward,
       (const float* go, const float* gm, const float* xh, const float* sd, float* gi, float* gg, float* bg, size_t n,
        size_t c, size_t sp, size_t groups),
       group_norm_backward(go, gm, xh, sd, gi, gg, bg, n, c, sp, groups))
PXR_BE(gru_lrp_hprev,
       (const float* hp, const float* w, const float* hn, const float* rb, const float* direct, float* out, size_t rows,
        size_t hidden, float eps),
       gru_lrp_hprev(hp, w, hn, rb, direct, out, rows, hidden, eps))

int pxr_be_recurrent_cell(int op, const float* const* in, float* const* out, float eps, size_t n) {
    return guarded([&] {
        RecurrentCellArgs a;
        std::copy(in, in + 10, a.in);
        std::copy(out, out + 6, a.out);
        a.eps = eps;
        driver_backend()->recurrent_cell(static_cast<RecurrentCellOp>(op), a, n);
    });
}

int pxr_be_ssm_pass(int op, const float* const* in, float* const* out, int64_t n, int64_t l, int64_t d, int64_t s,
                    float eps, float gamma) {
    return guarded([&] {
        SsmPassArgs a;
        std::copy(in, in + 12, a.in);
        std::copy(out, out + 10, a.out);
        a.n = n;
        a.l = l;
        a.d = d;
        a.s = s;
        a.eps = eps;
        a.gamma = gamma;
        driver_backend()->ssm_pass(static_cast<SsmPassOp>(op), a);
    });
}

int pxr_be_rl_rows(int op, const float* const* in, float* const* out, int64_t rows, int64_t cols, float scale,
                   float lower, float upper, float gamma, float tau, int64_t ignore_index) {
    return guarded([&] {
        RlRowArgs a;
        std::copy(in, in + 5, a.in);
        std::copy(out, out + 4, a.out);
        a.rows = rows;
        a.cols = cols;
        a.scale = scale;
        a.lower = lower;
        a.upper = upper;
        a.gamma = gamma;
        a.tau = tau;
        a.ignore_index = ignore_index;
        driver_backend()->rl_rows(static_cast<RlRowOp>(op), a);
    });
}

int pxr_be_synchronize(void) {
#ifdef PXR_ON_MI355X
    return guarded([&] { static_cast<MI355XBackend*>(driver_backend())->synchronize(); });
#else
    return 0;
#endif
}

int pxr_be_sum(const float* in, size_t n, float* out) {
    return guarded([&] { *out = driver_backend()->sum(in, n); });
}

int pxr_be_dot(const float* a, const float* b, size_t n, float* out) {
    return guarded([&] { *out = driver_backend()->dot(a, b, n); });
}

int pxr_be_allocate(size_t bytes, void** out) {
    return guarded([&] { *out = driver_backend()->allocate(bytes); });
}

void pxr_be_free(void* p) { driver_backend()->free(p); }

int pxr_be_device(void) { return static_cast<int>(driver_backend()->device()); }

}  // extern "C"
