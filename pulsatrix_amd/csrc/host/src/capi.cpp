// C ABI of the MI355X host framework (include/pulsatrix_amd.h).
#include "pulsatrix_amd.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <functional>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

#include "pulsatrix/causal_lm.hpp"
#include "pulsatrix/checkpoint.hpp"
#include "pulsatrix/mi355x_backend.hpp"
#include "pulsatrix/transformer_block.hpp"

using namespace pulsatrix;

namespace {

thread_local std::string g_error;

std::once_flag g_once;
std::unique_ptr<MI355XBackend> g_backend;

MI355XBackend* backend() {
    std::call_once(g_once, [] { g_backend = std::make_unique<MI355XBackend>(0); });
    return g_backend.get();
}

// Every entry point runs through guarded(): exceptions become -1 plus pxa_last_error(), and the
// model a call named (lm_handle) stops being the backend's current owner when the call returns.
template <typename F>
int guarded(F&& f) {
    int rc = 0;
    try {
        f();
    } catch (const std::exception& e) {
        g_error = e.what();
        rc = -1;
    }
    if (g_backend) g_backend->set_owner(0);
    return rc;
}

int64_t kv_heads(const px_model_config& c) { return c.num_kv_heads > 0 ? c.num_kv_heads : c.num_heads; }
int64_t head_dim(const px_model_config& c) { return c.head_dim > 0 ? c.head_dim : c.hidden_size / c.num_heads; }

// (size, is_norm_gamma) of each parameter of one block, in the flat blob's order.
std::vector<std::pair<int64_t, bool>> block_layout(const px_model_config& c) {
    const int64_t d = c.hidden_size, q = c.num_heads * head_dim(c), kv = kv_heads(c) * head_dim(c),
                  f = c.intermediate_size;
    std::vector<std::pair<int64_t, bool>> out{{d, true}};
    auto lin = [&](int64_t in, int64_t o, bool bias) {
        out.push_back({in * o, false});
        if (bias) out.push_back({o, false});
    };
    lin(d, q, c.qkv_bias);
    lin(d, kv, c.qkv_bias);
    lin(d, kv, c.qkv_bias);
    lin(q, d, c.out_bias);
    if (c.qk_norm) {
        out.push_back({head_dim(c), true});
        out.push_back({head_dim(c), true});
    }
    out.push_back({d, true});
    lin(d, f, c.mlp_bias);
    lin(d, f, c.mlp_bias);
    lin(f, d, c.mlp_bias);
    if (c.post_norms) {
        out.push_back({d, true});
        out.push_back({d, true});
    }
    return out;
}

std::vector<std::pair<int64_t, bool>> lm_layout(const px_model_config& c) {
    std::vector<std::pair<int64_t, bool>> out{{c.vocab_size * c.hidden_size, false}};
    for (int64_t i = 0; i < c.num_layers; ++i) {
        auto b = block_layout(c);
        out.insert(out.end(), b.begin(), b.end());
    }
    out.push_back({c.hidden_size, true});
    if (!c.tie_word_embeddings) out.push_back({c.hidden_size * c.vocab_size, false});
    return out;
}

int64_t total(const std::vector<std::pair<int64_t, bool>>& layout) {
    int64_t n = 0;
    for (const auto& e : layout) n += e.first;
    return n;
}

// The reference's HfModelConfig for a px_model_config (the fields ParseHfConfig fills).
HfModelConfig hf_config(const px_model_config& c) {
    if (c.hidden_act < 0 || c.hidden_act > 1) throw std::invalid_argument("model config: unknown hidden_act");
    if (c.rope_scaling < 0 || c.rope_scaling > 2) throw std::invalid_argument("model config: unknown rope_scaling");
    if (c.sliding_layers != 0 && c.num_layers > 64)
        throw std::invalid_argument("model config: sliding_layers names at most 64 layers");
    HfModelConfig hc;
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
    a.use_qk_norm = c.qk_norm != 0;
    a.qk_norm_eps = c.rms_norm_eps;
    a.qk_norm_weight_offset = c.norm_weight_offset;
    if (c.query_pre_attn_scalar > 0.0f)
        a.score_scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.query_pre_attn_scalar)));
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

std::vector<float> take(const float*& p, int64_t n) {
    std::vector<float> v(p, p + n);
    p += n;
    return v;
}

void load_linear(LinearModule& m, const float*& p) {
    m.set_weight(take(p, m.in_features() * m.out_features()));
    if (m.use_bias()) m.set_bias(take(p, m.out_features()));
}

void load_block(TransformerBlock& b, const float*& p) {
    b.norm1().set_gamma(take(p, b.norm1().num_features()));
    load_linear(b.mha().q_proj(), p);
    load_linear(b.mha().k_proj(), p);
    load_linear(b.mha().v_proj(), p);
    load_linear(b.mha().out_proj(), p);
    if (b.mha().config().use_qk_norm) {
        b.mha().q_norm().set_gamma(take(p, b.mha().q_norm().num_features()));
        b.mha().k_norm().set_gamma(take(p, b.mha().k_norm().num_features()));
    }
    b.norm2().set_gamma(take(p, b.norm2().num_features()));
    load_linear(b.swiglu().gate_proj(), p);
    load_linear(b.swiglu().up_proj(), p);
    load_linear(b.swiglu().down_proj(), p);
    if (b.has_post_norms()) {
        b.post_attn_norm().set_gamma(take(p, b.post_attn_norm().num_features()));
        b.post_mlp_norm().set_gamma(take(p, b.post_mlp_norm().num_features()));
    }
}

struct BlockHandle {
    std::unique_ptr<TransformerBlock> block;
    int64_t d = 0, n = 0, l = 0;
};

// A model handle. Its device blocks are allocated under its own owner tag, and its captured explain
// graph (declared after the model, so destroyed first) is validated against their frees.
struct LmHandle {
    uint64_t owner = 0;
    std::unique_ptr<CausalLM> lm;
    std::unique_ptr<CapturedGraph> graph;
    px_model_config cfg{};
    int64_t n = 0, l = 0;
};

// Live model handles: a destroyed or foreign handle is refused instead of dereferenced.
std::mutex g_lm_mutex;
std::unordered_set<const void*> g_lms;

LmHandle* new_lm_handle() {
    auto h = std::make_unique<LmHandle>();
    h->owner = backend()->new_owner();
    backend()->set_owner(h->owner);  // the model's buffers carry its tag
    return h.release();
}

LmHandle* register_lm(std::unique_ptr<LmHandle> h) {
    std::lock_guard<std::mutex> lock(g_lm_mutex);
    g_lms.insert(h.get());
    return h.release();
}

LmHandle* find_lm(const void* handle) {
    std::lock_guard<std::mutex> lock(g_lm_mutex);
    return g_lms.count(handle) ? static_cast<LmHandle*>(const_cast<void*>(handle)) : nullptr;
}

// The live model behind a handle, made the backend's current owner for the rest of the call.
LmHandle* lm_handle(const void* handle) {
    LmHandle* h = find_lm(handle);
    if (h == nullptr) throw std::invalid_argument("unknown or destroyed model handle");
    backend()->set_owner(h->owner);
    return h;
}

LmHandle* make_lm(const px_model_config& c, const float* params) {
    if (c.vocab_size <= 0 || c.num_layers <= 0) throw std::invalid_argument("model config: vocab_size and num_layers must be positive");
    const HfModelConfig hc = hf_config(c);
    if (!c.use_rope || !c.rope_rotate_half)
        throw std::invalid_argument("model config: the causal LM uses rotate-half RoPE (ToAttentionConfig)");
    std::unique_ptr<LmHandle> h(new_lm_handle());
    h->cfg = c;
    h->lm = std::make_unique<CausalLM>(hc, backend());
    const float* p = params;
    h->lm->embed_tokens().set_weight(take(p, c.vocab_size * c.hidden_size));
    for (int64_t i = 0; i < c.num_layers; ++i) load_block(h->lm->layer(i), p);
    h->lm->norm().set_gamma(take(p, c.hidden_size));
    if (!c.tie_word_embeddings) h->lm->lm_head()->set_weight(take(p, c.hidden_size * c.vocab_size));
    return register_lm(std::move(h));
}

LRPRuleConfig rule(float eps, int bias_in_denominator) {
    LRPRuleConfig r{eps};
    r.epsilon_bias_in_denominator = bias_in_denominator != 0;
    return r;
}

LRPRuleConfig rule(const px_lrp_rule* p) {
    if (p == nullptr) throw std::invalid_argument("LRP rule config is NULL");
    if (p->rule < 0 || p->rule > 3) throw std::invalid_argument("unknown LRPRule " + std::to_string(p->rule));
    LRPRuleConfig r{p->epsilon};
    r.rule = static_cast<LRPRule>(p->rule);
    r.gamma = p->gamma;
    r.alpha = p->alpha;
    r.beta = p->beta;
    r.low = p->low;
    r.high = p->high;
    r.epsilon_bias_in_denominator = p->bias_in_denominator != 0;
    return r;
}

// Runs `work` once eagerly, so that every buffer it uses exists at its final size, then captures
// it into the model's own graph (replacing any earlier one).
void capture(LmHandle* h, const std::function<void()>& work) {
    h->graph.reset();
    work();
    h->graph = backend()->capture(h->owner, work);
}

void block_relevance(void* handle, const float* r_out, const LRPRuleConfig& cfg, float* r_in) {
    auto* h = static_cast<BlockHandle*>(handle);
    if (h->n == 0) throw std::logic_error("TransformerBlock::propagate_relevance: called before any forward()");
    const int64_t count = h->n * h->l * h->d;
    Tensor r(Shape({h->n, h->l, h->d}), backend(), std::vector<float>(r_out, r_out + count));
    const std::vector<float> out = h->block->propagate_relevance(r, cfg).to_host_vector();
    std::copy(out.begin(), out.end(), r_in);
}

void lm_relevance(void* handle, const float* seed, const LRPRuleConfig& cfg, float* r_embed, float* r_tokens,
                  float* key_rel, float* value_rel) {
    LmHandle* h = lm_handle(handle);
    if (h->n == 0) throw std::logic_error("CausalLM::propagate_relevance_by_layer: called before any forward()");
    CausalLM& lm = *h->lm;
    const px_model_config& c = h->cfg;
    const int64_t count = h->n * h->l * c.vocab_size;
    Tensor s(Shape({h->n, h->l, c.vocab_size}), backend(), std::vector<float>(seed, seed + count));
    const std::vector<Tensor> bounds = lm.propagate_relevance_by_layer(s, cfg);
    auto to_host = [](const Tensor& t, float* dst) {
        const std::vector<float> v = t.to_host_vector();
        std::copy(v.begin(), v.end(), dst);
    };
    if (r_embed) to_host(bounds.front(), r_embed);
    if (r_tokens) to_host(lm.embed_tokens().propagate_relevance(bounds.front(), cfg), r_tokens);
    const int64_t kv = h->n * h->l * kv_heads(c) * head_dim(c);
    for (int64_t i = 0; i < lm.num_layers(); ++i) {
        if (key_rel) to_host(lm.layer(i).mha().key_relevance(), key_rel + i * kv);
        if (value_rel) to_host(lm.layer(i).mha().value_relevance(), value_rel + i * kv);
    }
}

}  // namespace

extern "C" {

const char* pxa_last_error(void) { return g_error.c_str(); }

int pxa_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

void* pxa_backend(void) {
    void* out = nullptr;
    guarded([&] { out = backend(); });
    return out;
}

void* pxa_backend_stream(void) {
    void* out = nullptr;
    guarded([&] { out = backend()->stream(); });
    return out;
}

int pxa_backend_synchronize(void) {
    return guarded([&] { backend()->synchronize(); });
}

int pxa_backend_memory(size_t* in_use, size_t* cached) {
    return guarded([&] {
        const auto st = backend()->allocator().stats();
        if (in_use) *in_use = st.in_use_bytes;
        if (cached) *cached = st.cached_bytes;
    });
}

int pxa_launch_log_start(void) {
    return guarded([&] { backend()->start_launch_log(); });
}

int pxa_launch_log_stop(int64_t* count) {
    return guarded([&] {
        backend()->stop_launch_log();
        if (count) *count = static_cast<int64_t>(backend()->launch_log().size());
    });
}

int pxa_launch_log_entry(int64_t index, char* kernel, size_t kernel_cap, char* family, size_t family_cap,
                         double* flops, double* bytes) {
    return guarded([&] {
        const auto& log = backend()->launch_log();
        if (index < 0 || static_cast<size_t>(index) >= log.size())
            throw std::invalid_argument("pxa_launch_log_entry: index outside the log");
        const LaunchRecord& r = log[static_cast<size_t>(index)];
        if (kernel && kernel_cap > 0) std::snprintf(kernel, kernel_cap, "%s", r.kernel.c_str());
        if (family && family_cap > 0) std::snprintf(family, family_cap, "%s", r.family.c_str());
        if (flops) *flops = r.flops;
        if (bytes) *bytes = r.bytes;
    });
}

int pxa_launch_log_dispatches(int64_t index, int32_t* count) {
    return guarded([&] {
        const auto& log = backend()->launch_log();
        if (index < 0 || static_cast<size_t>(index) >= log.size() || count == nullptr)
            throw std::invalid_argument("pxa_launch_log_dispatches: index outside the log, or count NULL");
        *count = log[static_cast<size_t>(index)].dispatches;
    });
}

int pxa_launch_log_time(int reps, double* seconds) {
    return guarded([&] {
        if (reps <= 0) throw std::invalid_argument("pxa_launch_log_time: reps must be positive");
        std::vector<double> t;
        backend()->time_launch_log(reps, t);
        if (seconds) std::copy(t.begin(), t.end(), seconds);
    });
}

void pxa_fill_normal(float* dst, size_t n, uint64_t seed, double stddev) {
    uint64_t state = seed;
    auto next = [&state]() {  // SplitMix64
        state += 0x9E3779B97F4A7C15ULL;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        return z ^ (z >> 31);
    };
    auto uniform = [&]() { return (static_cast<double>(next() >> 11) + 0.5) / static_cast<double>(1ULL << 53); };
    constexpr double kTwoPi = 6.28318530717958647692;
    for (size_t i = 0; i < n; ++i) {
        const double u1 = uniform();
        const double u2 = uniform();
        dst[i] = static_cast<float>(stddev * (std::sqrt(-2.0 * std::log(u1)) * std::cos(kTwoPi * u2)));
    }
}

int64_t pxa_param_count(const px_model_config* cfg) { return total(lm_layout(*cfg)); }
int64_t pxa_block_param_count(const px_model_config* cfg) { return total(block_layout(*cfg)); }

int pxa_synthetic_params(const px_model_config* cfg, int block, uint64_t seed, double stddev, float* dst) {
    return guarded([&] {
        const auto layout = block ? block_layout(*cfg) : lm_layout(*cfg);
        pxa_fill_normal(dst, static_cast<size_t>(total(layout)), seed, stddev);
        int64_t off = 0;
        const float g = 1.0f - cfg->norm_weight_offset;  // every RMSNorm's effective scale 1
        for (const auto& [size, gamma] : layout) {
            if (gamma)
                for (int64_t i = 0; i < size; ++i) dst[off + i] = g;
            off += size;
        }
    });
}

void* pxa_block_create(const px_model_config* cfg, const float* params) {
    BlockHandle* out = nullptr;
    guarded([&] {
        auto h = std::make_unique<BlockHandle>();
        h->block = std::make_unique<TransformerBlock>(attention_config(*cfg), cfg->intermediate_size, backend(),
                                                      block_options(*cfg));
        const float* p = params;
        load_block(*h->block, p);
        h->d = cfg->hidden_size;
        out = h.release();
    });
    return out;
}

int pxa_block_forward(void* handle, const float* x, int64_t n, int64_t l, float* y) {
    return guarded([&] {
        auto* h = static_cast<BlockHandle*>(handle);
        Tensor in(Shape({n, l, h->d}), backend(), std::vector<float>(x, x + n * l * h->d));
        const std::vector<float> out = h->block->forward(in).to_host_vector();
        std::copy(out.begin(), out.end(), y);
        h->n = n;
        h->l = l;
    });
}

int pxa_block_relevance(void* handle, const float* r_out, float eps, int bias_in_denominator, float* r_in) {
    return guarded([&] { block_relevance(handle, r_out, rule(eps, bias_in_denominator), r_in); });
}

int pxa_block_relevance_rule(void* handle, const float* r_out, const px_lrp_rule* p, float* r_in) {
    return guarded([&] { block_relevance(handle, r_out, rule(p), r_in); });
}

int pxa_linear_relevance_rule(const float* x, const float* w, const float* bias, int64_t n, int64_t in, int64_t out,
                              const float* r, const px_lrp_rule* p, float* y, float* r_in) {
    return guarded([&] {
        const LRPRuleConfig cfg = rule(p);
        LinearModule layer(in, out, backend(), bias != nullptr);
        layer.set_weight(std::vector<float>(w, w + in * out));
        if (bias) layer.set_bias(std::vector<float>(bias, bias + out));
        const std::vector<float> xs(x, x + n * in);
        const Tensor fy = layer.forward(Tensor(Shape({n, in}), backend(), xs));
        if (y) {
            const std::vector<float> v = fy.to_host_vector();
            std::copy(v.begin(), v.end(), y);
        }
        const Tensor rr(Shape({n, out}), backend(), std::vector<float>(r, r + n * out));
        const std::vector<float> v = layer.propagate_relevance(rr, cfg).to_host_vector();
        std::copy(v.begin(), v.end(), r_in);
    });
}

void pxa_block_destroy(void* handle) { delete static_cast<BlockHandle*>(handle); }

void* pxa_lm_create(const px_model_config* cfg, const float* params) {
    LmHandle* out = nullptr;
    guarded([&] { out = make_lm(*cfg, params); });
    return out;
}

void* pxa_lm_create_random(const px_model_config* cfg, uint64_t seed, double stddev) {
    LmHandle* out = nullptr;
    guarded([&] {
        std::vector<float> params(static_cast<size_t>(total(lm_layout(*cfg))));
        if (pxa_synthetic_params(cfg, 0, seed, stddev, params.data()) != 0) throw std::runtime_error(g_error);
        out = make_lm(*cfg, params.data());
    });
    return out;
}

void* pxa_lm_load(const char* directory, px_model_config* cfg_out) {
    LmHandle* out = nullptr;
    guarded([&] {
        if (directory == nullptr) throw std::invalid_argument("pxa_lm_load: directory is NULL");
        std::unique_ptr<LmHandle> h(new_lm_handle());
        h->lm = LoadCausalLM(directory, backend());
        const HfModelConfig& hc = h->lm->config();
        px_model_config& c = h->cfg;
        c.vocab_size = hc.vocab_size;
        c.hidden_size = hc.hidden_size;
        c.num_layers = hc.num_hidden_layers;
        c.num_heads = hc.num_attention_heads;
        c.num_kv_heads = hc.num_key_value_heads;
        c.head_dim = hc.head_dim;
        c.intermediate_size = hc.intermediate_size;
        c.rms_norm_eps = hc.rms_norm_eps;
        c.rope_theta = hc.rope_theta;
        c.use_rope = 1;
        c.rope_rotate_half = 1;
        c.causal = hc.causal ? 1 : 0;
        c.qkv_bias = hc.qkv_bias ? 1 : 0;
        c.out_bias = hc.out_bias ? 1 : 0;
        c.mlp_bias = hc.mlp_bias ? 1 : 0;
        c.tie_word_embeddings = hc.tie_word_embeddings ? 1 : 0;
        c.hidden_act = hc.hidden_act == "silu" ? 0 : 1;
        c.qk_norm = hc.qk_norm ? 1 : 0;
        c.post_norms = hc.post_norms ? 1 : 0;
        c.norm_weight_offset = hc.norm_weight_offset;
        c.embed_scale = hc.embed_scale;
        c.query_pre_attn_scalar = hc.query_pre_attn_scalar.value_or(0.0f);
        c.rope_local_base = hc.rope_local_base_freq.value_or(0.0f);
        if (hc.rope_scaling) {
            c.rope_scaling = hc.rope_scaling->type == "linear" ? 1 : 2;
            c.rope_factor = hc.rope_scaling->factor;
            c.rope_low_freq_factor = hc.rope_scaling->low_freq_factor;
            c.rope_high_freq_factor = hc.rope_scaling->high_freq_factor;
            c.rope_original_max_position = hc.rope_scaling->original_max_position_embeddings;
        }
        c.sliding_window = hc.sliding_window.value_or(0);
        for (size_t i = 0; i < hc.layer_types.size() && i < 64; ++i)
            if (hc.layer_types[i] == "sliding_attention") c.sliding_layers |= uint64_t{1} << i;
        if (cfg_out) *cfg_out = c;
        out = register_lm(std::move(h));
    });
    return out;
}

int pxa_lm_forward(void* handle, const int64_t* ids, int64_t n, int64_t l, float* logits) {
    return guarded([&] {
        LmHandle* h = lm_handle(handle);
        std::vector<float> f(static_cast<size_t>(n * l));
        for (size_t i = 0; i < f.size(); ++i) f[i] = static_cast<float>(ids[i]);
        Tensor out = h->lm->forward(Tensor(Shape({n, l}), backend(), f));
        h->n = n;
        h->l = l;
        if (logits) {
            const std::vector<float> v = out.to_host_vector();
            std::copy(v.begin(), v.end(), logits);
        }
    });
}

int pxa_lm_relevance(void* handle, const float* seed, float eps, int bias_in_denominator, float* r_embed,
                     float* r_tokens, float* key_rel, float* value_rel) {
    return guarded(
        [&] { lm_relevance(handle, seed, rule(eps, bias_in_denominator), r_embed, r_tokens, key_rel, value_rel); });
}

int pxa_lm_relevance_rule(void* handle, const float* seed, const px_lrp_rule* p, float* r_embed, float* r_tokens,
                          float* key_rel, float* value_rel) {
    return guarded([&] { lm_relevance(handle, seed, rule(p), r_embed, r_tokens, key_rel, value_rel); });
}

int pxa_lm_explain_device(void* handle, const float* ids, int64_t n, int64_t l, float eps, int bias_in_denominator,
                          float* token_rel, int64_t* targets, const int64_t* targets_in, int unit_seed) {
    return guarded([&] {
        LmHandle* h = lm_handle(handle);
        h->lm->explain_device(ids, n, l, rule(eps, bias_in_denominator), token_rel, targets, targets_in, unit_seed != 0);
    });
}

int pxa_lm_capture_explain(void* handle, const float* ids, int64_t n, int64_t l, float eps, int bias_in_denominator,
                           float* token_rel, int64_t* targets) {
    return guarded([&] {
        LmHandle* h = lm_handle(handle);
        const LRPRuleConfig cfg = rule(eps, bias_in_denominator);
        capture(h, [&] { h->lm->explain_device(ids, n, l, cfg, token_rel, targets, nullptr, false); });
    });
}

int pxa_lm_explain_device_rule(void* handle, const float* ids, int64_t n, int64_t l, const px_lrp_rule* p,
                               float* token_rel, int64_t* targets, const int64_t* targets_in, int unit_seed) {
    return guarded([&] {
        LmHandle* h = lm_handle(handle);
        h->lm->explain_device(ids, n, l, rule(p), token_rel, targets, targets_in, unit_seed != 0);
    });
}

int pxa_lm_capture_explain_rule(void* handle, const float* ids, int64_t n, int64_t l, const px_lrp_rule* p,
                                float* token_rel, int64_t* targets) {
    return guarded([&] {
        LmHandle* h = lm_handle(handle);
        const LRPRuleConfig cfg = rule(p);
        capture(h, [&] { h->lm->explain_device(ids, n, l, cfg, token_rel, targets, nullptr, false); });
    });
}

int pxa_lm_explain_rows_device(void* handle, const float* ids, int64_t n, int64_t l, const float* targets,
                               int64_t target_stride, const px_lrp_rule* p, float* token_rel, int64_t* targets_out,
                               int unit_seed) {
    return guarded([&] {
        lm_handle(handle)->lm->explain_rows_device(ids, n, l, targets, target_stride, rule(p), token_rel,
                                                                targets_out, unit_seed != 0);
    });
}

int pxa_lm_generate_device(void* handle, float* ids, int64_t n, int64_t prompt, int64_t new_tokens, int64_t ld_ids,
                           float* picked_logit) {
    return guarded([&] {
        lm_handle(handle)->lm->generate_greedy_device(ids, n, prompt, new_tokens, ld_ids, picked_logit);
    });
}

int pxa_lm_explain_generated_device(void* handle, const float* ids, int64_t n, int64_t prompt, int64_t new_tokens,
                                    int64_t ld_ids, const px_lrp_rule* p, float* token_rel, int unit_seed) {
    return guarded([&] {
        lm_handle(handle)->lm->explain_generated_device(ids, n, prompt, new_tokens, ld_ids, rule(p),
                                                                     token_rel, unit_seed != 0);
    });
}

namespace {
struct NextTokenHandle {
    NextTokenLogitsFn fn;
    int64_t vocab;
    const void* model;  // the LmHandle whose caches and buffers fn uses
};
}  // namespace

void* pxa_lm_next_token_logits_create(void* handle, int64_t max_length) {
    NextTokenHandle* out = nullptr;
    guarded([&] {
        LmHandle* h = lm_handle(handle);
        out = new NextTokenHandle{h->lm->next_token_logits(max_length), h->lm->config().vocab_size, h};
    });
    return out;
}

int pxa_lm_next_token_logits(void* f, const int64_t* tokens, int64_t n, float* logits, int64_t vocab) {
    return guarded([&] {
        auto* h = static_cast<NextTokenHandle*>(f);
        if (h == nullptr) throw std::invalid_argument("pxa_lm_next_token_logits: NULL function handle");
        (void)lm_handle(h->model);  // refuses a function whose model was destroyed
        if (vocab != h->vocab)
            throw std::invalid_argument("pxa_lm_next_token_logits: the logits buffer holds " + std::to_string(vocab) +
                                        " entries, the vocabulary " + std::to_string(h->vocab));
        if (n < 0) throw std::invalid_argument("pxa_lm_next_token_logits: negative length");
        const std::vector<float> out = h->fn(std::vector<int64_t>(tokens, tokens + n));
        std::copy(out.begin(), out.end(), logits);
    });
}

void pxa_lm_next_token_logits_destroy(void* f) { delete static_cast<NextTokenHandle*>(f); }

int pxa_lm_replay(void* handle) {
    return guarded([&] {
        LmHandle* h = lm_handle(handle);
        if (!h->graph) throw std::logic_error("pxa_lm_replay: nothing was captured for this model");
        h->graph->replay();
    });
}

int pxa_lm_check_device_ids(void* handle) {
    return guarded([&] {
        if (!lm_handle(handle)->lm->device_ids_valid())
            throw std::invalid_argument("EmbeddingModule::forward: index out of range [0, num_embeddings)");
    });
}

const float* pxa_lm_last_logits(void* handle) {
    LmHandle* h = find_lm(handle);
    return h ? h->lm->last_logits() : nullptr;
}
const float* pxa_lm_last_embedding_relevance(void* handle) {
    LmHandle* h = find_lm(handle);
    return h ? h->lm->last_embedding_relevance() : nullptr;
}

void pxa_lm_destroy(void* handle) {
    LmHandle* h = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_lm_mutex);
        if (g_lms.erase(handle) == 0) return;  // NULL, unknown or already destroyed
        h = static_cast<LmHandle*>(handle);
    }
    const uint64_t owner = h->owner;
    delete h;  // its graph first (after the stream drains), then the model's buffers
    if (g_backend) g_backend->forget_owner(owner);
}

}  // extern "C"
