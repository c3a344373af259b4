// CausalLM on MI355XBackend (src/causal_lm.cpp, src/hf_model.cpp:282-313).
#include "pulsatrix/causal_lm.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>

namespace pulsatrix {

bool HfModelConfig::is_sliding_layer(int64_t i) const {
    if (!sliding_window) return false;
    if (layer_types.empty()) return true;
    return i >= 0 && static_cast<size_t>(i) < layer_types.size() &&
           layer_types[static_cast<size_t>(i)] == "sliding_attention";
}

// Rotary inverse frequencies theta^(-2p / head_dim) for the pairs p < head_dim / 2, in double, then
// the two rope_scaling kinds the loader accepts. "linear" divides every frequency by the factor.
// "llama3" is Hugging Face's published llama3 rule (_compute_llama3_parameters): with the original
// context C, a frequency whose wavelength 2 pi / f exceeds C / low_freq_factor is divided by the
// factor, one whose wavelength is below C / high_freq_factor is kept, and the band between (both
// edges included) blends the two with t = (C / wavelength - low) / (high - low) as
// (1 - t) f / factor + t f, the operations in the order Hugging Face evaluates them.
std::vector<double> RopeInverseFrequencies(const HfModelConfig& config) {
    const double dim = static_cast<double>(config.head_dim);
    std::vector<double> freq;
    freq.reserve(static_cast<size_t>(config.head_dim / 2));
    for (int64_t pair = 0; pair < config.head_dim / 2; ++pair)
        freq.push_back(1.0 / std::pow(static_cast<double>(config.rope_theta), 2.0 * static_cast<double>(pair) / dim));
    if (!config.rope_scaling) return freq;
    const HfRopeScaling& rs = *config.rope_scaling;
    if (rs.type == "linear") {
        std::transform(freq.begin(), freq.end(), freq.begin(), [&](double f) { return f / rs.factor; });
        return freq;
    }
    if (rs.type != "llama3")
        throw std::invalid_argument("RopeInverseFrequencies: rope_scaling \"" + rs.type + "\" is not supported");
    const double context = static_cast<double>(rs.original_max_position_embeddings);
    const double stretch_above = context / rs.low_freq_factor;  // longer wavelengths: divided by the factor
    const double keep_below = context / rs.high_freq_factor;    // shorter wavelengths: unchanged
    const double full_turn = 2.0 * 3.14159265358979323846;
    std::transform(freq.begin(), freq.end(), freq.begin(), [&](double f) {
        const double wavelength = full_turn / f;
        if (wavelength > stretch_above) return f / rs.factor;
        if (wavelength < keep_below) return f;
        const double t = (context / wavelength - rs.low_freq_factor) / (rs.high_freq_factor - rs.low_freq_factor);
        return (1.0 - t) * f / rs.factor + t * f;
    });
    return freq;
}

AttentionConfig ToAttentionConfig(const HfModelConfig& config) {
    AttentionConfig a;
    a.d_model = config.hidden_size;
    a.num_heads = config.num_attention_heads;
    a.num_kv_heads = config.num_key_value_heads;
    a.head_dim = config.head_dim;
    a.use_rope = true;
    a.rope_layout = RoPELayout::RotateHalf;
    a.rope_base = config.rope_theta;
    if (config.rope_scaling) a.rope_inverse_frequencies = RopeInverseFrequencies(config);
    a.use_qk_norm = config.qk_norm;
    a.qk_norm_eps = config.rms_norm_eps;
    a.qkv_bias = config.qkv_bias;
    a.out_bias = config.out_bias;
    a.causal = config.causal;
    if (config.query_pre_attn_scalar)
        a.score_scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(*config.query_pre_attn_scalar)));
    a.qk_norm_weight_offset = config.norm_weight_offset;
    return a;
}

AttentionConfig ToAttentionConfig(const HfModelConfig& config, int64_t layer) {
    AttentionConfig a = ToAttentionConfig(config);
    if (!config.is_sliding_layer(layer)) return a;
    a.sliding_window = *config.sliding_window;
    if (config.rope_local_base_freq) {
        a.rope_base = *config.rope_local_base_freq;
        a.rope_inverse_frequencies.clear();
    }
    return a;
}

namespace {

const HfModelConfig& checked(const HfModelConfig& c) {
    if (c.hidden_size <= 0 || c.num_hidden_layers <= 0 || c.vocab_size <= 0 || c.intermediate_size <= 0)
        throw std::invalid_argument("CausalLM: hidden_size, num_hidden_layers, vocab_size and intermediate_size "
                                    "must be positive");
    if (c.hidden_act != "silu" && c.hidden_act != "gelu_pytorch_tanh" && c.hidden_act != "gelu_new")
        throw std::invalid_argument("CausalLM: the config needs features pulsatrix can't run yet: activation \"" +
                                    c.hidden_act + "\" in the MLP");
    return c;
}

TransformerBlockOptions block_options(const HfModelConfig& c) {  // causal_lm.cpp:36-41
    TransformerBlockOptions o;
    o.norm_eps = c.rms_norm_eps;
    o.mlp_bias = c.mlp_bias;
    o.mlp_activation = c.hidden_act == "silu" ? GatedActivation::Silu : GatedActivation::GeluTanh;
    o.post_norms = c.post_norms;
    o.norm_weight_offset = c.norm_weight_offset;
    return o;
}

}  // namespace

CausalLM::CausalLM(const HfModelConfig& config, DeviceBackend* backend)
    : config_(checked(config)),
      be_(detail::require_mi355x(backend, "CausalLM")),
      embed_(config.vocab_size, config.hidden_size, backend),
      norm_(config.hidden_size, backend, DeviceType::Hip, config.rms_norm_eps) {
    norm_.set_weight_offset(config.norm_weight_offset);
    // Each layer's own attention: Gemma 3 alternates sliding-window and full layers, each with its
    // own RoPE base (causal_lm.cpp:42-47).
    for (int64_t i = 0; i < config.num_hidden_layers; ++i)
        layers_.push_back(std::make_unique<TransformerBlock>(ToAttentionConfig(config, i), config.intermediate_size,
                                                             backend, block_options(config)));
    if (config.tie_word_embeddings)
        tied_head_ = std::make_unique<TiedLMHeadModule>(embed_, backend);
    else
        lm_head_ = std::make_unique<LinearModule>(config.hidden_size, config.vocab_size, backend, false);
}

const float* CausalLM::last_logits() const noexcept { return tied_head_ ? tied_head_->logits() : nullptr; }

const float* CausalLM::run_forward_hidden(const float* ids, int64_t n, int64_t l) {
    N_ = n;
    L_ = l;
    const int64_t M = n * l;
    const float* x = embed_.run_forward_device(ids, n, l);
    if (config_.embed_scale != 1.0f) {  // ScaleEmbeddings (causal_lm.cpp:56-61), in the gather's own buffer
        float* xs = const_cast<float*>(x);
        MI355XBackend::check(pxk_axpby(config_.embed_scale, xs, 0.0f, nullptr, xs, M * config_.hidden_size,
                                       be_->stream()),
                             "CausalLM::forward");
    }
    for (auto& layer : layers_) x = layer->run_forward(x, n, l);
    return norm_.run_forward(x, M);
}

const float* CausalLM::run_forward(const float* ids, int64_t n, int64_t l) {
    const int64_t M = n * l;
    const float* xn = run_forward_hidden(ids, n, l);
    return tied_head_ ? tied_head_->run_forward(xn, M) : lm_head_->run_forward(xn, M);
}

const float* CausalLM::forward_last_rows(const float* ids, int64_t n, int64_t l) {
    const int64_t d = config_.hidden_size;
    const float* xn = run_forward_hidden(ids, n, l);
    float* xl = last_x_.ensure(be_, n * d);
    be_->copy_2d(xl, static_cast<size_t>(d), xn + (l - 1) * d, static_cast<size_t>(l * d), static_cast<size_t>(n),
                 static_cast<size_t>(d));
    return tied_head_ ? tied_head_->run_forward(xl, n) : lm_head_->run_forward(xl, n);
}

const float* CausalLM::run_relevance(const float* seed, const LRPRuleConfig& config) {
    if (N_ == 0) throw std::logic_error("CausalLM::propagate_relevance_by_layer: called before any forward()");
    // The final RMSNorm passes relevance through unchanged (rms_norm_module.cpp:101-111). Each
    // residual sum's epsilon split (lrp_residual_split) runs inside the GEMM that produces the
    // sum's relevance: the head's for the top block's output, each block's q/k/v GEMM for the
    // output of the block below.
    const size_t nl = layers_.size();
    const detail::ResidualSplit top = nl > 0 ? layers_.back()->output_split(&config) : detail::ResidualSplit{};
    const float* r = tied_head_ ? tied_head_->run_relevance(seed, config, top)
                                : lm_head_->run_relevance(seed, config, nullptr, top);
    for (size_t i = nl; i-- > 0;)
        r = layers_[i]->run_relevance_split(config, i > 0 ? layers_[i - 1]->output_split(&config) : detail::ResidualSplit{});
    r_embed_ = r;
    return r;
}

void CausalLM::explain_device(const float* ids, int64_t n, int64_t l, const LRPRuleConfig& config,
                              float* token_relevance, int64_t* targets, const int64_t* targets_in, bool unit_seed) {
    const int64_t V = config_.vocab_size, M = n * l;
    const float* logits = run_forward(ids, n, l);
    if (tied_head_ && !detail::is_affine_rule(config)) {
        // The seed is one-hot at each sequence's last row, so the head's epsilon rule has one
        // nonzero row per sequence: those rows alone, straight into the top block's residual split.
        detail::validate_rule(config, "CausalLM");
        const size_t nl = layers_.size();
        const detail::ResidualSplit top = nl > 0 ? layers_.back()->output_split(&config) : detail::ResidualSplit{};
        const float* r = tied_head_->run_seeded_relevance(n, l, targets_in, targets, unit_seed, config, top);
        for (size_t i = nl; i-- > 0;)
            r = layers_[i]->run_relevance_split(config, i > 0 ? layers_[i - 1]->output_split(&config) : detail::ResidualSplit{});
        r_embed_ = r;
        embed_.token_relevance(r, M, token_relevance);
        return;
    }
    float* seed = seed_.ensure(be_, M * V);
    // the seed's zero fill (N L V floats) plus one scan of each sequence's last logit row
    const std::vector<int64_t> given = targets_in ? std::vector<int64_t>(targets_in, targets_in + n) : std::vector<int64_t>();
    be_->launch("lm_seed", "rows", 0.0, 4.0 * (M * V + n * V), "CausalLM::explain_device (seed)", [=](void* st) {
        return pxk_lm_seed(logits, n, l, V, given.empty() ? nullptr : given.data(), targets, seed, unit_seed, st);
    });
    embed_.token_relevance(run_relevance(seed, config), M, token_relevance);
}

void CausalLM::explain_rows_device(const float* ids, int64_t n, int64_t l, const float* targets, int64_t target_stride,
                                   const LRPRuleConfig& config, float* token_relevance, int64_t* targets_out,
                                   bool unit_seed) {
    if (n <= 0 || l <= 0) throw std::invalid_argument("CausalLM::explain_rows_device: n and l must be positive");
    explain_staggered_rows(ids, n, 1, l, targets, target_stride, config, token_relevance, targets_out, unit_seed,
                           false);
}

void CausalLM::explain_staggered_rows(const float* ids, int64_t n, int64_t groups, int64_t l, const float* targets,
                                      int64_t target_stride, const LRPRuleConfig& config, float* token_relevance,
                                      int64_t* targets_out, bool unit_seed, bool replicate) {
    const int64_t V = config_.vocab_size, d = config_.hidden_size, S = groups * n, M = S * l;
    void* st = be_->stream();
    // Layers and final norm over every row (once over n sequences and repeated when the copies are
    // identical); the head on the seeded row of each sequence only.
    const float* xn = nullptr;
    if (replicate) {
        xn = run_forward_hidden(ids, n, l);
        embed_.replicate_forward(groups);
        for (auto& layer : layers_) layer->replicate_forward(groups);
        norm_.replicate_forward(groups);
        N_ = S;
    } else {
        xn = run_forward_hidden(ids, S, l);
    }
    float* xl = last_x_.ensure(be_, S * d);
    for (int64_t g = 0; g < groups; ++g)
        be_->copy_2d(xl + g * n * d, static_cast<size_t>(d), xn + (g * n * l + l - groups + g) * d,
                     static_cast<size_t>(l * d), static_cast<size_t>(n), static_cast<size_t>(d));
    const float* logits = tied_head_ ? tied_head_->run_forward(xl, S) : lm_head_->run_forward(xl, S);
    float* seed = seed_.ensure(be_, S * V);
    for (int64_t g = 0; g < groups; ++g)
        MI355XBackend::check(pxk_seed_rows(logits + g * n * V, V, targets + g, target_stride, n, V, seed + g * n * V,
                                           targets_out ? targets_out + g * n : nullptr, unit_seed, st),
                             "CausalLM::explain_rows_device (seed)");
    // The head's rule on the seeded rows, then those rows' relevance placed at their rows of the
    // stack's output (every other row's is zero, as the dense pass computes it).
    const float* rl = tied_head_ ? tied_head_->run_relevance(seed, config) : lm_head_->run_relevance(seed, config);
    float* rtop = r_top_.ensure(be_, M * d);
    MI355XBackend::check(pxk_fill(rtop, 0.0f, M * d, st), "CausalLM::explain_rows_device");
    for (int64_t g = 0; g < groups; ++g)
        be_->copy_2d(rtop + (g * n * l + l - groups + g) * d, static_cast<size_t>(l * d), rl + g * n * d,
                     static_cast<size_t>(d), static_cast<size_t>(n), static_cast<size_t>(d));
    const float* r = rtop;
    if (!layers_.empty()) {  // the final RMSNorm passes relevance unchanged
        const detail::ResidualSplit top = layers_.back()->output_split();
        MI355XBackend::check(pxk_lrp_residual_split(top.a, top.b, rtop, top.r_a, top.r_b, M * d, config.epsilon, st),
                             "CausalLM::explain_rows_device");
        for (size_t i = layers_.size(); i-- > 0;)
            r = layers_[i]->run_relevance_split(config, i > 0 ? layers_[i - 1]->output_split(&config) : detail::ResidualSplit{});
    }
    r_embed_ = r;
    embed_.token_relevance(r, M, token_relevance);
}

void CausalLM::generate_greedy_device(float* ids, int64_t n, int64_t prompt, int64_t new_tokens, int64_t ld_ids,
                                      float* picked_logit) {
    if (!config_.causal)
        throw std::logic_error("CausalLM::next_token_logits: the model attends bidirectionally (a diffusion LM), so it "
                               "has no next-token cache");
    if (n <= 0 || prompt <= 0 || new_tokens <= 0)
        throw std::invalid_argument("CausalLM::generate: n, the prompt length and new_tokens must be positive");
    if (ld_ids < prompt + new_tokens)
        throw std::invalid_argument("CausalLM::generate: the id rows must hold the prompt and every new token");
    const int64_t V = config_.vocab_size;
    const int64_t positions = prompt + new_tokens - 1;  // the last generated token is never fed back
    void* st = be_->stream();
    // 1. the prompts: one forward fills every layer's cache; its last rows pick the first token.
    float* pid = prompt_ids_.ensure(be_, n * prompt);
    be_->copy_2d(pid, static_cast<size_t>(prompt), ids, static_cast<size_t>(ld_ids), static_cast<size_t>(n),
                 static_cast<size_t>(prompt));
    const float* logits = forward_last_rows(pid, n, prompt);
    caches_.resize(layers_.size());
    for (size_t i = 0; i < layers_.size(); ++i) layers_[i]->mha().export_kv(caches_[i], positions);
    auto* pos = reinterpret_cast<int32_t*>(pos_.ensure(be_, 1));
    const int32_t start = static_cast<int32_t>(prompt - 1);
    be_->copy(pos, &start, sizeof(start), CopyDirection::HostToDevice);
    float* cur = cur_ids_.ensure(be_, n);
    const size_t pick_bytes = pxk_decode_pick_workspace(n);
    void* pick_ws = pick_ws_.ensure(be_, static_cast<int64_t>(pick_bytes / sizeof(float)));
    auto pick = [&](const float* lg) {
        MI355XBackend::check(pxk_decode_pick(lg, V, n, V, ids, ld_ids, cur, picked_logit, ld_ids, pos, pick_ws,
                                             pick_bytes, st),
                             "CausalLM::generate (pick)");
        MI355XBackend::check(pxk_decode_advance(pos, st), "CausalLM::generate (advance)");
    };
    pick(logits);
    // 2. decode steps: the step's own token in, the next one out, at the device position.
    auto step = [&] { pick(decode_logits(cur, n, caches_, pos)); };
    if (new_tokens < 2) return;
    step();  // eagerly once: every buffer and workspace the step uses exists before the capture
    if (new_tokens < 3) return;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    auto hip = [](hipError_t e, const char* what) {
        if (e != hipSuccess) throw std::runtime_error(std::string("CausalLM::generate: ") + what + ": " + hipGetErrorString(e));
    };
    hip(hipStreamBeginCapture(static_cast<hipStream_t>(st), hipStreamCaptureModeThreadLocal), "begin capture");
    try {
        step();
    } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(static_cast<hipStream_t>(st), &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    hip(hipStreamEndCapture(static_cast<hipStream_t>(st), &graph), "end capture");
    const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (inst != hipSuccess) {
        (void)hipGraphDestroy(graph);
        hip(inst, "instantiate");
    }
    hipError_t rc = hipSuccess;
    for (int64_t t = 2; t < new_tokens && rc == hipSuccess; ++t) rc = hipGraphLaunch(exec, static_cast<hipStream_t>(st));
    // The graph is released only once its replays have run.
    const hipError_t done = hipStreamSynchronize(static_cast<hipStream_t>(st));
    (void)hipGraphExecDestroy(exec);
    (void)hipGraphDestroy(graph);
    hip(rc, "replay");
    hip(done, "synchronize");
}

const float* CausalLM::decode_logits(const float* cur, int64_t n, std::vector<KVCacheState>& caches,
                                     const int32_t* pos) {
    const int64_t d = config_.hidden_size;
    void* st = be_->stream();
    float* x = dec_x_.ensure(be_, n * d);
    MI355XBackend::check(pxk_gather_rows(embed_.weight_data(), cur, x, n, d, st), "CausalLM::decode");
    if (config_.embed_scale != 1.0f)
        MI355XBackend::check(pxk_axpby(config_.embed_scale, x, 0.0f, nullptr, x, n * d, st), "CausalLM::decode");
    const float* h = x;
    const float* hn = nullptr;  // norm1(h) of the next layer (or the final norm) when a block wrote it
    for (size_t i = 0; i < layers_.size(); ++i) {
        RMSNormModule* next = i + 1 < layers_.size() ? &layers_[i + 1]->norm1() : &norm_;
        h = layers_[i]->decode_step(h, hn, n, caches[i], pos, next, &hn);
    }
    if (!hn) hn = norm_.run_forward(h, n);
    return tied_head_ ? tied_head_->run_forward(hn, n) : lm_head_->run_forward(hn, n);
}

// The state a next_token_logits() function owns: its KV caches, the history and its logits, the
// step's device inputs (token id and position) and the captured graph of the step.
struct CausalLM::NextTokenState {
    explicit NextTokenState(int64_t max) : max_length(max) {}
    ~NextTokenState() { release_graph(); }
    NextTokenState(const NextTokenState&) = delete;
    NextTokenState& operator=(const NextTokenState&) = delete;
    void release_graph() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
    }
    int64_t max_length;
    std::vector<KVCacheState> caches;
    std::vector<int64_t> processed;
    std::vector<float> last_logits;
    detail::DevBuf cur, pos;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t epoch = 0;                   // the backend's allocation count the graph was captured at
    const float* graph_logits = nullptr;  // where the captured step writes its logits
};

NextTokenLogitsFn CausalLM::next_token_logits(int64_t max_length) {
    if (!config_.causal)
        throw std::logic_error("CausalLM::next_token_logits: the model attends bidirectionally (a diffusion LM), so it "
                               "has no next-token cache");
    if (max_length <= 0) throw std::invalid_argument("CausalLM::next_token_logits: max_length must be positive");
    auto state = std::make_shared<NextTokenState>(max_length);
    return [this, state](const std::vector<int64_t>& tokens) { return next_token_call(*state, tokens); };
}

std::vector<float> CausalLM::next_token_call(NextTokenState& s, const std::vector<int64_t>& tokens) {
    // Validation and history handling as MakeCachedNextTokenLogits (generation.cpp:214-236).
    if (tokens.empty()) throw std::invalid_argument("MakeCachedNextTokenLogits: the sequence is empty");
    const auto L = static_cast<int64_t>(tokens.size());
    if (L > s.max_length)
        throw std::invalid_argument("MakeCachedNextTokenLogits: " + std::to_string(L) + " tokens don't fit in caches of " +
                                    std::to_string(s.max_length));
    const int64_t V = config_.vocab_size;
    for (const int64_t t : tokens)
        if (t < 0 || t >= V) throw std::invalid_argument("EmbeddingModule::forward: index out of range [0, num_embeddings)");
    size_t shared = 0;
    while (shared < tokens.size() && shared < s.processed.size() && tokens[shared] == s.processed[shared]) ++shared;
    if (shared == tokens.size() && shared == s.processed.size()) return s.last_logits;  // the same sequence again
    if (shared == tokens.size()) --shared;  // a prefix of the history: rerun its last token for its logits
    // A short extension runs one decode step per new token over the caches (positions before
    // `shared` hold this sequence's keys and values already); anything else is one forward over
    // the whole sequence, whose keys and values then fill the caches.
    constexpr size_t kMaxSteps = 8;
    const float* logits = nullptr;
    void* st = be_->stream();
    if (shared == 0 || tokens.size() - shared > kMaxSteps) {
        std::vector<float> ids(tokens.begin(), tokens.end());
        float* pid = prompt_ids_.ensure(be_, L);
        be_->copy(pid, ids.data(), ids.size() * sizeof(float), CopyDirection::HostToDevice);
        logits = forward_last_rows(pid, 1, L);
        s.caches.resize(layers_.size());
        for (size_t i = 0; i < layers_.size(); ++i) layers_[i]->mha().export_kv(s.caches[i], s.max_length);
    } else {
        float* cur = s.cur.ensure(be_, 1);
        auto* pos = reinterpret_cast<int32_t*>(s.pos.ensure(be_, 1));
        for (size_t t = shared; t < tokens.size(); ++t) {
            const float id = static_cast<float>(tokens[t]);
            const int32_t p = static_cast<int32_t>(t);
            be_->copy(cur, &id, sizeof(id), CopyDirection::HostToDevice);
            be_->copy(pos, &p, sizeof(p), CopyDirection::HostToDevice);
            if (s.exec && s.epoch == be_->allocation_epoch()) {
                const hipError_t rc = hipGraphLaunch(s.exec, static_cast<hipStream_t>(st));
                if (rc != hipSuccess)
                    throw std::runtime_error(std::string("CausalLM::next_token_logits: replay: ") + hipGetErrorString(rc));
                logits = s.graph_logits;
                continue;
            }
            // Eager (its buffers now exist), then capture the same step for the calls that follow.
            s.release_graph();
            logits = decode_logits(cur, 1, s.caches, pos);
            hipGraph_t g = nullptr;
            if (hipStreamBeginCapture(static_cast<hipStream_t>(st), hipStreamCaptureModeThreadLocal) != hipSuccess)
                throw std::runtime_error("CausalLM::next_token_logits: begin capture");
            const float* captured = nullptr;
            try {
                captured = decode_logits(cur, 1, s.caches, pos);
            } catch (...) {
                (void)hipStreamEndCapture(static_cast<hipStream_t>(st), &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            if (hipStreamEndCapture(static_cast<hipStream_t>(st), &g) != hipSuccess)
                throw std::runtime_error("CausalLM::next_token_logits: end capture");
            s.graph = g;
            if (hipGraphInstantiate(&s.exec, g, nullptr, nullptr, 0) != hipSuccess) {
                s.release_graph();
                throw std::runtime_error("CausalLM::next_token_logits: instantiate");
            }
            s.graph_logits = captured;
            s.epoch = be_->allocation_epoch();
        }
    }
    s.last_logits.resize(static_cast<size_t>(V));
    be_->copy(s.last_logits.data(), logits, static_cast<size_t>(V) * sizeof(float), CopyDirection::DeviceToHost);
    s.processed = tokens;
    return s.last_logits;
}

void CausalLM::explain_generated_device(const float* ids, int64_t n, int64_t prompt, int64_t new_tokens, int64_t ld_ids,
                                        const LRPRuleConfig& config, float* token_relevance, bool unit_seed) {
    if (n <= 0 || prompt <= 0 || new_tokens <= 0 || ld_ids < prompt + new_tokens)
        throw std::invalid_argument("CausalLM::explain_generated_device: bad sizes");
    const int64_t W = prompt + new_tokens - 1;
    void* st = be_->stream();
    // Tokens t0 .. t1 go through one pass as G = t1 - t0 + 1 copies of the longest prefix (columns
    // 0 .. prompt + t1 - 1), copy g seeded at row prompt + t0 + g - 1 with the id that followed it.
    // The model is causal, so a row sees nothing after it and the relevance of a row seeded there
    // reaches no later row: copy g's relevance over its own prefix is that of the pass over the
    // prefix alone (the later rows carry zero). Groups hold up to 16384 rows (fewer for models wider
    // than 1024, so the pass's activations stay a few GiB). The longest group comes first; its size
    // sizes every forward buffer once, and each group then runs the forward once over the n
    // prefixes and repeats its activations G times.
    constexpr int64_t kMaxGroup = 32;
    int64_t rows = std::clamp<int64_t>(16384 * 1024 / std::max<int64_t>(1, config_.hidden_size), 1024, 16384);
    bool first = true;
    for (int64_t t1 = new_tokens - 1; t1 >= 0;) {
        const int64_t l = prompt + t1;
        const int64_t G = std::max<int64_t>(1, std::min<int64_t>({t1 + 1, kMaxGroup, rows / (n * l)}));
        const int64_t t0 = t1 - G + 1;
        if (first) {  // every later group holds no more rows (and no longer rows) than this one
            rows = std::max<int64_t>(G * n * l, 1);
            embed_.reserve_forward(G * n * l);
            for (auto& layer : layers_) layer->reserve_forward(G * n, l);
            norm_.reserve_forward(G * n * l);
            first = false;
        }
        float* pid = prompt_ids_.ensure(be_, n * l);
        be_->copy_2d(pid, static_cast<size_t>(l), ids, static_cast<size_t>(ld_ids), static_cast<size_t>(n),
                     static_cast<size_t>(l));
        float* tmp = tok_tmp_.ensure(be_, G * n * l);
        explain_staggered_rows(pid, n, G, l, ids + (l - G + 1), ld_ids, config, tmp, nullptr, unit_seed, true);
        for (int64_t g = 0; g < G; ++g) {
            const int64_t t = t0 + g, lt = prompt + t;
            float* out = token_relevance + t * n * W;
            MI355XBackend::check(pxk_fill(out, 0.0f, n * W, st), "CausalLM::explain_generated_device");
            be_->copy_2d(out, static_cast<size_t>(W), tmp + g * n * l, static_cast<size_t>(l), static_cast<size_t>(n),
                         static_cast<size_t>(lt));
        }
        t1 = t0 - 1;
    }
}

Tensor CausalLM::forward_impl(const Tensor& input) {
    if (input.rank() != 2) throw std::invalid_argument("CausalLM::forward: input must be (N, L) token ids");
    const int64_t n = input.shape().dim(0), l = input.shape().dim(1), V = config_.vocab_size;
    std::vector<float> raw = input.to_host_vector();
    for (float& v : raw) {  // EmbeddingModule::forward_impl's validation (embedding_module.cpp:48-59)
        const auto idx = static_cast<int64_t>(std::llround(static_cast<double>(v)));
        if (idx < 0 || idx >= V)
            throw std::invalid_argument("EmbeddingModule::forward: index out of range [0, num_embeddings)");
        v = static_cast<float>(idx);
    }
    float* ids = ids_.ensure(be_, n * l);
    be_->copy(ids, raw.data(), raw.size() * sizeof(float), CopyDirection::HostToDevice);
    return detail::copy_out(be_, run_forward(ids, n, l), Shape({n, l, V}));
}

std::vector<Tensor> CausalLM::propagate_relevance_by_layer(const Tensor& relevance_out, const LRPRuleConfig& config) {
    if (N_ == 0) throw std::logic_error("CausalLM::propagate_relevance_by_layer: called before any forward()");
    const int64_t V = config_.vocab_size, d = config_.hidden_size;
    if (relevance_out.numel() != N_ * L_ * V)
        throw std::invalid_argument("CausalLM::propagate_relevance_by_layer: relevance_out must be (N, L, vocab)");
    const Shape shape({N_, L_, d});
    std::vector<Tensor> bounds(layers_.size() + 1);
    const float* r = tied_head_ ? tied_head_->run_relevance(relevance_out.data(), config)
                                : lm_head_->run_relevance(relevance_out.data(), config);
    for (size_t i = layers_.size(); i-- > 0;) {
        bounds[i + 1] = detail::copy_out(be_, r, shape);
        r = layers_[i]->run_relevance(r, config);
    }
    bounds[0] = detail::copy_out(be_, r, shape);
    r_embed_ = r;
    return bounds;
}

Tensor CausalLM::propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) {
    if (N_ == 0) throw std::logic_error("CausalLM::propagate_relevance: called before any forward()");
    if (relevance_out.numel() != N_ * L_ * config_.vocab_size)
        throw std::invalid_argument("CausalLM::propagate_relevance: relevance_out must be (N, L, vocab)");
    const float* r = run_relevance(relevance_out.data(), config);
    Tensor out = Tensor::uninitialized(Shape({N_, L_}), be_);
    embed_.token_relevance(r, N_ * L_, out.data());
    return out;
}

}  // namespace pulsatrix
