/*
 * pulsatrix_amd.h -- C ABI of the MI355X host framework (libpulsatrix_amd.so).
 *
 * The C++17 surface (MI355XBackend, TransformerBlock, CausalLM, ... in
 * pulsatrix_amd/csrc/host/include/pulsatrix/) is what a C++ caller of Pulsatrix uses directly. This
 * header is the flat binding a foreign-language caller (ctypes, cgo, JNI) uses for the same path:
 * plain pointers and sizes, no C++ types. Entry points return 0 on success and -1 on failure;
 * pxa_last_error() then holds the message of the C++ exception (std::invalid_argument,
 * std::logic_error, std::runtime_error -- the reference's error behaviour).
 *
 * Weights travel as one flat float blob in the reference's parameter order and layout
 * (CausalLM::named_parameters(), causal_lm.cpp:115-125; Linear weights (in, out)):
 *   embed_tokens.weight (V, d)
 *   per layer: norm1.weight (d), mha.{q,k,v}_proj.weight (d, H*D | Hkv*D) [+ .bias when qkv_bias],
 *              mha.out_proj.weight (H*D, d) [+ .bias when out_bias], [mha.{q,k}_norm.weight (D) with
 *              qk_norm], norm2.weight (d), swiglu.{gate,up}_proj.weight (d, F) [+ .bias],
 *              swiglu.down_proj.weight (F, d) [+ .bias], [post_attn_norm.weight, post_mlp_norm.weight
 *              (d) with post_norms]
 *   norm.weight (d), lm_head.weight (d, V) when not tied.
 * A bare block uses the per-layer part alone.
 */
#ifndef PULSATRIX_AMD_H
#define PULSATRIX_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* HfModelConfig (include/pulsatrix/hf_model.hpp:33-101) + AttentionConfig/TransformerBlockOptions
 * fields the path reads; vocab_size == 0 describes a bare TransformerBlock. */
typedef struct px_model_config {
    int64_t vocab_size;
    int64_t hidden_size;
    int64_t num_layers;
    int64_t num_heads;
    int64_t num_kv_heads;
    int64_t head_dim;
    int64_t intermediate_size;
    float rms_norm_eps;
    float rope_theta;
    int32_t use_rope;
    int32_t rope_rotate_half;
    int32_t causal;
    int32_t qkv_bias;
    int32_t out_bias;
    int32_t mlp_bias;
    int32_t tie_word_embeddings;
    int32_t reserved;
    /* The architecture variants ToAttentionConfig and TransformerBlockOptions carry
     * (hf_model.cpp:282-313, causal_lm.cpp:30-54); all zero is the Llama family. */
    int32_t hidden_act;          /* 0 SiLU, 1 GeLU with the tanh approximation (gelu_pytorch_tanh) */
    int32_t qk_norm;             /* RMSNorm over each head's queries and keys, eps rms_norm_eps */
    int32_t post_norms;          /* Gemma 3 sandwich norms after the attention and after the MLP */
    int32_t rope_scaling;        /* full-attention layers: 0 none, 1 linear, 2 llama3 */
    float norm_weight_offset;    /* every RMSNorm scales by offset + gamma (Gemma 3: 1) */
    float embed_scale;           /* embeddings multiplied by this; 0 means 1 (Gemma 3: sqrt(hidden)) */
    float query_pre_attn_scalar; /* > 0: scores scaled by 1/sqrt(this), else by 1/sqrt(head_dim) */
    float rope_local_base;       /* > 0: the sliding layers' own RoPE base, without scaling */
    float rope_factor;           /* rope_scaling's factor, low_freq_factor, high_freq_factor */
    float rope_low_freq_factor;
    float rope_high_freq_factor;
    int32_t reserved2;
    int64_t rope_original_max_position; /* rope_scaling's original_max_position_embeddings */
    int64_t sliding_window;      /* > 0: a sliding layer's query i sees only keys j > i - window */
    uint64_t sliding_layers;     /* bit i: layer i slides (layer_types); 0 with a window: every layer */
} px_model_config;

/* LRPRuleConfig (include/pulsatrix/lrp_rule_config.hpp:72-115): rule in LRPRule order (0 Epsilon,
 * 1 Gamma, 2 AlphaBeta, 3 ZBox); epsilon is every rule's stabilizer. The config reaches every
 * Linear and the head, as the reference's modules pass it down; the attention, SwiGLU and residual
 * rules read only its epsilon. */
typedef struct px_lrp_rule {
    float epsilon;
    int32_t rule;
    float gamma;
    float alpha;
    float beta;
    float low;
    float high;
    int32_t bias_in_denominator;
} px_lrp_rule;

const char* pxa_last_error(void);
int pxa_device_count(void);

/* The process-wide MI355XBackend on device 0 (created on first use) that the block / LM handles
 * below run on; its HIP stream, and a wait for it. */
void* pxa_backend(void);
void* pxa_backend_stream(void);
int pxa_backend_synchronize(void);
/* Bytes the backend's caching allocator holds (in use, cached). */
int pxa_backend_memory(size_t* in_use, size_t* cached);

/* In-process kernel timing (a profiling aid with no reference counterpart; the reference times
 * whole calls only, docs/gpu-profiling.md). Between start and stop, every kernel launch the fused
 * path makes on the backend is recorded with its algorithmic work (dense FLOPs for GEMM and
 * attention kernels, HBM bytes for row kernels). pxa_launch_log_time replays the recorded
 * launches in their order `reps` times, every kernel recording its own start and end events
 * (pxk_timing_begin), and writes each launch's mean kernel time (the summed durations of its
 * kernels) in seconds. The replays rewrite the recorded passes' outputs; run them after reading
 * those. */
int pxa_launch_log_start(void);
int pxa_launch_log_stop(int64_t* count);
int pxa_launch_log_entry(int64_t index, char* kernel, size_t kernel_cap, char* family, size_t family_cap,
                         double* flops, double* bytes);
int pxa_launch_log_time(int reps, double* seconds);
/* The number of kernels launch `index` dispatched in the last pxa_launch_log_time replay (a split-K
 * GEMM dispatches two): how a profiler's per-dispatch records map back onto the launches. */
int pxa_launch_log_dispatches(int64_t index, int32_t* count);

/* Seeded N(0, stddev) on the host: SplitMix64 bits, Box-Muller in double (src/portable_random.hpp:11-29). */
void pxa_fill_normal(float* dst, size_t n, uint64_t seed, double stddev);
int64_t pxa_param_count(const px_model_config* cfg);
int64_t pxa_block_param_count(const px_model_config* cfg);
/* The flat blob of a random-init model: N(0, stddev) from seed, every RMSNorm's effective scale
 * (norm_weight_offset + gamma) 1. */
int pxa_synthetic_params(const px_model_config* cfg, int block, uint64_t seed, double stddev, float* dst);

/* ---- TransformerBlock (transformer_block.hpp) ; host tensors ---- */
void* pxa_block_create(const px_model_config* cfg, const float* params);
int pxa_block_forward(void* block, const float* x, int64_t n, int64_t l, float* y);
int pxa_block_relevance(void* block, const float* r_out, float eps, int bias_in_denominator, float* r_in);
int pxa_block_relevance_rule(void* block, const float* r_out, const px_lrp_rule* rule, float* r_in);
void pxa_block_destroy(void* block);

/* ---- LinearModule (linear_module.hpp) ; host tensors ----
 * x (n, in) through w (in, out) and bias (out, nullable: a layer without a bias) on the device,
 * then LinearModule::propagate_relevance of r (n, out) under `rule` into r_in (n, in); y (n, out,
 * nullable) receives the forward output. */
int pxa_linear_relevance_rule(const float* x, const float* w, const float* bias, int64_t n, int64_t in, int64_t out,
                              const float* r, const px_lrp_rule* rule, float* y, float* r_in);

/* ---- CausalLM (causal_lm.hpp) ---- */
void* pxa_lm_create(const px_model_config* cfg, const float* params);
void* pxa_lm_create_random(const px_model_config* cfg, uint64_t seed, double stddev);
/* LoadCausalLM (src/causal_lm.cpp:293-301): config.json and model.safetensors (or the shards of
 * model.safetensors.index.json) from `directory`, Llama / Qwen2 family; tensor bytes are copied
 * to HBM as stored and widened (BF16, F16, F8, F64) and transposed there. The model's settings
 * are written to cfg_out (nullable). NULL on failure, with the message in pxa_last_error(). */
void* pxa_lm_load(const char* directory, px_model_config* cfg_out);
/* Host ids (n, l) -> host logits (n, l, vocab) (nullable). CausalLM::forward. */
int pxa_lm_forward(void* lm, const int64_t* ids, int64_t n, int64_t l, float* logits);
/* Host seed (n, l, vocab) -> host outputs (each nullable): r_embed (n, l, d) =
 * propagate_relevance_by_layer()[0]; r_tokens (n, l); key_rel / value_rel per layer
 * (layers, n*l, Hkv*D) = MultiHeadAttentionModule::key_relevance() / value_relevance(). */
int pxa_lm_relevance(void* lm, const float* seed, float eps, int bias_in_denominator, float* r_embed,
                     float* r_tokens, float* key_rel, float* value_rel);
int pxa_lm_relevance_rule(void* lm, const float* seed, const px_lrp_rule* rule, float* r_embed, float* r_tokens,
                          float* key_rel, float* value_rel);
/* The device hot path (CausalLM::explain_device): ids (n*l floats) in HBM -> forward, argmax (or
 * targets_in, host, n entries, nullable) seed at each sequence's last position, relevance, per-token
 * sums into token_rel (n*l, HBM) and targets (n int64, HBM). Asynchronous on pxa_backend_stream(). */
int pxa_lm_explain_device(void* lm, const float* ids, int64_t n, int64_t l, float eps, int bias_in_denominator,
                          float* token_rel, int64_t* targets, const int64_t* targets_in, int unit_seed);
/* Runs one pxa_lm_explain_device call eagerly (so that every buffer it needs exists at its size),
 * then captures the same call into a HIP graph owned by this model, replacing the model's earlier
 * graph; pxa_lm_replay(lm) runs it. A capture whose work would still free device memory is refused.
 * The graph keeps the caller's ids / token_rel / targets pointers, which must stay valid. */
int pxa_lm_capture_explain(void* lm, const float* ids, int64_t n, int64_t l, float eps, int bias_in_denominator,
                           float* token_rel, int64_t* targets);
/* The same two under any rule. */
int pxa_lm_explain_device_rule(void* lm, const float* ids, int64_t n, int64_t l, const px_lrp_rule* rule,
                               float* token_rel, int64_t* targets, const int64_t* targets_in, int unit_seed);
int pxa_lm_capture_explain_rule(void* lm, const float* ids, int64_t n, int64_t l, const px_lrp_rule* rule,
                                float* token_rel, int64_t* targets);
/* Replays this model's captured graph on pxa_backend_stream(). Refused before any launch (-1,
 * pxa_last_error) when nothing was captured for it, when the handle is unknown or destroyed, or when
 * a device block the graph addresses has been freed or reallocated since the capture (a later pass
 * at a longer length, the shared split-K pool grown): capture again. */
int pxa_lm_replay(void* lm);
/* Forward over ids (n*l floats, HBM) and the LRP pass seeded at each sequence's last row only: the
 * target id targets[b * target_stride] (floats in HBM) with its logit (or 1 with unit_seed). The head
 * runs on those rows alone. token_rel (n*l) and targets_out (n int64, nullable) in HBM. */
int pxa_lm_explain_rows_device(void* lm, const float* ids, int64_t n, int64_t l, const float* targets,
                               int64_t target_stride, const px_lrp_rule* rule, float* token_rel, int64_t* targets_out,
                               int unit_seed);
/* Batched KV-cached greedy decode (MakeCachedNextTokenLogits + greedy Generate,
 * src/generation.cpp:189-258, for a batch): ids (n rows of ld_ids floats, HBM) hold each prompt in
 * the first `prompt` columns; columns prompt .. prompt + new_tokens - 1 receive the generated ids and
 * picked_logit (same layout, nullable) their logits. One HIP graph replay per token; returns when done. */
int pxa_lm_generate_device(void* lm, float* ids, int64_t n, int64_t prompt, int64_t new_tokens, int64_t ld_ids,
                           float* picked_logit);
/* AttnLRP of every generated token through a forward over its prefix (the reference's way to explain a
 * cached generation): token_rel (new_tokens, n, prompt + new_tokens - 1) in HBM, zero past each prefix. */
int pxa_lm_explain_generated_device(void* lm, const float* ids, int64_t n, int64_t prompt, int64_t new_tokens,
                                    int64_t ld_ids, const px_lrp_rule* rule, float* token_rel, int unit_seed);
/* CausalLM::next_token_logits(max_length) (include/pulsatrix/causal_lm.hpp:116): a cached next-token
 * function for the reference's Generate (generation.hpp:95-135), over the MI355X decode kernels.
 * _create returns NULL on error (pxa_last_error). pxa_lm_next_token_logits(f, tokens, n, logits,
 * vocab) writes the next token's logits after tokens[0 .. n) (host int64 ids) into logits (host,
 * vocab floats; vocab must be the model's); its signature is the callback a Generate() binding
 * takes, with f as the context. Calls after the model was destroyed are refused (-1). */
void* pxa_lm_next_token_logits_create(void* lm, int64_t max_length);
int pxa_lm_next_token_logits(void* f, const int64_t* tokens, int64_t n, float* logits, int64_t vocab);
void pxa_lm_next_token_logits_destroy(void* f);
/* After a device-side pass (explain or replay): 0 when every id was in [0, vocab), else -1 with
 * the reference's message ("EmbeddingModule::forward: index out of range [0, num_embeddings)") in
 * pxa_last_error(); an out-of-range id is gathered as id 0 so the pass itself completes. Waits for
 * the backend's stream. */
int pxa_lm_check_device_ids(void* lm);
/* Device pointers of the last pass: logits (n*l*vocab), embedding-level relevance (n*l*d). */
const float* pxa_lm_last_logits(void* lm);
const float* pxa_lm_last_embedding_relevance(void* lm);
/* Destroys the model and its captured graph (after the backend's stream drains). A destroyed handle
 * is refused by every entry point that returns a status (-1, "unknown or destroyed model handle");
 * destroying it again is a no-op. */
void pxa_lm_destroy(void* lm);

#ifdef __cplusplus
}
#endif

#endif /* PULSATRIX_AMD_H */
