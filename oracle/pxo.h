/*
 * pxo.h -- C API of the CPU oracle.
 *
 * TEST INFRASTRUCTURE ONLY. The oracle is a CPU restatement of Pulsatrix's CPUBackend and of
 * the causal-LM forward + AttnLRP relevance modules, used as the checker for the MI355X path.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the product
 * (pulsatrix_amd/) never does.
 *
 * Every entry point returns 0 on success and -1 on failure; pxo_last_error() then names the
 * problem (the reference throws std::invalid_argument / std::logic_error in those cases).
 */
#ifndef PXO_H
#define PXO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model shape and options. vocab_size == 0 describes a bare TransformerBlock.
 * Mirrors HfModelConfig (include/pulsatrix/hf_model.hpp:33-101), AttentionConfig
 * (include/pulsatrix/multihead_attention_module.hpp:31-63) and TransformerBlockOptions
 * (include/pulsatrix/transformer_block.hpp:20-32) for the fields the path reads. */
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

/* LRPRuleConfig (include/pulsatrix/lrp_rule_config.hpp:72-115): rule in LRPRule order
 * (0 Epsilon, 1 Gamma, 2 AlphaBeta, 3 ZBox); epsilon is every rule's stabilizer. */
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

const char* pxo_last_error(void);
void pxo_set_threads(int threads); /* GEMM worker threads; <= 0 restores hardware_concurrency() */
int pxo_get_threads(void);
/* Threads over the independent rows / slices of lrp_linear and lrp_bilinear_matmul, which
 * CPUBackend runs on one thread (default 1, its schedule). Results are identical for any count:
 * a checker may raise it to finish sooner; the CPU baseline keeps 1. */
void pxo_set_split_threads(int threads);

/* Seeded N(0, stddev) fill: SplitMix64 bits, Box-Muller in double (src/portable_random.hpp:11-29). */
void pxo_fill_normal(float* dst, size_t n, uint64_t seed, double stddev);

/* Number of floats in the flat parameter blob (layout: pulsatrix_amd.h, px_param_layout). */
int64_t pxo_param_count(const px_model_config* cfg);
int64_t pxo_block_param_count(const px_model_config* cfg);

/* ---- TransformerBlock (src/transformer_block.cpp) ---- */
void* pxo_block_create(const px_model_config* cfg, const float* params);
int pxo_block_forward(void* h, const float* x, int64_t n, int64_t l, float* y);
int pxo_block_relevance(void* h, const float* r_out, float eps, int bias_in_denominator, float* r_in);
int pxo_block_relevance_rule(void* h, const float* r_out, const px_lrp_rule* rule, float* r_in);
void pxo_block_destroy(void* h);

/* ---- CausalLM (src/causal_lm.cpp) ---- */
void* pxo_lm_create(const px_model_config* cfg, const float* params);
int pxo_lm_forward(void* h, const int64_t* ids, int64_t n, int64_t l, float* logits);
/* seed: (n, l, vocab) relevance at the logits. Outputs may be NULL.
 * r_embed (n, l, hidden): propagate_relevance_by_layer()[0]; r_tokens (n, l): the embedding's
 * per-token sum; key_rel / value_rel: per layer the MHA's key_relevance() / value_relevance(),
 * (layers, n*l, kv_heads*head_dim). */
int pxo_lm_relevance(void* h, const float* seed, float eps, int bias_in_denominator, float* r_embed,
                     float* r_tokens, float* key_rel, float* value_rel);
/* The same under any rule: the config reaches every Linear and the head, as the reference's modules
 * pass it down (the attention, SwiGLU and residual rules read only its epsilon). */
int pxo_lm_relevance_rule(void* h, const float* seed, const px_lrp_rule* rule, float* r_embed, float* r_tokens,
                          float* key_rel, float* value_rel);
void pxo_lm_destroy(void* h);

/* ---- Single Linear layer (src/linear_module.cpp + src/lrp_rules.cpp) ---- */
int pxo_linear_forward(const float* x, const float* w, const float* bias, int64_t n, int64_t in, int64_t out,
                       float* pre_bias, float* y);
int pxo_linear_relevance(const float* x, const float* w, const float* bias, const float* pre_bias, const float* r,
                         int64_t n, int64_t in, int64_t out, float eps, int bias_in_denominator, float* r_in);
/* LinearModule::propagate_relevance under any rule (lrp_rules::linear, lrp_rules.cpp:197-215); bias may
 * be NULL (a zero bias, as a bias-free layer holds). */
int pxo_linear_relevance_rule(const float* x, const float* w, const float* bias, const float* pre_bias,
                              const float* r, int64_t n, int64_t in, int64_t out, const px_lrp_rule* rule,
                              float* r_in);

/* ---- CPUBackend primitives (src/cpu_backend.cpp) ---- */
void pxo_gemm(const float* a, const float* b, float* out, size_t m, size_t k, size_t n);
void pxo_gemm_ex(const float* a, int transpose_a, const float* b, int transpose_b, float* out, size_t m, size_t k,
                 size_t n, float beta);
void pxo_elementwise(int op, const float* in, float* out, size_t n);
/* Backward rows of training (device_backend.hpp:428, 462, 557): ReLU as a select, the other
 * activations' slopes times the gradient; softmax dx = y (dy - sum y dy); RMSNorm's input
 * gradient and per-element gamma terms. */
void pxo_elementwise_backward(int op, const float* x, const float* grad_out, float* grad_in, size_t n);
void pxo_softmax_rows_backward(const float* y, const float* dy, float* dx, size_t rows, size_t cols);
void pxo_rms_norm_backward(const float* grad_out, const float* gamma, const float* in, const float* row_rms,
                           float* grad_in, float* gamma_terms, size_t rows, size_t cols);
void pxo_add(const float* a, const float* b, float* out, size_t n);
void pxo_mul(const float* a, const float* b, float* out, size_t n);
void pxo_axpby(float alpha, const float* x, float beta, const float* y, float* out, size_t n);
void pxo_add_row_vector(const float* in, const float* row, float* out, size_t rows, size_t cols);
void pxo_softmax_rows(const float* in, float* out, size_t rows, size_t cols);
void pxo_rms_norm_forward(const float* in, const float* gamma, float* out, float* row_rms, size_t rows, size_t cols,
                          float eps);
void pxo_rope_rotate(const float* in, const float* cos_t, const float* sin_t, float* out, size_t slices,
                     size_t seq_len, size_t head_dim, int inverse, int rotate_half);
void pxo_permute_0213(const float* in, float* out, size_t d0, size_t d1, size_t d2, size_t d3);
void pxo_attention_mask_fill(float* scores, const float* key_keep, size_t batch, size_t heads, size_t q_len,
                             size_t k_len, int causal, size_t q_offset, size_t window, float value);
void pxo_gather_rows(const float* table, const float* indices, float* out, size_t count, size_t dim);
void pxo_lrp_linear(const float* x, const float* w, const float* z, const float* r, float* r_in, size_t rows,
                    size_t in_features, size_t out_features, float eps);
void pxo_lrp_residual_split(const float* a, const float* b, const float* r, float* r_a, float* r_b, size_t n,
                            float eps);
void pxo_lrp_bilinear_elementwise(const float* a, const float* b, const float* r, float* r_out, size_t n, float eps);
void pxo_lrp_bilinear_matmul(const float* a, const float* b, const float* o, const float* r_o, float* r_a, float* r_b,
                             size_t slices, size_t m, size_t p, size_t q, float eps, int b_transposed);
void pxo_lrp_softmax_rows(const float* x, const float* y, const float* r, float* r_in, size_t rows, size_t cols);
void pxo_lrp_rope(const float* x, const float* y, const float* r, const float* cos_t, const float* sin_t, float* r_in,
                  size_t slices, size_t seq_len, size_t head_dim, float eps, int rotate_half);
void pxo_lrp_stabilized_divide(const float* r, const float* denom, const float* gate, float* out, size_t n, float eps,
                               int gate_mode);
void pxo_copy_2d(float* dst, size_t dst_stride, const float* src, size_t src_stride, size_t rows, size_t cols);
void pxo_accumulate_rows(const float* in, float* out, size_t rows, size_t cols);
void pxo_column_sums(const float* in, float* out, size_t rows, size_t cols, float beta);
float pxo_sum(const float* in, size_t n);
float pxo_dot(const float* a, const float* b, size_t n);
/* RoPE tables as RoPEModule::ensure_tables builds them (src/rope_module.cpp:83-101). */
void pxo_rope_tables(int64_t head_dim, float base, int64_t seq_len, int64_t offset, float* cos_t, float* sin_t);

#ifdef __cplusplus
}
#endif

#endif /* PXO_H */
