/** @file multihead_attention_module.hpp
 *  @brief Causal GQA multi-head attention with RoPE and its AttnLRP relevance
 *         (the surface of include/pulsatrix/multihead_attention_module.hpp).
 *
 *  MI355X layout: Q, K, V stay head-packed in the projections' (N*L, heads*D) row layout (no
 *  permutes, no repeat_kv copies: a query head reads its KV head through the GEMM's batch map);
 *  scores and P are (N, H, L, L). The forward is a fused QKV GEMM, one RoPE kernel, a causal
 *  scores GEMM (tiles above the diagonal skipped), the row softmax and a causal P V GEMM. The
 *  relevance is the reference's Eq. 15 / softmax rule sequence (multihead_attention_module.cpp:
 *  404-485) in GEMM form with the divides, RoPE rule and projection denominators fused into the
 *  GEMM epilogues.
 */
#pragma once

#include <cstdint>
#include <memory>
#include <vector>

#include "pulsatrix/detail/fused.hpp"
#include "pulsatrix/linear_module.hpp"
#include "pulsatrix/module.hpp"
#include "pulsatrix/rms_norm_module.hpp"

namespace pulsatrix {

/** @brief Pair layout of the rotary embedding: (2i, 2i+1) or Hugging Face's (i, i + D/2). */
enum class RoPELayout { AdjacentPairs, RotateHalf };

/** @brief AttentionConfig of include/pulsatrix/multihead_attention_module.hpp:31-63. */
struct AttentionConfig {
    int64_t d_model = 0;
    int64_t num_heads = 0;
    int64_t num_kv_heads = 0;
    int64_t head_dim = 0;
    bool use_rope = true;
    RoPELayout rope_layout = RoPELayout::AdjacentPairs;
    float rope_base = 10000.0f;
    std::vector<double> rope_inverse_frequencies;
    bool use_qk_norm = false;
    float qk_norm_eps = 1e-6f;
    bool qkv_bias = true;
    bool out_bias = true;
    bool causal = false;
    int64_t sliding_window = 0;
    float score_scale = 0.0f;
    float qk_norm_weight_offset = 0.0f;
};

/** @brief One layer's KV cache for a batched decode (the KVCache of kv_cache.cpp:18-39, for a
 *         batch): keys after QK-Norm and RoPE and values, sequence b's position p at row
 *         b * positions + p of (n * positions, kv_heads * head_dim). */
struct KVCacheState {
    detail::DevBuf k, v;
    int64_t n = 0, positions = 0;
};

class MultiHeadAttentionModule : public Module {
public:
    MultiHeadAttentionModule(const AttentionConfig& config, DeviceBackend* backend);
    MultiHeadAttentionModule(int64_t d_model, int64_t num_heads, DeviceBackend* backend, bool use_rope = true,
                             bool use_qk_norm = false);

    [[nodiscard]] Tensor propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) override;

    [[nodiscard]] LinearModule& q_proj() { return q_proj_; }
    [[nodiscard]] LinearModule& k_proj() { return k_proj_; }
    [[nodiscard]] LinearModule& v_proj() { return v_proj_; }
    [[nodiscard]] LinearModule& out_proj() { return out_proj_; }
    /** @brief QK-Norm's query and key RMSNorms (multihead_attention_module.cpp:116-121); throws
     *         std::logic_error when the module has none. */
    [[nodiscard]] RMSNormModule& q_norm();
    [[nodiscard]] RMSNormModule& k_norm();
    [[nodiscard]] const AttentionConfig& config() const noexcept { return config_; }
    /** @brief Relevance at the key / value projections' outputs, (N*L, Hkv*D), from the last
     *         propagate_relevance() (multihead_attention_module.cpp:488-496). */
    [[nodiscard]] const Tensor& key_relevance() const;
    [[nodiscard]] const Tensor& value_relevance() const;
    [[nodiscard]] float score_scale() const;

    /** @brief Fused-path forward. With `resid`, the output projection's epilogue also writes
     *         resid + attention output into `resid_out` (the block's first residual add). With
     *         `norm`, x is that RMSNorm's input and the q/k/v GEMM applies the norm itself
     *         (RMSNormModule::fold); the relevance pass then reads the norm's output the same way. */
    const float* run_forward(const float* x, int64_t n, int64_t l, const float* resid = nullptr,
                             float* resid_out = nullptr, RMSNormModule* norm = nullptr);
    /** @brief After run_forward over n sequences: repeats every activation the relevance pass reads
     *         `copies` times in place, as if the forward had run over copies * n sequences that
     *         repeat the n (storage from an earlier pass at least that large). */
    void replicate_forward(int64_t copies);
    /** @brief Sizes the buffers replicate_forward() repeats into for `n sequences of length l`, without computing. */
    void reserve_forward(int64_t n, int64_t l);
    /** @brief Fused-path relevance; `add` (nullable) is summed into the input relevance. `divided`:
     *         relevance_out already holds R / stab(z) of the output projection (a producer honoured
     *         relevance_denominator()), so no prologue divides it. */
    const float* run_relevance(const float* relevance_out, const LRPRuleConfig& config, const float* add = nullptr,
                               const detail::ResidualSplit& split = {}, bool divided = false);
    /** @brief The epsilon rule's denominator of the output projection for `config`: its pre-bias
     *         output z and, under the bias-in-denominator rule, its bias (else nullptr). */
    void relevance_denominator(const LRPRuleConfig& config, const float** den, const float** bias) const;
    /** @brief The attention output (after the output projection's bias) of the last forward. */
    [[nodiscard]] const float* output() const noexcept;

    /** @brief Fills `cache` (n sequences, `positions` each) with the last forward's keys and values:
     *         the prompt rows of a decode. Also sizes the RoPE tables for every cached position. */
    void export_kv(KVCacheState& cache, int64_t positions);
    /** @brief One decode step of n sequences (forward_cached, multihead_attention_module.cpp:501-587):
     *         x (n, d_model) at the device position *pos; the step's key and value join the cache.
     *         With `resid`, resid_out = resid + output. Returns the output (n, d_model). Launches the
     *         same kernels with the same arguments at every position (HIP-graph capturable). */
    const float* decode_step(const float* x, int64_t n, KVCacheState& cache, const int32_t* pos,
                             const float* resid = nullptr, float* resid_out = nullptr);

protected:
    Tensor forward_impl(const Tensor& input) override;

private:
    void pack_weights();
    void ensure_tables(int64_t l);
    void run_attention_unfused(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v, int64_t n,
                               int64_t l);
    void relevance_scores_unfused(const float* spv, float eps, bool bid, bool rel_only);
    /** @brief The sliding window that masks something at length l (0: none). */
    [[nodiscard]] int64_t window_for(int64_t l) const;
    /** @brief Whether the fused attention kernels take this layer at length l (head_dim up to 128,
     *         score rows within LDS, no active sliding window). */
    [[nodiscard]] bool fused_attention(int64_t l) const;

    AttentionConfig config_;
    int64_t d_, H_, Hkv_, D_;
    MI355XBackend* be_;
    LinearModule q_proj_, k_proj_, v_proj_, out_proj_;
    std::unique_ptr<RMSNormModule> q_norm_, k_norm_;
    uint64_t packed_version_ = ~uint64_t{0};
    detail::DevBuf wqkv_, bqkv_;
    int64_t table_len_ = -1;
    detail::DevBuf cos_, sin_;
    int64_t N_ = 0, L_ = 0;
    const float* x_ = nullptr;
    detail::DevBuf x_copy_, qkv_z_, qkv_y_, qk_norm_out_, qk_rot_, raw_, p_, ctx_, out_z_, out_y_;
    detail::DevBuf stats_;  // fused path: the softmax's max and 1 / sum per (sequence, head, row)
    RMSNormModule* norm_in_ = nullptr;  // the RMSNorm folded into the q/k/v GEMM by the last forward, if any
    detail::DevBuf wqkv_g_;             // [Wq | Wk | Wv] with the folded norm's gamma on its rows
    const RMSNormModule* wg_norm_ = nullptr;
    uint64_t wg_version_ = ~uint64_t{0}, wg_packed_ = ~uint64_t{0};
    const float* folded_weights(RMSNormModule* norm);
    detail::DevBuf spv_, ra_, g_, r_in_, rctx_;
    detail::DevBuf dec_z_, dec_y_, dec_qkn_, dec_q_, dec_ctx_, dec_oz_, dec_oy_, dec_ws_;
    detail::AffineRule out_rule_, qkv_rule_;
    Tensor key_rel_, value_rel_;
    bool has_relevance_ = false;
};

}  // namespace pulsatrix
