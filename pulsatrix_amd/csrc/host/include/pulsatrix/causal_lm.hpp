/** @file causal_lm.hpp
 *  @brief Llama-family decoder LM (the surface of include/pulsatrix/causal_lm.hpp:82-167):
 *         embedding -> blocks -> RMSNorm -> tied or untied head, with AttnLRP relevance back to
 *         the embeddings.
 *
 *  explain_device() is the MI355X hot path: ids already in HBM, forward, on-device argmax seed
 *  (or given targets), relevance and per-token sums, all queued on the backend's stream with no
 *  host round trip, on buffers whose addresses stay fixed for a given (N, L) -- so one call can
 *  be captured into a HIP graph and replayed.
 */
#pragma once

#include <memory>
#include <vector>

#include "pulsatrix/embedding_module.hpp"
#include "pulsatrix/generation.hpp"
#include "pulsatrix/hf_model.hpp"
#include "pulsatrix/linear_module.hpp"
#include "pulsatrix/rms_norm_module.hpp"
#include "pulsatrix/tied_lm_head_module.hpp"
#include "pulsatrix/transformer_block.hpp"

namespace pulsatrix {

class CausalLM : public Module {
public:
    CausalLM(const HfModelConfig& config, DeviceBackend* backend);

    /** @brief Relevance at the embeddings' input: per-token sums, (N, L). */
    [[nodiscard]] Tensor propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) override;
    /** @brief Relevance at every layer boundary, embeddings first: layers + 1 tensors (N, L, d). */
    [[nodiscard]] std::vector<Tensor> propagate_relevance_by_layer(const Tensor& relevance_out,
                                                                   const LRPRuleConfig& config);

    [[nodiscard]] const HfModelConfig& config() const noexcept { return config_; }
    [[nodiscard]] EmbeddingModule& embed_tokens() { return embed_; }
    [[nodiscard]] TransformerBlock& layer(int64_t i) { return *layers_.at(static_cast<size_t>(i)); }
    [[nodiscard]] int64_t num_layers() const noexcept { return static_cast<int64_t>(layers_.size()); }
    [[nodiscard]] RMSNormModule& norm() { return norm_; }
    [[nodiscard]] LinearModule* lm_head() { return lm_head_.get(); }

    /** @brief Forward + seed + relevance + per-token sums on device. ids (N*L floats) in HBM;
     *         token_relevance (N*L) and targets (N int64) written in HBM. targets_in (host, N
     *         entries, nullable): explain those ids at each sequence's last position instead of the
     *         argmax. unit_seed: one-hot seed (LRPSeed::OneHot) instead of the logit value. */
    void explain_device(const float* ids, int64_t n, int64_t l, const LRPRuleConfig& config, float* token_relevance,
                        int64_t* targets, const int64_t* targets_in = nullptr, bool unit_seed = false);
    /** @brief Forward over n x l ids in HBM, then the LRP pass seeded at each sequence's last row
     *         only: target id targets[b * target_stride] (a float id in HBM) with its logit as the
     *         value (or 1 with unit_seed). The head runs on the last rows alone (every other row's
     *         relevance is exactly zero: its seed row is zero), so no (n*l, vocab) logits or seed exist.
     *         token_relevance (n*l) and targets_out (n int64, nullable) in HBM. */
    void explain_rows_device(const float* ids, int64_t n, int64_t l, const float* targets, int64_t target_stride,
                             const LRPRuleConfig& config, float* token_relevance, int64_t* targets_out = nullptr,
                             bool unit_seed = false);
    /** @brief Batched KV-cached greedy decode on the device (MakeCachedNextTokenLogits and greedy
     *         Generate, generation.cpp:189-258, with a batch): ids (n rows of ld_ids floats in HBM)
     *         hold each prompt in its first `prompt` columns; columns prompt .. prompt + new_tokens - 1
     *         receive the generated ids and picked_logit (same layout, nullable) the logits that picked
     *         them. One forward over the prompts fills the KV caches; then each decode step is one HIP
     *         graph replay (the position lives on the device, so no host work between steps). Returns
     *         once the replays have run (the graph is then released). */
    void generate_greedy_device(float* ids, int64_t n, int64_t prompt, int64_t new_tokens, int64_t ld_ids,
                                float* picked_logit = nullptr);
    /** @brief AttnLRP of each generated token: token t (at column prompt + t) explained through a
     *         forward over its prefix (columns 0 .. prompt + t - 1), seeded with its id at the
     *         prefix's last row (explain_rows_device), as the reference explains a cached generation
     *         (forward_cached keeps no relevance state). Consecutive tokens share one pass over the
     *         longest of their prefixes, each seeded at its own row (a causal model's row sees no
     *         later row). token_relevance (new_tokens, n, W) in HBM with W = prompt + new_tokens - 1,
     *         zero past each prefix. */
    void explain_generated_device(const float* ids, int64_t n, int64_t prompt, int64_t new_tokens, int64_t ld_ids,
                                  const LRPRuleConfig& config, float* token_relevance, bool unit_seed = false);
    /** @brief A cached next-token function for the reference's Generate (causal_lm.hpp:116, built
     *         there as MakeCachedNextTokenLogits, generation.cpp:189-258): the first call (and any call
     *         that is not a short extension of the history) runs one forward over the sequence and
     *         fills KV caches of max_length positions; each call that extends the history by a few
     *         tokens runs one decode step per token, replaying a HIP graph of the step (recaptured
     *         whenever the backend has allocated since). The same sequence again returns the last
     *         logits; a prefix of the history reruns its last token. Holds this model, which must
     *         outlive it; one function per sequence being generated.
     *  @throws std::logic_error for a bidirectional model; (when called) std::invalid_argument for an
     *          empty sequence, one longer than max_length, or an id outside [0, vocab). */
    [[nodiscard]] NextTokenLogitsFn next_token_logits(int64_t max_length);
    /** @brief Whether every id of the last device-side pass was in [0, vocab) (waits for the
     *         stream). An out-of-range id is gathered as id 0, so its pass completes; the reference
     *         would have thrown "EmbeddingModule::forward: index out of range [0, num_embeddings)". */
    [[nodiscard]] bool device_ids_valid() { return embed_.device_ids_valid(); }
    /** @brief Device pointers of the last pass: logits (N*L*V), embedding-level relevance (N*L*d). */
    [[nodiscard]] const float* last_logits() const noexcept;
    [[nodiscard]] const float* last_embedding_relevance() const noexcept { return r_embed_; }

    /** @brief Fused-path forward from device ids; returns the logits pointer. */
    const float* run_forward(const float* ids, int64_t n, int64_t l);
    /** @brief Fused-path relevance from a device seed (N*L*V); returns the embedding-level relevance. */
    const float* run_relevance(const float* seed, const LRPRuleConfig& config);

protected:
    Tensor forward_impl(const Tensor& input) override;

private:
    HfModelConfig config_;
    MI355XBackend* be_;
    EmbeddingModule embed_;
    std::vector<std::unique_ptr<TransformerBlock>> layers_;
    RMSNormModule norm_;
    std::unique_ptr<TiedLMHeadModule> tied_head_;
    std::unique_ptr<LinearModule> lm_head_;
    /** @brief Layers, final norm and the head on the last row of each sequence: (n, vocab) logits. */
    const float* forward_last_rows(const float* ids, int64_t n, int64_t l);
    /** @brief explain_rows_device over groups * n sequences of length l (sequence g * n + b),
     *         seeded at row l - groups + g with the id targets[g + b * target_stride]. ids holds the
     *         groups * n sequences, or with `replicate` the n sequences every group repeats (the
     *         forward then runs once and its activations are repeated). */
    void explain_staggered_rows(const float* ids, int64_t n, int64_t groups, int64_t l, const float* targets,
                                int64_t target_stride, const LRPRuleConfig& config, float* token_relevance,
                                int64_t* targets_out, bool unit_seed, bool replicate);
    const float* run_forward_hidden(const float* ids, int64_t n, int64_t l);
    /** @brief One decode step of n sequences: token ids `cur` (n floats in HBM) at the device
     *         position *pos, through every layer's cache; returns the (n, vocab) logits. */
    const float* decode_logits(const float* cur, int64_t n, std::vector<KVCacheState>& caches, const int32_t* pos);
    struct NextTokenState;
    std::vector<float> next_token_call(NextTokenState& s, const std::vector<int64_t>& tokens);

    int64_t N_ = 0, L_ = 0;
    const float* r_embed_ = nullptr;
    detail::DevBuf ids_, seed_, last_x_, r_top_, prompt_ids_, dec_x_, cur_ids_, pos_, tok_tmp_, pick_ws_;
    std::vector<KVCacheState> caches_;
};

}  // namespace pulsatrix
