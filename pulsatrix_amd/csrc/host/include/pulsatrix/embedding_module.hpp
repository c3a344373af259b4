/** @file embedding_module.hpp
 *  @brief Token embedding (V, d) (the surface of include/pulsatrix/embedding_module.hpp).
 *         forward() validates ids on the host as the reference does (embedding_module.cpp:48-59);
 *         run_forward_device() takes ids resident in HBM and validates them there.
 */
#pragma once

#include <vector>

#include "pulsatrix/detail/fused.hpp"
#include "pulsatrix/module.hpp"

namespace pulsatrix {

class EmbeddingModule : public Module {
public:
    EmbeddingModule(int64_t num_embeddings, int64_t embedding_dim, DeviceBackend* backend);

    /** @brief Each token's relevance: the sum of its embedding row's relevance, (N, L). */
    [[nodiscard]] Tensor propagate_relevance(const Tensor& relevance_out, const LRPRuleConfig& config) override;

    void set_weight(const std::vector<float>& values);
    /** @brief Mutable access counts as a change (the tied head's rule weights are rebuilt). */
    [[nodiscard]] Tensor& weight() noexcept {
        ++version_;
        return weight_;
    }
    [[nodiscard]] const Tensor& weight() const noexcept { return weight_; }
    [[nodiscard]] const float* weight_data() const noexcept { return weight_.data(); }
    [[nodiscard]] uint64_t version() const noexcept { return version_; }
    [[nodiscard]] int64_t num_embeddings() const noexcept { return V_; }
    [[nodiscard]] int64_t embedding_dim() const noexcept { return d_; }

    /** @brief Gathers rows for n x l ids (floats, rounded as llround does) into a module-owned
     *         (n*l, d) buffer. The ids are validated on the device: an id outside [0, V) gathers
     *         row 0 instead and is reported by device_ids_valid(). */
    const float* run_forward_device(const float* ids, int64_t n, int64_t l);
    /** @brief After run_forward over n sequences: repeats every activation the relevance pass reads
     *         `copies` times in place, as if the forward had run over copies * n sequences that
     *         repeat the n (storage from an earlier pass at least that large). */
    void replicate_forward(int64_t copies);
    /** @brief Sizes the buffers replicate_forward() repeats into for `count ids`, without computing. */
    void reserve_forward(int64_t count);
    /** @brief Whether every id of the last run_forward_device() was in range (waits for the stream). */
    [[nodiscard]] bool device_ids_valid();
    /** @brief Per-token sums of a (count, d) relevance into out (count). */
    void token_relevance(const float* relevance, int64_t count, float* out);

protected:
    Tensor forward_impl(const Tensor& input) override;

private:
    int64_t V_, d_;
    MI355XBackend* be_;
    Tensor weight_;
    uint64_t version_ = 0;
    Shape last_shape_;
    detail::DevBuf ids_, out_, ids_checked_, ids_status_;
};

}  // namespace pulsatrix
