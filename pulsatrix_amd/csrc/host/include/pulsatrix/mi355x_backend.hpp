/** @file mi355x_backend.hpp
 *  @brief MI355XBackend: the DeviceBackend of one MI355X (gfx950), over libpxk_gfx950's C ABI.
 *
 *  Replaces Pulsatrix's HIPBackend (src/hip_backend.hip, include/pulsatrix/hip_backend.hpp) for the
 *  causal-LM forward + AttnLRP path. Every path op is a hand-written gfx950 kernel (include/pxk.h);
 *  no hipBLAS. One in-order HIP stream per backend; the host waits only on host copies, dot() and
 *  sum() (hip_backend.hpp:64-71). Device memory comes from a size-class caching allocator with
 *  Pulsatrix's contract (pulsatrix/mi355x_allocator.hpp; hip_backend.hip:36-54).
 *  DeviceBackend virtuals outside that path (convolution, pooling, batch/group norm, recurrent
 *  and state-space cells, RL, optimizer steps, dropout, losses, backward passes) run simple
 *  gfx950 kernels (training.hip, module_ops.hip) that add in the reference CPUBackend's order.
 */
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "pulsatrix/device_backend.hpp"
#include "pulsatrix/mi355x_allocator.hpp"
#include "pxk.h"

namespace pulsatrix {

using mi355x::CachingAllocator;

/** @brief One kernel launch of the fused path, kept while a launch log is open so the launches of
 *         a pass can be timed in place (MI355XBackend::time_launch_log). */
struct LaunchRecord {
    std::string kernel;  ///< kernel and variant, e.g. "gemm 32x64d NN pro0 epi2"
    std::string family;  ///< "gemm", "attention" or "rows"
    double flops = 0;    ///< algorithmic FLOPs of the launch (dense, as the reference computes them)
    double bytes = 0;    ///< algorithmic HBM bytes of the launch (memory-bound kernels)
    std::function<int(void* stream)> run;  ///< relaunches it with the same arguments
    int dispatches = 0;  ///< kernels it dispatched in the last time_launch_log replay
};

class MI355XBackend;

/** @brief A HIP graph of work captured on an MI355XBackend's stream for one owner (a model).
 *
 *  The graph addresses the device blocks its launches used at capture time. replay() refuses,
 *  before launching anything, once any block that existed when the owner last captured and that
 *  was allocated for this owner (or the backend's shared split-K pool) has been freed: a longer
 *  pass regrew a buffer, the pool grew, or the owner released its buffers. Destroying the graph
 *  waits for the backend's stream first. */
class CapturedGraph {
public:
    ~CapturedGraph();
    CapturedGraph(const CapturedGraph&) = delete;
    CapturedGraph& operator=(const CapturedGraph&) = delete;
    /** @brief Launches the graph on the backend's stream; throws std::logic_error if it is stale. */
    void replay();
    /** @brief Whether every block the graph may address is still the one it captured. */
    [[nodiscard]] bool valid() const noexcept;

private:
    friend class MI355XBackend;
    CapturedGraph() = default;
    MI355XBackend* be_ = nullptr;
    void* exec_ = nullptr;
    uint64_t owner_ = 0;
    uint64_t owner_retired_ = 0;   // the owner's freed pre-capture blocks at capture time
    uint64_t shared_retired_ = 0;  // the shared pool's, likewise
};

class MI355XBackend : public DeviceBackend {
public:
    /** @brief Binds device `device_index`, creates the backend's stream (default priority). */
    explicit MI355XBackend(int device_index = 0);
    ~MI355XBackend() override;
    MI355XBackend(const MI355XBackend&) = delete;
    MI355XBackend& operator=(const MI355XBackend&) = delete;

    [[nodiscard]] DeviceType device() const noexcept override { return DeviceType::Hip; }
    [[nodiscard]] void* allocate(size_t bytes) override;
    void free(void* ptr) noexcept override;
    void copy(void* dst, const void* src, size_t bytes, CopyDirection dir) override;
    void fill(void* ptr, float value, size_t n) override;
    void gemm(const float* a, const float* b, float* out, size_t m, size_t k, size_t n) override;
    void elementwise(ElementwiseOp op, const float* in, float* out, size_t n) override;
    void add(const float* a, const float* b, float* out, size_t n) override;
    void mul(const float* a, const float* b, float* out, size_t n) override;
    void gemm_ex(const float* a, bool transpose_a, const float* b, bool transpose_b, float* out, size_t m, size_t k,
                 size_t n, float beta) override;
    void gemm_strided_batched(const float* a, bool transpose_a, size_t stride_a, const float* b, bool transpose_b,
                              size_t stride_b, float* out, size_t stride_out, size_t m, size_t k, size_t n,
                              size_t batch, float beta = 0.0f) override;
    void column_sums(const float* in, float* out, size_t rows, size_t cols, float beta) override;
    void add_row_vector(const float* in, const float* row, float* out, size_t rows, size_t cols) override;
    void elementwise_backward(ElementwiseOp op, const float* x, const float* grad_out, float* grad_in,
                              size_t n) override;
    void axpby(float alpha, const float* x, float beta, const float* y, float* out, size_t n) override;
    [[nodiscard]] float dot(const float* a, const float* b, size_t n) override;
    void dot_into(const float* a, const float* b, size_t n, float* out) override;
    void softmax_rows(const float* in, float* out, size_t rows, size_t cols) override;
    void softmax_rows_backward(const float* y, const float* dy, float* dx, size_t rows, size_t cols) override;
    void logsumexp_rows(const float* in, float* out, size_t rows, size_t cols) override;
    void adam_step(float* param, const float* grad, float* m, float* v, size_t n, float lr, float beta1, float beta2,
                   float eps, float bias_correction1, float bias_correction2) override;
    [[nodiscard]] float sum(const float* in, size_t n) override;
    void dropout_forward(const float* in, float* out, float* mask, size_t n, float p, float scale, uint64_t seed,
                         uint64_t offset) override;
    void bce_with_logits(const float* logits, const float* target, float* out, size_t n) override;
    void bce_with_logits_grad(const float* logits, const float* target, float* grad, size_t n, float scale) override;
    void layer_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                            float* row_std, size_t rows, size_t cols, float eps) override;
    void layer_norm_backward(const float* grad_out, const float* gamma, const float* xhat, const float* row_std,
                             float* grad_in, size_t rows, size_t cols) override;
    void rms_norm_forward(const float* in, const float* gamma, float* out, float* row_rms, size_t rows, size_t cols,
                          float eps) override;
    void rms_norm_backward(const float* grad_out, const float* gamma, const float* in, const float* row_rms,
                           float* grad_in, float* gamma_terms, size_t rows, size_t cols) override;
    void rope_rotate(const float* in, const float* cos_table, const float* sin_table, float* out, size_t num_slices,
                     size_t seq_len, size_t head_dim, bool inverse, bool rotate_half) override;
    void permute_0213(const float* in, float* out, size_t d0, size_t d1, size_t d2, size_t d3) override;
    void attention_mask_fill(float* scores, const float* key_keep, size_t batch, size_t heads, size_t q_len,
                             size_t k_len, bool causal, size_t q_offset, size_t window, float value) override;
    void gather_rows(const float* table, const float* indices, float* out, size_t count, size_t dim) override;
    void scatter_add_rows(const float* src, const float* indices, float* table, size_t count, size_t dim) override;
    void tanh_gaussian_forward(const float* mean, const float* log_std, const float* eps, float* action,
                               float* std_cache, float* log_prob, size_t rows, size_t cols, float stabilizer,
                               double half_log_two_pi) override;
    void tanh_gaussian_backward(const float* action, const float* std_cache, const float* eps,
                                const float* grad_action, const float* grad_log_prob, float* grad_mean,
                                float* grad_log_std, size_t n, float stabilizer) override;
    void lrp_linear(const float* x, const float* w, const float* z, const float* r, float* r_in, size_t rows,
                    size_t in_features, size_t out_features, float eps) override;
    void lrp_residual_split(const float* a, const float* b, const float* r, float* r_a, float* r_b, size_t n,
                            float eps) override;
    void lrp_bilinear_elementwise(const float* a, const float* b, const float* r, float* r_out, size_t n,
                                  float eps) override;
    void lrp_bilinear_matmul(const float* a, const float* b, const float* o, const float* r_o, float* r_a, float* r_b,
                             size_t slices, size_t m, size_t p, size_t q, float eps, bool b_transposed) override;
    void lrp_softmax_rows(const float* x, const float* y, const float* r, float* r_in, size_t rows,
                          size_t cols) override;
    void lrp_rope(const float* x, const float* y, const float* r, const float* cos_table, const float* sin_table,
                  float* r_in, size_t slices, size_t seq_len, size_t head_dim, float eps, bool rotate_half) override;
    void logic_pointwise(LogicOp op, int norm, const float* a, const float* b, const float* g_or_r, const float* y,
                         float* out_a, float* out_b, size_t n, float eps) override;
    void aggregator_forward(const float* x, float* mean_pow, float* out, size_t n, size_t cols, float p) override;
    void aggregator_backward(const float* x, const float* mean_pow, const float* grad_out, float* grad_in, size_t n,
                             size_t cols, float p) override;
    void aggregator_lrp(const float* x, const float* mean_pow, const float* r_out, float* r_in, size_t n, size_t cols,
                        float p, float eps) override;
    void im2col(const float* in, float* col, size_t n, size_t c, size_t h, size_t w,
                const ConvGeometry& geometry) override;
    void col2im_add(const float* col, float* out, size_t n, size_t c, size_t h, size_t w,
                    const ConvGeometry& geometry) override;
    void add_channel_vector(const float* in, const float* vec, float* out, size_t n, size_t c, size_t inner) override;
    void lrp_conv(const float* col, const float* kernel, const float* pre_bias, const float* r, float* r_col,
                  size_t n, size_t out_channels, size_t p, size_t q, float eps) override;
    void lrp_stabilized_divide(const float* r, const float* denom, const float* gate, float* out, size_t n, float eps,
                               LrpGate gate_mode) override;
    void max_pool_forward(const float* in, float* out, float* argmax, size_t planes, size_t h, size_t w, size_t kh,
                          size_t kw, size_t sh, size_t sw, size_t ph, size_t pw) override;
    void max_unpool(const float* src, const float* argmax, float* dst, size_t planes, size_t h, size_t w, size_t kh,
                    size_t kw, size_t sh, size_t sw, size_t ph, size_t pw) override;
    void avg_pool_forward(const float* in, float* out, size_t planes, size_t h, size_t w, size_t kh,
                          size_t kw) override;
    void avg_pool_backward(const float* grad_out, float* grad_in, size_t planes, size_t h, size_t w, size_t kh,
                           size_t kw) override;
    void lrp_avg_pool(const float* x, const float* r, float* r_in, size_t planes, size_t h, size_t w, size_t kh,
                      size_t kw, float eps) override;
    void batch_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                            float* channel_std, size_t n, size_t c, size_t spatial, float eps) override;
    void batch_norm_backward(const float* grad_out, const float* gamma, const float* xhat, const float* channel_std,
                             float* grad_in, float* gamma_grad, float* beta_grad, size_t n, size_t c,
                             size_t spatial) override;
    void batch_norm_update_running(const float* in, float* running_mean, float* running_var, size_t n, size_t c,
                                   size_t spatial, float momentum) override;
    void batch_norm_eval_forward(const float* in, const float* gamma, const float* beta, const float* running_mean,
                                 const float* running_var, float* xhat, float* out, float* channel_std, size_t n,
                                 size_t c, size_t spatial, float eps) override;
    void batch_norm_eval_backward(const float* grad_out, const float* gamma, const float* xhat,
                                  const float* channel_std, float* grad_in, float* gamma_grad, float* beta_grad,
                                  size_t n, size_t c, size_t spatial) override;
    void group_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                            float* group_std, size_t n, size_t c, size_t spatial, size_t num_groups,
                            float eps) override;
    void group_norm_backward(const float* grad_out, const float* gamma, const float* xhat, const float* group_std,
                             float* grad_in, float* gamma_grad, float* beta_grad, size_t n, size_t c, size_t spatial,
                             size_t num_groups) override;
    void copy_2d(float* dst, size_t dst_stride, const float* src, size_t src_stride, size_t rows,
                 size_t cols) override;
    void accumulate_rows(const float* in, float* out, size_t rows, size_t cols) override;
    void recurrent_cell(RecurrentCellOp op, const RecurrentCellArgs& args, size_t n) override;
    void gru_lrp_hprev(const float* h_prev, const float* w_hn, const float* hn, const float* r_term_b,
                       const float* direct, float* r_hprev, size_t rows, size_t hidden, float eps) override;
    void ssm_pass(SsmPassOp op, const SsmPassArgs& args) override;
    void rl_rows(RlRowOp op, const RlRowArgs& args) override;
    void top_k_rows(const float* in, float* values, float* indices, size_t rows, size_t cols, size_t k,
                    bool largest) override;

    // ---- MI355X extensions used by the fused module path ----------------------------------
    /** @brief The backend's HIP stream (hipStream_t as void*). */
    [[nodiscard]] void* stream() const noexcept { return stream_; }
    /** @brief Waits for everything queued on the stream. */
    void synchronize();
    /** @brief Runs one fused GEMM, supplying the split-K workspace from the backend's own pool. */
    void run_gemm(pxk_gemm_desc& d);
    /** @brief Throws (std::invalid_argument / std::runtime_error) unless rc == PXK_OK. */
    static void check(int rc, const char* what);
    /** @brief Captures what `work` queues on the stream into a HIP graph owned by the caller, on
     *         behalf of `owner` (work runs with that owner current). Nothing runs on the device. The
     *         capture is refused (std::logic_error, no graph) if the work frees device memory while it
     *         is captured: a captured launch may address the freed block. Run the work once eagerly
     *         at the same shapes first, so that every buffer it uses already exists. */
    std::unique_ptr<CapturedGraph> capture(uint64_t owner, const std::function<void()>& work);
    /** @brief A fresh owner tag (never 0). Blocks allocated while an owner is current carry its tag;
     *         graphs and launch logs are validated against the frees of their owner's blocks. */
    uint64_t new_owner() noexcept { return ++owner_count_; }
    /** @brief Sets the current owner (0: none) and returns the previous one. */
    uint64_t set_owner(uint64_t owner) noexcept {
        const uint64_t prev = owner_;
        owner_ = owner;
        return prev;
    }
    /** @brief Drops an owner's bookkeeping (its model is gone; its graphs must be gone first). */
    void forget_owner(uint64_t owner);
    CachingAllocator& allocator() { return *allocator_; }
    /** @brief Counts the backend's allocations (allocate() and workspace growth). A graph captured
     *         at one count still addresses live buffers while the count is unchanged: a buffer that
     *         moved was reallocated. */
    [[nodiscard]] uint64_t allocation_epoch() const noexcept { return allocations_; }

    /** @brief Runs `f(stream)` (a pxk_* launch returning its status) and, while a launch log is
     *         open, records it with its algorithmic work. */
    template <class F>
    void launch(const char* kernel, const char* family, double flops, double bytes, const char* what, F&& f) {
        check(f(stream_), what);
        if (logging_) {
            log_.push_back(LaunchRecord{kernel, family, flops, bytes, std::function<int(void*)>(f)});
            if (owner_ != 0) log_owner_ = owner_;  // the model whose buffers the log addresses
        }
        if (sync_debug_) synchronize();
    }
    /** @brief Opens (clearing) / closes the launch log. Every buffer a logged launch touches must
     *         outlive the log: module buffers do; the GEMM workspace is pinned while it is open.
     *         Closing it snapshots the current owner's blocks as a capture does, and
     *         time_launch_log refuses once one of them has been freed. */
    void start_launch_log();
    void stop_launch_log();
    [[nodiscard]] const std::vector<LaunchRecord>& launch_log() const noexcept { return log_; }
    /** @brief Replays the logged launches in order, `reps` times, each dispatch recording its own
     *         start and end events (pxk_timing_*); seconds[i] = mean summed duration of launch i's
     *         kernels. Logged launches rewrite their outputs. */
    void time_launch_log(int reps, std::vector<double>& seconds);

private:
    friend class CapturedGraph;
    struct Block {
        uint64_t serial;  // allocation order
        uint64_t owner;   // the owner current at allocation; kSharedOwner for the split-K pool
    };
    struct OwnerState {
        uint64_t captured_serial = 0;  // blocks up to this serial existed at the owner's last capture
        uint64_t retired = 0;          // how many of those have been freed since
    };
    static constexpr uint64_t kSharedOwner = ~uint64_t{0};
    float* workspace(size_t bytes);
    void* track(void* p, uint64_t owner);
    void untrack(void* p) noexcept;
    void snapshot(uint64_t owner, uint64_t& owner_retired, uint64_t& shared_retired);
    [[nodiscard]] bool unchanged(uint64_t owner, uint64_t owner_retired, uint64_t shared_retired) const noexcept;

    int device_ = 0;
    void* stream_ = nullptr;
    std::unique_ptr<CachingAllocator> allocator_;
    float* ws_ = nullptr;
    size_t ws_bytes_ = 0;
    uint64_t allocations_ = 0;
    float* reduce_ = nullptr;  // dot/sum partials + result slot
    bool sync_debug_ = false;
    uint64_t owner_ = 0, owner_count_ = 0;
    std::unordered_map<void*, Block> blocks_;             // live allocations
    std::unordered_map<uint64_t, OwnerState> owners_;     // owners that captured a graph or a log
    uint64_t shared_captured_serial_ = 0, shared_retired_ = 0;
    bool capturing_ = false;
    uint64_t frees_in_capture_ = 0;
    uint64_t log_owner_ = 0, log_owner_retired_ = 0, log_shared_retired_ = 0;
    bool logging_ = false;
    std::vector<LaunchRecord> log_;
    std::vector<float*> retired_ws_;  // workspaces outgrown while a log was open (logged GEMMs use them)
};

}  // namespace pulsatrix
