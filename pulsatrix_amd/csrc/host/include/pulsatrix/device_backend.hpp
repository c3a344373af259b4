/** @file device_backend.hpp
 *  @brief The DeviceBackend plug-in interface: the boundary every Pulsatrix module computes through.
 *
 *  The enums, argument structs and virtual signatures are those of Pulsatrix's
 *  include/pulsatrix/device_backend.hpp:17-838 (same names, order, parameter types and defaults),
 *  so a backend written against this header compiles against the reference's and the reference's
 *  modules can run on it. The contract each virtual carries (aliasing, beta semantics, "throw,
 *  never return null") is restated in the comments.
 */
#pragma once

#include <cstddef>
#include <cstdint>

namespace pulsatrix {

/** @brief Where a Tensor's buffer lives (device_backend.hpp:17-21). */
enum class DeviceType { Cpu, Cuda, Hip };

/** @brief Direction of DeviceBackend::copy() (device_backend.hpp:24-29). */
enum class CopyDirection { HostToDevice, DeviceToHost, DeviceToDevice, HostToHost };

/** @brief Unary ops of DeviceBackend::elementwise(), in the reference's order (device_backend.hpp:39-48). */
enum class ElementwiseOp { Relu, Neg, Tanh, Sigmoid, Silu, Exp, GeluTanh, Gelu };

/** @brief Which elements lrp_stabilized_divide() passes (device_backend.hpp:55-59). */
enum class LrpGate { None, Positive, Negative };

/** @brief Fuzzy-logic module passes (device_backend.hpp:66-73). */
enum class LogicOp {
    ConjunctionForward,
    ConjunctionBackward,
    ConjunctionLrp,
    DisjunctionForward,
    DisjunctionBackward,
    DisjunctionLrp
};

/** @brief Recurrent-cell passes (device_backend.hpp:89). */
enum class RecurrentCellOp { RnnBackward, LstmForward, LstmBackward, LstmLrp, GruBackward, GruLrp };

struct RecurrentCellArgs {
    const float* in[10] = {};
    float* out[6] = {};
    float eps = 0.0f;
};

/** @brief State-space-model passes (device_backend.hpp:126-146). */
enum class SsmPassOp {
    MambaForward,
    MambaBackward,
    MambaGradBC,
    MambaLrp,
    RwkvTokenShift,
    RwkvForward,
    RwkvBackward,
    RwkvShiftBackward,
    RwkvLrp,
    RwkvShiftLrp,
    StabilizedDiv,
    RetnetForward,
    RetnetStateGrad,
    RetnetGradQK,
    RetnetGradV,
    RetnetScores,
    RetnetReadout,
    RetnetLrpInput,
    ReverseTimeSum
};

struct SsmPassArgs {
    const float* in[12] = {};
    float* out[10] = {};
    int64_t n = 0;
    int64_t l = 0;
    int64_t d = 0;
    int64_t s = 0;
    float eps = 0.0f;
    float gamma = 0.0f;
};

struct ConvGeometry {
    size_t kh;
    size_t kw;
    size_t stride_h = 1;
    size_t stride_w = 1;
    size_t pad_h = 0;
    size_t pad_w = 0;
};

enum class RlRowOp { DqnLoss, DqnGrad, PgLoss, PgGrad, PpoLoss, PpoGrad, DqnTarget, PolyakBlend, TokenCeLoss };

struct RlRowArgs {
    const float* in[5] = {};
    float* out[4] = {};
    int64_t rows = 0;
    int64_t cols = 0;
    float scale = 0.0f;
    float lower = 0.0f;
    float upper = 0.0f;
    float gamma = 0.0f;
    float tau = 0.0f;
    int64_t ignore_index = -100;
};

struct AdamTensorStep {
    float* param = nullptr;
    const float* grad = nullptr;
    float* m = nullptr;
    float* v = nullptr;
    size_t n = 0;
    float lr = 0.0f;
    float bias_correction1 = 1.0f;
    float bias_correction2 = 1.0f;
    float decay = 1.0f;
    float l2 = 0.0f;
};

/**
 * @brief Vendor-specific memory and compute behind raw float pointers. Implementations keep
 *        identical numeric semantics and error behaviour: failures throw, allocate() never returns
 *        null for a nonzero request (device_backend.hpp:241-247).
 */
class DeviceBackend {
public:
    virtual ~DeviceBackend() = default;

    [[nodiscard]] virtual DeviceType device() const noexcept = 0;
    /** @brief nullptr for 0 bytes; throws on failure. */
    [[nodiscard]] virtual void* allocate(size_t bytes) = 0;
    /** @brief Safe with nullptr. */
    virtual void free(void* ptr) noexcept = 0;
    virtual void copy(void* dst, const void* src, size_t bytes, CopyDirection dir) = 0;
    virtual void fill(void* ptr, float value, size_t n) = 0;

    /** @brief out (m x n) = a (m x k) * b (k x n), row-major. */
    virtual void gemm(const float* a, const float* b, float* out, size_t m, size_t k, size_t n) = 0;
    /** @brief out may alias in. */
    virtual void elementwise(ElementwiseOp op, const float* in, float* out, size_t n) = 0;
    /** @brief out may alias a or b. */
    virtual void add(const float* a, const float* b, float* out, size_t n) = 0;
    virtual void mul(const float* a, const float* b, float* out, size_t n) = 0;

    /** @brief out = op(a) op(b) + beta out; beta == 0 never reads out; out must not alias a or b. */
    virtual void gemm_ex(const float* a, bool transpose_a, const float* b, bool transpose_b, float* out, size_t m,
                         size_t k, size_t n, float beta) = 0;

    /** @brief batch independent gemm_ex() products at strides (a stride of 0 shares a matrix). */
    virtual void gemm_strided_batched(const float* a, bool transpose_a, size_t stride_a, const float* b,
                                      bool transpose_b, size_t stride_b, float* out, size_t stride_out, size_t m,
                                      size_t k, size_t n, size_t batch, float beta = 0.0f) {
        for (size_t i = 0; i < batch; ++i) {
            if (!transpose_a && !transpose_b && beta == 0.0f) {
                gemm(a + i * stride_a, b + i * stride_b, out + i * stride_out, m, k, n);
            } else {
                gemm_ex(a + i * stride_a, transpose_a, b + i * stride_b, transpose_b, out + i * stride_out, m, k, n,
                        beta);
            }
        }
    }

    /** @brief acc += parts[0], += parts[1], ... in order. */
    virtual void accumulate_parts(const float* parts, size_t count, size_t n, float* acc) {
        for (size_t i = 0; i < count; ++i) add(acc, parts + i * n, acc, n);
    }

    /** @brief out[j] = beta out[j] + sum_i in[i][j]; out must not alias in. */
    virtual void column_sums(const float* in, float* out, size_t rows, size_t cols, float beta) = 0;
    /** @brief out[i][j] = in[i][j] + row[j]; out may alias in. */
    virtual void add_row_vector(const float* in, const float* row, float* out, size_t rows, size_t cols) = 0;
    virtual void add_row_vector_relu(const float* in, const float* row, float* z, float* out, size_t rows,
                                     size_t cols) {
        add_row_vector(in, row, z, rows, cols);
        elementwise(ElementwiseOp::Relu, z, out, rows * cols);
    }
    virtual void elementwise_backward(ElementwiseOp op, const float* x, const float* grad_out, float* grad_in,
                                      size_t n) = 0;
    /** @brief out = alpha x + beta y; beta == 0 does not read y; out may alias x or y. */
    virtual void axpby(float alpha, const float* x, float beta, const float* y, float* out, size_t n) = 0;
    /** @brief Synchronizes; fixed-order reduction. */
    [[nodiscard]] virtual float dot(const float* a, const float* b, size_t n) = 0;
    virtual void dot_into(const float* a, const float* b, size_t n, float* out) {
        const float result = dot(a, b, n);
        copy(out, &result, sizeof(float), CopyDirection::HostToDevice);
    }
    /** @brief Max-subtracted row softmax; out may alias in. */
    virtual void softmax_rows(const float* in, float* out, size_t rows, size_t cols) = 0;
    virtual void softmax_rows_backward(const float* y, const float* dy, float* dx, size_t rows, size_t cols) = 0;
    virtual void logsumexp_rows(const float* in, float* out, size_t rows, size_t cols) = 0;
    virtual void adam_step(float* param, const float* grad, float* m, float* v, size_t n, float lr, float beta1,
                           float beta2, float eps, float bias_correction1, float bias_correction2) = 0;
    virtual void adam_step_multi(const AdamTensorStep* tensors, size_t count, float beta1, float beta2, float eps) {
        for (size_t t = 0; t < count; ++t) {
            const AdamTensorStep& s = tensors[t];
            if (s.n == 0) continue;
            if (s.decay != 1.0f) axpby(s.decay, s.param, 0.0f, s.param, s.param, s.n);
            const float* grad = s.grad;
            void* decayed = nullptr;
            if (s.l2 != 0.0f) {
                decayed = allocate(s.n * sizeof(float));
                axpby(s.l2, s.param, 1.0f, s.grad, static_cast<float*>(decayed), s.n);
                grad = static_cast<const float*>(decayed);
            }
            adam_step(s.param, grad, s.m, s.v, s.n, s.lr, beta1, beta2, eps, s.bias_correction1, s.bias_correction2);
            free(decayed);
        }
    }
    /** @brief Synchronizes; same reduction order as dot(). */
    [[nodiscard]] virtual float sum(const float* in, size_t n) = 0;
    virtual void dropout_forward(const float* in, float* out, float* mask, size_t n, float p, float scale,
                                 uint64_t seed, uint64_t offset) = 0;
    virtual void bce_with_logits(const float* logits, const float* target, float* out, size_t n) = 0;
    virtual void bce_with_logits_grad(const float* logits, const float* target, float* grad, size_t n,
                                      float scale) = 0;
    virtual void layer_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                                    float* row_std, size_t rows, size_t cols, float eps) = 0;
    virtual void layer_norm_backward(const float* grad_out, const float* gamma, const float* xhat,
                                     const float* row_std, float* grad_in, size_t rows, size_t cols) = 0;
    /** @brief out = gamma x / sqrt(mean(x^2) + eps) per row; row_rms receives each row's rms. */
    virtual void rms_norm_forward(const float* in, const float* gamma, float* out, float* row_rms, size_t rows,
                                  size_t cols, float eps) = 0;
    virtual void rms_norm_backward(const float* grad_out, const float* gamma, const float* in, const float* row_rms,
                                   float* grad_in, float* gamma_terms, size_t rows, size_t cols) = 0;
    /** @brief Rotary embedding over (num_slices, seq_len, head_dim); out must not alias in. */
    virtual void rope_rotate(const float* in, const float* cos_table, const float* sin_table, float* out,
                             size_t num_slices, size_t seq_len, size_t head_dim, bool inverse, bool rotate_half) = 0;
    /** @brief (d0, d1, d2, d3) -> (d0, d2, d1, d3); out must not alias in. */
    virtual void permute_0213(const float* in, float* out, size_t d0, size_t d1, size_t d2, size_t d3) = 0;
    virtual void attention_mask_fill(float* scores, const float* key_keep, size_t batch, size_t heads, size_t q_len,
                                     size_t k_len, bool causal, size_t q_offset, size_t window, float value) = 0;
    virtual void gather_rows(const float* table, const float* indices, float* out, size_t count, size_t dim) = 0;
    virtual void scatter_add_rows(const float* src, const float* indices, float* table, size_t count, size_t dim) = 0;
    virtual void tanh_gaussian_forward(const float* mean, const float* log_std, const float* eps, float* action,
                                       float* std_cache, float* log_prob, size_t rows, size_t cols,
                                       float stabilizer, double half_log_two_pi) = 0;
    virtual void tanh_gaussian_backward(const float* action, const float* std_cache, const float* eps,
                                        const float* grad_action, const float* grad_log_prob, float* grad_mean,
                                        float* grad_log_std, size_t n, float stabilizer) = 0;
    /** @brief r_in[n][i] = sum_j (x[n][i] w[i][j] / stab(z[n][j])) r[n][j]. */
    virtual void lrp_linear(const float* x, const float* w, const float* z, const float* r, float* r_in, size_t rows,
                            size_t in_features, size_t out_features, float eps) = 0;
    virtual void lrp_residual_split(const float* a, const float* b, const float* r, float* r_a, float* r_b, size_t n,
                                    float eps) = 0;
    virtual void lrp_bilinear_elementwise(const float* a, const float* b, const float* r, float* r_out, size_t n,
                                          float eps) = 0;
    /** @brief AttnLRP Eq. 15 for slices of O = A B; r_a, r_b overwritten. */
    virtual void lrp_bilinear_matmul(const float* a, const float* b, const float* o, const float* r_o, float* r_a,
                                     float* r_b, size_t slices, size_t m, size_t p, size_t q, float eps,
                                     bool b_transposed) = 0;
    virtual void lrp_softmax_rows(const float* x, const float* y, const float* r, float* r_in, size_t rows,
                                  size_t cols) = 0;
    virtual void lrp_rope(const float* x, const float* y, const float* r, const float* cos_table,
                          const float* sin_table, float* r_in, size_t slices, size_t seq_len, size_t head_dim,
                          float eps, bool rotate_half) = 0;
    virtual void logic_pointwise(LogicOp op, int norm, const float* a, const float* b, const float* g_or_r,
                                 const float* y, float* out_a, float* out_b, size_t n, float eps) = 0;
    virtual void aggregator_forward(const float* x, float* mean_pow, float* out, size_t n, size_t cols, float p) = 0;
    virtual void aggregator_backward(const float* x, const float* mean_pow, const float* grad_out, float* grad_in,
                                     size_t n, size_t cols, float p) = 0;
    virtual void aggregator_lrp(const float* x, const float* mean_pow, const float* r_out, float* r_in, size_t n,
                                size_t cols, float p, float eps) = 0;
    virtual void im2col(const float* in, float* col, size_t n, size_t c, size_t h, size_t w,
                        const ConvGeometry& geometry) = 0;
    virtual void col2im_add(const float* col, float* out, size_t n, size_t c, size_t h, size_t w,
                            const ConvGeometry& geometry) = 0;
    virtual void add_channel_vector(const float* in, const float* vec, float* out, size_t n, size_t c,
                                    size_t inner) = 0;
    virtual void lrp_conv(const float* col, const float* kernel, const float* pre_bias, const float* r, float* r_col,
                          size_t n, size_t out_channels, size_t p, size_t q, float eps) = 0;
    /** @brief out = passes(gate) ? r / stab(denom) : 0; out may alias r or denom. */
    virtual void lrp_stabilized_divide(const float* r, const float* denom, const float* gate, float* out, size_t n,
                                       float eps, LrpGate gate_mode) = 0;
    virtual void max_pool_forward(const float* in, float* out, float* argmax, size_t planes, size_t h, size_t w,
                                  size_t kh, size_t kw, size_t sh, size_t sw, size_t ph, size_t pw) = 0;
    virtual void max_unpool(const float* src, const float* argmax, float* dst, size_t planes, size_t h, size_t w,
                            size_t kh, size_t kw, size_t sh, size_t sw, size_t ph, size_t pw) = 0;
    virtual void avg_pool_forward(const float* in, float* out, size_t planes, size_t h, size_t w, size_t kh,
                                  size_t kw) = 0;
    virtual void avg_pool_backward(const float* grad_out, float* grad_in, size_t planes, size_t h, size_t w, size_t kh,
                                   size_t kw) = 0;
    virtual void lrp_avg_pool(const float* x, const float* r, float* r_in, size_t planes, size_t h, size_t w, size_t kh,
                              size_t kw, float eps) = 0;
    virtual void batch_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                                    float* channel_std, size_t n, size_t c, size_t spatial, float eps) = 0;
    virtual void batch_norm_backward(const float* grad_out, const float* gamma, const float* xhat,
                                     const float* channel_std, float* grad_in, float* gamma_grad, float* beta_grad,
                                     size_t n, size_t c, size_t spatial) = 0;
    virtual void batch_norm_update_running(const float* in, float* running_mean, float* running_var, size_t n,
                                           size_t c, size_t spatial, float momentum) = 0;
    virtual void batch_norm_eval_forward(const float* in, const float* gamma, const float* beta,
                                         const float* running_mean, const float* running_var, float* xhat, float* out,
                                         float* channel_std, size_t n, size_t c, size_t spatial, float eps) = 0;
    virtual void batch_norm_eval_backward(const float* grad_out, const float* gamma, const float* xhat,
                                          const float* channel_std, float* grad_in, float* gamma_grad,
                                          float* beta_grad, size_t n, size_t c, size_t spatial) = 0;
    virtual void group_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                                    float* group_std, size_t n, size_t c, size_t spatial, size_t num_groups,
                                    float eps) = 0;
    virtual void group_norm_backward(const float* grad_out, const float* gamma, const float* xhat,
                                     const float* group_std, float* grad_in, float* gamma_grad, float* beta_grad,
                                     size_t n, size_t c, size_t spatial, size_t num_groups) = 0;
    virtual void copy_2d(float* dst, size_t dst_stride, const float* src, size_t src_stride, size_t rows,
                         size_t cols) = 0;
    /** @brief out[j] += in[i][j] for i in order. */
    virtual void accumulate_rows(const float* in, float* out, size_t rows, size_t cols) = 0;
    virtual void recurrent_cell(RecurrentCellOp op, const RecurrentCellArgs& args, size_t n) = 0;
    virtual void gru_lrp_hprev(const float* h_prev, const float* w_hn, const float* hn, const float* r_term_b,
                               const float* direct, float* r_hprev, size_t rows, size_t hidden, float eps) = 0;
    virtual void ssm_pass(SsmPassOp op, const SsmPassArgs& args) = 0;
    virtual void rl_rows(RlRowOp op, const RlRowArgs& args) = 0;
    virtual void top_k_rows(const float* in, float* values, float* indices, size_t rows, size_t cols, size_t k,
                            bool largest) = 0;
};

}  // namespace pulsatrix
