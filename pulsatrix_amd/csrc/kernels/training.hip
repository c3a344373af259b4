// training.hip -- the DeviceBackend ops of training and of the non-LLM modules that are rows or
// elements (include/pxk.h): activation, softmax and RMSNorm backward, the embedding's scatter-add,
// LayerNorm, log-sum-exp, Adam, dropout, BCE-with-logits, the tanh-Gaussian policy and top-k.
// Simple, correct kernels: one thread per element, or one wave64 per row with the row's sums
// reduced across the wave in a fixed order (deterministic, no atomics). Each computes the
// reference's per-element expression (src/cpu_backend.cpp, src/row_math.hpp,
// src/pointwise_math.hpp, src/top_k_math.hpp); sums over a row run in another order than the
// reference's sequential loop, so they agree to rounding.
#include <cmath>
#include <cstdint>

#include "common.hpp"

namespace pxk {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / kWave;

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }  // cpu_backend.cpp:29

// d/dx of the tanh-approximated GeLU, 0.5 x (1 + tanh(b (x + k x^3))), b = sqrt(2 / pi), k = 0.044715.
__device__ __forceinline__ float gelu_tanh_slope(float x) {
    const float b = 0.7978845608028654f, k = 0.044715f;
    const float x2 = x * x;
    const float t = tanhf(b * (x + k * x2 * x));
    return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * b * (1.0f + 3.0f * k * x2);
}

// d/dx of x Phi(x): Phi(x) + x phi(x).
__device__ __forceinline__ float gelu_slope(float x) {
    return 0.5f * (1.0f + erff(x * 0.7071067811865476f)) + x * 0.3989422804014327f * expf(-0.5f * x * x);
}

// elementwise_backward (cpu_backend.cpp:226-270): grad_in = grad_out * f'(x); ReLU selects, so a
// non-finite gradient where x <= 0 still gives 0.
__global__ void __launch_bounds__(kThreads) act_backward_kernel(int op, const float* x, const float* gy, float* gx,
                                                                int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const float v = x[i], g = gy[i];
        float d;
        switch (op) {
            case 0: gx[i] = v > 0.0f ? g : 0.0f; continue;  // Relu
            case 1: d = -1.0f; break;                        // Neg
            case 2: {                                        // Tanh
                const float t = tanhf(v);
                d = 1.0f - t * t;
                break;
            }
            case 3: {  // Sigmoid
                const float s = sigm(v);
                d = s * (1.0f - s);
                break;
            }
            case 4: {  // Silu: s + x s (1 - s)
                const float s = sigm(v);
                d = s + v * s * (1.0f - s);
                break;
            }
            case 5: d = expf(v); break;               // Exp
            case 6: d = gelu_tanh_slope(v); break;    // GeluTanh
            default: d = gelu_slope(v); break;        // Gelu
        }
        gx[i] = g * d;
    }
}

// One wave per row: lanes stride over the columns; wave_sum reduces in a fixed lane order.
#define PXK_ROW_LOOP(rows)                                                                    \
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6); \
    const int lane = threadIdx.x & 63;                                                        \
    if (row >= (rows)) return;

// softmax_rows_backward (cpu_backend.cpp:312-323): dx = y (dy - sum(y dy)).
__global__ void __launch_bounds__(kThreads) softmax_backward_kernel(const float* y, const float* dy, float* dx,
                                                                    int64_t rows, int64_t cols) {
    PXK_ROW_LOOP(rows)
    const float* yr = y + row * cols;
    const float* gr = dy + row * cols;
    float dot = 0.0f;
    for (int64_t j = lane; j < cols; j += kWave) dot += yr[j] * gr[j];
    dot = wave_sum(dot);
    for (int64_t j = lane; j < cols; j += kWave) dx[row * cols + j] = yr[j] * (gr[j] - dot);
}

// rms_norm_backward (row_math.hpp:75-86): gamma_terms = g x / rms; grad_in = g gamma / rms
// - x / (D rms^3) sum(g gamma x).
__global__ void __launch_bounds__(kThreads) rms_backward_kernel(const float* gy, const float* gamma, const float* x,
                                                                const float* row_rms, float* gx, float* gterms,
                                                                int64_t rows, int64_t cols) {
    PXK_ROW_LOOP(rows)
    const int64_t off = row * cols;
    const float rms = row_rms[row], D = static_cast<float>(cols);
    float dot = 0.0f;
    for (int64_t j = lane; j < cols; j += kWave) dot += gy[off + j] * gamma[j] * x[off + j];
    dot = wave_sum(dot);
    for (int64_t j = lane; j < cols; j += kWave) {
        gterms[off + j] = gy[off + j] * x[off + j] / rms;
        gx[off + j] = gy[off + j] * gamma[j] / rms - (x[off + j] / (D * rms * rms * rms)) * dot;
    }
}

// layer_norm_forward (row_math.hpp:15-38): mean, then the mean of squared deviations, std =
// sqrt(var + eps); xhat = (x - mu) / std, out = gamma xhat + beta.
__global__ void __launch_bounds__(kThreads) layer_norm_kernel(const float* x, const float* gamma, const float* beta,
                                                              float* xhat, float* out, float* row_std, int64_t rows,
                                                              int64_t cols, float eps) {
    PXK_ROW_LOOP(rows)
    const int64_t off = row * cols;
    const float D = static_cast<float>(cols);
    float s = 0.0f;
    for (int64_t j = lane; j < cols; j += kWave) s += x[off + j];
    const float mu = wave_sum(s) / D;
    float q = 0.0f;
    for (int64_t j = lane; j < cols; j += kWave) {
        const float d = x[off + j] - mu;
        q += d * d;
    }
    const float sd = sqrtf(wave_sum(q) / D + eps);
    if (lane == 0) row_std[row] = sd;
    for (int64_t j = lane; j < cols; j += kWave) {
        const float xh = (x[off + j] - mu) / sd;
        xhat[off + j] = xh;
        out[off + j] = gamma[j] * xh + beta[j];
    }
}

// layer_norm_backward (row_math.hpp:40-56): with g = grad_out gamma,
// grad_in = (D g - sum g - xhat sum(g xhat)) / (D std).
__global__ void __launch_bounds__(kThreads) layer_norm_backward_kernel(const float* gy, const float* gamma,
                                                                       const float* xhat, const float* row_std,
                                                                       float* gx, int64_t rows, int64_t cols) {
    PXK_ROW_LOOP(rows)
    const int64_t off = row * cols;
    const float D = static_cast<float>(cols);
    float s1 = 0.0f, s2 = 0.0f;
    for (int64_t j = lane; j < cols; j += kWave) {
        const float g = gy[off + j] * gamma[j];
        s1 += g;
        s2 += g * xhat[off + j];
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float den = D * row_std[row];
    for (int64_t j = lane; j < cols; j += kWave) {
        const float g = gy[off + j] * gamma[j];
        gx[off + j] = (D * g - s1 - xhat[off + j] * s2) / den;
    }
}

// logsumexp_rows (cpu_backend.cpp:325-338): max + log(sum exp(x - max)).
__global__ void __launch_bounds__(kThreads) logsumexp_kernel(const float* in, float* out, int64_t rows, int64_t cols) {
    PXK_ROW_LOOP(rows)
    const float* x = in + row * cols;
    float m = -INFINITY;
    for (int64_t j = lane; j < cols; j += kWave) m = fmaxf(m, x[j]);
    m = wave_max(m);
    float s = 0.0f;
    for (int64_t j = lane; j < cols; j += kWave) s += expf(x[j] - m);
    s = wave_sum(s);
    if (lane == 0) out[row] = m + logf(s);
}

// scatter_add_rows (cpu_backend.cpp:468-475): table[idx[i]] += src[i] for i ascending. A thread
// owns one column and walks every source row in order, so rows that share an index add up in the
// reference's order without atomics.
__global__ void __launch_bounds__(kThreads) scatter_add_kernel(const float* src, const float* idx, float* table,
                                                               int64_t count, int64_t dim) {
    const int64_t j = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
    if (j >= dim) return;
    for (int64_t i = 0; i < count; ++i) {
        const int64_t r = static_cast<int64_t>(idx[i]);
        table[r * dim + j] += src[i * dim + j];
    }
}

// adam_step (cpu_backend.cpp:340-351).
__global__ void __launch_bounds__(kThreads) adam_kernel(float* p, const float* g, float* m, float* v, int64_t n,
                                                        float lr, float b1, float b2, float eps, float c1, float c2) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const float gi = g[i];
        const float mi = b1 * m[i] + (1.0f - b1) * gi;
        const float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
        m[i] = mi;
        v[i] = vi;
        p[i] -= lr * (mi / c1) / (sqrtf(vi / c2) + eps);
    }
}

// A counter-based uniform in [0, 1): the SplitMix64 finalizer (Steele, Lea and Flood, 2014) of
// seed + (k + 1) * 0x9E3779B97F4A7C15, its top 24 bits as a float mantissa, so element k's draw
// depends on (seed, k) alone whatever the thread schedule.
__device__ __forceinline__ float counter_uniform(uint64_t seed, uint64_t k) {
    uint64_t z = seed + (k + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return static_cast<float>(z >> 40) * (1.0f / 16777216.0f);
}

// dropout_forward (cpu_backend.cpp:362-369): keep unless u < p; out = keep ? x scale : 0.
__global__ void __launch_bounds__(kThreads) dropout_kernel(const float* in, float* out, float* mask, int64_t n, float p,
                                                           float scale, uint64_t seed, uint64_t offset) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const bool keep = !(counter_uniform(seed, offset + static_cast<uint64_t>(i)) < p);
        mask[i] = keep ? 1.0f : 0.0f;
        out[i] = keep ? in[i] * scale : 0.0f;
    }
}

// The logistic function without overflow: the exponent's argument is never positive.
__device__ __forceinline__ float sigm_stable(float x) {
    if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
    const float e = expf(x);
    return e / (1.0f + e);
}

// bce_with_logits (cpu_backend.cpp:371-375): max(x, 0) - x y + log1p(exp(-|x|)), the max as a
// select so -0 and NaN behave as std::max does; with grad: (sigmoid(x) - y) scale.
__global__ void __launch_bounds__(kThreads) bce_kernel(const float* x, const float* y, float* out, int64_t n, int grad,
                                                       float scale) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const float xi = x[i], yi = y[i];
        if (grad)
            out[i] = (sigm_stable(xi) - yi) * scale;
        else
            out[i] = ((xi < 0.0f) ? 0.0f : xi) - xi * yi + log1pf(expf(-fabsf(xi)));
    }
}

// tanh_gaussian_forward (row_math.hpp:131-150): a = tanh(mean + exp(log_std) eps) per element and
// the row's log-probability accumulated in double.
__global__ void __launch_bounds__(kThreads) tanh_gaussian_kernel(const float* mean, const float* log_std, const float* e,
                                                                 float* action, float* std_cache, float* log_prob,
                                                                 int64_t rows, int64_t cols, float stabilizer,
                                                                 double half_log_two_pi) {
    PXK_ROW_LOOP(rows)
    const int64_t off = row * cols;
    double lp = 0.0;
    for (int64_t j = lane; j < cols; j += kWave) {
        const float sd = expf(log_std[off + j]);
        const float a = tanhf(mean[off + j] + sd * e[off + j]);
        std_cache[off + j] = sd;
        action[off + j] = a;
        const double ev = static_cast<double>(e[off + j]);
        const double corr = log(1.0 - static_cast<double>(a) * static_cast<double>(a) + static_cast<double>(stabilizer));
        lp += -0.5 * ev * ev - static_cast<double>(log_std[off + j]) - half_log_two_pi - corr;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lp += __shfl_xor(lp, o, kWave);
    if (lane == 0) log_prob[row] = static_cast<float>(lp);
}

// tanh_gaussian_backward (row_math.hpp:152-160), per element.
__global__ void __launch_bounds__(kThreads) tanh_gaussian_backward_kernel(const float* action, const float* std_cache,
                                                                          const float* e, const float* ga,
                                                                          const float* glp, float* gm, float* gls,
                                                                          int64_t n, float stabilizer) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const float a = action[i];
        const float om = 1.0f - a * a;
        const float dlp = 2.0f * a * om / (om + stabilizer);
        const float gu = ga[i] * om + glp[i] * dlp;
        gm[i] = gu;
        gls[i] = gu * std_cache[i] * e[i] - glp[i];
    }
}

// top_k_rows (top_k_math.hpp:20-48): one thread per row inserts each column into the k-long output
// row; NaN ranks above every number and equal values keep the lower column first.
__device__ __forceinline__ bool topk_above(float a, float b) { return (a != a && b == b) || a > b; }
__device__ __forceinline__ bool topk_beats(float a, float b, bool largest) {
    return largest ? topk_above(a, b) : topk_above(b, a);
}
__global__ void __launch_bounds__(kThreads) top_k_kernel(const float* in, float* values, float* indices, int64_t rows,
                                                         int64_t cols, int64_t k, int largest) {
    const int64_t row = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
    if (row >= rows) return;
    const float* x = in + row * cols;
    float* v = values + row * k;
    float* ix = indices + row * k;
    int64_t filled = 0;
    for (int64_t j = 0; j < cols; ++j) {
        const float xj = x[j];
        if (filled == k && !topk_beats(xj, v[k - 1], largest != 0)) continue;
        int64_t p = filled < k ? filled++ : k - 1;
        while (p > 0 && topk_beats(xj, v[p - 1], largest != 0)) {
            v[p] = v[p - 1];
            ix[p] = ix[p - 1];
            --p;
        }
        v[p] = xj;
        ix[p] = static_cast<float>(j);
    }
}

unsigned rows_grid(int64_t rows) { return static_cast<unsigned>(cdiv(rows, kRowsPerBlock)); }

bool bad_rows(const char* what, int64_t rows, int64_t cols, int* rc) {
    if (rows < 0 || cols < 0) {
        *rc = fail(PXK_ERR_INVALID, "%s: negative size", what);
        return true;
    }
    if (rows > (int64_t{1} << 36)) {
        *rc = fail(PXK_ERR_INVALID, "%s: too many rows", what);
        return true;
    }
    *rc = PXK_OK;
    return rows == 0 || cols == 0;
}

}  // namespace
}  // namespace pxk

using namespace pxk;

extern "C" {

int pxk_elementwise_backward(int op, const float* x, const float* grad_out, float* grad_in, int64_t n, void* stream) {
    if (op < 0 || op > 7) return fail(PXK_ERR_INVALID, "pxk_elementwise_backward: unknown op %d", op);
    if (n < 0) return fail(PXK_ERR_INVALID, "pxk_elementwise_backward: negative size");
    if (n == 0) return PXK_OK;
    PXK_LAUNCH(act_backward_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, S(stream), op, x, grad_out, grad_in,
               n);
    return launched("pxk_elementwise_backward");
}

int pxk_softmax_rows_backward(const float* y, const float* dy, float* dx, int64_t rows, int64_t cols, void* stream) {
    int rc;
    if (bad_rows("pxk_softmax_rows_backward", rows, cols, &rc)) return rc;
    PXK_LAUNCH(softmax_backward_kernel, dim3(rows_grid(rows)), dim3(kThreads), 0, S(stream), y, dy, dx, rows, cols);
    return launched("pxk_softmax_rows_backward");
}

int pxk_rms_norm_backward(const float* grad_out, const float* gamma, const float* in, const float* row_rms,
                          float* grad_in, float* gamma_terms, int64_t rows, int64_t cols, void* stream) {
    int rc;
    if (bad_rows("pxk_rms_norm_backward", rows, cols, &rc)) return rc;
    PXK_LAUNCH(rms_backward_kernel, dim3(rows_grid(rows)), dim3(kThreads), 0, S(stream), grad_out, gamma, in, row_rms,
               grad_in, gamma_terms, rows, cols);
    return launched("pxk_rms_norm_backward");
}

int pxk_layer_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                           float* row_std, int64_t rows, int64_t cols, float eps, void* stream) {
    int rc;
    if (bad_rows("pxk_layer_norm_forward", rows, cols, &rc)) return rc;
    PXK_LAUNCH(layer_norm_kernel, dim3(rows_grid(rows)), dim3(kThreads), 0, S(stream), in, gamma, beta, xhat, out,
               row_std, rows, cols, eps);
    return launched("pxk_layer_norm_forward");
}

int pxk_layer_norm_backward(const float* grad_out, const float* gamma, const float* xhat, const float* row_std,
                            float* grad_in, int64_t rows, int64_t cols, void* stream) {
    int rc;
    if (bad_rows("pxk_layer_norm_backward", rows, cols, &rc)) return rc;
    PXK_LAUNCH(layer_norm_backward_kernel, dim3(rows_grid(rows)), dim3(kThreads), 0, S(stream), grad_out, gamma, xhat,
               row_std, grad_in, rows, cols);
    return launched("pxk_layer_norm_backward");
}

int pxk_logsumexp_rows(const float* in, float* out, int64_t rows, int64_t cols, void* stream) {
    int rc;
    if (cols == 0 && rows > 0) return fail(PXK_ERR_INVALID, "pxk_logsumexp_rows: empty rows");
    if (bad_rows("pxk_logsumexp_rows", rows, cols, &rc)) return rc;
    PXK_LAUNCH(logsumexp_kernel, dim3(rows_grid(rows)), dim3(kThreads), 0, S(stream), in, out, rows, cols);
    return launched("pxk_logsumexp_rows");
}

int pxk_scatter_add_rows(const float* src, const float* indices, float* table, int64_t count, int64_t dim,
                         void* stream) {
    int rc;
    if (bad_rows("pxk_scatter_add_rows", count, dim, &rc)) return rc;
    PXK_LAUNCH(scatter_add_kernel, dim3(static_cast<unsigned>(cdiv(dim, kThreads))), dim3(kThreads), 0, S(stream), src,
               indices, table, count, dim);
    return launched("pxk_scatter_add_rows");
}

int pxk_adam_step(float* param, const float* grad, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                  float eps, float bias_correction1, float bias_correction2, void* stream) {
    if (n < 0) return fail(PXK_ERR_INVALID, "pxk_adam_step: negative size");
    if (n == 0) return PXK_OK;
    PXK_LAUNCH(adam_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, S(stream), param, grad, m, v, n, lr, beta1,
               beta2, eps, bias_correction1, bias_correction2);
    return launched("pxk_adam_step");
}

int pxk_dropout_forward(const float* in, float* out, float* mask, int64_t n, float p, float scale, uint64_t seed,
                        uint64_t offset, void* stream) {
    if (n < 0) return fail(PXK_ERR_INVALID, "pxk_dropout_forward: negative size");
    if (n == 0) return PXK_OK;
    PXK_LAUNCH(dropout_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, S(stream), in, out, mask, n, p, scale, seed,
               offset);
    return launched("pxk_dropout_forward");
}

int pxk_bce_with_logits(const float* logits, const float* target, float* out, int64_t n, int grad, float scale,
                        void* stream) {
    if (n < 0) return fail(PXK_ERR_INVALID, "pxk_bce_with_logits: negative size");
    if (n == 0) return PXK_OK;
    PXK_LAUNCH(bce_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, S(stream), logits, target, out, n, grad,
               scale);
    return launched("pxk_bce_with_logits");
}

int pxk_tanh_gaussian_forward(const float* mean, const float* log_std, const float* eps, float* action,
                              float* std_cache, float* log_prob, int64_t rows, int64_t cols, float stabilizer,
                              double half_log_two_pi, void* stream) {
    int rc;
    if (bad_rows("pxk_tanh_gaussian_forward", rows, cols, &rc)) return rc;
    PXK_LAUNCH(tanh_gaussian_kernel, dim3(rows_grid(rows)), dim3(kThreads), 0, S(stream), mean, log_std, eps, action,
               std_cache, log_prob, rows, cols, stabilizer, half_log_two_pi);
    return launched("pxk_tanh_gaussian_forward");
}

int pxk_tanh_gaussian_backward(const float* action, const float* std_cache, const float* eps, const float* grad_action,
                               const float* grad_log_prob, float* grad_mean, float* grad_log_std, int64_t n,
                               float stabilizer, void* stream) {
    if (n < 0) return fail(PXK_ERR_INVALID, "pxk_tanh_gaussian_backward: negative size");
    if (n == 0) return PXK_OK;
    PXK_LAUNCH(tanh_gaussian_backward_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, S(stream), action,
               std_cache, eps, grad_action, grad_log_prob, grad_mean, grad_log_std, n, stabilizer);
    return launched("pxk_tanh_gaussian_backward");
}

int pxk_top_k_rows(const float* in, float* values, float* indices, int64_t rows, int64_t cols, int64_t k, int largest,
                   void* stream) {
    if (rows < 0 || cols < 0 || k < 1 || k > cols)
        return fail(PXK_ERR_INVALID, "pxk_top_k_rows: needs 1 <= k <= cols");
    if (rows == 0) return PXK_OK;
    PXK_LAUNCH(top_k_kernel, dim3(static_cast<unsigned>(cdiv(rows, kThreads))), dim3(kThreads), 0, S(stream), in, values,
               indices, rows, cols, k, largest);
    return launched("pxk_top_k_rows");
}

}  // extern "C"
