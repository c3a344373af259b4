// pxo.cpp -- CPU oracle for the causal-LM forward + AttnLRP relevance path.
//
// TEST INFRASTRUCTURE ONLY (the checker, never the product): a restatement of Pulsatrix's
// CPUBackend (src/cpu_backend.cpp) and of the modules on the path, keeping the reference's loop
// orders and float expressions so that, built with the same flags, its results are bit-identical
// to the reference CPUBackend. Each function cites the reference lines it follows.
//
// Pinning (see tests/test_oracle.py): every module is checked against oracle/_ref (the reference
// CPUBackend and modules compiled from /root/reference by oracle/Makefile) bit for bit, and
// against the reference's own fixtures: hf_tiny golden logits (transformers) and AttnLRP
// relevance (LXT 2.1), and the LXT MHA / TransformerBlock values of tests/lrp_reference_test.cpp.

#include "pxo.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_error;
int g_threads = 0;
int g_split_threads = 1;  // threads for the ops CPUBackend runs single-threaded (split_outer)

using Buf = std::vector<float>;

// ---- scalar helpers (src/lrp_math.hpp, src/pointwise_math.hpp, src/cpu_backend.cpp:29) ----

float sigmoid(float z) { return 1.0f / (1.0f + std::exp(-z)); }  // cpu_backend.cpp:29

// z + eps * sign(z), sign(0) = +1 (lrp_math.hpp:17)
float stabilize(float z, float eps) { return z + eps * ((z >= 0.0f) ? 1.0f : -1.0f); }

float gelu_tanh(float x) {  // pointwise_math.hpp:32-36
    const float kBeta = 0.7978845608028654f;
    const float kKappa = 0.044715f;
    return 0.5f * x * (1.0f + tanhf(kBeta * (x + kKappa * x * x * x)));
}

float gelu(float x) {  // pointwise_math.hpp:50-53
    const float kInvSqrt2 = 0.7071067811865476f;
    return 0.5f * x * (1.0f + erff(x * kInvSqrt2));
}

// ---- GEMM (cpu_backend.cpp:38-77, 110-118, 181-206) ----

size_t worker_threads() {
    if (g_threads > 0) return static_cast<size_t>(g_threads);
    return std::max<size_t>(1, std::thread::hardware_concurrency());
}

// Column ranges over [0, n): every output element is owned by one thread and summed in one order,
// so the result does not depend on the thread count (cpu_backend.cpp:38-59).
template <typename Body>
void column_ranges(size_t m, size_t k, size_t n, const Body& body) {
    const size_t min_work = size_t{1} << 21, min_cols = 64;
    size_t threads = std::min({worker_threads(), (m * k * n) / min_work, n / min_cols});
    if (threads <= 1) {
        body(size_t{0}, n);
        return;
    }
    const size_t chunk = (n + threads - 1) / threads;
    std::vector<std::thread> pool;
    for (size_t t = 1; t < threads; ++t) {
        const size_t j0 = std::min(n, t * chunk), j1 = std::min(n, j0 + chunk);
        pool.emplace_back([&body, j0, j1] { body(j0, j1); });
    }
    body(size_t{0}, std::min(n, chunk));
    for (auto& t : pool) t.join();
}

// Row i of op(A)*B over columns [j0, j1): acc starts at 0 and adds a_ip * b_pj for p ascending
// (the i-p-j order of cpu_backend.cpp:67-77).
void gemm_row(const float* a, bool ta, const float* b, float* acc, size_t i, size_t m, size_t k, size_t n, size_t j0,
              size_t j1) {
    std::fill(acc, acc + (j1 - j0), 0.0f);
    for (size_t p = 0; p < k; ++p) {
        const float a_ip = ta ? a[p * m + i] : a[i * k + p];
        const float* brow = b + p * n + j0;
        for (size_t j = 0; j < j1 - j0; ++j) acc[j] += a_ip * brow[j];
    }
}

void gemm(const float* a, const float* b, float* out, size_t m, size_t k, size_t n) {
    column_ranges(m, k, n, [&](size_t j0, size_t j1) {
        Buf acc(j1 - j0);
        for (size_t i = 0; i < m; ++i) {
            gemm_row(a, false, b, acc.data(), i, m, k, n, j0, j1);
            std::copy(acc.begin(), acc.end(), out + i * n + j0);
        }
    });
}

void gemm_ex(const float* a, bool ta, const float* b, bool tb, float* out, size_t m, size_t k, size_t n, float beta) {
    auto store = [&](float* dst, float acc) { *dst = (beta == 0.0f) ? acc : beta * *dst + acc; };
    column_ranges(m, k, n, [&](size_t j0, size_t j1) {
        if (tb) {
            for (size_t i = 0; i < m; ++i) {
                for (size_t j = j0; j < j1; ++j) {
                    float acc = 0.0f;
                    for (size_t p = 0; p < k; ++p) {
                        const float a_ip = ta ? a[p * m + i] : a[i * k + p];
                        acc += a_ip * b[j * k + p];
                    }
                    store(&out[i * n + j], acc);
                }
            }
            return;
        }
        Buf acc(j1 - j0);
        for (size_t i = 0; i < m; ++i) {
            gemm_row(a, ta, b, acc.data(), i, m, k, n, j0, j1);
            for (size_t j = j0; j < j1; ++j) store(&out[i * n + j], acc[j - j0]);
        }
    });
}

// ---- elementwise and row primitives (cpu_backend.cpp) ----

void elementwise(int op, const float* in, float* out, size_t n) {  // cpu_backend.cpp:120-163
    for (size_t i = 0; i < n; ++i) {
        const float x = in[i];
        switch (op) {
            case 0: out[i] = std::max(x, 0.0f); break;
            case 1: out[i] = -x; break;
            case 2: out[i] = std::tanh(x); break;
            case 3: out[i] = sigmoid(x); break;
            case 4: out[i] = x * sigmoid(x); break;
            case 5: out[i] = std::exp(x); break;
            case 6: out[i] = gelu_tanh(x); break;
            case 7: out[i] = gelu(x); break;
            default: throw std::invalid_argument("elementwise: unknown op");
        }
    }
}

// ---- backward of the activation, softmax and RMSNorm rows (training; not on the explain path) ----

float gelu_tanh_slope(float x) {  // pointwise_math.hpp:39-45: 0.5 (1 + t) + 0.5 x (1 - t^2) b (1 + 3 k x^2)
    const float kBeta = 0.7978845608028654f;
    const float kKappa = 0.044715f;
    const float x2 = x * x;
    const float t = std::tanh(kBeta * (x + kKappa * x2 * x));
    return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * kBeta * (1.0f + 3.0f * kKappa * x2);
}

float gelu_slope(float x) {  // pointwise_math.hpp:55-60: Phi(x) + x phi(x)
    const float kInvSqrt2 = 0.7071067811865476f;
    const float kInvSqrt2Pi = 0.3989422804014327f;
    return 0.5f * (1.0f + std::erf(x * kInvSqrt2)) + x * kInvSqrt2Pi * std::exp(-0.5f * x * x);
}

void elementwise_backward(int op, const float* x, const float* gy, float* gx, size_t n) {  // cpu_backend.cpp:226-270
    for (size_t i = 0; i < n; ++i) {
        const float v = x[i], g = gy[i];
        float d = 0.0f;
        switch (op) {
            case 0: gx[i] = v > 0.0f ? g : 0.0f; continue;
            case 1: d = -1.0f; break;
            case 2: {
                const float t = std::tanh(v);
                d = 1.0f - t * t;
                break;
            }
            case 3: {
                const float sg = sigmoid(v);
                d = sg * (1.0f - sg);
                break;
            }
            case 4: {
                const float sg = sigmoid(v);
                d = sg + v * sg * (1.0f - sg);
                break;
            }
            case 5: d = std::exp(v); break;
            case 6: d = gelu_tanh_slope(v); break;
            case 7: d = gelu_slope(v); break;
            default: throw std::invalid_argument("elementwise_backward: unknown op");
        }
        gx[i] = g * d;
    }
}

void softmax_rows_backward(const float* y, const float* dy, float* dx, size_t rows, size_t cols) {  // :312-323
    for (size_t r = 0; r < rows; ++r) {
        const size_t base = r * cols;
        float dot = 0.0f;
        for (size_t j = 0; j < cols; ++j) dot += y[base + j] * dy[base + j];
        for (size_t j = 0; j < cols; ++j) dx[base + j] = y[base + j] * (dy[base + j] - dot);
    }
}

void rms_norm_backward(const float* gy, const float* gamma, const float* x, const float* row_rms, float* gx,
                       float* gterms, size_t rows, size_t cols) {  // cpu_backend.cpp:410-417, row_math.hpp:75-86
    const float D = static_cast<float>(cols);
    for (size_t r = 0; r < rows; ++r) {
        const size_t o = r * cols;
        const float rms = row_rms[r];
        float dot = 0.0f;
        for (size_t i = 0; i < cols; ++i) dot += gy[o + i] * gamma[i] * x[o + i];
        for (size_t i = 0; i < cols; ++i) {
            gterms[o + i] = gy[o + i] * x[o + i] / rms;
            gx[o + i] = gy[o + i] * gamma[i] / rms - (x[o + i] / (D * rms * rms * rms)) * dot;
        }
    }
}

void add(const float* a, const float* b, float* out, size_t n) {  // :165-169
    for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

void mul(const float* a, const float* b, float* out, size_t n) {  // :171-175
    for (size_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}

void axpby(float alpha, const float* x, float beta, const float* y, float* out, size_t n) {  // :272-282
    if (beta == 0.0f) {
        for (size_t i = 0; i < n; ++i) out[i] = alpha * x[i];
        return;
    }
    for (size_t i = 0; i < n; ++i) out[i] = alpha * x[i] + beta * y[i];
}

void add_row_vector(const float* in, const float* row, float* out, size_t rows, size_t cols) {  // :218-224
    for (size_t i = 0; i < rows; ++i)
        for (size_t j = 0; j < cols; ++j) out[i * cols + j] = in[i * cols + j] + row[j];
}

void softmax_rows(const float* in, float* out, size_t rows, size_t cols) {  // :292-310
    for (size_t r = 0; r < rows; ++r) {
        const float* x = in + r * cols;
        float* y = out + r * cols;
        float mx = x[0];
        for (size_t j = 1; j < cols; ++j) mx = std::max(mx, x[j]);
        float s = 0.0f;
        for (size_t j = 0; j < cols; ++j) {
            const float e = std::exp(x[j] - mx);
            y[j] = e;
            s += e;
        }
        for (size_t j = 0; j < cols; ++j) y[j] /= s;
    }
}

void rms_norm_forward(const float* in, const float* gamma, float* out, float* row_rms, size_t rows, size_t cols,
                      float eps) {  // cpu_backend.cpp:393-399, row_math.hpp:59-71
    for (size_t r = 0; r < rows; ++r) {
        const float* x = in + r * cols;
        float* o = out + r * cols;
        float ss = 0.0f;
        for (size_t i = 0; i < cols; ++i) ss += x[i] * x[i];
        const float ms = ss / static_cast<float>(cols);
        const float rms = sqrtf(ms + eps);
        row_rms[r] = rms;
        for (size_t i = 0; i < cols; ++i) o[i] = gamma[i] * x[i] / rms;
    }
}

void rope_rotate(const float* in, const float* cs, const float* sn, float* out, size_t slices, size_t seq,
                 size_t hd, bool inverse, bool half_layout) {  // cpu_backend.cpp:419-427, row_math.hpp:93-110
    const size_t half = hd / 2;
    for (size_t row = 0; row < slices * seq; ++row) {
        const size_t pos = row % seq;
        const float* x = in + row * hd;
        float* o = out + row * hd;
        for (size_t i = 0; i < half; ++i) {
            const float c = cs[pos * half + i], s = sn[pos * half + i];
            const size_t lo = half_layout ? i : 2 * i, hi = half_layout ? i + half : 2 * i + 1;
            const float x0 = x[lo], x1 = x[hi];
            if (inverse) {
                o[lo] = x0 * c + x1 * s;
                o[hi] = -x0 * s + x1 * c;
            } else {
                o[lo] = x0 * c - x1 * s;
                o[hi] = x0 * s + x1 * c;
            }
        }
    }
}

void permute_0213(const float* in, float* out, size_t d0, size_t d1, size_t d2, size_t d3) {  // :445-457
    for (size_t a = 0; a < d0; ++a)
        for (size_t b = 0; b < d1; ++b)
            for (size_t c = 0; c < d2; ++c) {
                const float* src = in + ((a * d1 + b) * d2 + c) * d3;
                float* dst = out + ((a * d2 + c) * d1 + b) * d3;
                for (size_t e = 0; e < d3; ++e) dst[e] = src[e];
            }
}

bool attention_masked(const float* keep, size_t b, size_t i, size_t j, size_t k_len, bool causal, size_t q_offset,
                      size_t window) {  // row_math.hpp:117-126
    if (causal && j > i + q_offset) return true;
    if (causal && window > 0 && j + window <= i + q_offset) return true;
    return keep != nullptr && keep[b * k_len + j] == 0.0f;
}

void attention_mask_fill(float* scores, const float* keep, size_t batch, size_t heads, size_t q_len, size_t k_len,
                         bool causal, size_t q_offset, size_t window, float value) {  // cpu_backend.cpp:429-443
    for (size_t b = 0; b < batch; ++b)
        for (size_t h = 0; h < heads; ++h)
            for (size_t i = 0; i < q_len; ++i) {
                float* row = scores + ((b * heads + h) * q_len + i) * k_len;
                for (size_t j = 0; j < k_len; ++j)
                    if (attention_masked(keep, b, i, j, k_len, causal, q_offset, window)) row[j] = value;
            }
}

void gather_rows(const float* table, const float* idx, float* out, size_t count, size_t dim) {  // :459-466
    for (size_t i = 0; i < count; ++i) {
        const float* row = table + static_cast<size_t>(idx[i]) * dim;
        for (size_t d = 0; d < dim; ++d) out[i * dim + d] = row[d];
    }
}

// ---- LRP primitives (cpu_backend.cpp:499-566, 681-687; lrp_math.hpp) ----

// Independent outer iterations [0, count) over g_split_threads threads (1 = in order on the calling
// thread, as CPUBackend runs these ops). Each output element is still produced by one thread in
// one order, so the results do not depend on the thread count.
template <typename Body>
void split_outer(size_t count, const Body& body) {
    const size_t threads = std::min<size_t>(g_split_threads > 1 ? static_cast<size_t>(g_split_threads) : 1, count);
    if (threads <= 1) {
        for (size_t i = 0; i < count; ++i) body(i);
        return;
    }
    std::vector<std::thread> pool;
    for (size_t t = 0; t < threads; ++t)
        pool.emplace_back([&body, t, threads, count] {
            for (size_t i = t; i < count; i += threads) body(i);
        });
    for (auto& th : pool) th.join();
}

void lrp_linear(const float* x, const float* w, const float* z, const float* r, float* r_in, size_t rows, size_t in,
                size_t out, float eps) {  // cpu_backend.cpp:499-508, lrp_math.hpp:21-30
    split_outer(rows, [&](size_t n) {
        for (size_t i = 0; i < in; ++i) {
            float acc = 0.0f;
            const float x_i = x[n * in + i];
            for (size_t j = 0; j < out; ++j) {
                const float denom = stabilize(z[n * out + j], eps);
                acc += (x_i * w[i * out + j] / denom) * r[n * out + j];
            }
            r_in[n * in + i] = acc;
        }
    });
}

void lrp_residual_split(const float* a, const float* b, const float* r, float* ra, float* rb, size_t n,
                        float eps) {  // lrp_math.hpp:33-38
    for (size_t i = 0; i < n; ++i) {
        const float y = a[i] + b[i];
        const float denom = stabilize(y, eps);
        ra[i] = (a[i] / denom) * r[i];
        rb[i] = (b[i] / denom) * r[i];
    }
}

void lrp_bilinear_elementwise(const float* a, const float* b, const float* r, float* out, size_t n,
                              float eps) {  // lrp_math.hpp:41-45
    for (size_t i = 0; i < n; ++i) {
        const float c = a[i] * b[i];
        const float denom = 2.0f * c + eps * ((c >= 0.0f) ? 1.0f : -1.0f);
        out[i] = (a[i] * b[i] / denom) * r[i];
    }
}

float bilinear_scaled_r(const float* o, const float* r_o, size_t idx, float eps) {  // lrp_math.hpp:57-61
    const float o_ik = o[idx];
    const float denom = 2.0f * o_ik + eps * ((o_ik >= 0.0f) ? 1.0f : -1.0f);
    return r_o[idx] / denom;
}

void lrp_bilinear_matmul(const float* a, const float* b, const float* o, const float* r_o, float* r_a, float* r_b,
                         size_t slices, size_t m, size_t p, size_t q, float eps,
                         bool bt) {  // cpu_backend.cpp:524-546, lrp_math.hpp:63-86
    split_outer(slices, [&](size_t s) {
        const float* as = a + s * m * p;
        const float* bs = b + s * p * q;
        const float* os = o + s * m * q;
        const float* rs = r_o + s * m * q;
        auto b_at = [&](size_t j, size_t k) { return bt ? bs[k * p + j] : bs[j * q + k]; };
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < p; ++j) {
                float acc = 0.0f;
                for (size_t k = 0; k < q; ++k) acc += as[i * p + j] * b_at(j, k) * bilinear_scaled_r(os, rs, i * q + k, eps);
                r_a[s * m * p + i * p + j] = acc;
            }
        for (size_t j = 0; j < p; ++j)
            for (size_t k = 0; k < q; ++k) {
                float acc = 0.0f;
                for (size_t i = 0; i < m; ++i) acc += as[i * p + j] * b_at(j, k) * bilinear_scaled_r(os, rs, i * q + k, eps);
                r_b[s * p * q + (bt ? k * p + j : j * q + k)] = acc;
            }
    });
}

void lrp_softmax_rows(const float* x, const float* y, const float* r, float* r_in, size_t rows,
                      size_t cols) {  // lrp_math.hpp:89-98
    for (size_t row = 0; row < rows; ++row) {
        const size_t off = row * cols;
        float rs = 0.0f;
        for (size_t j = 0; j < cols; ++j) rs += r[off + j];
        for (size_t i = 0; i < cols; ++i) r_in[off + i] = x[off + i] * (r[off + i] - y[off + i] * rs);
    }
}

void lrp_rope(const float* x, const float* y, const float* r, const float* cs, const float* sn, float* r_in,
              size_t slices, size_t seq, size_t hd, float eps, bool half_layout) {  // lrp_math.hpp:104-123
    const size_t half = hd / 2;
    for (size_t row = 0; row < slices * seq; ++row) {
        const size_t pos = row % seq, off = row * hd;
        for (size_t i = 0; i < half; ++i) {
            const float c = cs[pos * half + i], s = sn[pos * half + i];
            const size_t lo = off + (half_layout ? i : 2 * i), hi = off + (half_layout ? i + half : 2 * i + 1);
            const float d0 = stabilize(y[lo], eps), d1 = stabilize(y[hi], eps);
            float rlo = 0.0f, rhi = 0.0f;
            rlo += (x[lo] * c / d0) * r[lo];
            rhi += (x[hi] * -s / d0) * r[lo];
            rlo += (x[lo] * s / d1) * r[hi];
            rhi += (x[hi] * c / d1) * r[hi];
            r_in[lo] = rlo;
            r_in[hi] = rhi;
        }
    }
}

void lrp_stabilized_divide(const float* r, const float* denom, const float* gate, float* out, size_t n, float eps,
                           int mode) {  // cpu_backend.cpp:681-687, lrp_math.hpp:312-315
    for (size_t i = 0; i < n; ++i) {
        const float g = mode == 0 ? 0.0f : gate[i];
        const bool passes = mode == 0 || (mode == 1 && g > 0.0f) || (mode == 2 && g < 0.0f);
        out[i] = passes ? r[i] / stabilize(denom[i], eps) : 0.0f;
    }
}

void copy_2d(float* dst, size_t ds, const float* src, size_t ss, size_t rows, size_t cols) {  // :852-857
    for (size_t r = 0; r < rows; ++r) std::memcpy(dst + r * ds, src + r * ss, cols * sizeof(float));
}

void accumulate_rows(const float* in, float* out, size_t rows, size_t cols) {  // :859-865
    for (size_t r = 0; r < rows; ++r)
        for (size_t j = 0; j < cols; ++j) out[j] += in[r * cols + j];
}

// RoPEModule tables (rope_module.cpp:67-69 inverse frequencies, :83-101 tables in double).
void rope_tables(int64_t hd, float base, int64_t seq, int64_t offset, float* cs, float* sn) {
    const int64_t half = hd / 2;
    std::vector<double> inv(static_cast<size_t>(half));
    for (int64_t i = 0; i < half; ++i)
        inv[static_cast<size_t>(i)] = std::pow(static_cast<double>(base), -2.0 * static_cast<double>(i) / static_cast<double>(hd));
    for (int64_t pos = 0; pos < seq; ++pos)
        for (int64_t i = 0; i < half; ++i) {
            const double theta = static_cast<double>(offset + pos) * inv[static_cast<size_t>(i)];
            cs[pos * half + i] = static_cast<float>(std::cos(theta));
            sn[pos * half + i] = static_cast<float>(std::sin(theta));
        }
}

// RoPEModule built from an inverse-frequency list (rope_module.cpp:36-51): the same tables.
void rope_tables_inv(const std::vector<double>& inv, int64_t hd, int64_t seq, int64_t offset, float* cs, float* sn) {
    const int64_t half = hd / 2;
    for (int64_t pos = 0; pos < seq; ++pos)
        for (int64_t i = 0; i < half; ++i) {
            const double theta = static_cast<double>(offset + pos) * inv[static_cast<size_t>(i)];
            cs[pos * half + i] = static_cast<float>(std::cos(theta));
            sn[pos * half + i] = static_cast<float>(std::sin(theta));
        }
}

// RopeInverseFrequencies (hf_model.cpp:258-287): 1 / theta^(2i/D), then linear or llama3 scaling.
std::vector<double> rope_inverse_frequencies(const px_model_config& c, int64_t hd) {
    const int64_t half = hd / 2;
    std::vector<double> inv(static_cast<size_t>(half));
    for (int64_t i = 0; i < half; ++i)
        inv[static_cast<size_t>(i)] =
            1.0 / std::pow(static_cast<double>(c.rope_theta), 2.0 * static_cast<double>(i) / static_cast<double>(hd));
    if (c.rope_scaling == 1) {
        for (double& f : inv) f /= c.rope_factor;
        return inv;
    }
    const double old_len = static_cast<double>(c.rope_original_max_position);
    const double low_wavelen = old_len / c.rope_low_freq_factor;
    const double high_wavelen = old_len / c.rope_high_freq_factor;
    constexpr double kPi = 3.14159265358979323846;
    for (double& f : inv) {
        const double wavelen = 2.0 * kPi / f;
        if (wavelen > low_wavelen) {
            f /= c.rope_factor;
        } else if (wavelen >= high_wavelen) {
            const double smooth =
                (old_len / wavelen - c.rope_low_freq_factor) / (c.rope_high_freq_factor - c.rope_low_freq_factor);
            f = (1.0 - smooth) * f / c.rope_factor + smooth * f;
        }
    }
    return inv;
}

// ---- modules -------------------------------------------------------------------------------

// LRPRuleConfig (include/pulsatrix/lrp_rule_config.hpp:72-115); rule in LRPRule order.
enum Rule { kEpsilon = 0, kGamma = 1, kAlphaBeta = 2, kZBox = 3 };

struct RuleConfig {
    float eps;
    bool bias_in_denominator;
    int rule = kEpsilon;
    float gamma = 0.25f, alpha = 1.0f, beta = 0.0f, low = 0.0f, high = 1.0f;
};

// ---- Zennit-compatible affine rules (src/lrp_rules.cpp:13-160) ----------------------------------
// An affine layer seen abstractly (lrp_rules.hpp:35-52): forward(x, w) -> output-shaped,
// backward(g, w) -> input-shaped, add_bias(y, b) -> y + b. Each rule is composed from the
// primitives above in the order lrp_rules.cpp issues them, each step into a fresh zero-filled
// buffer as the reference's Tensor scratch is.
struct Affine {
    size_t n_in = 0, n_out = 0, n_w = 0, n_b = 0;
    std::function<void(const float*, const float*, float*)> forward, backward, add_bias;
};

Buf rule_pos(const float* v, size_t n) {  // lrp_rules.cpp:18-22, max(v, 0)
    Buf out(n, 0.0f);
    elementwise(0, v, out.data(), n);
    return out;
}

Buf rule_neg(const float* v, size_t n) {  // :24-29, v - max(v, 0)
    Buf out = rule_pos(v, n);
    axpby(1.0f, v, -1.0f, out.data(), out.data(), n);
    return out;
}

Buf rule_plus_scaled(const float* a, float scale, const Buf& b) {  // :31-36, a + scale b
    Buf out(b.size(), 0.0f);
    axpby(1.0f, a, scale, b.data(), out.data(), b.size());
    return out;
}

Buf rule_affine(const Affine& op, const float* x, const float* w, const float* bias) {  // :38-46
    Buf out(op.n_out, 0.0f);
    op.forward(x, w, out.data());
    if (bias) op.add_bias(out.data(), bias, out.data());
    return out;
}

Buf rule_divide(const Affine& op, const float* r, const float* den, const float* gate, int mode, float eps) {  // :48-53
    Buf out(op.n_out, 0.0f);
    lrp_stabilized_divide(r, den, gate, out.data(), op.n_out, eps, mode);
    return out;
}

// acc = (first ? 0 : acc) + scale * (x_mod * backward(g, w))  (:55-62)
void rule_term(const Affine& op, const float* x_mod, const float* g, const float* w, float scale, float* acc,
               bool first) {
    Buf t(op.n_in, 0.0f);
    op.backward(g, w, t.data());
    mul(x_mod, t.data(), t.data(), op.n_in);
    axpby(scale, t.data(), first ? 0.0f : 1.0f, acc, acc, op.n_in);
}

void rule_epsilon(const Affine& op, const float* x, const float* w, const float* b, const float* pre, const float* r,
                  float* r_in, float eps) {  // :64-70
    Buf z(op.n_out, 0.0f);
    op.add_bias(pre, b, z.data());
    const Buf g = rule_divide(op, r, z.data(), nullptr, 0, eps);
    rule_term(op, x, g.data(), w, 1.0f, r_in, true);
}

void rule_alpha_beta(const Affine& op, const float* x, const float* w, const float* b, const float* r, float* r_in,
                     const RuleConfig& c) {  // :72-111
    const Buf xp = rule_pos(x, op.n_in), xn = rule_neg(x, op.n_in);
    const Buf wp = rule_pos(w, op.n_w), wn = rule_neg(w, op.n_w);
    const Buf bp = rule_pos(b, op.n_b), bn = rule_neg(b, op.n_b);
    Buf zp = rule_affine(op, xp.data(), wp.data(), bp.data());
    const Buf zp_rest = rule_affine(op, xn.data(), wn.data(), nullptr);
    add(zp.data(), zp_rest.data(), zp.data(), op.n_out);
    const Buf gp = rule_divide(op, r, zp.data(), nullptr, 0, c.eps);
    Buf positive(op.n_in, 0.0f);
    rule_term(op, xp.data(), gp.data(), wp.data(), 1.0f, positive.data(), true);
    rule_term(op, xn.data(), gp.data(), wn.data(), 1.0f, positive.data(), false);
    if (c.beta == 0.0f) {
        axpby(c.alpha, positive.data(), 0.0f, positive.data(), r_in, op.n_in);
        return;
    }
    Buf zn = rule_affine(op, xp.data(), wn.data(), bn.data());
    const Buf zn_rest = rule_affine(op, xn.data(), wp.data(), nullptr);
    add(zn.data(), zn_rest.data(), zn.data(), op.n_out);
    const Buf gn = rule_divide(op, r, zn.data(), nullptr, 0, c.eps);
    Buf negative(op.n_in, 0.0f);
    rule_term(op, xp.data(), gn.data(), wn.data(), 1.0f, negative.data(), true);
    rule_term(op, xn.data(), gn.data(), wp.data(), 1.0f, negative.data(), false);
    axpby(c.alpha, positive.data(), -c.beta, negative.data(), r_in, op.n_in);
}

void rule_gamma(const Affine& op, const float* x, const float* w, const float* b, const float* pre, const float* r,
                float* r_in, const RuleConfig& c) {  // :113-140
    const float g = c.gamma;
    const Buf xp = rule_pos(x, op.n_in), xn = rule_neg(x, op.n_in);
    const Buf wa = rule_plus_scaled(w, g, rule_pos(w, op.n_w)), wb = rule_plus_scaled(w, g, rule_neg(w, op.n_w));
    const Buf ba = rule_plus_scaled(b, g, rule_pos(b, op.n_b)), bb = rule_plus_scaled(b, g, rule_neg(b, op.n_b));
    Buf z(op.n_out, 0.0f);  // the original output selects the pair that explains each unit
    op.add_bias(pre, b, z.data());
    Buf den_pos = rule_affine(op, xp.data(), wa.data(), ba.data());
    const Buf o1 = rule_affine(op, xn.data(), wb.data(), nullptr);
    add(den_pos.data(), o1.data(), den_pos.data(), op.n_out);
    Buf den_neg = rule_affine(op, xp.data(), wb.data(), bb.data());
    const Buf o3 = rule_affine(op, xn.data(), wa.data(), nullptr);
    add(den_neg.data(), o3.data(), den_neg.data(), op.n_out);
    const Buf gp = rule_divide(op, r, den_pos.data(), z.data(), 1, c.eps);
    const Buf gn = rule_divide(op, r, den_neg.data(), z.data(), 2, c.eps);
    rule_term(op, xp.data(), gp.data(), wa.data(), 1.0f, r_in, true);
    rule_term(op, xn.data(), gp.data(), wb.data(), 1.0f, r_in, false);
    rule_term(op, xp.data(), gn.data(), wb.data(), 1.0f, r_in, false);
    rule_term(op, xn.data(), gn.data(), wa.data(), 1.0f, r_in, false);
}

void rule_zbox(const Affine& op, const float* x, const float* w, const float* pre, const float* r, float* r_in,
               const RuleConfig& c) {  // :142-160, constant bounds (no fill_bound for dense layers)
    const Buf wp = rule_pos(w, op.n_w), wn = rule_neg(w, op.n_w);
    const Buf lo(op.n_in, c.low), hi(op.n_in, c.high);
    Buf den(op.n_out, 0.0f);
    const Buf lo_out = rule_affine(op, lo.data(), wp.data(), nullptr);
    const Buf hi_out = rule_affine(op, hi.data(), wn.data(), nullptr);
    axpby(1.0f, pre, -1.0f, lo_out.data(), den.data(), op.n_out);
    axpby(1.0f, den.data(), -1.0f, hi_out.data(), den.data(), op.n_out);
    const Buf g = rule_divide(op, r, den.data(), nullptr, 0, c.eps);
    rule_term(op, x, g.data(), w, 1.0f, r_in, true);
    rule_term(op, lo.data(), g.data(), wp.data(), -1.0f, r_in, false);
    rule_term(op, hi.data(), g.data(), wn.data(), -1.0f, r_in, false);
}

// lrp_rules::validate (:164-176)
void rule_validate(const RuleConfig& c, const char* module) {
    if (c.rule < kEpsilon || c.rule > kZBox) throw std::invalid_argument("lrp_rules::apply: unknown LRPRule");
    if (c.rule != kAlphaBeta) return;
    if (!(c.alpha >= 0.0f) || !(c.beta >= 0.0f))
        throw std::invalid_argument(std::string(module) +
                                    "::propagate_relevance: AlphaBeta rule needs alpha >= 0 and beta >= 0");
    if (c.alpha - c.beta != 1.0f)
        throw std::invalid_argument(std::string(module) + "::propagate_relevance: AlphaBeta rule needs alpha - beta == 1");
}

// lrp_rules::apply (:178-195)
void rule_apply(const Affine& op, const float* x, const float* w, const float* b, const float* pre, const float* r,
                float* r_in, const RuleConfig& c) {
    switch (c.rule) {
        case kEpsilon: rule_epsilon(op, x, w, b, pre, r, r_in, c.eps); return;
        case kAlphaBeta: rule_alpha_beta(op, x, w, b, r, r_in, c); return;
        case kGamma: rule_gamma(op, x, w, b, pre, r, r_in, c); return;
        case kZBox: rule_zbox(op, x, w, pre, r, r_in, c); return;
        default: throw std::invalid_argument("lrp_rules::apply: unknown LRPRule");
    }
}

// LinearModule (linear_module.cpp:189-228 forward; 333-341 relevance -> lrp_rules::linear,
// lrp_rules.cpp:197-220). The bias tensor always exists; it is zero when the layer has none
// (the constructor zero-fills it, linear_module.cpp:24).
struct Linear {
    int64_t in = 0, out = 0;
    bool has_bias = false;
    Buf w, b;  // w (in, out); b (out)
    Buf x, z;  // cached input and pre-bias output
    int64_t n = 0;

    void init(int64_t in_, int64_t out_, bool bias, const float*& p) {
        in = in_;
        out = out_;
        has_bias = bias;
        w.assign(p, p + in * out);
        p += in * out;
        b.assign(static_cast<size_t>(out), 0.0f);
        if (bias) {
            b.assign(p, p + out);
            p += out;
        }
    }

    Buf forward(const Buf& input, int64_t rows) {
        n = rows;
        x = input;
        z.assign(static_cast<size_t>(rows * out), 0.0f);
        gemm(x.data(), w.data(), z.data(), rows, in, out);
        if (!has_bias) return z;
        Buf y(z.size());
        add_row_vector(z.data(), b.data(), y.data(), rows, out);
        return y;
    }

    Buf relevance(const Buf& r, const RuleConfig& cfg) const {
        rule_validate(cfg, "LinearModule");
        Buf r_in(static_cast<size_t>(n * in), 0.0f);
        const size_t N = n, I = in, O = out;
        if (cfg.rule == kEpsilon && !cfg.bias_in_denominator) {  // legacy pre-bias epsilon rule: lrp_linear
            lrp_linear(x.data(), w.data(), z.data(), r.data(), r_in.data(), N, I, O, cfg.eps);
            return r_in;
        }
        // lrp_rules::linear (lrp_rules.cpp:197-215): x (N, in) through w (in, out).
        Affine op;
        op.n_in = N * I;
        op.n_out = N * O;
        op.n_w = I * O;
        op.n_b = O;
        op.forward = [=](const float* xs, const float* ws, float* y) { gemm(xs, ws, y, N, I, O); };
        op.backward = [=](const float* g, const float* ws, float* gx) { gemm_ex(g, false, ws, true, gx, N, O, I, 0.0f); };
        op.add_bias = [=](const float* y, const float* bb, float* o) { add_row_vector(y, bb, o, N, O); };
        rule_apply(op, x.data(), w.data(), b.data(), z.data(), r.data(), r_in.data(), cfg);
        return r_in;
    }
};

// RMSNormModule (rms_norm_module.cpp:51-68 forward; 101-111 relevance = identity).
struct RMSNorm {
    int64_t d = 0;
    float eps = 1e-6f;
    float offset = 0.0f;  // EffectiveGamma (rms_norm_module.cpp:40-49): fill(offset), then add gamma
    Buf gamma;
    void init(int64_t d_, float eps_, float offset_, const float*& p) {
        d = d_;
        eps = eps_;
        offset = offset_;
        gamma.assign(p, p + d);
        p += d;
    }
    Buf forward(const Buf& x, int64_t rows) const {
        Buf out(x.size()), rms(static_cast<size_t>(rows));
        Buf g = gamma;
        if (offset != 0.0f)
            for (size_t i = 0; i < g.size(); ++i) g[i] = offset + gamma[i];
        rms_norm_forward(x.data(), g.data(), out.data(), rms.data(), rows, d, eps);
        return out;
    }
};

struct ModelShape {
    int64_t d, H, Hkv, D, F;
    float norm_eps, theta;
    bool rope, half_layout, causal, qkv_bias, out_bias, mlp_bias;
    // Variants (ToAttentionConfig(config, layer), hf_model.cpp:289-313; TransformerBlockOptions)
    int act = 0;                 // 0 SiLU, 1 GeLU tanh
    bool qk_norm = false, post_norms = false;
    float norm_offset = 0.0f;
    float score_scale = 0.0f;    // 0: 1/sqrt(D)
    size_t window = 0;           // this layer's sliding window (0: none)
    std::vector<double> inv_freq;  // non-empty: the RoPE inverse frequencies (else theta's schedule)
};

// MultiHeadAttentionModule (multihead_attention_module.cpp:204-310 forward, 404-485 relevance).
struct MHA {
    ModelShape s;
    Linear q, k, v, o;
    RMSNorm q_norm, k_norm;
    int64_t N = 0, L = 0;
    Buf q_in, q_out, k_in, k_out;  // RoPE caches (RoPEModule last_input_/last_output_)
    Buf cos_t, sin_t;
    Buf Q, K, V, raw, scaled, attn, ctx;  // K, V after repeat_kv
    Buf key_rel, value_rel;

    void init(const ModelShape& sh, const float*& p) {
        s = sh;
        q.init(s.d, s.H * s.D, s.qkv_bias, p);
        k.init(s.d, s.Hkv * s.D, s.qkv_bias, p);
        v.init(s.d, s.Hkv * s.D, s.qkv_bias, p);
        o.init(s.H * s.D, s.d, s.out_bias, p);
        if (s.qk_norm) {  // qk_norm_eps = rms_norm_eps, offset = norm_weight_offset (hf_model.cpp:299-311)
            q_norm.init(s.D, s.norm_eps, s.norm_offset, p);
            k_norm.init(s.D, s.norm_eps, s.norm_offset, p);
        }
    }

    // repeat_kv (:154-171): head h reads KV head h / group.
    Buf repeat_kv(const Buf& t) const {
        const int64_t group = s.H / s.Hkv;
        if (group == 1) return t;
        const size_t slice = static_cast<size_t>(L * s.D);
        Buf out(static_cast<size_t>(N * s.H) * slice, 0.0f);
        for (int64_t g = 0; g < group; ++g)
            copy_2d(out.data() + g * slice, slice * group, t.data(), slice, static_cast<size_t>(N * s.Hkv), slice);
        return out;
    }

    // sum_kv_groups (:173-188): accumulate_rows over each group, in order.
    Buf sum_kv_groups(const Buf& t) const {
        const int64_t group = s.H / s.Hkv;
        if (group == 1) return t;
        const size_t slice = static_cast<size_t>(L * s.D);
        Buf out(static_cast<size_t>(N * s.Hkv) * slice, 0.0f);
        for (int64_t r = 0; r < N * s.Hkv; ++r)
            accumulate_rows(t.data() + r * group * slice, out.data() + r * slice, group, slice);
        return out;
    }

    void fill_masked(Buf& scores, float value) const {  // :194-202
        if (!s.causal) return;
        attention_mask_fill(scores.data(), nullptr, N, s.H, L, L, true, 0, s.window, value);
    }

    Buf forward(const Buf& input, int64_t n_, int64_t l_) {
        N = n_;
        L = l_;
        const int64_t H = s.H, Hkv = s.Hkv, D = s.D;
        Buf qf = q.forward(input, N * L), kf = k.forward(input, N * L), vf = v.forward(input, N * L);
        Buf qh(qf.size()), kh(kf.size()), vh(vf.size());
        permute_0213(qf.data(), qh.data(), N, L, H, D);
        permute_0213(kf.data(), kh.data(), N, L, Hkv, D);
        permute_0213(vf.data(), vh.data(), N, L, Hkv, D);
        if (s.qk_norm) {  // step 3, QK-Norm over each (head, position) row of D
            qh = q_norm.forward(qh, N * H * L);
            kh = k_norm.forward(kh, N * Hkv * L);
        }
        if (s.rope) {
            cos_t.assign(static_cast<size_t>(L * D / 2), 0.0f);
            sin_t.assign(cos_t.size(), 0.0f);
            if (s.inv_freq.empty())
                rope_tables(D, s.theta, L, 0, cos_t.data(), sin_t.data());
            else
                rope_tables_inv(s.inv_freq, D, L, 0, cos_t.data(), sin_t.data());
            q_in = qh;
            k_in = kh;
            q_out.assign(qh.size(), 0.0f);
            k_out.assign(kh.size(), 0.0f);
            rope_rotate(q_in.data(), cos_t.data(), sin_t.data(), q_out.data(), N * H, L, D, false, s.half_layout);
            rope_rotate(k_in.data(), cos_t.data(), sin_t.data(), k_out.data(), N * Hkv, L, D, false, s.half_layout);
            qh = q_out;
            kh = k_out;
        }
        Q = qh;
        K = repeat_kv(kh);
        V = repeat_kv(vh);
        const size_t LL = static_cast<size_t>(L * L), LD = static_cast<size_t>(L * D);
        raw.assign(static_cast<size_t>(N * H) * LL, 0.0f);
        scaled.assign(raw.size(), 0.0f);
        // score_scale(), :190-192
        const float scale = s.score_scale > 0.0f ? s.score_scale : 1.0f / std::sqrt(static_cast<float>(D));
        for (int64_t nh = 0; nh < N * H; ++nh)
            gemm_ex(Q.data() + nh * LD, false, K.data() + nh * LD, true, raw.data() + nh * LL, L, D, L, 0.0f);
        axpby(scale, raw.data(), 0.0f, nullptr, scaled.data(), raw.size());
        fill_masked(scaled, std::numeric_limits<float>::lowest());
        attn.assign(raw.size(), 0.0f);
        softmax_rows(scaled.data(), attn.data(), N * H * L, L);  // SoftmaxModule (softmax_module.cpp:39-51)
        ctx.assign(static_cast<size_t>(N * H) * LD, 0.0f);
        for (int64_t nh = 0; nh < N * H; ++nh)
            gemm(attn.data() + nh * LL, V.data() + nh * LD, ctx.data() + nh * LD, L, L, D);
        Buf merged(ctx.size());
        permute_0213(ctx.data(), merged.data(), N, H, L, D);
        return o.forward(merged, N * L);
    }

    Buf relevance(const Buf& r_out, const RuleConfig& cfg) {
        const int64_t H = s.H, Hkv = s.Hkv, D = s.D;
        Buf r_merged = o.relevance(r_out, cfg);
        Buf r_ctx(r_merged.size());
        permute_0213(r_merged.data(), r_ctx.data(), N, L, H, D);
        Buf r_attn(attn.size()), r_v(V.size());
        lrp_bilinear_matmul(attn.data(), V.data(), ctx.data(), r_ctx.data(), r_attn.data(), r_v.data(), N * H, L, L, D,
                            cfg.eps, false);
        Buf r_scores(attn.size());
        lrp_softmax_rows(scaled.data(), attn.data(), r_attn.data(), r_scores.data(), N * H * L, L);
        fill_masked(r_scores, 0.0f);
        Buf r_q(Q.size()), r_k(K.size());
        lrp_bilinear_matmul(Q.data(), K.data(), raw.data(), r_scores.data(), r_q.data(), r_k.data(), N * H, L, D, L,
                            cfg.eps, true);
        r_k = sum_kv_groups(r_k);
        r_v = sum_kv_groups(r_v);
        if (s.rope) {  // RoPEModule::propagate_relevance (rope_module.cpp:142-160)
            Buf rq(r_q.size()), rk(r_k.size());
            lrp_rope(q_in.data(), q_out.data(), r_q.data(), cos_t.data(), sin_t.data(), rq.data(), N * H, L, D, cfg.eps,
                     s.half_layout);
            lrp_rope(k_in.data(), k_out.data(), r_k.data(), cos_t.data(), sin_t.data(), rk.data(), N * Hkv, L, D,
                     cfg.eps, s.half_layout);
            r_q = rq;
            r_k = rk;
        }
        Buf rqf(r_q.size()), rkf(r_k.size()), rvf(r_v.size());
        permute_0213(r_q.data(), rqf.data(), N, H, L, D);
        permute_0213(r_k.data(), rkf.data(), N, Hkv, L, D);
        permute_0213(r_v.data(), rvf.data(), N, Hkv, L, D);
        Buf r_in = q.relevance(rqf, cfg);
        Buf rk_in = k.relevance(rkf, cfg), rv_in = v.relevance(rvf, cfg);
        add(r_in.data(), rk_in.data(), r_in.data(), r_in.size());  // Tensor::accumulate
        add(r_in.data(), rv_in.data(), r_in.data(), r_in.size());
        key_rel = rkf;
        value_rel = rvf;
        return r_in;
    }
};

// SwiGLUModule (swiglu_module.cpp:70-102 forward, 139-170 relevance), Silu gate.
struct SwiGLU {
    Linear gate, up, down;
    Buf gate_post, up_out;
    int64_t rows = 0;
    int act = 0;

    void init(const ModelShape& s, const float*& p) {
        act = s.act;
        gate.init(s.d, s.F, s.mlp_bias, p);
        up.init(s.d, s.F, s.mlp_bias, p);
        down.init(s.F, s.d, s.mlp_bias, p);
    }

    Buf forward(const Buf& x, int64_t n_flat) {
        rows = n_flat;
        Buf gp = gate.forward(x, rows);
        gate_post.assign(gp.size(), 0.0f);
        elementwise(act == 1 ? 6 : 4, gp.data(), gate_post.data(), gp.size());  // GeluTanh or Silu
        up_out = up.forward(x, rows);
        Buf hidden(gp.size());
        mul(gate_post.data(), up_out.data(), hidden.data(), hidden.size());
        return down.forward(hidden, rows);
    }

    Buf relevance(const Buf& r_out, const RuleConfig& cfg) const {
        Buf r_hidden = down.relevance(r_out, cfg);
        Buf r_gate(r_hidden.size());
        lrp_bilinear_elementwise(gate_post.data(), up_out.data(), r_hidden.data(), r_gate.data(), r_gate.size(),
                                 cfg.eps);
        Buf r_from_gate = gate.relevance(r_gate, cfg), r_from_up = up.relevance(r_gate, cfg);
        Buf r_in(r_from_gate.size());
        add(r_from_gate.data(), r_from_up.data(), r_in.data(), r_in.size());
        return r_in;
    }
};

// TransformerBlock (transformer_block.cpp:99-133 forward, 189-227 relevance), pre-norm.
struct Block {
    ModelShape s;
    RMSNorm norm1, norm2, post_attn_norm, post_mlp_norm;
    MHA mha;
    SwiGLU mlp;
    Buf last_x, last_attn, last_y1, last_ffn;
    int64_t N = 0, L = 0;

    void init(const ModelShape& sh, const float*& p) {  // named_parameters order (transformer_block.cpp:240-249)
        s = sh;
        norm1.init(s.d, s.norm_eps, s.norm_offset, p);
        mha.init(s, p);
        norm2.init(s.d, s.norm_eps, s.norm_offset, p);
        mlp.init(s, p);
        if (s.post_norms) {
            post_attn_norm.init(s.d, s.norm_eps, s.norm_offset, p);
            post_mlp_norm.init(s.d, s.norm_eps, s.norm_offset, p);
        }
    }

    Buf forward(const Buf& x, int64_t n_, int64_t l_) {
        N = n_;
        L = l_;
        const int64_t rows = N * L;
        Buf attn_out = mha.forward(norm1.forward(x, rows), N, L);
        if (s.post_norms) attn_out = post_attn_norm.forward(attn_out, rows);  // PostNorm (:99-133)
        Buf y1(x.size());
        add(x.data(), attn_out.data(), y1.data(), y1.size());
        Buf ffn = mlp.forward(norm2.forward(y1, rows), rows);
        if (s.post_norms) ffn = post_mlp_norm.forward(ffn, rows);
        Buf y2(x.size());
        add(y1.data(), ffn.data(), y2.data(), y2.size());
        last_x = x;
        last_attn = attn_out;
        last_y1 = y1;
        last_ffn = ffn;
        return y2;
    }

    Buf relevance(const Buf& r, const RuleConfig& cfg) {
        const size_t n = r.size();
        Buf r_y1_direct(n), r_ffn(n);
        lrp_residual_split(last_y1.data(), last_ffn.data(), r.data(), r_y1_direct.data(), r_ffn.data(), n, cfg.eps);
        Buf r_norm2 = mlp.relevance(r_ffn, cfg);  // RMSNorm relevance is the identity
        Buf r_y1(n);
        add(r_y1_direct.data(), r_norm2.data(), r_y1.data(), n);
        Buf r_x_direct(n), r_attn(n);
        lrp_residual_split(last_x.data(), last_attn.data(), r_y1.data(), r_x_direct.data(), r_attn.data(), n, cfg.eps);
        Buf r_norm1 = mha.relevance(r_attn, cfg);
        Buf r_x(n);
        add(r_x_direct.data(), r_norm1.data(), r_x.data(), n);
        return r_x;
    }
};

ModelShape shape_of(const px_model_config& c) {
    ModelShape s;
    s.d = c.hidden_size;
    s.H = c.num_heads;
    s.Hkv = c.num_kv_heads > 0 ? c.num_kv_heads : c.num_heads;
    s.D = c.head_dim > 0 ? c.head_dim : c.hidden_size / c.num_heads;
    s.F = c.intermediate_size;
    s.norm_eps = c.rms_norm_eps;
    s.theta = c.rope_theta;
    s.rope = c.use_rope != 0;
    s.half_layout = c.rope_rotate_half != 0;
    s.causal = c.causal != 0;
    s.qkv_bias = c.qkv_bias != 0;
    s.out_bias = c.out_bias != 0;
    s.mlp_bias = c.mlp_bias != 0;
    s.act = c.hidden_act;
    s.qk_norm = c.qk_norm != 0;
    s.post_norms = c.post_norms != 0;
    s.norm_offset = c.norm_weight_offset;
    if (c.query_pre_attn_scalar > 0.0f)
        s.score_scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(c.query_pre_attn_scalar)));
    if (c.rope_scaling != 0) s.inv_freq = rope_inverse_frequencies(c, s.D);
    return s;
}

// is_sliding_layer (hf_model.cpp:249-253) and ToAttentionConfig(config, layer) (:305-313): a
// sliding layer gets the window and, when given, its own unscaled RoPE base.
bool sliding_layer(const px_model_config& c, int64_t i) {
    if (c.sliding_window <= 0) return false;
    return c.sliding_layers == 0 || (i < 64 && ((c.sliding_layers >> i) & 1u) != 0);
}

ModelShape shape_of_layer(const px_model_config& c, int64_t i) {
    ModelShape s = shape_of(c);
    if (!sliding_layer(c, i)) return s;
    s.window = static_cast<size_t>(c.sliding_window);
    if (c.rope_local_base > 0.0f) {
        s.theta = c.rope_local_base;
        s.inv_freq.clear();
    }
    return s;
}

void validate(const px_model_config& c, bool lm) {
    if (c.hidden_size <= 0 || c.num_heads <= 0 || c.intermediate_size <= 0)
        throw std::invalid_argument("model config: hidden_size, num_heads and intermediate_size must be positive");
    const ModelShape s = shape_of(c);
    if (s.H % s.Hkv != 0) throw std::invalid_argument("model config: num_heads must be a multiple of num_kv_heads");
    if (s.rope && s.D % 2 != 0) throw std::invalid_argument("model config: RoPE needs an even head_dim");
    if (lm && (c.vocab_size <= 0 || c.num_layers <= 0))
        throw std::invalid_argument("model config: vocab_size and num_layers must be positive");
    if (c.hidden_act < 0 || c.hidden_act > 1) throw std::invalid_argument("model config: unknown hidden_act");
    if (c.rope_scaling < 0 || c.rope_scaling > 2) throw std::invalid_argument("model config: unknown rope_scaling");
    if (c.sliding_layers != 0 && c.num_layers > 64)
        throw std::invalid_argument("model config: sliding_layers names at most 64 layers");
}

int64_t block_params(const ModelShape& s) {
    const int64_t q = s.H * s.D, kv = s.Hkv * s.D;
    int64_t n = 2 * s.d + s.d * q + 2 * s.d * kv + q * s.d + 3 * s.d * s.F;
    if (s.qkv_bias) n += q + 2 * kv;
    if (s.out_bias) n += s.d;
    if (s.mlp_bias) n += 2 * s.F + s.d;
    if (s.qk_norm) n += 2 * s.D;
    if (s.post_norms) n += 2 * s.d;
    return n;
}

// CausalLM (causal_lm.cpp:30-54 assembly, 63-80 forward, 94-113 relevance), Llama family.
struct LM {
    px_model_config c;
    ModelShape s;
    Buf embed;  // (V, d)
    std::vector<std::unique_ptr<Block>> layers;
    RMSNorm norm;
    Linear head;  // untied: (d, V)
    int64_t N = 0, L = 0;
    Buf ids_f;
    Buf head_x, logits;  // tied head caches (tied_lm_head_module.cpp:30-53)

    void init(const px_model_config& cfg, const float* p) {
        c = cfg;
        s = shape_of(cfg);
        embed.assign(p, p + c.vocab_size * s.d);
        p += c.vocab_size * s.d;
        for (int64_t i = 0; i < c.num_layers; ++i) {
            layers.push_back(std::make_unique<Block>());
            layers.back()->init(shape_of_layer(c, i), p);
        }
        norm.init(s.d, s.norm_eps, s.norm_offset, p);
        if (!c.tie_word_embeddings) head.init(s.d, c.vocab_size, false, p);
    }

    Buf forward(const int64_t* ids, int64_t n_, int64_t l_) {
        N = n_;
        L = l_;
        const int64_t rows = N * L;
        ids_f.assign(static_cast<size_t>(rows), 0.0f);
        for (int64_t i = 0; i < rows; ++i) {  // EmbeddingModule::forward_impl validation (embedding_module.cpp:48-59)
            if (ids[i] < 0 || ids[i] >= c.vocab_size)
                throw std::invalid_argument("EmbeddingModule::forward: index out of range [0, num_embeddings)");
            ids_f[static_cast<size_t>(i)] = static_cast<float>(ids[i]);
        }
        Buf x(static_cast<size_t>(rows * s.d));
        gather_rows(embed.data(), ids_f.data(), x.data(), rows, s.d);
        if (c.embed_scale != 0.0f && c.embed_scale != 1.0f)  // ScaleEmbeddings (causal_lm.cpp:56-61)
            axpby(c.embed_scale, x.data(), 0.0f, nullptr, x.data(), x.size());
        for (auto& layer : layers) x = layer->forward(x, N, L);
        head_x = norm.forward(x, rows);
        if (!c.tie_word_embeddings) return head.forward(head_x, rows);
        logits.assign(static_cast<size_t>(rows * c.vocab_size), 0.0f);
        gemm_ex(head_x.data(), false, embed.data(), true, logits.data(), rows, s.d, c.vocab_size, 0.0f);
        return logits;
    }

    // TiedLMHeadModule::propagate_relevance (tied_lm_head_module.cpp:76-111): the table E (V, d)
    // as an affine layer x E^T with a zero bias; the pre-bias epsilon rule becomes the
    // bias-in-denominator one.
    Buf head_relevance(const Buf& r, const RuleConfig& cfg) const {
        const size_t M = N * L, V = c.vocab_size, D = s.d;
        if (!c.tie_word_embeddings) return head.relevance(r, cfg);
        rule_validate(cfg, "TiedLMHeadModule");
        Affine op;
        op.n_in = M * D;
        op.n_out = M * V;
        op.n_w = V * D;
        op.n_b = V;
        op.forward = [=](const float* xs, const float* w, float* y) { gemm_ex(xs, false, w, true, y, M, D, V, 0.0f); };
        op.backward = [=](const float* g, const float* w, float* gx) { gemm(g, w, gx, M, V, D); };
        op.add_bias = [=](const float* y, const float* bb, float* o) { add_row_vector(y, bb, o, M, V); };
        RuleConfig rule = cfg;
        if (rule.rule == kEpsilon) rule.bias_in_denominator = true;
        const Buf zero(V, 0.0f);
        Buf r_in(M * D, 0.0f);
        rule_apply(op, head_x.data(), embed.data(), zero.data(), logits.data(), r.data(), r_in.data(), rule);
        return r_in;
    }

    Buf relevance(const Buf& seed, const RuleConfig& cfg, float* key_rel, float* value_rel) {
        Buf r = head_relevance(seed, cfg);
        const size_t kv = static_cast<size_t>(N * L * s.Hkv * s.D);
        for (size_t i = layers.size(); i-- > 0;) {
            r = layers[i]->relevance(r, cfg);
            if (key_rel) std::copy(layers[i]->mha.key_rel.begin(), layers[i]->mha.key_rel.end(), key_rel + i * kv);
            if (value_rel)
                std::copy(layers[i]->mha.value_rel.begin(), layers[i]->mha.value_rel.end(), value_rel + i * kv);
        }
        return r;
    }
};

// EmbeddingModule::propagate_relevance (embedding_module.cpp:100-124): a gemm against a ones
// column, so each token's sum runs over features in order.
void token_sums(const float* r, float* out, size_t count, size_t dim) {
    Buf ones(dim, 1.0f);
    gemm_ex(r, false, ones.data(), false, out, count, dim, 1, 0.0f);
}

RuleConfig rule_config(const px_lrp_rule& r) {
    RuleConfig c{r.epsilon, r.bias_in_denominator != 0};
    c.rule = r.rule;
    c.gamma = r.gamma;
    c.alpha = r.alpha;
    c.beta = r.beta;
    c.low = r.low;
    c.high = r.high;
    return c;
}

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

}  // namespace

extern "C" {

const char* pxo_last_error(void) { return g_error.c_str(); }
void pxo_set_threads(int threads) { g_threads = threads > 0 ? threads : 0; }
void pxo_set_split_threads(int threads) { g_split_threads = threads > 1 ? threads : 1; }
int pxo_get_threads(void) { return static_cast<int>(worker_threads()); }

void pxo_fill_normal(float* dst, size_t n, uint64_t seed, double stddev) {
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

int64_t pxo_block_param_count(const px_model_config* cfg) { return block_params(shape_of(*cfg)); }

int64_t pxo_param_count(const px_model_config* cfg) {
    const ModelShape s = shape_of(*cfg);
    int64_t n = cfg->vocab_size * s.d + cfg->num_layers * block_params(s) + s.d;
    if (!cfg->tie_word_embeddings) n += s.d * cfg->vocab_size;
    return n;
}

void* pxo_block_create(const px_model_config* cfg, const float* params) {
    Block* b = nullptr;
    if (guarded([&] {
            validate(*cfg, false);
            auto blk = std::make_unique<Block>();
            const float* p = params;
            blk->init(shape_of_layer(*cfg, 0), p);
            b = blk.release();
        }) != 0)
        return nullptr;
    return b;
}

int pxo_block_forward(void* h, const float* x, int64_t n, int64_t l, float* y) {
    return guarded([&] {
        Block* b = static_cast<Block*>(h);
        Buf in(x, x + n * l * b->s.d);
        Buf out = b->forward(in, n, l);
        std::copy(out.begin(), out.end(), y);
    });
}

int pxo_block_relevance(void* h, const float* r_out, float eps, int bias_in_denominator, float* r_in) {
    return guarded([&] {
        Block* b = static_cast<Block*>(h);
        if (b->N == 0) throw std::logic_error("TransformerBlock::propagate_relevance: called before any forward()");
        Buf r(r_out, r_out + b->N * b->L * b->s.d);
        Buf out = b->relevance(r, RuleConfig{eps, bias_in_denominator != 0});
        std::copy(out.begin(), out.end(), r_in);
    });
}

int pxo_block_relevance_rule(void* h, const float* r_out, const px_lrp_rule* rule, float* r_in) {
    return guarded([&] {
        auto* b = static_cast<Block*>(h);
        if (b->N == 0) throw std::logic_error("TransformerBlock::propagate_relevance: called before any forward()");
        Buf r(r_out, r_out + b->N * b->L * b->s.d);
        Buf out = b->relevance(r, rule_config(*rule));
        std::copy(out.begin(), out.end(), r_in);
    });
}

void pxo_block_destroy(void* h) { delete static_cast<Block*>(h); }

void* pxo_lm_create(const px_model_config* cfg, const float* params) {
    LM* m = nullptr;
    if (guarded([&] {
            validate(*cfg, true);
            auto lm = std::make_unique<LM>();
            lm->init(*cfg, params);
            m = lm.release();
        }) != 0)
        return nullptr;
    return m;
}

int pxo_lm_forward(void* h, const int64_t* ids, int64_t n, int64_t l, float* logits) {
    return guarded([&] {
        LM* m = static_cast<LM*>(h);
        Buf out = m->forward(ids, n, l);
        if (logits) std::copy(out.begin(), out.end(), logits);
    });
}

int pxo_lm_relevance(void* h, const float* seed, float eps, int bias_in_denominator, float* r_embed, float* r_tokens,
                     float* key_rel, float* value_rel) {
    return guarded([&] {
        LM* m = static_cast<LM*>(h);
        if (m->N == 0) throw std::logic_error("CausalLM::propagate_relevance_by_layer: called before any forward()");
        const size_t rows = static_cast<size_t>(m->N * m->L);
        Buf s(seed, seed + rows * m->c.vocab_size);
        Buf r = m->relevance(s, RuleConfig{eps, bias_in_denominator != 0}, key_rel, value_rel);
        if (r_embed) std::copy(r.begin(), r.end(), r_embed);
        if (r_tokens) token_sums(r.data(), r_tokens, rows, m->s.d);
    });
}

int pxo_lm_relevance_rule(void* h, const float* seed, const px_lrp_rule* rule, float* r_embed, float* r_tokens,
                          float* key_rel, float* value_rel) {
    return guarded([&] {
        LM* m = static_cast<LM*>(h);
        if (m->N == 0) throw std::logic_error("CausalLM::propagate_relevance_by_layer: called before any forward()");
        const size_t rows = static_cast<size_t>(m->N * m->L);
        Buf s(seed, seed + rows * m->c.vocab_size);
        Buf r = m->relevance(s, rule_config(*rule), key_rel, value_rel);
        if (r_embed) std::copy(r.begin(), r.end(), r_embed);
        if (r_tokens) token_sums(r.data(), r_tokens, rows, m->s.d);
    });
}

void pxo_lm_destroy(void* h) { delete static_cast<LM*>(h); }

int pxo_linear_forward(const float* x, const float* w, const float* bias, int64_t n, int64_t in, int64_t out,
                       float* pre_bias, float* y) {
    return guarded([&] {
        gemm(x, w, pre_bias, n, in, out);
        if (bias) add_row_vector(pre_bias, bias, y, n, out);
        else std::copy(pre_bias, pre_bias + n * out, y);
    });
}

int pxo_linear_relevance(const float* x, const float* w, const float* bias, const float* pre_bias, const float* r,
                         int64_t n, int64_t in, int64_t out, float eps, int bias_in_denominator, float* r_in) {
    return guarded([&] {
        Linear lin;
        lin.in = in;
        lin.out = out;
        lin.n = n;
        lin.has_bias = bias != nullptr;
        lin.w.assign(w, w + in * out);
        lin.b.assign(static_cast<size_t>(out), 0.0f);
        if (bias) lin.b.assign(bias, bias + out);
        lin.x.assign(x, x + n * in);
        lin.z.assign(pre_bias, pre_bias + n * out);
        Buf rr(r, r + n * out);
        Buf res = lin.relevance(rr, RuleConfig{eps, bias_in_denominator != 0});
        std::copy(res.begin(), res.end(), r_in);
    });
}

int pxo_linear_relevance_rule(const float* x, const float* w, const float* bias, const float* pre_bias,
                              const float* r, int64_t n, int64_t in, int64_t out, const px_lrp_rule* rule,
                              float* r_in) {
    return guarded([&] {
        Linear lin;
        lin.in = in;
        lin.out = out;
        lin.n = n;
        lin.has_bias = bias != nullptr;
        lin.w.assign(w, w + in * out);
        lin.b.assign(static_cast<size_t>(out), 0.0f);
        if (bias) lin.b.assign(bias, bias + out);
        lin.x.assign(x, x + n * in);
        lin.z.assign(pre_bias, pre_bias + n * out);
        Buf rr(r, r + n * out);
        Buf res = lin.relevance(rr, rule_config(*rule));
        std::copy(res.begin(), res.end(), r_in);
    });
}

void pxo_gemm(const float* a, const float* b, float* out, size_t m, size_t k, size_t n) { gemm(a, b, out, m, k, n); }
void pxo_gemm_ex(const float* a, int ta, const float* b, int tb, float* out, size_t m, size_t k, size_t n, float beta) {
    gemm_ex(a, ta != 0, b, tb != 0, out, m, k, n, beta);
}
void pxo_elementwise(int op, const float* in, float* out, size_t n) { elementwise(op, in, out, n); }
void pxo_elementwise_backward(int op, const float* x, const float* gy, float* gx, size_t n) {
    elementwise_backward(op, x, gy, gx, n);
}
void pxo_softmax_rows_backward(const float* y, const float* dy, float* dx, size_t rows, size_t cols) {
    softmax_rows_backward(y, dy, dx, rows, cols);
}
void pxo_rms_norm_backward(const float* gy, const float* gamma, const float* x, const float* row_rms, float* gx,
                           float* gterms, size_t rows, size_t cols) {
    rms_norm_backward(gy, gamma, x, row_rms, gx, gterms, rows, cols);
}
void pxo_add(const float* a, const float* b, float* out, size_t n) { add(a, b, out, n); }
void pxo_mul(const float* a, const float* b, float* out, size_t n) { mul(a, b, out, n); }
void pxo_axpby(float alpha, const float* x, float beta, const float* y, float* out, size_t n) {
    axpby(alpha, x, beta, y, out, n);
}
void pxo_add_row_vector(const float* in, const float* row, float* out, size_t rows, size_t cols) {
    add_row_vector(in, row, out, rows, cols);
}
void pxo_softmax_rows(const float* in, float* out, size_t rows, size_t cols) { softmax_rows(in, out, rows, cols); }
void pxo_rms_norm_forward(const float* in, const float* gamma, float* out, float* row_rms, size_t rows, size_t cols,
                          float eps) {
    rms_norm_forward(in, gamma, out, row_rms, rows, cols, eps);
}
void pxo_rope_rotate(const float* in, const float* cs, const float* sn, float* out, size_t slices, size_t seq,
                     size_t hd, int inverse, int half_layout) {
    rope_rotate(in, cs, sn, out, slices, seq, hd, inverse != 0, half_layout != 0);
}
void pxo_permute_0213(const float* in, float* out, size_t d0, size_t d1, size_t d2, size_t d3) {
    permute_0213(in, out, d0, d1, d2, d3);
}
void pxo_attention_mask_fill(float* scores, const float* keep, size_t batch, size_t heads, size_t q_len, size_t k_len,
                             int causal, size_t q_offset, size_t window, float value) {
    attention_mask_fill(scores, keep, batch, heads, q_len, k_len, causal != 0, q_offset, window, value);
}
void pxo_gather_rows(const float* table, const float* idx, float* out, size_t count, size_t dim) {
    gather_rows(table, idx, out, count, dim);
}
void pxo_lrp_linear(const float* x, const float* w, const float* z, const float* r, float* r_in, size_t rows,
                    size_t in, size_t out, float eps) {
    lrp_linear(x, w, z, r, r_in, rows, in, out, eps);
}
void pxo_lrp_residual_split(const float* a, const float* b, const float* r, float* ra, float* rb, size_t n, float eps) {
    lrp_residual_split(a, b, r, ra, rb, n, eps);
}
void pxo_lrp_bilinear_elementwise(const float* a, const float* b, const float* r, float* out, size_t n, float eps) {
    lrp_bilinear_elementwise(a, b, r, out, n, eps);
}
void pxo_lrp_bilinear_matmul(const float* a, const float* b, const float* o, const float* r_o, float* r_a, float* r_b,
                             size_t slices, size_t m, size_t p, size_t q, float eps, int bt) {
    lrp_bilinear_matmul(a, b, o, r_o, r_a, r_b, slices, m, p, q, eps, bt != 0);
}
void pxo_lrp_softmax_rows(const float* x, const float* y, const float* r, float* r_in, size_t rows, size_t cols) {
    lrp_softmax_rows(x, y, r, r_in, rows, cols);
}
void pxo_lrp_rope(const float* x, const float* y, const float* r, const float* cs, const float* sn, float* r_in,
                  size_t slices, size_t seq, size_t hd, float eps, int half_layout) {
    lrp_rope(x, y, r, cs, sn, r_in, slices, seq, hd, eps, half_layout != 0);
}
void pxo_lrp_stabilized_divide(const float* r, const float* denom, const float* gate, float* out, size_t n, float eps,
                               int mode) {
    lrp_stabilized_divide(r, denom, gate, out, n, eps, mode);
}
void pxo_copy_2d(float* dst, size_t ds, const float* src, size_t ss, size_t rows, size_t cols) {
    copy_2d(dst, ds, src, ss, rows, cols);
}
void pxo_accumulate_rows(const float* in, float* out, size_t rows, size_t cols) { accumulate_rows(in, out, rows, cols); }
void pxo_column_sums(const float* in, float* out, size_t rows, size_t cols, float beta) {  // cpu_backend.cpp:208-216
    for (size_t j = 0; j < cols; ++j) {
        float acc = 0.0f;
        for (size_t i = 0; i < rows; ++i) acc += in[i * cols + j];
        out[j] = (beta == 0.0f) ? acc : beta * out[j] + acc;
    }
}
float pxo_sum(const float* in, size_t n) {  // cpu_backend.cpp:354-360
    float acc = 0.0f;
    for (size_t i = 0; i < n; ++i) acc += in[i];
    return acc;
}
float pxo_dot(const float* a, const float* b, size_t n) {  // cpu_backend.cpp:284-290
    float acc = 0.0f;
    for (size_t i = 0; i < n; ++i) acc += a[i] * b[i];
    return acc;
}
void pxo_rope_tables(int64_t hd, float base, int64_t seq, int64_t offset, float* cs, float* sn) {
    rope_tables(hd, base, seq, offset, cs, sn);
}

}  // extern "C"
