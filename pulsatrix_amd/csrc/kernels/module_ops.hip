// module_ops.hip -- the DeviceBackend ops of the reference's non-LLM modules (include/pxk.h): the
// fuzzy-logic gates and the power-mean aggregator, convolution patches, pooling, batch and group
// normalisation, the RNN/LSTM/GRU cell passes, the Mamba / RWKV / RetNet scans and the
// reinforcement-learning row losses. None is on the LM's hot path, so each is a simple kernel: one
// thread per independent output, lane or row, which owns every sum it makes and adds its terms in
// the reference's loop order (src/lrp_math.hpp, cnn_math.hpp, recurrent_math.hpp, ssm_math.hpp,
// rl_math.hpp; src/cpu_backend.cpp). Deterministic, no atomics; the GPU's exp/log/pow/tanh and its
// fused multiply-adds make results agree with CPUBackend to rounding, not bit for bit.
#include <cmath>
#include <cstdint>

#include "common.hpp"

namespace pxk {
namespace {

constexpr int kThreads = 256;

template <class F>
__global__ void __launch_bounds__(kThreads) lanes_kernel(int64_t count, F f) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < count;
         i += static_cast<int64_t>(gridDim.x) * kThreads)
        f(i);
}

// Runs f(i) for i in [0, count) on the stream.
template <class F>
int run_lanes(const char* what, int64_t count, void* stream, F f) {
    if (count < 0) return fail(PXK_ERR_INVALID, "%s: negative size", what);
    if (count == 0) return PXK_OK;
    PXK_LAUNCH(lanes_kernel<F>, dim3(grid_for(count, kThreads)), dim3(kThreads), 0, S(stream), count, f);
    return launched(what);
}

__device__ __forceinline__ float logistic(float z) { return 1.0f / (1.0f + expf(-z)); }
__device__ __forceinline__ float softplus(float z) { return z > 20.0f ? z : log1pf(expf(z)); }
// std::max / std::min as libstdc++ defines them (which operand a NaN comparison returns).
__device__ __forceinline__ float lmax(float a, float b) { return a < b ? b : a; }
__device__ __forceinline__ float lmin(float a, float b) { return b < a ? b : a; }

// ---- fuzzy logic (lrp_math.hpp:125-270): norm 0 product, 1 Lukasiewicz, 2 Godel -------------------
// The winner-takes-all rules of the Godel norm hand the whole share to the winning operand (ties to a).
__device__ void logic_element(int op, int norm, float a, float b, float g, float y, float eps, float* oa, float* ob) {
    const bool conj = op < 3;
    const int pass = op % 3;  // 0 forward, 1 backward, 2 LRP
    if (pass == 0) {
        float v;
        if (norm == 0) {
            v = conj ? a * b : a + b - a * b;
        } else if (norm == 1) {
            const float z = conj ? a + b - 1.0f : a + b;
            v = conj ? (z > 0.0f ? z : 0.0f) : (z < 1.0f ? z : 1.0f);
        } else {
            v = conj ? (a <= b ? a : b) : (a >= b ? a : b);
        }
        *oa = v;
        return;
    }
    if (norm == 2) {
        const bool a_wins = conj ? a <= b : a >= b;
        *oa = a_wins ? g : 0.0f;
        *ob = a_wins ? 0.0f : g;
        return;
    }
    if (norm == 1) {  // the active region passes (backward) or shares by the pre-bias sum a + b (LRP)
        const bool active = conj ? a + b - 1.0f > 0.0f : a + b < 1.0f;
        if (!active) {
            *oa = 0.0f;
            *ob = 0.0f;
        } else if (pass == 1) {
            *oa = g;
            *ob = g;
        } else {
            const float den = stab(a + b, eps);
            *oa = (a / den) * g;
            *ob = (b / den) * g;
        }
        return;
    }
    if (pass == 1) {  // product
        *oa = conj ? b * g : (1.0f - b) * g;
        *ob = conj ? a * g : (1.0f - a) * g;
    } else if (conj) {  // a b: the bilinear half-and-half share
        const float share = (a * b / (2.0f * y + eps * (y >= 0.0f ? 1.0f : -1.0f))) * g;
        *oa = share;
        *ob = share;
    } else {  // a + b - a b split as a (2 - b) / 2 and b (2 - a) / 2
        const float den = stab(y, eps);
        *oa = ((a * (2.0f - b) * 0.5f) / den) * g;
        *ob = ((b * (2.0f - a) * 0.5f) / den) * g;
    }
}

// ---- conv2d patches (cnn_math.hpp:21-93) -----------------------------------------------------------
struct Geo {
    int64_t kh, kw, sh, sw, ph, pw, out_h, out_w;
};

Geo geo_of(const pxk_conv_geometry& g, int64_t h, int64_t w) {
    Geo o{g.kh, g.kw, g.stride_h, g.stride_w, g.pad_h, g.pad_w, 0, 0};
    o.out_h = (h + 2 * g.pad_h - g.kh) / g.stride_h + 1;
    o.out_w = (w + 2 * g.pad_w - g.kw) / g.stride_w + 1;
    return o;
}

bool bad_geometry(const char* what, const pxk_conv_geometry* g, int64_t h, int64_t w, int* rc) {
    if (g == nullptr || g->kh <= 0 || g->kw <= 0 || g->stride_h <= 0 || g->stride_w <= 0 || g->pad_h < 0 ||
        g->pad_w < 0 || h + 2 * g->pad_h < g->kh || w + 2 * g->pad_w < g->kw) {
        *rc = fail(PXK_ERR_INVALID, "%s: bad window geometry", what);
        return true;
    }
    return false;
}

// ---- the per-channel normalisations (cnn_math.hpp:186-413) -----------------------------------------
// Element (e, c, s) of (n, c, spatial) data lives at (e * C + c) * spatial + s.
struct Planes {
    int64_t N, C, sp;
    __device__ int64_t at(int64_t e, int64_t c, int64_t s) const { return (e * C + c) * sp + s; }
};

}  // namespace
}  // namespace pxk

using namespace pxk;

extern "C" {

int pxk_logic_pointwise(int op, int norm, const float* a, const float* b, const float* g_or_r, const float* y,
                        float* out_a, float* out_b, int64_t n, float eps, void* stream) {
    if (op < 0 || op > 5 || norm < 0 || norm > 2) return fail(PXK_ERR_INVALID, "pxk_logic_pointwise: unknown op or norm");
    return run_lanes("pxk_logic_pointwise", n, stream, [=] __device__(int64_t i) {
        float sink = 0.0f;
        logic_element(op, norm, a[i], b[i], op % 3 ? g_or_r[i] : 0.0f, op % 3 == 2 ? y[i] : 0.0f, eps, out_a + i,
                      op % 3 ? out_b + i : &sink);
    });
}

// AggregatorModule's power mean over the leading axis, one thread per column, rows in order
// (lrp_math.hpp:272-306).
int pxk_aggregator_forward(const float* x, float* mean_pow, float* out, int64_t n, int64_t cols, float p,
                           void* stream) {
    return run_lanes("pxk_aggregator_forward", cols, stream, [=] __device__(int64_t j) {
        float sum = 0.0f;
        for (int64_t i = 0; i < n; ++i) sum += powf(x[i * cols + j], p);
        const float m = sum / static_cast<float>(n);
        mean_pow[j] = m;
        out[j] = powf(m, 1.0f / p);
    });
}

int pxk_aggregator_backward(const float* x, const float* mean_pow, const float* grad_out, float* grad_in, int64_t n,
                            int64_t cols, float p, void* stream) {
    return run_lanes("pxk_aggregator_backward", cols, stream, [=] __device__(int64_t j) {
        const float scale = powf(mean_pow[j], 1.0f / p - 1.0f);
        for (int64_t i = 0; i < n; ++i)
            grad_in[i * cols + j] = grad_out[j] * (scale * powf(x[i * cols + j], p - 1.0f)) / static_cast<float>(n);
    });
}

int pxk_aggregator_lrp(const float* x, const float* mean_pow, const float* r_out, float* r_in, int64_t n, int64_t cols,
                       float p, float eps, void* stream) {
    return run_lanes("pxk_aggregator_lrp", cols, stream, [=] __device__(int64_t j) {
        const float den = stab(mean_pow[j] * static_cast<float>(n), eps);
        for (int64_t i = 0; i < n; ++i) r_in[i * cols + j] = (powf(x[i * cols + j], p) / den) * r_out[j];
    });
}

// One thread per patch entry (e, p, q) with p = (c kh + i) kw + j over the (out_h, out_w) grid q.
int pxk_im2col(const float* in, float* col, int64_t n, int64_t c, int64_t h, int64_t w, const pxk_conv_geometry* g,
               void* stream) {
    int rc;
    if (bad_geometry("pxk_im2col", g, h, w, &rc)) return rc;
    const Geo o = geo_of(*g, h, w);
    const int64_t P = c * o.kh * o.kw, Q = o.out_h * o.out_w;
    return run_lanes("pxk_im2col", n * P * Q, stream, [=] __device__(int64_t idx) {
        const int64_t q = idx % Q, p = (idx / Q) % P, e = idx / (P * Q);
        const int64_t j = p % o.kw, i = (p / o.kw) % o.kh, ch = p / (o.kw * o.kh);
        const int64_t ih = (q / o.out_w) * o.sh - o.ph + i, iw = (q % o.out_w) * o.sw - o.pw + j;
        col[idx] = (ih < 0 || ih >= h || iw < 0 || iw >= w) ? 0.0f : in[((e * c + ch) * h + ih) * w + iw];
    });
}

// One thread per input pixel: the pixel's window taps in the order the CPU scatter adds them (kernel
// row, then column, descending), added to the pixel's value.
int pxk_col2im_add(const float* col, float* out, int64_t n, int64_t c, int64_t h, int64_t w,
                   const pxk_conv_geometry* g, void* stream) {
    int rc;
    if (bad_geometry("pxk_col2im_add", g, h, w, &rc)) return rc;
    const Geo o = geo_of(*g, h, w);
    const int64_t P = c * o.kh * o.kw, Q = o.out_h * o.out_w;
    return run_lanes("pxk_col2im_add", n * c * h * w, stream, [=] __device__(int64_t idx) {
        const int64_t iw = idx % w, ih = (idx / w) % h, ch = (idx / (w * h)) % c, e = idx / (w * h * c);
        const float* pc = col + e * P * Q;
        float acc = out[idx];
        for (int64_t i = o.kh - 1; i >= 0; --i) {
            const int64_t t = ih + o.ph - i;
            if (t < 0 || t % o.sh != 0 || t / o.sh >= o.out_h) continue;
            for (int64_t j = o.kw - 1; j >= 0; --j) {
                const int64_t u = iw + o.pw - j;
                if (u < 0 || u % o.sw != 0 || u / o.sw >= o.out_w) continue;
                acc += pc[((ch * o.kh + i) * o.kw + j) * Q + (t / o.sh) * o.out_w + u / o.sw];
            }
        }
        out[idx] = acc;
    });
}

int pxk_add_channel_vector(const float* in, const float* vec, float* out, int64_t n, int64_t c, int64_t inner,
                           void* stream) {
    if (c <= 0 || inner <= 0) return n * c * inner == 0 ? PXK_OK : fail(PXK_ERR_INVALID, "pxk_add_channel_vector: bad sizes");
    return run_lanes("pxk_add_channel_vector", n * c * inner, stream,
                     [=] __device__(int64_t i) { out[i] = in[i] + vec[(i / inner) % c]; });
}

// Conv2D's epsilon rule per patch entry: output channels in order (cnn_math.hpp:84-93).
int pxk_lrp_conv(const float* col, const float* kernel, const float* pre_bias, const float* r, float* r_col, int64_t n,
                 int64_t out_channels, int64_t p, int64_t q, float eps, void* stream) {
    return run_lanes("pxk_lrp_conv", n * p * q, stream, [=] __device__(int64_t idx) {
        const int64_t qi = idx % q, pi = (idx / q) % p, e = idx / (p * q);
        const float a = col[idx];
        const float* z = pre_bias + e * out_channels * q;
        const float* rr = r + e * out_channels * q;
        float acc = 0.0f;
        for (int64_t oc = 0; oc < out_channels; ++oc) acc += (a * kernel[oc * p + pi] / stab(z[oc * q + qi], eps)) * rr[oc * q + qi];
        r_col[idx] = acc;
    });
}

// Max pooling with padding that never wins; argmax = first maximum's flat in-plane index.
int pxk_max_pool_forward(const float* in, float* out, float* argmax, int64_t planes, int64_t h, int64_t w, int64_t kh,
                         int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, void* stream) {
    const pxk_conv_geometry g{kh, kw, sh, sw, ph, pw};
    int rc;
    if (bad_geometry("pxk_max_pool_forward", &g, h, w, &rc)) return rc;
    const Geo o = geo_of(g, h, w);
    return run_lanes("pxk_max_pool_forward", planes * o.out_h * o.out_w, stream, [=] __device__(int64_t idx) {
        const int64_t ow = idx % o.out_w, oh = (idx / o.out_w) % o.out_h, pl = idx / (o.out_w * o.out_h);
        const float* plane = in + pl * h * w;
        float best = -INFINITY;
        int64_t at = -1;
        for (int64_t i = 0; i < kh; ++i) {
            const int64_t y = oh * sh - ph + i;
            if (y < 0 || y >= h) continue;
            for (int64_t j = 0; j < kw; ++j) {
                const int64_t x = ow * sw - pw + j;
                if (x < 0 || x >= w) continue;
                const float v = plane[y * w + x];
                if (at < 0 || v > best) {
                    best = v;
                    at = y * w + x;
                }
            }
        }
        out[idx] = best;
        argmax[idx] = static_cast<float>(at < 0 ? 0 : at);
    });
}

// Each input position gathers the pooled values whose argmax it is, over the windows holding it.
int pxk_max_unpool(const float* src, const float* argmax, float* dst, int64_t planes, int64_t h, int64_t w, int64_t kh,
                   int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, void* stream) {
    const pxk_conv_geometry g{kh, kw, sh, sw, ph, pw};
    int rc;
    if (bad_geometry("pxk_max_unpool", &g, h, w, &rc)) return rc;
    const Geo o = geo_of(g, h, w);
    return run_lanes("pxk_max_unpool", planes * h * w, stream, [=] __device__(int64_t idx) {
        const int64_t x = idx % w, y = (idx / w) % h, pl = idx / (w * h);
        const float* ps = src + pl * o.out_h * o.out_w;
        const float* pa = argmax + pl * o.out_h * o.out_w;
        const float me = static_cast<float>(y * w + x);
        const int64_t lo_h = y + ph - kh + 1, lo_w = x + pw - kw + 1;
        const int64_t oh0 = lo_h <= 0 ? 0 : (lo_h + sh - 1) / sh, ow0 = lo_w <= 0 ? 0 : (lo_w + sw - 1) / sw;
        const int64_t hh = (y + ph) / sh, ww = (x + pw) / sw;
        const int64_t oh1 = hh < o.out_h - 1 ? hh : o.out_h - 1, ow1 = ww < o.out_w - 1 ? ww : o.out_w - 1;
        float sum = 0.0f;
        for (int64_t oh = oh0; oh <= oh1; ++oh)
            for (int64_t ow = ow0; ow <= ow1; ++ow)
                if (pa[oh * o.out_w + ow] == me) sum += ps[oh * o.out_w + ow];
        dst[idx] = sum;
    });
}

// Non-overlapping average pooling (stride = window, no padding), its gradient and its epsilon rule:
// one thread per window.
int pxk_avg_pool_forward(const float* in, float* out, int64_t planes, int64_t h, int64_t w, int64_t kh, int64_t kw,
                         void* stream) {
    if (kh <= 0 || kw <= 0 || kh > h || kw > w) return fail(PXK_ERR_INVALID, "pxk_avg_pool_forward: bad window");
    const int64_t out_h = (h - kh) / kh + 1, out_w = (w - kw) / kw + 1;
    return run_lanes("pxk_avg_pool_forward", planes * out_h * out_w, stream, [=] __device__(int64_t idx) {
        const int64_t ow = idx % out_w, oh = (idx / out_w) % out_h, pl = idx / (out_w * out_h);
        const float* plane = in + pl * h * w;
        float sum = 0.0f;
        for (int64_t i = 0; i < kh; ++i)
            for (int64_t j = 0; j < kw; ++j) sum += plane[(oh * kh + i) * w + ow * kw + j];
        out[idx] = sum / static_cast<float>(kh * kw);
    });
}

int pxk_avg_pool_backward(const float* grad_out, float* grad_in, int64_t planes, int64_t h, int64_t w, int64_t kh,
                          int64_t kw, void* stream) {
    if (kh <= 0 || kw <= 0 || kh > h || kw > w) return fail(PXK_ERR_INVALID, "pxk_avg_pool_backward: bad window");
    const int64_t out_h = (h - kh) / kh + 1, out_w = (w - kw) / kw + 1;
    return run_lanes("pxk_avg_pool_backward", planes * out_h * out_w, stream, [=] __device__(int64_t idx) {
        const int64_t ow = idx % out_w, oh = (idx / out_w) % out_h, pl = idx / (out_w * out_h);
        const float gv = grad_out[idx] / static_cast<float>(kh * kw);
        for (int64_t i = 0; i < kh; ++i)
            for (int64_t j = 0; j < kw; ++j) grad_in[pl * h * w + (oh * kh + i) * w + ow * kw + j] = gv;
    });
}

int pxk_lrp_avg_pool(const float* x, const float* r, float* r_in, int64_t planes, int64_t h, int64_t w, int64_t kh,
                     int64_t kw, float eps, void* stream) {
    if (kh <= 0 || kw <= 0 || kh > h || kw > w) return fail(PXK_ERR_INVALID, "pxk_lrp_avg_pool: bad window");
    const int64_t out_h = (h - kh) / kh + 1, out_w = (w - kw) / kw + 1;
    return run_lanes("pxk_lrp_avg_pool", planes * out_h * out_w, stream, [=] __device__(int64_t idx) {
        const int64_t ow = idx % out_w, oh = (idx / out_w) % out_h, pl = idx / (out_w * out_h);
        const float* plane = x + pl * h * w;
        const float inv_k = 1.0f / static_cast<float>(kh * kw);
        float z = 0.0f;
        for (int64_t i = 0; i < kh; ++i)
            for (int64_t j = 0; j < kw; ++j) z += plane[(oh * kh + i) * w + ow * kw + j] * inv_k;
        const float den = stab(z, eps), rv = r[idx];
        for (int64_t i = 0; i < kh; ++i)
            for (int64_t j = 0; j < kw; ++j) {
                const int64_t k = (oh * kh + i) * w + ow * kw + j;
                r_in[pl * h * w + k] = (plane[k] * inv_k / den) * rv;
            }
    });
}

// BatchNorm over (n, spatial) per channel: one thread per channel, examples then positions in order.
int pxk_batch_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                           float* channel_std, int64_t n, int64_t c, int64_t spatial, float eps, void* stream) {
    const Planes P{n, c, spatial};
    return run_lanes("pxk_batch_norm_forward", c, stream, [=] __device__(int64_t ch) {
        const float M = static_cast<float>(n * spatial);
        float sum = 0.0f;
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) sum += in[P.at(e, ch, s)];
        const float mu = sum / M;
        float ss = 0.0f;
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) {
                const float d = in[P.at(e, ch, s)] - mu;
                ss += d * d;
            }
        const float sd = sqrtf(ss / M + eps);
        channel_std[ch] = sd;
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                const float xh = (in[k] - mu) / sd;
                xhat[k] = xh;
                out[k] = gamma[ch] * xh + beta[ch];
            }
    });
}

int pxk_batch_norm_backward(const float* grad_out, const float* gamma, const float* xhat, const float* channel_std,
                            float* grad_in, float* gamma_grad, float* beta_grad, int64_t n, int64_t c, int64_t spatial,
                            void* stream) {
    const Planes P{n, c, spatial};
    return run_lanes("pxk_batch_norm_backward", c, stream, [=] __device__(int64_t ch) {
        const float M = static_cast<float>(n * spatial), sd = channel_std[ch], gm = gamma[ch];
        float gs = 0.0f, bs = 0.0f;
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                gs += grad_out[k] * xhat[k];
                bs += grad_out[k];
            }
        gamma_grad[ch] = gs;
        beta_grad[ch] = bs;
        float sg = 0.0f, sgx = 0.0f;
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                const float gx = grad_out[k] * gm;
                sg += gx;
                sgx += gx * xhat[k];
            }
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                grad_in[k] = (M * (grad_out[k] * gm) - sg - xhat[k] * sgx) / (M * sd);
            }
    });
}

// PyTorch's momentum rule with the unbiased batch variance; one value per channel keeps the variance.
int pxk_batch_norm_update_running(const float* in, float* running_mean, float* running_var, int64_t n, int64_t c,
                                  int64_t spatial, float momentum, void* stream) {
    const Planes P{n, c, spatial};
    return run_lanes("pxk_batch_norm_update_running", c, stream, [=] __device__(int64_t ch) {
        const int64_t count = n * spatial;
        const float M = static_cast<float>(count);
        float sum = 0.0f;
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) sum += in[P.at(e, ch, s)];
        const float mu = sum / M;
        running_mean[ch] = (1.0f - momentum) * running_mean[ch] + momentum * mu;
        if (count < 2) return;
        float ss = 0.0f;
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) {
                const float d = in[P.at(e, ch, s)] - mu;
                ss += d * d;
            }
        running_var[ch] = (1.0f - momentum) * running_var[ch] + momentum * (ss / (M - 1.0f));
    });
}

int pxk_batch_norm_eval_forward(const float* in, const float* gamma, const float* beta, const float* running_mean,
                                const float* running_var, float* xhat, float* out, float* channel_std, int64_t n,
                                int64_t c, int64_t spatial, float eps, void* stream) {
    const Planes P{n, c, spatial};
    return run_lanes("pxk_batch_norm_eval_forward", c, stream, [=] __device__(int64_t ch) {
        const float mu = running_mean[ch], sd = sqrtf(running_var[ch] + eps);
        channel_std[ch] = sd;
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                const float xh = (in[k] - mu) / sd;
                xhat[k] = xh;
                out[k] = gamma[ch] * xh + beta[ch];
            }
    });
}

int pxk_batch_norm_eval_backward(const float* grad_out, const float* gamma, const float* xhat,
                                 const float* channel_std, float* grad_in, float* gamma_grad, float* beta_grad,
                                 int64_t n, int64_t c, int64_t spatial, void* stream) {
    const Planes P{n, c, spatial};
    return run_lanes("pxk_batch_norm_eval_backward", c, stream, [=] __device__(int64_t ch) {
        const float scale = gamma[ch] / channel_std[ch];
        float gs = 0.0f, bs = 0.0f;
        for (int64_t e = 0; e < n; ++e)
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                gs += grad_out[k] * xhat[k];
                bs += grad_out[k];
                grad_in[k] = grad_out[k] * scale;
            }
        gamma_grad[ch] = gs;
        beta_grad[ch] = bs;
    });
}

// GroupNorm per (example, group): one thread per pair; then the gamma/beta gradients one thread per
// channel, per-example sums added over the examples in order.
int pxk_group_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                           float* group_std, int64_t n, int64_t c, int64_t spatial, int64_t groups, float eps,
                           void* stream) {
    if (groups <= 0 || c % groups != 0) return fail(PXK_ERR_INVALID, "pxk_group_norm_forward: groups must divide channels");
    const Planes P{n, c, spatial};
    const int64_t gsize = c / groups;
    return run_lanes("pxk_group_norm_forward", n * groups, stream, [=] __device__(int64_t lane) {
        const int64_t e = lane / groups, g = lane % groups, c0 = g * gsize;
        const float Ng = static_cast<float>(gsize * spatial);
        float sum = 0.0f;
        for (int64_t ch = c0; ch < c0 + gsize; ++ch)
            for (int64_t s = 0; s < spatial; ++s) sum += in[P.at(e, ch, s)];
        const float mu = sum / Ng;
        float ss = 0.0f;
        for (int64_t ch = c0; ch < c0 + gsize; ++ch)
            for (int64_t s = 0; s < spatial; ++s) {
                const float d = in[P.at(e, ch, s)] - mu;
                ss += d * d;
            }
        const float sd = sqrtf(ss / Ng + eps);
        group_std[lane] = sd;
        for (int64_t ch = c0; ch < c0 + gsize; ++ch)
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                const float xh = (in[k] - mu) / sd;
                xhat[k] = xh;
                out[k] = gamma[ch] * xh + beta[ch];
            }
    });
}

int pxk_group_norm_backward(const float* grad_out, const float* gamma, const float* xhat, const float* group_std,
                            float* grad_in, float* gamma_grad, float* beta_grad, int64_t n, int64_t c, int64_t spatial,
                            int64_t groups, void* stream) {
    if (groups <= 0 || c % groups != 0) return fail(PXK_ERR_INVALID, "pxk_group_norm_backward: groups must divide channels");
    const Planes P{n, c, spatial};
    const int64_t gsize = c / groups;
    int rc = run_lanes("pxk_group_norm_backward", n * groups, stream, [=] __device__(int64_t lane) {
        const int64_t e = lane / groups, g = lane % groups, c0 = g * gsize;
        const float Ng = static_cast<float>(gsize * spatial), sd = group_std[lane];
        float sg = 0.0f, sgx = 0.0f;
        for (int64_t ch = c0; ch < c0 + gsize; ++ch)
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                const float gx = grad_out[k] * gamma[ch];
                sg += gx;
                sgx += gx * xhat[k];
            }
        for (int64_t ch = c0; ch < c0 + gsize; ++ch)
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                grad_in[k] = (Ng * (grad_out[k] * gamma[ch]) - sg - xhat[k] * sgx) / (Ng * sd);
            }
    });
    if (rc != PXK_OK) return rc;
    return run_lanes("pxk_group_norm_backward (parameters)", c, stream, [=] __device__(int64_t ch) {
        float ga = 0.0f, ba = 0.0f;
        for (int64_t e = 0; e < n; ++e) {
            float gs = 0.0f, bs = 0.0f;
            for (int64_t s = 0; s < spatial; ++s) {
                const int64_t k = P.at(e, ch, s);
                gs += grad_out[k] * xhat[k];
                bs += grad_out[k];
            }
            ga += gs;
            ba += bs;
        }
        gamma_grad[ch] = ga;
        beta_grad[ch] = ba;
    });
}

// RNN / LSTM / GRU per-element cell passes (recurrent_math.hpp:18-106); slots per op in pxk.h.
int pxk_recurrent_cell(int op, const pxk_recurrent_args* args, int64_t n, void* stream) {
    if (op < 0 || op > 5 || args == nullptr) return fail(PXK_ERR_INVALID, "pxk_recurrent_cell: unknown op");
    const pxk_recurrent_args a = *args;
    return run_lanes("pxk_recurrent_cell", n, stream, [=] __device__(int64_t i) {
        const float dh = a.in[0][i] + a.in[1][i];  // upstream gradient / relevance plus the next step's
        switch (op) {
            case 0: {  // RNN: dz = dh (1 - h^2)
                const float h = a.in[2][i];
                a.out[0][i] = dh * (1.0f - h * h);
                return;
            }
            case 1: {  // LSTM forward from the activated gates
                const float ig = a.in[0][i], fg = a.in[1][i], gg = a.in[2][i], og = a.in[3][i];
                const float cc = fg * a.in[4][i] + ig * gg, tc = tanhf(cc);
                a.out[0][i] = cc;
                a.out[1][i] = tc;
                a.out[2][i] = og * tc;
                return;
            }
            case 2: {  // LSTM backward
                const float ig = a.in[3][i], fg = a.in[4][i], gg = a.in[5][i], og = a.in[6][i], tc = a.in[7][i];
                const float dc = dh * og * (1.0f - tc * tc) + a.in[2][i];
                a.out[3][i] = dh * tc * og * (1.0f - og);
                a.out[1][i] = dc * a.in[8][i] * fg * (1.0f - fg);
                a.out[0][i] = dc * gg * ig * (1.0f - ig);
                a.out[2][i] = dc * ig * (1.0f - gg * gg);
                a.out[4][i] = dc * fg;
                return;
            }
            case 3: {  // LSTM epsilon rule through c = f c_prev + i g
                const float rc = dh + a.in[2][i];
                const float den = stab(a.in[7][i], a.eps);
                a.out[1][i] = (a.in[4][i] * a.in[6][i] / den) * rc;
                a.out[0][i] = (a.in[3][i] * a.in[5][i] / den) * rc;
                return;
            }
            case 4: {  // GRU backward
                const float z = a.in[2][i], r = a.in[3][i], nn = a.in[4][i], hn = a.in[5][i], hp = a.in[6][i];
                a.out[0][i] = dh * (1.0f - z);
                a.out[1][i] = dh * (nn - hp) * z * (1.0f - z);
                const float dnp = dh * z * (1.0f - nn * nn);
                a.out[2][i] = dnp;
                a.out[3][i] = dnp * hn * r * (1.0f - r);
                a.out[4][i] = dnp * r;
                return;
            }
            default: {  // GRU epsilon rule through h = (1 - z) h_prev + z n and n's r * hn term
                const float z = a.in[2][i], r = a.in[3][i], nn = a.in[4][i], hn = a.in[5][i], hp = a.in[6][i];
                const float hd = stab(a.in[7][i], a.eps);
                a.out[0][i] = ((1.0f - z) * hp / hd) * dh;
                const float rn = (z * nn / hd) * dh;
                a.out[1][i] = rn;
                a.out[2][i] = (r * hn / stab(a.in[8][i], a.eps)) * rn;
                return;
            }
        }
    });
}

// GRU's R_hprev: the epsilon-rule sum through W_hn over k ascending, the element's own direct term
// added just before term kk (recurrent_math.hpp:108-124).
int pxk_gru_lrp_hprev(const float* h_prev, const float* w_hn, const float* hn, const float* r_term_b,
                      const float* direct, float* r_hprev, int64_t rows, int64_t hidden, float eps, void* stream) {
    return run_lanes("pxk_gru_lrp_hprev", rows * hidden, stream, [=] __device__(int64_t idx) {
        const int64_t kk = idx % hidden, row = idx / hidden;
        const float* hr = hn + row * hidden;
        const float* rb = r_term_b + row * hidden;
        const float hp = h_prev[idx];
        float acc = 0.0f;
        for (int64_t k = 0; k < hidden; ++k) {
            if (k == kk) acc += direct[idx];
            acc += (hp * w_hn[kk * hidden + k] / stab(hr[k], eps)) * rb[k];
        }
        r_hprev[idx] = acc;
    });
}

}  // extern "C"

// ---- Mamba / RWKV / RetNet (ssm_math.hpp) -----------------------------------------------------------
namespace pxk {
namespace {

// Lanes of each SsmPassOp (ssm_math.hpp:30-58).
int64_t ssm_lanes(int op, const pxk_ssm_args& a) {
    switch (op) {
        case 0: case 1: case 3: case 5: case 6: case 8: case 11: return a.n * a.d;
        case 2: case 13: return a.n * a.l * a.s;
        case 12: return a.n * a.s * a.d;
        case 15: return a.n * a.l * a.l;
        case 18: return a.d;
        default: return a.n * a.l * a.d;  // 4, 7, 9, 10, 14, 16, 17
    }
}

__device__ void mamba_forward(const pxk_ssm_args& a, int64_t lane) {
    const int64_t L = a.l, D = a.d, S = a.s, b = lane / D, d = lane % D;
    float* st = a.out[3];
    for (int64_t t = 0; t < L; ++t) {
        const int64_t x_at = (b * L + t) * D + d, bc = (b * L + t) * S;
        const float dl = softplus(a.in[1][x_at]), x = a.in[0][x_at];
        a.out[0][x_at] = dl;
        float y = a.in[5][d] * x;
        for (int64_t s = 0; s < S; ++s) {
            const float ab = expf(dl * a.in[4][d * S + s]), bb = dl * a.in[2][bc + s];
            a.out[1][x_at * S + s] = ab;
            a.out[2][x_at * S + s] = bb;
            const float h = ab * st[((b * (L + 1) + t) * D + d) * S + s] + bb * x;
            st[((b * (L + 1) + t + 1) * D + d) * S + s] = h;
            y += a.in[3][bc + s] * h;
        }
        a.out[4][x_at] = y;
    }
}

__device__ void mamba_backward(const pxk_ssm_args& a, int64_t lane) {
    const int64_t L = a.l, D = a.d, S = a.s, b = lane / D, d = lane % D;
    float* carry = a.out[4] + (b * D + d) * S;
    for (int64_t t = L - 1; t >= 0; --t) {
        const int64_t x_at = (b * L + t) * D + d, bc = (b * L + t) * S;
        const float gy = a.in[0][x_at], x = a.in[1][x_at], dl = a.in[2][x_at];
        float dx = 0.0f;
        dx += gy * a.in[10][d];
        float ddl = 0.0f;
        for (int64_t s = 0; s < S; ++s) {
            const int64_t k = x_at * S + s;
            const float hp = a.in[4][((b * (L + 1) + t) * D + d) * S + s], ab = a.in[5][k], bb = a.in[6][k];
            const float tot = gy * a.in[8][bc + s] + carry[s];
            carry[s] = tot * ab;
            a.out[2][k] = tot;
            const float dab = tot * hp, dbb = tot * x;
            dx += tot * bb;
            ddl += dbb * a.in[7][bc + s];
            ddl += dab * ab * a.in[9][d * S + s];
            a.out[3][k] = dab * ab * dl;
        }
        a.out[1][x_at] = ddl * logistic(a.in[3][x_at]);
        a.out[0][x_at] = dx;
    }
}

__device__ void mamba_grad_bc(const pxk_ssm_args& a, int64_t lane) {
    const int64_t L = a.l, D = a.d, S = a.s, bt = lane / S, s = lane % S, b = bt / L, t = bt % L;
    float db = 0.0f, dc = 0.0f;
    for (int64_t d = 0; d < D; ++d) {
        const int64_t x_at = bt * D + d;
        dc += a.in[0][x_at] * a.in[3][((b * (L + 1) + t + 1) * D + d) * S + s];
        db += a.in[4][x_at * S + s] * a.in[1][x_at] * a.in[2][x_at];
    }
    a.out[0][lane] = db;
    a.out[1][lane] = dc;
}

__device__ void mamba_lrp(const pxk_ssm_args& a, int64_t lane) {
    const int64_t L = a.l, D = a.d, S = a.s, b = lane / D, d = lane % D;
    float* carry = a.out[1] + (b * D + d) * S;
    for (int64_t t = L - 1; t >= 0; --t) {
        const int64_t x_at = (b * L + t) * D + d, bc = (b * L + t) * S;
        const float x = a.in[0][x_at], dy = stab(a.in[1][x_at], a.eps), ry = a.in[2][x_at];
        float rx = 0.0f;
        rx += (a.in[7][d] * x / dy) * ry;
        for (int64_t s = 0; s < S; ++s) {
            const int64_t k = x_at * S + s;
            const float ht = a.in[3][((b * (L + 1) + t + 1) * D + d) * S + s];
            const float hp = a.in[3][((b * (L + 1) + t) * D + d) * S + s];
            const float rh = (a.in[6][bc + s] * ht / dy) * ry + carry[s];
            const float dh = stab(ht, a.eps);
            carry[s] = (a.in[4][k] * hp / dh) * rh;
            rx += (a.in[5][k] * x / dh) * rh;
        }
        a.out[0][x_at] = rx;
    }
}

__device__ void rwkv_forward(const pxk_ssm_args& a, int64_t lane) {
    const int64_t L = a.l, D = a.d, b = lane / D, d = lane % D;
    const float u = a.in[3][d], w = a.in[4][d];
    for (int64_t t = 0; t < L; ++t) {
        const int64_t x_at = (b * L + t) * D + d, s0 = (b * (L + 1) + t) * D + d, s1 = s0 + D;
        const float r = logistic(a.in[0][x_at]), k = a.in[1][x_at], v = a.in[2][x_at];
        a.out[0][x_at] = r;
        const float ap = a.out[6][s0], bp = a.out[7][s0];
        const float e = expf(u + k), num = ap + e * v, den = bp + e, wkv = num / den;
        a.out[1][x_at] = e;
        a.out[2][x_at] = num;
        a.out[3][x_at] = den;
        a.out[4][x_at] = wkv;
        const float decay = expf(-w), kk = expf(k);
        a.out[5][x_at] = kk;
        a.out[6][s1] = decay * ap + kk * v;
        a.out[7][s1] = decay * bp + kk;
        a.out[8][x_at] = r * wkv;
    }
}

__device__ void rwkv_backward(const pxk_ssm_args& a, int64_t lane) {
    const int64_t L = a.l, D = a.d, b = lane / D, d = lane % D;
    const float w = a.in[10][d];
    float ca = 0.0f, cb = 0.0f;  // carries into a_{t+1}, b_{t+1}
    for (int64_t t = L - 1; t >= 0; --t) {
        const int64_t x_at = (b * L + t) * D + d, s0 = (b * (L + 1) + t) * D + d;
        const float r = a.in[1][x_at], v = a.in[2][x_at], e = a.in[3][x_at], kk = a.in[4][x_at];
        const float num = a.in[5][x_at], den = a.in[6][x_at], ap = a.in[7][s0], bp = a.in[8][s0];
        const float decay = expf(-w), g = a.in[0][x_at];
        const float dr = g * a.in[9][x_at], dwkv = g * r;
        const float dnum = dwkv / den, dden = -dwkv * num / (den * den);
        float dap = dnum, dbp = dden;
        const float de = dnum * v + dden;
        float dv = dnum * e;
        float dk = de * e;
        a.out[3][x_at] = de * e;
        const float from_a = ca * ap;
        dap += ca * decay;
        float dkk = ca * v;
        dv += ca * kk;
        const float from_b = cb * bp;
        dbp += cb * decay;
        dkk += cb;
        a.out[4][x_at] = (from_a + from_b) * (-decay);
        dk += dkk * kk;
        ca = dap;
        cb = dbp;
        a.out[1][x_at] = dk;
        a.out[2][x_at] = dv;
        a.out[0][x_at] = dr * r * (1.0f - r);
    }
}

__device__ void rwkv_lrp(const pxk_ssm_args& a, int64_t lane) {
    const int64_t L = a.l, D = a.d, b = lane / D, d = lane % D;
    const float w = a.in[7][d];
    float ra = 0.0f;  // relevance of a_{t+1}
    for (int64_t t = L - 1; t >= 0; --t) {
        const int64_t x_at = (b * L + t) * D + d, s0 = (b * (L + 1) + t) * D + d;
        const float rw = a.in[0][x_at], ap = a.in[1][s0], an = a.in[1][s0 + D], den = a.in[2][x_at];
        const float e = a.in[3][x_at], v = a.in[4][x_at], decay = expf(-w), kk = a.in[6][x_at];
        const float dw = stab(a.in[5][x_at], a.eps), dn = stab(an, a.eps);
        const float a_read = (ap / den / dw) * rw, v_read = (e * v / den / dw) * rw;
        const float a_state = (decay * ap / dn) * ra, v_state = (kk * v / dn) * ra;
        ra = a_read + a_state;
        a.out[0][x_at] = v_read + v_state;
    }
}

__device__ void retnet_forward(const pxk_ssm_args& a, int64_t lane) {
    const int64_t L = a.l, D = a.d, K = a.s, b = lane / D, j = lane % D;
    for (int64_t t = 0; t < L; ++t) {
        float acc = 0.0f;
        for (int64_t i = 0; i < K; ++i) {
            const float sc = a.gamma * a.out[0][((b * (L + 1) + t) * K + i) * D + j] +
                             a.in[1][(b * L + t) * K + i] * a.in[2][(b * L + t) * D + j];
            a.out[0][((b * (L + 1) + t + 1) * K + i) * D + j] = sc;
            acc += a.in[0][(b * L + t) * K + i] * sc;
        }
        a.out[1][(b * L + t) * D + j] = acc;
    }
}

__device__ void ssm_lane(int op, const pxk_ssm_args& a, int64_t lane) {
    const int64_t L = a.l, D = a.d, K = a.s;
    switch (op) {
        case 0: mamba_forward(a, lane); return;
        case 1: mamba_backward(a, lane); return;
        case 2: mamba_grad_bc(a, lane); return;
        case 3: mamba_lrp(a, lane); return;
        case 4: {  // RWKV token shift, x_{-1} = 0
            const int64_t t = (lane / D) % L, e = lane % D;
            const float xc = a.in[0][lane], xp = t > 0 ? a.in[0][lane - D] : 0.0f;
            for (int m = 0; m < 3; ++m) a.out[m][lane] = a.in[1 + m][e] * xc + (1.0f - a.in[1 + m][e]) * xp;
            return;
        }
        case 5: rwkv_forward(a, lane); return;
        case 6: rwkv_backward(a, lane); return;
        case 7: {  // token-shift backward: step t+1's x_{t-1} share first, then the direct share
            const int64_t t = (lane / D) % L, d = lane % D;
            const float diff = a.in[0][lane] - (t > 0 ? a.in[0][lane - D] : 0.0f);
            for (int m = 0; m < 3; ++m) a.out[1 + m][lane] = a.in[1 + m][lane] * diff;
            const float mr = a.in[4][d], mk = a.in[5][d], mv = a.in[6][d];
            float acc = 0.0f;
            if (t + 1 < L) {
                const int64_t nx = lane + D;
                acc += a.in[1][nx] * (1.0f - mr) + a.in[2][nx] * (1.0f - mk) + a.in[3][nx] * (1.0f - mv);
            }
            acc += a.in[1][lane] * mr + a.in[2][lane] * mk + a.in[3][lane] * mv;
            a.out[0][lane] = acc;
            return;
        }
        case 8: rwkv_lrp(a, lane); return;
        case 9: {  // value token-shift epsilon rule, gathered in the same order
            const int64_t t = (lane / D) % L, e = lane % D;
            const float mu = a.in[3][e], x = a.in[0][lane];
            float acc = 0.0f;
            if (t + 1 < L) {
                const float xn = a.in[1][lane + D];
                acc += ((1.0f - mu) * x / stab(xn, a.eps)) * (xn * a.in[2][lane + D]);
            }
            const float xv = a.in[1][lane];
            acc += (mu * x / stab(xv, a.eps)) * (xv * a.in[2][lane]);
            a.out[0][lane] = acc;
            return;
        }
        case 10: a.out[0][lane] = a.in[0][lane] / stab(a.in[1][lane], a.eps); return;
        case 11: retnet_forward(a, lane); return;
        case 12: {  // undecayed state gradient over t descending, carry dS gamma
            const int64_t j = lane % D, bi = lane / D, b = bi / K, i = bi % K;
            float carry = 0.0f;
            for (int64_t t = L - 1; t >= 0; --t) {
                const float ds = a.in[0][(b * L + t) * D + j] * a.in[1][(b * L + t) * K + i] + carry;
                a.out[0][((b * L + t) * K + i) * D + j] = ds;
                carry = ds * a.gamma;
            }
            return;
        }
        case 13: {  // dQ from the readout, dK from the outer product, j ascending
            const int64_t bt = lane / K, i = lane % K, b = bt / L, t = bt % L;
            float dq = 0.0f, dk = 0.0f;
            for (int64_t j = 0; j < D; ++j) dq += a.in[0][bt * D + j] * a.in[1][((b * (L + 1) + t + 1) * K + i) * D + j];
            for (int64_t j = 0; j < D; ++j) dk += a.in[2][lane * D + j] * a.in[3][bt * D + j];
            a.out[0][lane] = dq;
            a.out[1][lane] = dk;
            return;
        }
        case 14: {  // dV over i ascending
            const int64_t bt = lane / D, j = lane % D;
            float acc = 0.0f;
            for (int64_t i = 0; i < K; ++i) acc += a.in[0][(bt * K + i) * D + j] * a.in[1][bt * K + i];
            a.out[0][lane] = acc;
            return;
        }
        case 15: {  // QK and the decayed scores, zero above the diagonal; the decay multiplied down from t
            const int64_t bt = lane / L, s = lane % L, b = bt / L, t = bt % L;
            if (s > t) {
                a.out[0][lane] = 0.0f;
                a.out[1][lane] = 0.0f;
                return;
            }
            float dot = 0.0f;
            for (int64_t i = 0; i < K; ++i) dot += a.in[0][bt * K + i] * a.in[1][(b * L + s) * K + i];
            float decay = 1.0f;
            for (int64_t u = t; u > s; --u) decay *= a.gamma;
            a.out[0][lane] = dot;
            a.out[1][lane] = decay * dot;
            return;
        }
        case 16: {  // Y = G V over s <= t
            const int64_t bt = lane / D, j = lane % D, b = bt / L, t = bt % L;
            float acc = 0.0f;
            for (int64_t s = 0; s <= t; ++s) acc += a.in[0][bt * L + s] * a.in[1][(b * L + s) * D + j];
            a.out[0][lane] = acc;
            return;
        }
        case 17: {  // the Q/K/V projections' epsilon rule into one input slot: Q then K per i, then V per j
            const int64_t bt = lane / D, e = lane % D;
            const float x = a.in[0][lane];
            float acc = 0.0f;
            for (int64_t i = 0; i < K; ++i) {
                acc += (x * a.in[1][e * K + i] / stab(a.in[4][bt * K + i], a.eps)) * a.in[7][bt * K + i];
                acc += (x * a.in[2][e * K + i] / stab(a.in[5][bt * K + i], a.eps)) * a.in[8][bt * K + i];
            }
            for (int64_t j = 0; j < D; ++j)
                acc += (x * a.in[3][e * D + j] / stab(a.in[6][bt * D + j], a.eps)) * a.in[9][bt * D + j];
            a.out[0][lane] = acc;
            return;
        }
        default: {  // sum over t descending, then the batch ascending (a parameter gradient's order)
            float acc = 0.0f;
            for (int64_t t = L - 1; t >= 0; --t)
                for (int64_t b = 0; b < a.n; ++b) acc += a.in[0][(b * L + t) * D + lane];
            a.out[0][lane] = acc;
            return;
        }
    }
}

// ---- reinforcement-learning rows (rl_math.hpp) -------------------------------------------------------
// Stabilised softmax of logits row b into probs; returns the log-probability of the row's action.
__device__ float softmax_row(const float* logits, const float* action, float* probs, int64_t cols, int64_t b) {
    const float* row = logits + b * cols;
    float mx = row[0];
    for (int64_t k = 1; k < cols; ++k) mx = lmax(mx, row[k]);
    float es = 0.0f;
    for (int64_t k = 0; k < cols; ++k) es += expf(row[k] - mx);
    const float lse = logf(es);
    for (int64_t k = 0; k < cols; ++k) probs[b * cols + k] = expf(row[k] - mx) / es;
    return row[static_cast<int64_t>(action[b])] - mx - lse;
}

__device__ void rl_row(int op, const pxk_rl_args& a, int64_t b) {
    const int64_t C = a.cols;
    switch (op) {
        case 0: {  // DQN loss: squared TD error of the taken action
            const float diff = a.in[0][b * C + static_cast<int64_t>(a.in[1][b])] - a.in[2][b];
            a.out[0][b] = diff * diff;
            return;
        }
        case 1: {  // DQN gradient: the taken action's element only
            const int64_t k = static_cast<int64_t>(a.in[1][b]);
            a.out[0][b * C + k] = a.scale * (a.in[0][b * C + k] - a.in[2][b]);
            return;
        }
        case 2:  // policy-gradient loss
            a.out[1][b] = -softmax_row(a.in[0], a.in[1], a.out[0], C, b) * a.in[2][b];
            return;
        case 3: {  // policy-gradient gradient: weight (p - 1{k = a_b})
            const int64_t act = static_cast<int64_t>(a.in[1][b]);
            const float wgt = a.in[2][b] * a.scale;
            for (int64_t k = 0; k < C; ++k) a.out[0][b * C + k] = wgt * (a.in[0][b * C + k] - (k == act ? 1.0f : 0.0f));
            return;
        }
        case 4: {  // PPO clipped surrogate
            const float ratio = expf(softmax_row(a.in[0], a.in[1], a.out[0], C, b) - a.in[2][b]);
            const float adv = a.in[3][b];
            a.out[1][b] = -lmin(ratio * adv, lmin(lmax(ratio, a.lower), a.upper) * adv);
            const bool out_of_range = (adv >= 0.0f && ratio > a.upper) || (adv < 0.0f && ratio < a.lower);
            a.out[2][b] = ratio;
            a.out[3][b] = out_of_range ? 0.0f : 1.0f;
            return;
        }
        case 5: {  // PPO gradient: weight (1{k = a_b} - p)
            const int64_t act = static_cast<int64_t>(a.in[1][b]);
            const float wgt = -a.in[4][b] * a.in[2][b] * a.in[3][b] * a.scale;
            for (int64_t k = 0; k < C; ++k) a.out[0][b * C + k] = wgt * ((k == act ? 1.0f : 0.0f) - a.in[0][b * C + k]);
            return;
        }
        case 6: {  // (double) DQN target: argmax of the selection row (first maximum) read in the evaluation row
            const float* sel = a.in[0] + b * C;
            int64_t best = 0;
            for (int64_t k = 1; k < C; ++k)
                if (sel[k] > sel[best]) best = k;
            a.out[0][b] = a.in[2][b] + a.gamma * (1.0f - a.in[3][b]) * a.in[1][b * C + best];
            return;
        }
        case 7:  // Polyak blend, one element
            a.out[0][b] = a.tau * a.in[0][b] + (1.0f - a.tau) * a.in[1][b];
            return;
        default: {  // token cross-entropy with on-device target checks; statistics row of four
            const float e = a.in[1][b], rounded = roundf(e);
            float index = 0.0f, weight = 0.0f, bad_int = 0.0f, bad_range = 0.0f;
            if (!(fabsf(e - rounded) <= 1e-4f)) {
                bad_int = 1.0f;
            } else {
                const int64_t i = static_cast<int64_t>(rounded);
                if (i != a.ignore_index) {
                    if (i < 0 || i >= C) {
                        bad_range = 1.0f;
                    } else {
                        index = static_cast<float>(i);
                        weight = 1.0f;
                    }
                }
            }
            a.out[2][b] = index;
            a.out[3][b] = weight;
            const float lp = softmax_row(a.in[0], a.out[2], a.out[0], C, b);
            float* st = a.out[1] + b * 4;
            st[0] = -lp * weight;
            st[1] = weight;
            st[2] = bad_int;
            st[3] = bad_range;
            return;
        }
    }
}

}  // namespace
}  // namespace pxk

extern "C" {

int pxk_ssm_pass(int op, const pxk_ssm_args* args, void* stream) {
    if (op < 0 || op > 18 || args == nullptr) return fail(PXK_ERR_INVALID, "pxk_ssm_pass: unknown op");
    const pxk_ssm_args a = *args;
    if (a.n < 0 || a.l < 0 || a.d < 0 || a.s < 0) return fail(PXK_ERR_INVALID, "pxk_ssm_pass: negative size");
    return run_lanes("pxk_ssm_pass", ssm_lanes(op, a), stream, [=] __device__(int64_t lane) { ssm_lane(op, a, lane); });
}

int pxk_rl_rows(int op, const pxk_rl_args* args, void* stream) {
    if (op < 0 || op > 8 || args == nullptr) return fail(PXK_ERR_INVALID, "pxk_rl_rows: unknown op");
    const pxk_rl_args a = *args;
    if (a.cols <= 0 && op != 7) return a.rows == 0 ? PXK_OK : fail(PXK_ERR_INVALID, "pxk_rl_rows: no columns");
    return run_lanes("pxk_rl_rows", a.rows, stream, [=] __device__(int64_t b) { rl_row(op, a, b); });
}

}  // extern "C"
