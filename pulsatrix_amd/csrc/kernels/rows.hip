// rows.hip -- row-wise and attention kernels for gfx950 (include/pxk.h).
//
// Row reductions run one wave64 per row (four rows per 256-thread workgroup) with lane-strided
// loads and a cross-lane shuffle tree, so each row's sum or max is a fixed-order reduction (the
// same every run). The reference's HIP backend ran these one thread per row (gpu_kernels.cuh:
// 315-334, 609-615), leaving almost all of a 256-CU device idle.
#include <algorithm>
#include <cstring>

#include "common.hpp"

namespace pxk {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / kWave;

__device__ __forceinline__ int64_t row_id() {
    return static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
}
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// ---- RMSNorm (row_math.hpp:59-71) -------------------------------------------------------------
__global__ void __launch_bounds__(kThreads) rms_norm_kernel(const float* in, const float* gamma, float* out,
                                                            float* row_rms, int64_t rows, int64_t cols, float eps) {
    const int64_t r = row_id();
    if (r >= rows) return;
    const int lane = lane_id();
    const float* x = in + r * cols;
    float ss = 0.0f;
    for (int64_t i = lane; i < cols; i += kWave) ss += x[i] * x[i];
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / static_cast<float>(cols) + eps);
    if (row_rms && lane == 0) row_rms[r] = rms;
    float* o = out + r * cols;
    for (int64_t i = lane; i < cols; i += kWave) o[i] = gamma[i] * x[i] / rms;
}

// The same row with 128-bit accesses and the row held in registers between the two passes: lane l
// owns float4 columns l, l + 64, ..., so x is read from HBM once. Needs cols % 4 == 0, 16-byte
// aligned rows, and cols <= 256 * NV. NT: streaming (non-temporal) cache policy for x and out, for
// tensors far larger than the caches.
template <int NV, bool NT>
__global__ void __launch_bounds__(kThreads) rms_norm_vec_kernel(const float* in, const float* gamma, float* out,
                                                                float* row_rms, int64_t rows, int cols4, float eps) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int64_t r = row_id();
    if (r >= rows) return;
    const int lane = lane_id();
    const f4* x = reinterpret_cast<const f4*>(in) + r * cols4;
    f4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = lane + j * kWave;
        if (c < cols4) {
            if constexpr (NT) v[j] = __builtin_nontemporal_load(x + c);
            else v[j] = x[c];
        } else {
            v[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / static_cast<float>(4 * cols4) + eps);
    if (row_rms && lane == 0) row_rms[r] = rms;
    f4* o = reinterpret_cast<f4*>(out) + r * cols4;
    const f4* g = reinterpret_cast<const f4*>(gamma);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = lane + j * kWave;
        if (c < cols4) {
            const f4 gv = g[c];
            f4 y;
            y.x = gv.x * v[j].x / rms;
            y.y = gv.y * v[j].y / rms;
            y.z = gv.z * v[j].z / rms;
            y.w = gv.w * v[j].w / rms;
            if constexpr (NT) __builtin_nontemporal_store(y, o + c);
            else o[c] = y;
        }
    }
}

// ---- a sublayer's post-norm and residual add, then the next norm (Gemma 3 sandwich blocks) --------
// y = x + g_a * a / rms(a), and yn = g_y * y / rms(y) when g_y is given: the post-attention (or
// post-MLP) RMSNorm, the residual sum and the norm that reads the sum next, each with RMSNorm's and
// the add's own expressions. One wave per row; a row of a and of y stays in registers (lane l owns
// float4 columns l, l + 64, ...).
struct NormAddArgs {
    const float* x;
    const float* a;
    const float* ga;
    float* y;
    const float* gy;
    float* yn;
    int64_t rows;
    int cols4;
    float ea, ey;
};

template <int NV>
__global__ void __launch_bounds__(kThreads) rms_norm_add_vec_kernel(const NormAddArgs g) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int64_t r = row_id();
    if (r >= g.rows) return;
    const int lane = lane_id();
    const int64_t base = r * g.cols4;
    const f4* a = reinterpret_cast<const f4*>(g.a) + base;
    const f4* x = reinterpret_cast<const f4*>(g.x) + base;
    const f4* ga = reinterpret_cast<const f4*>(g.ga);
    f4 v[NV];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = lane + j * kWave;
        v[j] = c < g.cols4 ? a[c] : f4{0.0f, 0.0f, 0.0f, 0.0f};
        ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    }
    ss = wave_sum(ss);
    const float rms_a = sqrtf(ss / static_cast<float>(4 * g.cols4) + g.ea);
    f4* y = reinterpret_cast<f4*>(g.y) + base;
    float sy = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = lane + j * kWave;
        if (c < g.cols4) {
            const f4 gv = ga[c], xv = x[c];
            f4 t;
            t.x = xv.x + gv.x * v[j].x / rms_a;
            t.y = xv.y + gv.y * v[j].y / rms_a;
            t.z = xv.z + gv.z * v[j].z / rms_a;
            t.w = xv.w + gv.w * v[j].w / rms_a;
            y[c] = t;
            v[j] = t;
            sy += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
        }
    }
    if (!g.yn) return;
    sy = wave_sum(sy);
    const float rms_y = sqrtf(sy / static_cast<float>(4 * g.cols4) + g.ey);
    const f4* gy = reinterpret_cast<const f4*>(g.gy);
    f4* yn = reinterpret_cast<f4*>(g.yn) + base;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = lane + j * kWave;
        if (c < g.cols4) {
            const f4 gv = gy[c];
            f4 t;
            t.x = gv.x * v[j].x / rms_y;
            t.y = gv.y * v[j].y / rms_y;
            t.z = gv.z * v[j].z / rms_y;
            t.w = gv.w * v[j].w / rms_y;
            yn[c] = t;
        }
    }
}

// Any width: the same steps reading the rows from memory (cols = 4 * cols4 is not assumed).
__global__ void __launch_bounds__(kThreads) rms_norm_add_kernel(const NormAddArgs g, int64_t cols) {
    const int64_t r = row_id();
    if (r >= g.rows) return;
    const int lane = lane_id();
    const float* a = g.a + r * cols;
    const float* x = g.x + r * cols;
    float* y = g.y + r * cols;
    float ss = 0.0f;
    for (int64_t i = lane; i < cols; i += kWave) ss += a[i] * a[i];
    ss = wave_sum(ss);
    const float rms_a = sqrtf(ss / static_cast<float>(cols) + g.ea);
    float sy = 0.0f;
    for (int64_t i = lane; i < cols; i += kWave) {
        const float t = x[i] + g.ga[i] * a[i] / rms_a;
        y[i] = t;
        sy += t * t;
    }
    if (!g.yn) return;
    sy = wave_sum(sy);
    const float rms_y = sqrtf(sy / static_cast<float>(cols) + g.ey);
    float* yn = g.yn + r * cols;
    for (int64_t i = lane; i < cols; i += kWave) yn[i] = g.gy[i] * y[i] / rms_y;  // own lane's writes
}

// ---- softmax_rows (cpu_backend.cpp:292-310) ---------------------------------------------------
__global__ void __launch_bounds__(kThreads) softmax_kernel(const float* in, float* out, int64_t rows, int64_t cols) {
    const int64_t r = row_id();
    if (r >= rows) return;
    const int lane = lane_id();
    const float* x = in + r * cols;
    float* y = out + r * cols;
    float mx = -INFINITY;
    for (int64_t j = lane; j < cols; j += kWave) mx = fmaxf(mx, x[j]);
    mx = wave_max(mx);
    float s = 0.0f;
    for (int64_t j = lane; j < cols; j += kWave) s += expf(x[j] - mx);
    s = wave_sum(s);
    for (int64_t j = lane; j < cols; j += kWave) y[j] = expf(x[j] - mx) / s;
}

// ---- lrp_softmax_rows (lrp_math.hpp:89-98) ----------------------------------------------------
__global__ void __launch_bounds__(kThreads) lrp_softmax_kernel(const float* x, const float* y, const float* r,
                                                               float* r_in, int64_t rows, int64_t cols) {
    const int64_t row = row_id();
    if (row >= rows) return;
    const int lane = lane_id();
    const int64_t off = row * cols;
    float s = 0.0f;
    for (int64_t j = lane; j < cols; j += kWave) s += r[off + j];
    s = wave_sum(s);
    for (int64_t j = lane; j < cols; j += kWave) r_in[off + j] = x[off + j] * (r[off + j] - y[off + j] * s);
}

__global__ void __launch_bounds__(kThreads) row_sums_kernel(const float* in, float* out, int64_t rows, int64_t cols) {
    const int64_t r = row_id();
    if (r >= rows) return;
    const int lane = lane_id();
    float s = 0.0f;
    for (int64_t j = lane; j < cols; j += kWave) s += in[r * cols + j];
    s = wave_sum(s);
    if (lane == 0) out[r] = s;
}

// ---- deterministic two-pass sum / dot ---------------------------------------------------------
constexpr int kReduceBlocks = 1024;

__device__ float block_sum(float v) {
    __shared__ float part[kThreads / kWave];
    v = wave_sum(v);
    if (lane_id() == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / kWave; ++w) t += part[w];
    return t;
}

__global__ void __launch_bounds__(kThreads) reduce_pass1(const float* a, const float* b, int64_t n, float* partials) {
    float s = 0.0f;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
        s += b ? a[i] * b[i] : a[i];
    const float t = block_sum(s);
    if (threadIdx.x == 0) partials[blockIdx.x] = t;
}

__global__ void __launch_bounds__(kThreads) reduce_pass2(const float* partials, int count, float* out) {
    float s = 0.0f;
    for (int i = threadIdx.x; i < count; i += kThreads) s += partials[i];
    const float t = block_sum(s);
    if (threadIdx.x == 0) out[0] = t;
}

// ---- attention -----------------------------------------------------------------------------------
// Keys [lo, vis) a query row i sees: all of them, the causal prefix, or its last `window` keys
// (attention_masked, row_math.hpp:117-126: j masked when j > i or j + window <= i).
__device__ __forceinline__ void visible_keys(int64_t i, int64_t L, int causal, int64_t window, int64_t& lo,
                                             int64_t& vis) {
    vis = causal ? i + 1 : L;
    lo = (causal && window > 0 && i + 1 > window) ? i + 1 - window : 0;
}

// P = softmax(scale * raw) over visible keys; masked entries of P written 0.
__global__ void __launch_bounds__(kThreads) attention_softmax_kernel(const float* raw, float* p, int64_t rows,
                                                                     int64_t L, float scale, int causal,
                                                                     int64_t window) {
    const int64_t r = row_id();
    if (r >= rows) return;
    const int lane = lane_id();
    int64_t lo, vis;
    visible_keys(r % L, L, causal, window, lo, vis);
    const float* x = raw + r * L;
    float* y = p + r * L;
    float mx = -INFINITY;
    for (int64_t j = lo + lane; j < vis; j += kWave) mx = fmaxf(mx, scale * x[j]);
    mx = wave_max(mx);
    float s = 0.0f;
    for (int64_t j = lo + lane; j < vis; j += kWave) s += expf(scale * x[j] - mx);
    s = wave_sum(s);
    for (int64_t j = lane; j < L; j += kWave) y[j] = (j >= lo && j < vis) ? expf(scale * x[j] - mx) / s : 0.0f;
}

// s = [x * (r - P * sum r)] / (2 raw + eps sign raw), x = scale * raw; 0 where masked.
__global__ void __launch_bounds__(kThreads) attention_lrp_scores_kernel(const float* r_attn, const float* p,
                                                                        const float* raw, float* s_out, int64_t rows,
                                                                        int64_t L, float scale, float eps, int causal,
                                                                        int64_t window) {
    const int64_t r = row_id();
    if (r >= rows) return;
    const int lane = lane_id();
    int64_t lo, vis;
    visible_keys(r % L, L, causal, window, lo, vis);
    const int64_t off = r * L;
    float sum = 0.0f;
    for (int64_t j = lo + lane; j < vis; j += kWave) sum += r_attn[off + j];
    sum = wave_sum(sum);
    for (int64_t j = lane; j < L; j += kWave) {
        float v = 0.0f;
        if (j >= lo && j < vis) {
            const float o = raw[off + j];
            const float rs = (scale * o) * (r_attn[off + j] - p[off + j] * sum);
            v = rs / (2.0f * o + eps * ((o >= 0.0f) ? 1.0f : -1.0f));
        }
        s_out[off + j] = v;
    }
}

// RMSNorm over each head's D values of head-packed rows (QK-Norm, multihead_attention_module.cpp
// step 3): wave per (row, head); in row m, head h at in + m * ld_in + h * D.
__global__ void __launch_bounds__(kThreads) rms_norm_heads_kernel(const float* in, int64_t ld_in, float* out,
                                                                  int64_t ld_out, const float* gamma, int64_t rows,
                                                                  int64_t heads, int64_t D, float eps) {
    const int64_t r = row_id();
    if (r >= rows * heads) return;
    const int lane = lane_id();
    const int64_t m = r / heads, h = r - m * heads;
    const float* x = in + m * ld_in + h * D;
    float ss = 0.0f;
    for (int64_t i = lane; i < D; i += kWave) ss += x[i] * x[i];
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / static_cast<float>(D) + eps);
    float* o = out + m * ld_out + h * D;
    for (int64_t i = lane; i < D; i += kWave) o[i] = gamma[i] * x[i] / rms;
}

// The RoPE epsilon rule (lrp_math.hpp:104-123) on token-major head-packed rows, then the
// projection's stabilised divide: r = y * s_acc (the bilinear share, y the rotated values),
// r_in per pair from x (before rotation), and g = r_in / stab(z + bias) -- or g = r_in under
// rel_only. One thread per (row, head, pair).
struct RopeRelArgs {
    const float* acc;  // (rows, heads*D) sums s @ K for the queries
    int64_t ld_acc;
    const float* x;
    int64_t ldx;
    const float* y;
    int64_t ldy;
    const float* z;
    int64_t ldz;
    const float* bias;
    const float* cos_t;
    const float* sin_t;
    float* g;
    int64_t ldg;
    int64_t rows, L, heads, D;
    float eps;
    int rotate_half, rel_only;
};

__global__ void __launch_bounds__(kThreads) rope_rel_rows_kernel(const RopeRelArgs a) {
    const int64_t half = a.D / 2, n = a.rows * a.heads * half;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; t < n; t += stride) {
        const int64_t i = t % half, h = (t / half) % a.heads, m = t / (half * a.heads);
        const int64_t pos = m % a.L;
        const int64_t lo = h * a.D + (a.rotate_half ? i : 2 * i), hi = h * a.D + (a.rotate_half ? i + half : 2 * i + 1);
        const float y_lo = a.y[m * a.ldy + lo], y_hi = a.y[m * a.ldy + hi];
        const float r_lo = y_lo * a.acc[m * a.ld_acc + lo], r_hi = y_hi * a.acc[m * a.ld_acc + hi];
        const float c = a.cos_t[pos * half + i], sn = a.sin_t[pos * half + i];
        const float d0 = stab(y_lo, a.eps), d1 = stab(y_hi, a.eps);
        const float x_lo = a.x[m * a.ldx + lo], x_hi = a.x[m * a.ldx + hi];
        float in_lo = 0.0f, in_hi = 0.0f;
        in_lo += (x_lo * c / d0) * r_lo;
        in_lo += (x_lo * sn / d1) * r_hi;
        in_hi += (x_hi * -sn / d0) * r_lo;
        in_hi += (x_hi * c / d1) * r_hi;
        if (a.rel_only) {
            a.g[m * a.ldg + lo] = in_lo;
            a.g[m * a.ldg + hi] = in_hi;
        } else {
            const float zl = a.bias ? a.z[m * a.ldz + lo] + a.bias[lo] : a.z[m * a.ldz + lo];
            const float zh = a.bias ? a.z[m * a.ldz + hi] + a.bias[hi] : a.z[m * a.ldz + hi];
            a.g[m * a.ldg + lo] = in_lo / stab(zl, a.eps);
            a.g[m * a.ldg + hi] = in_hi / stab(zh, a.eps);
        }
    }
}

// RoPE of q and k from the packed projection buffer into head-packed (rows, heads*D) outputs.
__global__ void __launch_bounds__(kThreads) rope_qk_kernel(const float* q_in, const float* k_in, int64_t ld,
                                                           float* q_out, float* k_out, int64_t ld_out,
                                                           const float* cos_t,
                                                           const float* sin_t, int64_t rows, int64_t L, int64_t H,
                                                           int64_t Hkv, int64_t D, int rotate_half) {
    const int64_t half = D / 2;
    const int64_t nq = rows * H * half, nk = rows * Hkv * half;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; t < nq + nk; t += stride) {
        const bool is_q = t < nq;
        const int64_t u = is_q ? t : t - nq;
        const int64_t heads = is_q ? H : Hkv;
        const int64_t i = u % half, h = (u / half) % heads, row = u / (half * heads);
        const int64_t pos = row % L;
        const int64_t lo = rotate_half ? i : 2 * i, hi = rotate_half ? i + half : 2 * i + 1;
        const float* src = (is_q ? q_in : k_in) + row * ld + h * D;
        float* dst = (is_q ? q_out : k_out) + row * ld_out + h * D;
        const float c = cos_t[pos * half + i], s = sin_t[pos * half + i];
        const float x0 = src[lo], x1 = src[hi];
        dst[lo] = x0 * c - x1 * s;
        dst[hi] = x0 * s + x1 * c;
    }
}

__global__ void __launch_bounds__(kThreads) rope_rotate_kernel(const float* in, const float* cos_t, const float* sin_t,
                                                               float* out, int64_t slices, int64_t L, int64_t D,
                                                               int inverse, int rotate_half) {
    const int64_t half = D / 2, n = slices * L * half;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; t < n; t += stride) {
        const int64_t i = t % half, row = t / half, pos = row % L;
        const int64_t lo = row * D + (rotate_half ? i : 2 * i), hi = row * D + (rotate_half ? i + half : 2 * i + 1);
        const float c = cos_t[pos * half + i], s = sin_t[pos * half + i];
        const float x0 = in[lo], x1 = in[hi];
        if (inverse) {
            out[lo] = x0 * c + x1 * s;
            out[hi] = -x0 * s + x1 * c;
        } else {
            out[lo] = x0 * c - x1 * s;
            out[hi] = x0 * s + x1 * c;
        }
    }
}

// lrp_math.hpp:104-123, one thread per pair.
__global__ void __launch_bounds__(kThreads) lrp_rope_kernel(const float* x, const float* y, const float* r,
                                                            const float* cos_t, const float* sin_t, float* r_in,
                                                            int64_t slices, int64_t L, int64_t D, float eps,
                                                            int rotate_half) {
    const int64_t half = D / 2, n = slices * L * half;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; t < n; t += stride) {
        const int64_t i = t % half, row = t / half, pos = row % L;
        const int64_t lo = row * D + (rotate_half ? i : 2 * i), hi = row * D + (rotate_half ? i + half : 2 * i + 1);
        const float c = cos_t[pos * half + i], s = sin_t[pos * half + i];
        const float d0 = stab(y[lo], eps), d1 = stab(y[hi], eps);
        float rl = 0.0f, rh = 0.0f;
        rl += (x[lo] * c / d0) * r[lo];
        rh += (x[hi] * -s / d0) * r[lo];
        rl += (x[lo] * s / d1) * r[hi];
        rh += (x[hi] * c / d1) * r[hi];
        r_in[lo] = rl;
        r_in[hi] = rh;
    }
}

__global__ void __launch_bounds__(kThreads) permute_kernel(const float* in, float* out, int64_t d0, int64_t d1,
                                                           int64_t d2, int64_t d3) {
    const int64_t n = d0 * d1 * d2 * d3, stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; t < n; t += stride) {
        // t indexes the output (a, c, b, e)
        const int64_t e = t % d3, b = (t / d3) % d1, c = (t / (d3 * d1)) % d2, a = t / (d3 * d1 * d2);
        out[t] = in[((a * d1 + b) * d2 + c) * d3 + e];
    }
}

__global__ void __launch_bounds__(kThreads) mask_fill_kernel(float* scores, const float* keep, int64_t batch,
                                                             int64_t heads, int64_t q_len, int64_t k_len, int causal,
                                                             int64_t q_offset, int64_t window, float value) {
    const int64_t n = batch * heads * q_len * k_len, stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; t < n; t += stride) {
        const int64_t j = t % k_len, i = (t / k_len) % q_len, b = t / (k_len * q_len * heads);
        bool masked = causal && j > i + q_offset;  // row_math.hpp:117-126
        masked = masked || (causal && window > 0 && j + window <= i + q_offset);
        masked = masked || (keep != nullptr && keep[b * k_len + j] == 0.0f);
        if (masked) scores[t] = value;
    }
}

// ---- LM seeding --------------------------------------------------------------------------------
struct Targets {
    int64_t t[64];
};

constexpr int kSeedThreads = 1024;

// One workgroup per sequence scans the last position's logits: each thread keeps the first
// maximum of its strided share (indices ascending), loading eight values ahead of the compares so
// the scan is not one memory round trip per element; the shares then merge in LDS, larger value
// first and the lower index on ties.
__global__ void __launch_bounds__(kSeedThreads) lm_seed_kernel(const float* logits, int64_t L, int64_t V,
                                                               int use_given, Targets given, int64_t* targets_out,
                                                               float* seed, int unit) {
    const int64_t n = blockIdx.x;
    const float* row = logits + (n * L + (L - 1)) * V;
    __shared__ float bv[kSeedThreads];
    __shared__ int64_t bi[kSeedThreads];
    float best = -INFINITY;
    int64_t idx = V;  // "none yet"
    if (use_given) {
        if (threadIdx.x == 0) {
            best = row[given.t[n]];
            idx = given.t[n];
        }
    } else {
        constexpr int kAhead = 8;
        for (int64_t j0 = threadIdx.x; j0 < V; j0 += static_cast<int64_t>(kAhead) * kSeedThreads) {
            float v[kAhead];
#pragma unroll
            for (int u = 0; u < kAhead; ++u) {
                const int64_t j = j0 + static_cast<int64_t>(u) * kSeedThreads;
                v[u] = row[j < V ? j : V - 1];
            }
#pragma unroll
            for (int u = 0; u < kAhead; ++u) {  // j ascends: ties keep the first index
                const int64_t j = j0 + static_cast<int64_t>(u) * kSeedThreads;
                if (j < V && (idx == V || v[u] > best)) {
                    best = v[u];
                    idx = j;
                }
            }
        }
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (int s = kSeedThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            const float ov = bv[threadIdx.x + s];
            const int64_t oi = bi[threadIdx.x + s];
            const float cv = bv[threadIdx.x];
            const int64_t ci = bi[threadIdx.x];
            // larger value wins; equal values keep the lower index; "none" (index V) always loses
            const bool take = (ci == V) || (oi != V && (ov > cv || (ov == cv && oi < ci)));
            if (take) {
                bv[threadIdx.x] = ov;
                bi[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int64_t t = bi[0];
        targets_out[n] = t;
        if (seed) seed[(n * L + (L - 1)) * V + t] = unit ? 1.0f : row[t];
    }
}

// The tied head's epsilon rule for a seed that is one-hot at the last position of each sequence
// (tied_lm_head_module.cpp:76-111 through lrp_rules::epsilon_with_bias): g = R / stab(z) is zero
// except at (row, target), so (g E)[row, :] = g_t * E[t, :] and every other row is exactly zero. One
// workgroup per row; the seeded row reads its target (written by lm_seed_kernel), its logit and
// E's row t. With a residual split the row's relevance r becomes r_a = a / stab(a + b) * r and
// r_b = b / stab(a + b) * r (lrp_residual_split, lrp_math.hpp:33-38), with s = a + b as the forward
// stored it; zero rows split into zeros.
struct SeedHeadArgs {
    const float* logits;
    const float* x;
    const float* e;
    const int64_t* targets;
    float* r;
    const float* a;
    const float* b;
    const float* s;
    float* r_a;
    float* r_b;
    const float* b_den;
    const float* b_den_bias;
    int64_t l, vocab, d;
    float eps;
    int unit;
};

__global__ void __launch_bounds__(kThreads) seed_head_rows_kernel(const SeedHeadArgs g) {
    const int64_t row = blockIdx.x;
    const bool seeded = row % g.l == g.l - 1;
    const int64_t off = row * g.d;
    float gt = 0.0f;
    const float* er = nullptr;
    if (seeded) {
        const int64_t t = g.targets[row / g.l];
        const float z = g.logits[row * g.vocab + t];
        gt = (g.unit ? 1.0f : z) / stab(z, g.eps);
        er = g.e + t * g.d;
    }
    for (int64_t j = threadIdx.x; j < g.d; j += kThreads) {
        const float r = seeded ? g.x[off + j] * (gt * er[j]) : 0.0f;
        if (g.r_a) {
            if (seeded) {
                const float den = stab(g.s[off + j], g.eps);
                g.r_a[off + j] = (g.a[off + j] / den) * r;
                float rb = (g.b[off + j] / den) * r;
                if (g.b_den) rb = rb / stab(g.b_den_bias ? g.b_den[off + j] + g.b_den_bias[j] : g.b_den[off + j], g.eps);
                g.r_b[off + j] = rb;
            } else {
                g.r_a[off + j] = 0.0f;
                g.r_b[off + j] = 0.0f;
            }
        } else {
            g.r[off + j] = r;
        }
    }
}

template <bool NT>
void launch_rms_vec(int64_t nv, dim3 grid, dim3 block, hipStream_t st, const float* in, const float* gamma, float* out,
                    float* row_rms, int64_t rows, int cols4, float eps) {
    if (nv <= 2)
        PXK_LAUNCH((rms_norm_vec_kernel<2, NT>), grid, block, 0, st, in, gamma, out, row_rms, rows, cols4, eps);
    else if (nv <= 3)
        PXK_LAUNCH((rms_norm_vec_kernel<3, NT>), grid, block, 0, st, in, gamma, out, row_rms, rows, cols4, eps);
    else if (nv <= 4)
        PXK_LAUNCH((rms_norm_vec_kernel<4, NT>), grid, block, 0, st, in, gamma, out, row_rms, rows, cols4, eps);
    else if (nv <= 8)
        PXK_LAUNCH((rms_norm_vec_kernel<8, NT>), grid, block, 0, st, in, gamma, out, row_rms, rows, cols4, eps);
    else
        PXK_LAUNCH((rms_norm_vec_kernel<16, NT>), grid, block, 0, st, in, gamma, out, row_rms, rows, cols4, eps);
}

unsigned rows_grid(int64_t rows) { return static_cast<unsigned>(cdiv(rows, kRowsPerBlock)); }

bool sizes_ok(const char* what, int64_t a, int64_t b, int* rc) {
    if (a < 0 || b < 0) {
        *rc = fail(PXK_ERR_INVALID, "%s: negative size", what);
        return false;
    }
    *rc = PXK_OK;
    return a > 0 && b > 0;
}

}  // namespace
}  // namespace pxk

using namespace pxk;

extern "C" {

int pxk_rms_norm_forward(const float* in, const float* gamma, float* out, float* row_rms, int64_t rows, int64_t cols,
                         float eps, void* stream) {
    int rc;
    if (!sizes_ok("pxk_rms_norm_forward", rows, cols, &rc)) return rc;
    const dim3 grid(rows_grid(rows)), block(kThreads);
    const int64_t c4 = cols / 4, nv = cdiv(c4, kWave);
    if (cols % 4 == 0 && nv <= 16 && aligned16(in) && aligned16(gamma) && aligned16(out)) {
        const int cols4 = static_cast<int>(c4);
        if (rows * cols >= (int64_t{1} << 22))
            launch_rms_vec<true>(nv, grid, block, S(stream), in, gamma, out, row_rms, rows, cols4, eps);
        else
            launch_rms_vec<false>(nv, grid, block, S(stream), in, gamma, out, row_rms, rows, cols4, eps);
    } else {
        PXK_LAUNCH(rms_norm_kernel, grid, block, 0, S(stream), in, gamma, out, row_rms, rows, cols, eps);
    }
    return launched("pxk_rms_norm_forward");
}

int pxk_rms_norm_add(const float* x, const float* a, const float* gamma_a, float eps_a, float* y,
                     const float* gamma_y, float eps_y, float* y_norm, int64_t rows, int64_t cols, void* stream) {
    int rc;
    if (!sizes_ok("pxk_rms_norm_add", rows, cols, &rc)) return rc;
    if (!x || !a || !gamma_a || !y || (y_norm && !gamma_y))
        return fail(PXK_ERR_INVALID, "pxk_rms_norm_add: a required operand is NULL");
    const NormAddArgs g{x, a, gamma_a, y, gamma_y, y_norm, rows, static_cast<int>(std::min<int64_t>(cols / 4, 1 << 30)),
                        eps_a, eps_y};
    const dim3 grid(rows_grid(rows)), block(kThreads);
    const int64_t nv = cdiv(cols / 4, kWave);
    const bool vec = cols % 4 == 0 && nv <= 8 && aligned16(x) && aligned16(a) && aligned16(gamma_a) && aligned16(y) &&
                     (!y_norm || (aligned16(gamma_y) && aligned16(y_norm)));
    if (vec && nv <= 2)
        PXK_LAUNCH(rms_norm_add_vec_kernel<2>, grid, block, 0, S(stream), g);
    else if (vec && nv <= 4)
        PXK_LAUNCH(rms_norm_add_vec_kernel<4>, grid, block, 0, S(stream), g);
    else if (vec)
        PXK_LAUNCH(rms_norm_add_vec_kernel<8>, grid, block, 0, S(stream), g);
    else
        PXK_LAUNCH(rms_norm_add_kernel, grid, block, 0, S(stream), g, cols);
    return launched("pxk_rms_norm_add");
}

int pxk_softmax_rows(const float* in, float* out, int64_t rows, int64_t cols, void* stream) {
    int rc;
    if (!sizes_ok("pxk_softmax_rows", rows, cols, &rc)) return rc;
    PXK_LAUNCH(softmax_kernel, dim3(rows_grid(rows)), dim3(kThreads), 0, S(stream), in, out, rows, cols);
    return launched("pxk_softmax_rows");
}

int pxk_lrp_softmax_rows(const float* x, const float* y, const float* r, float* r_in, int64_t rows, int64_t cols,
                         void* stream) {
    int rc;
    if (!sizes_ok("pxk_lrp_softmax_rows", rows, cols, &rc)) return rc;
    PXK_LAUNCH(lrp_softmax_kernel, dim3(rows_grid(rows)), dim3(kThreads), 0, S(stream), x, y, r, r_in, rows,
                       cols);
    return launched("pxk_lrp_softmax_rows");
}

int pxk_row_sums(const float* in, float* out, int64_t rows, int64_t cols, void* stream) {
    int rc;
    if (!sizes_ok("pxk_row_sums", rows, cols, &rc)) {
        if (rc == PXK_OK && rows > 0) return pxk_fill(out, 0.0f, rows, stream);
        return rc;
    }
    PXK_LAUNCH(row_sums_kernel, dim3(rows_grid(rows)), dim3(kThreads), 0, S(stream), in, out, rows, cols);
    return launched("pxk_row_sums");
}

size_t pxk_reduce_partials(int64_t) { return kReduceBlocks * sizeof(float); }

static int reduce(const char* what, const float* a, const float* b, int64_t n, float* out, float* partials,
                  void* stream) {
    if (n < 0) return fail(PXK_ERR_INVALID, "%s: negative size", what);
    if (n == 0) return pxk_fill(out, 0.0f, 1, stream);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(kReduceBlocks, cdiv(n, kThreads)));
    PXK_LAUNCH(reduce_pass1, dim3(blocks), dim3(kThreads), 0, S(stream), a, b, n, partials);
    if (const int rc = launched(what)) return rc;
    PXK_LAUNCH(reduce_pass2, dim3(1), dim3(kThreads), 0, S(stream), partials, static_cast<int>(blocks), out);
    return launched(what);
}

int pxk_sum(const float* in, int64_t n, float* out, float* partials, void* stream) {
    return reduce("pxk_sum", in, nullptr, n, out, partials, stream);
}

int pxk_dot(const float* a, const float* b, int64_t n, float* out, float* partials, void* stream) {
    return reduce("pxk_dot", a, b, n, out, partials, stream);
}

int pxk_attention_softmax(const float* raw, float* p, int64_t slices, int64_t l, float scale, int causal,
                          int64_t window, void* stream) {
    int rc;
    if (!sizes_ok("pxk_attention_softmax", slices, l, &rc)) return rc;
    if (window < 0) return fail(PXK_ERR_INVALID, "pxk_attention_softmax: negative window");
    PXK_LAUNCH(attention_softmax_kernel, dim3(rows_grid(slices * l)), dim3(kThreads), 0, S(stream), raw, p,
                       slices * l, l, scale, causal, window);
    return launched("pxk_attention_softmax");
}

int pxk_attention_lrp_scores(const float* r_attn, const float* p, const float* raw, float* s, int64_t slices,
                             int64_t l, float scale, float eps, int causal, int64_t window, void* stream) {
    int rc;
    if (!sizes_ok("pxk_attention_lrp_scores", slices, l, &rc)) return rc;
    if (window < 0) return fail(PXK_ERR_INVALID, "pxk_attention_lrp_scores: negative window");
    PXK_LAUNCH(attention_lrp_scores_kernel, dim3(rows_grid(slices * l)), dim3(kThreads), 0, S(stream), r_attn,
                       p, raw, s, slices * l, l, scale, eps, causal, window);
    return launched("pxk_attention_lrp_scores");
}

int pxk_rms_norm_heads(const float* in, int64_t ld_in, float* out, int64_t ld_out, const float* gamma, int64_t rows,
                       int64_t heads, int64_t head_dim, float eps, void* stream) {
    if (rows < 0 || heads <= 0 || head_dim <= 0 || ld_in < heads * head_dim || ld_out < heads * head_dim)
        return fail(PXK_ERR_INVALID, "pxk_rms_norm_heads: bad sizes or row strides");
    if (rows == 0) return PXK_OK;
    if (!in || !out || !gamma) return fail(PXK_ERR_INVALID, "pxk_rms_norm_heads: NULL operand");
    PXK_LAUNCH(rms_norm_heads_kernel, dim3(rows_grid(rows * heads)), dim3(kThreads), 0, S(stream), in, ld_in,
                       out, ld_out, gamma, rows, heads, head_dim, eps);
    return launched("pxk_rms_norm_heads");
}

int pxk_lrp_rope_rows(const float* acc, int64_t ld_acc, const float* x, int64_t ldx, const float* y, int64_t ldy,
                      const float* z, int64_t ldz, const float* bias, const float* cos_t, const float* sin_t, float* g,
                      int64_t ldg, int64_t rows, int64_t seq_len, int64_t heads, int64_t head_dim, float eps,
                      int rotate_half, int rel_only, void* stream) {
    const int64_t w = heads * head_dim;
    if (rows < 0 || seq_len <= 0 || heads <= 0 || head_dim <= 0 || head_dim % 2 != 0 || ld_acc < w || ldx < w ||
        ldy < w || ldg < w || (!rel_only && ldz < w))
        return fail(PXK_ERR_INVALID, "pxk_lrp_rope_rows: bad sizes or row strides");
    if (rows == 0) return PXK_OK;
    if (!acc || !x || !y || !cos_t || !sin_t || !g || (!rel_only && !z))
        return fail(PXK_ERR_INVALID, "pxk_lrp_rope_rows: a required operand is NULL");
    const RopeRelArgs a{acc, ld_acc, x, ldx, y, ldy, z, ldz, bias, cos_t, sin_t, g, ldg, rows, seq_len, heads,
                        head_dim, eps, rotate_half, rel_only};
    PXK_LAUNCH(rope_rel_rows_kernel, dim3(grid_for(rows * heads * (head_dim / 2), kThreads)), dim3(kThreads), 0,
                       S(stream), a);
    return launched("pxk_lrp_rope_rows");
}

int pxk_rope_qk(const float* q_in, const float* k_in, int64_t ld_in, float* q_out, float* k_out, int64_t ld_out,
                const float* cos_t, const float* sin_t, int64_t rows, int64_t seq_len, int64_t heads, int64_t kv_heads,
                int64_t head_dim, int rotate_half, void* stream) {
    if (rows < 0 || seq_len <= 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0)
        return fail(PXK_ERR_INVALID, "pxk_rope_qk: bad sizes");
    if (ld_in < heads * head_dim || ld_in < kv_heads * head_dim || ld_out < heads * head_dim)
        return fail(PXK_ERR_INVALID, "pxk_rope_qk: row strides must hold every head");
    if (rows == 0) return PXK_OK;
    const int64_t work = rows * (heads + kv_heads) * (head_dim / 2);
    PXK_LAUNCH(rope_qk_kernel, dim3(grid_for(work, kThreads)), dim3(kThreads), 0, S(stream), q_in, k_in, ld_in,
                       q_out, k_out, ld_out, cos_t, sin_t, rows, seq_len, heads, kv_heads, head_dim, rotate_half);
    return launched("pxk_rope_qk");
}

int pxk_rope_rotate(const float* in, const float* cos_t, const float* sin_t, float* out, int64_t slices,
                    int64_t seq_len, int64_t head_dim, int inverse, int rotate_half, void* stream) {
    if (slices < 0 || seq_len < 0 || head_dim <= 0 || head_dim % 2 != 0)
        return fail(PXK_ERR_INVALID, "pxk_rope_rotate: bad sizes");
    const int64_t work = slices * seq_len * (head_dim / 2);
    if (work == 0) return PXK_OK;
    PXK_LAUNCH(rope_rotate_kernel, dim3(grid_for(work, kThreads)), dim3(kThreads), 0, S(stream), in, cos_t,
                       sin_t, out, slices, seq_len, head_dim, inverse, rotate_half);
    return launched("pxk_rope_rotate");
}

int pxk_lrp_rope(const float* x, const float* y, const float* r, const float* cos_t, const float* sin_t, float* r_in,
                 int64_t slices, int64_t seq_len, int64_t head_dim, float eps, int rotate_half, void* stream) {
    if (slices < 0 || seq_len < 0 || head_dim <= 0 || head_dim % 2 != 0)
        return fail(PXK_ERR_INVALID, "pxk_lrp_rope: bad sizes");
    const int64_t work = slices * seq_len * (head_dim / 2);
    if (work == 0) return PXK_OK;
    PXK_LAUNCH(lrp_rope_kernel, dim3(grid_for(work, kThreads)), dim3(kThreads), 0, S(stream), x, y, r, cos_t,
                       sin_t, r_in, slices, seq_len, head_dim, eps, rotate_half);
    return launched("pxk_lrp_rope");
}

int pxk_permute_0213(const float* in, float* out, int64_t d0, int64_t d1, int64_t d2, int64_t d3, void* stream) {
    if (d0 < 0 || d1 < 0 || d2 < 0 || d3 < 0) return fail(PXK_ERR_INVALID, "pxk_permute_0213: negative size");
    const int64_t n = d0 * d1 * d2 * d3;
    if (n == 0) return PXK_OK;
    PXK_LAUNCH(permute_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, S(stream), in, out, d0, d1, d2,
                       d3);
    return launched("pxk_permute_0213");
}

int pxk_attention_mask_fill(float* scores, const float* key_keep, int64_t batch, int64_t heads, int64_t q_len,
                            int64_t k_len, int causal, int64_t q_offset, int64_t window, float value, void* stream) {
    if (batch < 0 || heads < 0 || q_len < 0 || k_len < 0 || q_offset < 0 || window < 0)
        return fail(PXK_ERR_INVALID, "pxk_attention_mask_fill: negative size");
    const int64_t n = batch * heads * q_len * k_len;
    if (n == 0 || (!causal && key_keep == nullptr)) return PXK_OK;
    PXK_LAUNCH(mask_fill_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, S(stream), scores, key_keep,
                       batch, heads, q_len, k_len, causal, q_offset, window, value);
    return launched("pxk_attention_mask_fill");
}

int pxk_lm_seed(const float* logits, int64_t n, int64_t l, int64_t vocab, const int64_t* targets_in,
                int64_t* targets_out, float* seed, int unit, void* stream) {
    if (n <= 0 || l <= 0 || vocab <= 0) return fail(PXK_ERR_INVALID, "pxk_lm_seed: sizes must be positive");
    Targets given{};
    if (targets_in) {
        if (n > 64) return fail(PXK_ERR_INVALID, "pxk_lm_seed: at most 64 sequences with explicit targets");
        for (int64_t i = 0; i < n; ++i) {
            if (targets_in[i] < 0 || targets_in[i] >= vocab)
                return fail(PXK_ERR_INVALID, "pxk_lm_seed: target %lld outside the vocabulary",
                            static_cast<long long>(targets_in[i]));
            given.t[i] = targets_in[i];
        }
    }
    if (const int rc = pxk_fill(seed, 0.0f, n * l * vocab, stream)) return rc;
    PXK_LAUNCH(lm_seed_kernel, dim3(static_cast<unsigned>(n)), dim3(kSeedThreads), 0, S(stream), logits, l, vocab,
                       targets_in ? 1 : 0, given, targets_out, seed, unit);
    return launched("pxk_lm_seed");
}

int pxk_lm_seed_head_relevance(const pxk_seed_head_desc* d, void* stream) {
    if (d == nullptr) return fail(PXK_ERR_INVALID, "pxk_lm_seed_head_relevance: descriptor is NULL");
    if (d->n <= 0 || d->l <= 0 || d->vocab <= 0 || d->d <= 0)
        return fail(PXK_ERR_INVALID, "pxk_lm_seed_head_relevance: sizes must be positive");
    if (!d->logits || !d->x || !d->e || !d->targets_out)
        return fail(PXK_ERR_INVALID, "pxk_lm_seed_head_relevance: logits, x, e and targets_out are required");
    const bool split = d->r_a != nullptr;
    if (split ? (!d->r_b || !d->a || !d->b || !d->s) : d->r == nullptr)
        return fail(PXK_ERR_INVALID, "pxk_lm_seed_head_relevance: needs r, or a, b, s, r_a and r_b for the split");
    if (d->n * d->l > (int64_t{1} << 31) - 1) return fail(PXK_ERR_INVALID, "pxk_lm_seed_head_relevance: too many rows");
    if ((d->b_den || d->b_den_bias) && (!split || !d->b_den))
        return fail(PXK_ERR_INVALID, "pxk_lm_seed_head_relevance: b_den belongs to the split, its bias only with b_den");
    Targets given{};
    if (d->targets_in) {
        if (d->n > 64) return fail(PXK_ERR_INVALID, "pxk_lm_seed_head_relevance: at most 64 sequences with given targets");
        for (int64_t i = 0; i < d->n; ++i) {
            if (d->targets_in[i] < 0 || d->targets_in[i] >= d->vocab)
                return fail(PXK_ERR_INVALID, "pxk_lm_seed_head_relevance: target %lld outside the vocabulary",
                            static_cast<long long>(d->targets_in[i]));
            given.t[i] = d->targets_in[i];
        }
    }
    PXK_LAUNCH(lm_seed_kernel, dim3(static_cast<unsigned>(d->n)), dim3(kSeedThreads), 0, S(stream), d->logits, d->l,
               d->vocab, d->targets_in ? 1 : 0, given, d->targets_out, static_cast<float*>(nullptr), d->unit);
    if (const int rc = launched("pxk_lm_seed_head_relevance (targets)")) return rc;
    const SeedHeadArgs a{d->logits, d->x, d->e, d->targets_out, d->r, d->a, d->b, d->s, d->r_a, d->r_b,
                         d->b_den, d->b_den_bias, d->l, d->vocab, d->d, d->eps, d->unit};
    PXK_LAUNCH(seed_head_rows_kernel, dim3(static_cast<unsigned>(d->n * d->l)), dim3(kThreads), 0, S(stream), a);
    return launched("pxk_lm_seed_head_relevance");
}

}  // extern "C"
