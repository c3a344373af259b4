// elementwise.hip -- memory-bound elementwise kernels (include/pxk.h). Grid-stride loops over
// 128-bit (float4) accesses when every operand is 16-byte aligned, scalar otherwise; each element's
// arithmetic is the reference's expression for that element (src/cpu_backend.cpp, lrp_math.hpp).
#include <algorithm>
#include <cstdarg>
#include <cstring>
#include <string>

#include <vector>

#include "common.hpp"

namespace pxk {

namespace {
thread_local std::string g_error;
}

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int launched(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(PXK_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return PXK_OK;
}

namespace {
// The calling thread's timing window: 2 events per slot, created on first need and kept.
struct TimingWindow {
    std::vector<hipEvent_t> events;
    int used = 0;
    bool open = false;
};
thread_local TimingWindow g_timing;
}  // namespace

bool timing_slot(hipEvent_t* start, hipEvent_t* stop) {
    TimingWindow& w = g_timing;
    if (!w.open || 2 * (static_cast<size_t>(w.used) + 1) > w.events.size()) return false;
    *start = w.events[2 * w.used];
    *stop = w.events[2 * w.used + 1];
    ++w.used;
    return true;
}

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }  // cpu_backend.cpp:29

__device__ __forceinline__ float apply_op(int op, float x) {
    switch (op) {
        case 0: return fmaxf(x, 0.0f);
        case 1: return -x;
        case 2: return tanhf(x);
        case 3: return sigmoidf_(x);
        case 4: return x * sigmoidf_(x);
        case 5: return expf(x);
        case 6: {  // pointwise_math.hpp:32-36
            const float kBeta = 0.7978845608028654f, kKappa = 0.044715f;
            return 0.5f * x * (1.0f + tanhf(kBeta * (x + kKappa * x * x * x)));
        }
        default: {  // 7: exact GELU, pointwise_math.hpp:50-53
            const float kInvSqrt2 = 0.7071067811865476f;
            return 0.5f * x * (1.0f + erff(x * kInvSqrt2));
        }
    }
}

// Pointer arrays travel by value inside a small struct (kernel arguments, no device allocation).
template <int NIN, int NOUT>
struct Ptrs {
    const float* in[NIN > 0 ? NIN : 1];
    float* out[NOUT];
};

typedef float f4 __attribute__((ext_vector_type(4)));

// Streaming loads and stores (the `nt` cache policy) for operands far larger than the caches, so a
// pass over them does not evict what the next kernel re-reads; plain accesses otherwise.
template <bool NT>
__device__ __forceinline__ f4 ld4(const f4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <bool NT>
__device__ __forceinline__ void st4(f4* p, f4 v) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// Float4 elements per thread per grid-stride iteration of the vector path: all of a thread's
// loads are issued before the first use, which keeps enough bytes in flight to saturate HBM.
constexpr int kUnroll = 4;

template <typename F, int NIN, int NOUT, bool VEC, bool NT>
__global__ void __launch_bounds__(kThreads) map_kernel_p(F f, Ptrs<NIN, NOUT> p, int64_t n) {
    if constexpr (VEC) {
        const int64_t n4 = n / 4;
        const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads * kUnroll;
        for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x; base < n4;
             base += stride) {
            f4 a[kUnroll][NIN > 0 ? NIN : 1];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t i = base + u * kThreads;
                if (i < n4) {
#pragma unroll
                    for (int j = 0; j < NIN; ++j) a[u][j] = ld4<NT>(reinterpret_cast<const f4*>(p.in[j]) + i);
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t i = base + u * kThreads;
                if (i < n4) {
                    f4 o[NOUT];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float x[NIN > 0 ? NIN : 1], y[NOUT];
#pragma unroll
                        for (int j = 0; j < NIN; ++j) x[j] = a[u][j][e];
                        f(x, y);
#pragma unroll
                        for (int j = 0; j < NOUT; ++j) o[j][e] = y[j];
                    }
#pragma unroll
                    for (int j = 0; j < NOUT; ++j) st4<NT>(reinterpret_cast<f4*>(p.out[j]) + i, o[j]);
                }
            }
        }
        const int64_t tstride = static_cast<int64_t>(gridDim.x) * kThreads;
        for (int64_t i = n4 * 4 + blockIdx.x * kThreads + threadIdx.x; i < n; i += tstride) {
            float x[NIN > 0 ? NIN : 1], y[NOUT];
#pragma unroll
            for (int j = 0; j < NIN; ++j) x[j] = p.in[j][i];
            f(x, y);
#pragma unroll
            for (int j = 0; j < NOUT; ++j) p.out[j][i] = y[j];
        }
    } else {
        const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
        for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
            float x[NIN > 0 ? NIN : 1], y[NOUT];
#pragma unroll
            for (int j = 0; j < NIN; ++j) x[j] = p.in[j][i];
            f(x, y);
#pragma unroll
            for (int j = 0; j < NOUT; ++j) p.out[j][i] = y[j];
        }
    }
}

template <int NIN, int NOUT, typename F>
int run_map(const char* what, F f, Ptrs<NIN, NOUT> p, int64_t n, void* stream) {
    if (n < 0) return fail(PXK_ERR_INVALID, "%s: negative size", what);
    if (n == 0) return PXK_OK;
    bool vec = true;
    for (int j = 0; j < NIN; ++j) {
        if (p.in[j] == nullptr) return fail(PXK_ERR_INVALID, "%s: null input", what);
        vec = vec && aligned16(p.in[j]);
    }
    for (int j = 0; j < NOUT; ++j) {
        if (p.out[j] == nullptr) return fail(PXK_ERR_INVALID, "%s: null output", what);
        vec = vec && aligned16(p.out[j]);
    }
    if (vec) {
        // One unrolled iteration per thread up to 32768 workgroups; streaming cache policy once an
        // operand reaches 16 MiB (beyond what the L2s hold).
        const int64_t g = std::max<int64_t>(1, std::min<int64_t>(cdiv(cdiv(n, 4), kThreads * kUnroll), 32768));
        if (n >= (int64_t{1} << 22))
            PXK_LAUNCH((map_kernel_p<F, NIN, NOUT, true, true>), dim3(static_cast<unsigned>(g)), dim3(kThreads),
                               0, S(stream), f, p, n);
        else
            PXK_LAUNCH((map_kernel_p<F, NIN, NOUT, true, false>), dim3(static_cast<unsigned>(g)),
                               dim3(kThreads), 0, S(stream), f, p, n);
    } else {
        PXK_LAUNCH((map_kernel_p<F, NIN, NOUT, false, false>), dim3(grid_for(n, kThreads)), dim3(kThreads), 0,
                           S(stream), f, p, n);
    }
    return launched(what);
}

struct FillF {
    float v;
    __device__ void operator()(const float*, float* y) const { y[0] = v; }
};
struct OpF {
    int op;
    __device__ void operator()(const float* x, float* y) const { y[0] = apply_op(op, x[0]); }
};
struct AddF {
    __device__ void operator()(const float* x, float* y) const { y[0] = x[0] + x[1]; }
};
struct MulF {
    __device__ void operator()(const float* x, float* y) const { y[0] = x[0] * x[1]; }
};
struct ScaleF {
    float a;
    __device__ void operator()(const float* x, float* y) const { y[0] = a * x[0]; }
};
struct AxpbyF {
    float a, b;
    __device__ void operator()(const float* x, float* y) const { y[0] = a * x[0] + b * x[1]; }
};
struct ResidualSplitF {  // lrp_math.hpp:33-38
    float eps;
    __device__ void operator()(const float* x, float* y) const {
        const float s = x[0] + x[1];
        const float denom = stab(s, eps);
        y[0] = (x[0] / denom) * x[2];
        y[1] = (x[1] / denom) * x[2];
    }
};
struct BilinearF {  // lrp_math.hpp:41-45
    float eps;
    __device__ void operator()(const float* x, float* y) const {
        const float c = x[0] * x[1];
        const float denom = 2.0f * c + eps * ((c >= 0.0f) ? 1.0f : -1.0f);
        y[0] = (x[0] * x[1] / denom) * x[2];
    }
};
struct BilinearScaleF {  // lrp_math.hpp:57-61
    float eps;
    __device__ void operator()(const float* x, float* y) const {
        const float o = x[1];
        y[0] = x[0] / (2.0f * o + eps * ((o >= 0.0f) ? 1.0f : -1.0f));
    }
};
struct DivideF {  // lrp_math.hpp:312-315, gate mode None
    float eps;
    __device__ void operator()(const float* x, float* y) const { y[0] = x[0] / stab(x[1], eps); }
};
struct DivideGatedF {
    float eps;
    int mode;
    __device__ void operator()(const float* x, float* y) const {
        const bool pass = (mode == 1 && x[2] > 0.0f) || (mode == 2 && x[2] < 0.0f);
        y[0] = pass ? x[0] / stab(x[1], eps) : 0.0f;
    }
};

// add_row_vector: out[i][j] = in[i][j] + row[j].
__global__ void __launch_bounds__(kThreads) add_row_kernel(const float* in, const float* row, float* out, int64_t rows,
                                                           int64_t cols) {
    const int64_t n = rows * cols, stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) out[i] = in[i] + row[i % cols];
}

// scale_rows: out[i][j] = in[i][j] * scale[i].
__global__ void __launch_bounds__(kThreads) scale_rows_kernel(const float* in, const float* scale, float* out,
                                                              int64_t rows, int64_t cols) {
    const int64_t n = rows * cols, stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) out[i] = in[i] * scale[i / cols];
}

// SwiGLU gate over a [gate | up] row block (swiglu_module.cpp:80-88).
__global__ void __launch_bounds__(kThreads) swiglu_kernel(const float* gu, int64_t ld, float* gate_post, float* hidden,
                                                          int64_t rows, int64_t f, int act) {
    const int64_t n = rows * f, stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / f, c = i % f;
        const float x = gu[r * ld + c];
        const float gp = gate_activation(x, act);
        gate_post[i] = gp;
        hidden[i] = gp * gu[r * ld + f + c];
    }
}

__global__ void __launch_bounds__(kThreads) copy2d_kernel(float* dst, int64_t ds, const float* src, int64_t ss,
                                                          int64_t rows, int64_t cols) {
    const int64_t n = rows * cols, stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / cols, c = i % cols;
        dst[r * ds + c] = src[r * ss + c];
    }
}

// buf[k * count + i] = buf[i] for k = 1 .. copies - 1: each thread reads a float4 of the first block
// once and writes it into every further block.
__global__ void __launch_bounds__(kThreads) repeat_block_vec_kernel(float* buf, int64_t count4, int64_t copies) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4* b = reinterpret_cast<f4*>(buf);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count4; i += stride) {
        const f4 v = b[i];
        for (int64_t k = 1; k < copies; ++k) b[k * count4 + i] = v;
    }
}
__global__ void __launch_bounds__(kThreads) repeat_block_kernel(float* buf, int64_t count, int64_t copies) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count; i += stride) {
        const float v = buf[i];
        for (int64_t k = 1; k < copies; ++k) buf[k * count + i] = v;
    }
}

// out[j] += in[i][j] for i in order: one thread per column keeps the reference's order.
__global__ void __launch_bounds__(kThreads) accumulate_rows_kernel(const float* in, float* out, int64_t rows,
                                                                   int64_t cols) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j >= cols) return;
    float acc = out[j];
    for (int64_t r = 0; r < rows; ++r) acc += in[r * cols + j];
    out[j] = acc;
}

__global__ void __launch_bounds__(kThreads) column_sums_kernel(const float* in, float* out, int64_t rows, int64_t cols,
                                                               float beta) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j >= cols) return;
    float acc = 0.0f;
    for (int64_t r = 0; r < rows; ++r) acc += in[r * cols + j];
    out[j] = (beta == 0.0f) ? acc : beta * out[j] + acc;
}

__global__ void __launch_bounds__(kThreads) gather_kernel(const float* table, const float* idx, float* out,
                                                          int64_t count, int64_t dim) {
    const int64_t n = count * dim, stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const int64_t r = i / dim, c = i % dim;
        out[i] = table[static_cast<int64_t>(idx[r]) * dim + c];
    }
}

constexpr int kIdThreads = 1024;

__global__ void __launch_bounds__(kIdThreads) embedding_ids_kernel(const float* ids, int64_t count, int64_t vocab,
                                                                   float* ids_out, int32_t* status) {
    int bad = 0;
    for (int64_t i = threadIdx.x; i < count; i += kIdThreads) {
        const float r = roundf(ids[i]);  // llround's rounding: halves away from zero
        const bool ok = r >= 0.0f && r < static_cast<float>(vocab);  // NaN and infinities fail
        ids_out[i] = ok ? r : 0.0f;
        bad |= !ok;
    }
    bad = __syncthreads_or(bad);
    if (threadIdx.x == 0) *status = bad ? 1 : 0;
}

}  // namespace
}  // namespace pxk

using namespace pxk;

extern "C" {

const char* pxk_last_error(void) { return g_error.c_str(); }

const char* pxk_version(void) { return "pxk_gfx950 1.0 (fp32 MFMA 16x16x4, wave64)"; }

int pxk_timing_begin(int capacity) {
    if (capacity <= 0 || capacity > (1 << 20)) return fail(PXK_ERR_INVALID, "pxk_timing_begin: bad capacity %d", capacity);
    TimingWindow& w = g_timing;
    if (w.open) return fail(PXK_ERR_INVALID, "pxk_timing_begin: a window is already open on this thread");
    while (w.events.size() < 2 * static_cast<size_t>(capacity)) {
        hipEvent_t e = nullptr;
        const hipError_t r = hipEventCreate(&e);
        if (r != hipSuccess) return fail(PXK_ERR_LAUNCH, "pxk_timing_begin: hipEventCreate: %s", hipGetErrorString(r));
        w.events.push_back(e);
    }
    w.used = 0;
    w.open = true;
    return PXK_OK;
}

int pxk_timing_count(void) { return g_timing.used; }

int pxk_timing_end(float* ms, int capacity) {
    TimingWindow& w = g_timing;
    if (!w.open) return fail(PXK_ERR_INVALID, "pxk_timing_end: no window is open on this thread");
    w.open = false;
    const int n = std::min(w.used, capacity);
    for (int i = 0; i < n; ++i) {
        hipError_t r = hipEventSynchronize(w.events[2 * i + 1]);
        if (r == hipSuccess) r = hipEventElapsedTime(ms + i, w.events[2 * i], w.events[2 * i + 1]);
        if (r != hipSuccess) return fail(PXK_ERR_LAUNCH, "pxk_timing_end: launch %d: %s", i, hipGetErrorString(r));
    }
    return PXK_OK;
}

int pxk_fill(float* ptr, float value, int64_t n, void* stream) {
    Ptrs<0, 1> p{{nullptr}, {ptr}};
    return run_map<0, 1>("pxk_fill", FillF{value}, p, n, stream);
}

int pxk_elementwise(int op, const float* in, float* out, int64_t n, void* stream) {
    if (op < 0 || op > 7) return fail(PXK_ERR_INVALID, "pxk_elementwise: unknown op %d", op);
    return run_map<1, 1>("pxk_elementwise", OpF{op}, Ptrs<1, 1>{{in}, {out}}, n, stream);
}

int pxk_add(const float* a, const float* b, float* out, int64_t n, void* stream) {
    return run_map<2, 1>("pxk_add", AddF{}, Ptrs<2, 1>{{a, b}, {out}}, n, stream);
}

int pxk_mul(const float* a, const float* b, float* out, int64_t n, void* stream) {
    return run_map<2, 1>("pxk_mul", MulF{}, Ptrs<2, 1>{{a, b}, {out}}, n, stream);
}

int pxk_axpby(float alpha, const float* x, float beta, const float* y, float* out, int64_t n, void* stream) {
    if (beta == 0.0f)  // y is not read (device_backend.hpp:433-435)
        return run_map<1, 1>("pxk_axpby", ScaleF{alpha}, Ptrs<1, 1>{{x}, {out}}, n, stream);
    return run_map<2, 1>("pxk_axpby", AxpbyF{alpha, beta}, Ptrs<2, 1>{{x, y}, {out}}, n, stream);
}

int pxk_add_row_vector(const float* in, const float* row, float* out, int64_t rows, int64_t cols, void* stream) {
    if (rows < 0 || cols < 0) return fail(PXK_ERR_INVALID, "pxk_add_row_vector: negative size");
    if (rows * cols == 0) return PXK_OK;
    PXK_LAUNCH(add_row_kernel, dim3(grid_for(rows * cols, kThreads)), dim3(kThreads), 0, S(stream), in, row,
                       out, rows, cols);
    return launched("pxk_add_row_vector");
}

int pxk_scale_rows(const float* in, const float* scale, float* out, int64_t rows, int64_t cols, void* stream) {
    if (rows < 0 || cols < 0) return fail(PXK_ERR_INVALID, "pxk_scale_rows: negative size");
    if (rows * cols == 0) return PXK_OK;
    if (in == nullptr || scale == nullptr || out == nullptr) return fail(PXK_ERR_INVALID, "pxk_scale_rows: NULL operand");
    PXK_LAUNCH(scale_rows_kernel, dim3(grid_for(rows * cols, kThreads)), dim3(kThreads), 0, S(stream), in, scale, out,
               rows, cols);
    return launched("pxk_scale_rows");
}

int pxk_lrp_residual_split(const float* a, const float* b, const float* r, float* r_a, float* r_b, int64_t n,
                           float eps, void* stream) {
    return run_map<3, 2>("pxk_lrp_residual_split", ResidualSplitF{eps}, Ptrs<3, 2>{{a, b, r}, {r_a, r_b}}, n, stream);
}

int pxk_lrp_bilinear_elementwise(const float* a, const float* b, const float* r, float* r_out, int64_t n, float eps,
                                 void* stream) {
    return run_map<3, 1>("pxk_lrp_bilinear_elementwise", BilinearF{eps}, Ptrs<3, 1>{{a, b, r}, {r_out}}, n, stream);
}

int pxk_lrp_bilinear_scale(const float* r, const float* o, float* s, int64_t n, float eps, void* stream) {
    return run_map<2, 1>("pxk_lrp_bilinear_scale", BilinearScaleF{eps}, Ptrs<2, 1>{{r, o}, {s}}, n, stream);
}

int pxk_lrp_stabilized_divide(const float* r, const float* denom, const float* gate, float* out, int64_t n, float eps,
                              int gate_mode, void* stream) {
    if (gate_mode < 0 || gate_mode > 2) return fail(PXK_ERR_INVALID, "pxk_lrp_stabilized_divide: bad gate mode");
    if (gate_mode == 0)
        return run_map<2, 1>("pxk_lrp_stabilized_divide", DivideF{eps}, Ptrs<2, 1>{{r, denom}, {out}}, n, stream);
    return run_map<3, 1>("pxk_lrp_stabilized_divide", DivideGatedF{eps, gate_mode}, Ptrs<3, 1>{{r, denom, gate}, {out}},
                         n, stream);
}

int pxk_swiglu_forward(const float* gu, int64_t ld, float* gate_post, float* hidden, int64_t rows, int64_t f, int act,
                       void* stream) {
    if (rows < 0 || f < 0 || ld < 2 * f) return fail(PXK_ERR_INVALID, "pxk_swiglu_forward: bad sizes");
    if (act < 0 || act > 1) return fail(PXK_ERR_INVALID, "pxk_swiglu_forward: unknown gate activation %d", act);
    if (rows * f == 0) return PXK_OK;
    PXK_LAUNCH(swiglu_kernel, dim3(grid_for(rows * f, kThreads)), dim3(kThreads), 0, S(stream), gu, ld,
                       gate_post, hidden, rows, f, act);
    return launched("pxk_swiglu_forward");
}

int pxk_copy_2d(float* dst, int64_t ds, const float* src, int64_t ss, int64_t rows, int64_t cols, void* stream) {
    if (rows < 0 || cols < 0) return fail(PXK_ERR_INVALID, "pxk_copy_2d: negative size");
    if (rows * cols == 0) return PXK_OK;
    PXK_LAUNCH(copy2d_kernel, dim3(grid_for(rows * cols, kThreads)), dim3(kThreads), 0, S(stream), dst, ds, src,
                       ss, rows, cols);
    return launched("pxk_copy_2d");
}

int pxk_repeat_block(float* buf, int64_t count, int64_t copies, void* stream) {
    if (count < 0 || copies < 1) return fail(PXK_ERR_INVALID, "pxk_repeat_block: bad sizes");
    if (count == 0 || copies == 1) return PXK_OK;
    if (!buf) return fail(PXK_ERR_INVALID, "pxk_repeat_block: NULL buffer");
    if (count % 4 == 0 && aligned16(buf))
        PXK_LAUNCH(repeat_block_vec_kernel, dim3(grid_for(count / 4, kThreads)), dim3(kThreads), 0, S(stream),
                           buf, count / 4, copies);
    else
        PXK_LAUNCH(repeat_block_kernel, dim3(grid_for(count, kThreads)), dim3(kThreads), 0, S(stream), buf,
                           count, copies);
    return launched("pxk_repeat_block");
}

int pxk_accumulate_rows(const float* in, float* out, int64_t rows, int64_t cols, void* stream) {
    if (rows < 0 || cols < 0) return fail(PXK_ERR_INVALID, "pxk_accumulate_rows: negative size");
    if (cols == 0) return PXK_OK;
    PXK_LAUNCH(accumulate_rows_kernel, dim3(static_cast<unsigned>(cdiv(cols, kThreads))), dim3(kThreads), 0,
                       S(stream), in, out, rows, cols);
    return launched("pxk_accumulate_rows");
}

int pxk_column_sums(const float* in, float* out, int64_t rows, int64_t cols, float beta, void* stream) {
    if (rows < 0 || cols < 0) return fail(PXK_ERR_INVALID, "pxk_column_sums: negative size");
    if (cols == 0) return PXK_OK;
    PXK_LAUNCH(column_sums_kernel, dim3(static_cast<unsigned>(cdiv(cols, kThreads))), dim3(kThreads), 0,
                       S(stream), in, out, rows, cols, beta);
    return launched("pxk_column_sums");
}

int pxk_embedding_ids(const float* ids, int64_t count, int64_t vocab, float* ids_out, int32_t* status, void* stream) {
    if (count < 0 || vocab <= 0 || vocab > (int64_t{1} << 24))
        return fail(PXK_ERR_INVALID, "pxk_embedding_ids: count must be >= 0 and vocab in [1, 2^24]");
    if (!status || (count > 0 && (!ids || !ids_out))) return fail(PXK_ERR_INVALID, "pxk_embedding_ids: NULL operand");
    PXK_LAUNCH(embedding_ids_kernel, dim3(1), dim3(kIdThreads), 0, S(stream), ids, count, vocab, ids_out,
                       status);
    return launched("pxk_embedding_ids");
}

int pxk_gather_rows(const float* table, const float* indices, float* out, int64_t count, int64_t dim, void* stream) {
    if (count < 0 || dim < 0) return fail(PXK_ERR_INVALID, "pxk_gather_rows: negative size");
    if (count * dim == 0) return PXK_OK;
    PXK_LAUNCH(gather_kernel, dim3(grid_for(count * dim, kThreads)), dim3(kThreads), 0, S(stream), table,
                       indices, out, count, dim);
    return launched("pxk_gather_rows");
}

}  // extern "C"
