// Internal helpers shared by the gfx950 kernel translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "pxk.h"

namespace pxk {

constexpr int kWave = 64;  // CDNA wavefront width

// Records a message for pxk_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);
// PXK_OK, or PXK_ERR_LAUNCH with the HIP error string after a launch.
int launched(const char* what);

inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

// Per-dispatch timing (pxk_timing_begin / pxk_timing_end): while a window is open on the calling
// thread, each launch takes the next pair of events and records the kernel's own start and end
// with it (hipExtLaunchKernelGGL), so the host can read every kernel's duration as the GPU ran it.
// Returns false (a plain launch) when no window is open or its events are used up.
bool timing_slot(hipEvent_t* start, hipEvent_t* stop);

// Every kernel launch of the library goes through here.
#define PXK_LAUNCH(kernel, grid, block, shmem, stream, ...)                                                 \
    do {                                                                                                    \
        hipEvent_t pxk_ev0_ = nullptr, pxk_ev1_ = nullptr;                                                  \
        if (::pxk::timing_slot(&pxk_ev0_, &pxk_ev1_))                                                       \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, pxk_ev0_, pxk_ev1_, 0u, __VA_ARGS__); \
        else                                                                                                \
            hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                            \
    } while (0)

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Blocks for a grid-stride elementwise kernel: enough to fill 256 CUs several times over.
inline unsigned grid_for(int64_t work, int threads) {
    int64_t g = cdiv(work, threads);
    if (g > 8192) g = 8192;
    if (g < 1) g = 1;
    return static_cast<unsigned>(g);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// z + eps * sign(z), sign(0) = +1: the stabilizer of every epsilon rule (src/lrp_math.hpp:17).
__device__ __forceinline__ float stab(float z, float eps) { return z + eps * ((z >= 0.0f) ? 1.0f : -1.0f); }

// SwiGLU gate activations: SiLU x / (1 + e^-x) (cpu_backend.cpp:29) and GeLU with the tanh
// approximation (pointwise_math.hpp:32-36), selected by act (0 SiLU, 1 GeLU tanh).
__device__ __forceinline__ float gate_activation(float x, int act) {
    if (act == 1) {
        const float kBeta = 0.7978845608028654f, kKappa = 0.044715f;
        return 0.5f * x * (1.0f + tanhf(kBeta * (x + kKappa * x * x * x)));
    }
    return x * (1.0f / (1.0f + expf(-x)));
}

// Sum / max over a full wave64 with cross-lane shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

}  // namespace pxk
