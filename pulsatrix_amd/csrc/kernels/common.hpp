// Internal helpers shared by the gfx950 kernel translation units.
#pragma once

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
