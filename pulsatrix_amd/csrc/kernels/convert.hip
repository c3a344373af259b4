// convert.hip -- checkpoint tensors widened to fp32 (and transposed) on the device (include/pxk.h).
//
// A checkpoint's raw little-endian bytes are copied to HBM as they are (half the bytes of fp32 for
// BF16 / F16, a quarter for F8), then widened here, exactly, as SafetensorsFile::tensor does on
// the host (src/safetensors.cpp:676-740): BF16 is the top half of a float32; F16, F8_E4M3 ("fn":
// no infinities, only S.1111.111 is NaN) and F8_E5M2 (IEEE-style) widen bit by bit with
// subnormals, infinities and NaN; F64 rounds to nearest. The Linear weights' (out, in) -> (in, out)
// transpose of the Hugging Face mapping (src/causal_lm.cpp:257-291) goes through 32 x 32 LDS tiles
// so reads and writes both stay coalesced.
#include "common.hpp"

namespace pxk {
namespace {

constexpr int kTile = 32;

// An IEEE-style binary float of the given widths, widened exactly to float (the reference's
// WidenFloat): every such value is a float.
__device__ float widen_bits(uint32_t v, int exp_bits, int man_bits, bool ieee_specials) {
    const uint32_t sign = (v >> (exp_bits + man_bits)) & 1u;
    const uint32_t exp = (v >> man_bits) & ((1u << exp_bits) - 1u);
    const uint32_t man = v & ((1u << man_bits) - 1u);
    const int bias = (1 << (exp_bits - 1)) - 1;
    const uint32_t exp_max = (1u << exp_bits) - 1u;
    const float s = sign ? -1.0f : 1.0f;
    if (ieee_specials && exp == exp_max) return man == 0 ? s * __builtin_inff() : __builtin_nanf("");
    if (!ieee_specials && exp == exp_max && man == (1u << man_bits) - 1u) return __builtin_nanf("");
    if (exp == 0) return s * ldexpf(static_cast<float>(man), 1 - bias - man_bits);
    return s * ldexpf(static_cast<float>((1u << man_bits) | man), static_cast<int>(exp) - bias - man_bits);
}

__device__ __forceinline__ float load_widened(const uint8_t* src, int64_t i, int dtype) {
    switch (dtype) {
        case PXK_DTYPE_F32: return __uint_as_float(reinterpret_cast<const uint32_t*>(src)[i]);
        case PXK_DTYPE_BF16: return __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(src)[i]) << 16);
        case PXK_DTYPE_F16: return widen_bits(reinterpret_cast<const uint16_t*>(src)[i], 5, 10, true);
        case PXK_DTYPE_F64: return static_cast<float>(reinterpret_cast<const double*>(src)[i]);
        case PXK_DTYPE_F8_E4M3: return widen_bits(src[i], 4, 3, false);
        default: return widen_bits(src[i], 5, 2, true);  // PXK_DTYPE_F8_E5M2
    }
}

__global__ void __launch_bounds__(256) widen_kernel(const uint8_t* src, int dtype, int64_t n, float* dst) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
        dst[i] = load_widened(src, i, dtype);
}

// dst (cols x rows) = widened src (rows x cols)^T, one 32 x 32 tile per workgroup (32 x 8 threads).
__global__ void __launch_bounds__(256) widen_transpose_kernel(const uint8_t* src, int dtype, int64_t rows,
                                                              int64_t cols, float* dst) {
    __shared__ float t[kTile][kTile + 1];
    const int64_t tiles_c = (cols + kTile - 1) / kTile;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) / tiles_c * kTile;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) % tiles_c * kTile;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int y = ty; y < kTile; y += 8) {
        const int64_t r = r0 + y, c = c0 + tx;
        if (r < rows && c < cols) t[y][tx] = load_widened(src, r * cols + c, dtype);
    }
    __syncthreads();
    for (int y = ty; y < kTile; y += 8) {
        const int64_t c = c0 + y, r = r0 + tx;  // dst row c, column r
        if (c < cols && r < rows) dst[c * rows + r] = t[tx][y];
    }
}

}  // namespace
}  // namespace pxk

using namespace pxk;

extern "C" int pxk_convert_weight(const void* src, int dtype, int64_t rows, int64_t cols, int transpose, float* dst,
                                  void* stream) {
    if (rows < 0 || cols < 0) return fail(PXK_ERR_INVALID, "pxk_convert_weight: negative size");
    if (dtype < PXK_DTYPE_F32 || dtype > PXK_DTYPE_F8_E5M2)
        return fail(PXK_ERR_INVALID, "pxk_convert_weight: unknown dtype %d", dtype);
    const int64_t n = rows * cols;
    if (n == 0) return PXK_OK;
    if (!src || !dst) return fail(PXK_ERR_INVALID, "pxk_convert_weight: NULL operand");
    const auto* s = static_cast<const uint8_t*>(src);
    if (transpose) {
        const int64_t tiles = ((rows + kTile - 1) / kTile) * ((cols + kTile - 1) / kTile);
        if (tiles > (int64_t{1} << 31) - 1) return fail(PXK_ERR_INVALID, "pxk_convert_weight: matrix too large");
        PXK_LAUNCH(widen_transpose_kernel, dim3(static_cast<unsigned>(tiles)), dim3(256), 0, S(stream), s, dtype,
                           rows, cols, dst);
    } else {
        PXK_LAUNCH(widen_kernel, dim3(grid_for(n, 256)), dim3(256), 0, S(stream), s, dtype, n, dst);
    }
    return launched("pxk_convert_weight");
}
