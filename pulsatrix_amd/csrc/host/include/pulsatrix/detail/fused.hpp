/** @file fused.hpp
 *  @brief Internals shared by the MI355X modules: module-owned device buffers and GEMM
 *         descriptor helpers.
 */
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>

#include "pulsatrix/mi355x_backend.hpp"
#include "pulsatrix/tensor.hpp"

namespace pulsatrix::detail {

/** @brief A module-owned device buffer with capacity semantics: its storage (and address) is kept
 *         while the requested size fits, so repeated passes at one shape launch on the same
 *         addresses (and can be captured into a HIP graph once), and passes at shorter lengths
 *         (a generation's growing prefixes, explained longest first) reuse the longest one's
 *         storage instead of allocating per length. */
class DevBuf {
public:
    float* ensure(DeviceBackend* be, int64_t n) {
        if (t_.numel() < n || t_.backend() != be || (n == 0 && t_.numel() != 0)) t_ = Tensor::uninitialized(Shape({n}), be);
        n_ = n;
        return t_.data();
    }
    [[nodiscard]] float* data() noexcept { return t_.data(); }
    [[nodiscard]] const float* data() const noexcept { return t_.data(); }
    /** @brief The size of the last ensure() (the storage may be larger). */
    [[nodiscard]] int64_t size() const noexcept { return n_; }
    /** @brief Repeats the first `count` floats `copies` times in place (pxk_repeat_block), within
     *         the storage an earlier, larger ensure() left; throws if that storage is too small. */
    void repeat(MI355XBackend* be, int64_t count, int64_t copies, const char* who);
    void release() {
        t_ = Tensor();
        n_ = 0;
    }

private:
    Tensor t_;
    int64_t n_ = 0;
};

/** @brief The MI355X modules compute through MI355XBackend's fused kernels. */
inline MI355XBackend* require_mi355x(DeviceBackend* be, const char* module) {
    auto* m = dynamic_cast<MI355XBackend*>(be);
    if (m == nullptr) throw std::invalid_argument(std::string(module) + ": needs an MI355XBackend");
    return m;
}

/** @brief A fresh tensor holding a copy of device data (the reference's modules return new tensors). */
Tensor copy_out(MI355XBackend* be, const float* src, Shape shape);
/** @brief Copies a caller's tensor into a module buffer (a module keeps its input for relevance). */
const float* keep_input(MI355XBackend* be, DevBuf& buf, const Tensor& t);

inline pxk_operand mat(const float* p, int64_t ld, int64_t batch_stride = 0, int64_t inner_stride = 0,
                       int64_t inner_div = 0, int64_t group_stride = 0) {
    return pxk_operand{p, ld, batch_stride, inner_stride, inner_div, group_stride};
}

inline pxk_gemm_desc gemm_desc(int64_t m, int64_t n, int64_t k) {
    pxk_gemm_desc d{};
    d.m = m;
    d.n = n;
    d.k = k;
    d.batch = d.inner = d.kgroups = 1;
    return d;
}

/** @brief The stabilizer bias a rule puts in a Linear's denominator: the layer's bias under the
 *         bias-in-denominator epsilon rule, none under the pre-bias rule (lrp_rules.cpp:197-220). */
inline const float* rule_bias(const float* bias, bool use_bias, bool bias_in_denominator) {
    return (use_bias && bias_in_denominator) ? bias : nullptr;
}

/** @brief The epsilon split of a residual sum s = a + b (lrp_residual_split, lrp_math.hpp:33-38)
 *         requested from the GEMM that produces the relevance of s: with a request, that GEMM
 *         writes r_a = (a / stab(s)) r and r_b = (b / stab(s)) r (PXK_EPI_MUL_X_SPLIT) instead of r.
 *         s must be the forward's stored a + b. */
struct ResidualSplit {
    const float* a = nullptr;
    const float* b = nullptr;
    const float* s = nullptr;
    float* r_a = nullptr;
    float* r_b = nullptr;
    /** Nullable: r_b is written divided by stab(b_den + b_den_bias[n]), the stabilised denominator
     *  of the epsilon-rule GEMM that reads r_b next, which then runs without its DIV_STAB prologue.
     *  Laid out like r_b; only epsilon-rule producers (GEMM epilogues, the seeded head) honour it. */
    const float* b_den = nullptr;
    const float* b_den_bias = nullptr;
    [[nodiscard]] bool requested() const noexcept { return r_a != nullptr; }
};

/** @brief Turns a MUL_X relevance GEMM (C = X * acc [+ Y], row stride ld) into its split form. */
inline void apply_split(pxk_gemm_desc& d, const ResidualSplit& sp, int64_t ld, float eps) {
    if (!sp.requested()) return;
    d.epilogue = PXK_EPI_MUL_X_SPLIT;
    d.eps = eps;
    d.c = mat(sp.r_a, ld);
    d.c2 = mat(sp.r_b, ld);
    d.z2 = mat(sp.a, ld);
    d.z3 = mat(sp.b, ld);
    d.w = mat(sp.s, ld);
    if (sp.b_den) {
        d.c2_den = mat(sp.b_den, ld);
        if (sp.b_den_bias) d.c2_den_bias = mat(sp.b_den_bias, 0);
    }
}

}  // namespace pulsatrix::detail
