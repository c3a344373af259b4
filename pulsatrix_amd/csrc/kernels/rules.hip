// rules.hip -- the Zennit-compatible affine LRP rules (Gamma, AlphaBeta, ZBox) around two MFMA
// GEMMs over stacked weights (include/pxk.h). The weight transforms and the ZBox column sums use
// round-to-nearest intrinsics so no product is fused into an add: the stacked weights and bound
// sums are bit-identical to the reference's axpby and gemm results (lrp_rules.cpp:13-160).
#include "common.hpp"

namespace pxk {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float pos_part(float v) { return v > 0.0f ? v : 0.0f; }

// The Gamma pair (Wa, Wb) = (w + g w+, w + g w-) or the AlphaBeta pair (w+, w-) of one weight.
__device__ __forceinline__ void rule_pair(int rule, float w, float gamma, float& p, float& q) {
    const float wp = pos_part(w), wn = __fsub_rn(w, wp);
    if (rule == PXK_RULE_GAMMA) {
        p = __fadd_rn(w, __fmul_rn(gamma, wp));
        q = __fadd_rn(w, __fmul_rn(gamma, wn));
    } else {
        p = wp;
        q = wn;
    }
}

struct WeightArgs {
    const float* w;
    int64_t ld, in, cols, col0, out;
    int rule;
    float gamma, low, high;
    float* w2;
};

// One 32 x 32 tile of one column block: read along the stored contiguity (rows of W, or rows of
// the transposed table), transposed through LDS when needed, written along W2's rows.
template <bool TRANS>
__global__ void __launch_bounds__(kThreads) rule_weights_kernel(const WeightArgs a) {
    __shared__ float t[32][33];
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    const int64_t i0 = static_cast<int64_t>(blockIdx.y) * 32, j0 = static_cast<int64_t>(blockIdx.x) * 32;
    for (int r = ty; r < 32; r += 8) {
        if constexpr (TRANS) {
            const int64_t j = j0 + r, i = i0 + tx;
            t[tx][r] = (i < a.in && j < a.cols) ? a.w[j * a.ld + i] : 0.0f;
        } else {
            const int64_t i = i0 + r, j = j0 + tx;
            t[r][tx] = (i < a.in && j < a.cols) ? a.w[i * a.ld + j] : 0.0f;
        }
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int64_t i = i0 + r, j = j0 + tx;
        if (i >= a.in || j >= a.cols) continue;
        const float v = t[r][tx];
        const int64_t jj = a.col0 + j;
        if (a.rule == PXK_RULE_ZBOX) {
            const float vp = pos_part(v), vn = __fsub_rn(v, vp);
            a.w2[i * a.out + jj] = v;
            a.w2[(a.in + i) * a.out + jj] = __fadd_rn(__fmul_rn(a.low, vp), __fmul_rn(a.high, vn));
        } else {
            float p, q;
            rule_pair(a.rule, v, a.gamma, p, q);
            const int64_t ld2 = 2 * a.out;
            a.w2[i * ld2 + jj] = p;
            a.w2[i * ld2 + a.out + jj] = q;
            a.w2[(a.in + i) * ld2 + jj] = q;
            a.w2[(a.in + i) * ld2 + a.out + jj] = p;
        }
    }
}

struct BiasArgs {
    const float* w;
    int64_t ld;
    int trans;
    const float* bias;
    int64_t in, cols, col0, out;
    int rule;
    float gamma, low, high;
    float* b2;
};

// b2 for one column block: Gamma / AlphaBeta's bias pair, or ZBox's bound sums low 1 W+ and
// high 1 W- accumulated over the inputs in increasing order from 0, as CPUBackend's gemm does.
__global__ void __launch_bounds__(kThreads) rule_bias_kernel(const BiasArgs a) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j >= a.cols) return;
    const int64_t jj = a.col0 + j;
    if (a.rule == PXK_RULE_ZBOX) {
        float lo = 0.0f, hi = 0.0f;
        for (int64_t i = 0; i < a.in; ++i) {
            const float v = a.trans ? a.w[j * a.ld + i] : a.w[i * a.ld + j];
            const float vp = pos_part(v), vn = __fsub_rn(v, vp);
            lo = __fadd_rn(lo, __fmul_rn(a.low, vp));
            hi = __fadd_rn(hi, __fmul_rn(a.high, vn));
        }
        a.b2[jj] = lo;
        a.b2[a.out + jj] = hi;
        return;
    }
    float p, q;
    rule_pair(a.rule, a.bias ? a.bias[j] : 0.0f, a.gamma, p, q);
    a.b2[jj] = p;
    a.b2[a.out + jj] = q;
}

__global__ void __launch_bounds__(kThreads) sign_split_kernel(const float* x, int64_t ldx, int64_t rows, int64_t in,
                                                                 float* out) {
    const int64_t total = rows * in;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t m = idx / in, i = idx - m * in;
        const float v = x[m * ldx + i], vp = pos_part(v);
        out[m * 2 * in + i] = vp;
        out[m * 2 * in + in + i] = __fsub_rn(v, vp);
    }
}

struct DivideArgs {
    const float* r;
    int64_t ldr, r_cols;
    const float* den;
    int64_t ld_den;
    const float* z;
    int64_t ldz;
    const float* bias;
    const float* b2;
    int64_t rows, out;
    float* g;
    int64_t ldg;
    int rule;
    float eps, alpha, beta;
};

__global__ void __launch_bounds__(kThreads) rule_divide_kernel(const DivideArgs a) {
    const int64_t total = a.rows * a.out;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t m = idx / a.out, j = idx - m * a.out;
        const float r = a.r[m * a.ldr + j % a.r_cols];
        if (a.rule == PXK_RULE_ZBOX) {
            // den = (x W - L W+) - H W-, two axpby passes in the reference.
            const float den = __fsub_rn(__fsub_rn(a.z[m * a.ldz + j], a.b2[j]), a.b2[a.out + j]);
            a.g[m * a.ldg + j] = r / stab(den, a.eps);
            continue;
        }
        const float d0 = a.den[m * a.ld_den + j] + a.b2[j];
        const float d1 = a.den[m * a.ld_den + a.out + j] + a.b2[a.out + j];
        float g0, g1;
        if (a.rule == PXK_RULE_GAMMA) {
            // The original output's sign selects the pair that explains each unit; the other
            // quotient is a hard 0 (lrp_math.hpp:312-315).
            const float zz = a.bias ? a.z[m * a.ldz + j] + a.bias[j] : a.z[m * a.ldz + j];
            g0 = zz > 0.0f ? r / stab(d0, a.eps) : 0.0f;
            g1 = zz < 0.0f ? r / stab(d1, a.eps) : 0.0f;
        } else {
            g0 = a.alpha * (r / stab(d0, a.eps));
            g1 = a.beta == 0.0f ? 0.0f : -a.beta * (r / stab(d1, a.eps));  // beta 0: no negative branch
        }
        a.g[m * a.ldg + j] = g0;
        a.g[m * a.ldg + a.out + j] = g1;
    }
}

struct CombineArgs {
    const float* x;
    int64_t ldx;
    const float* c;
    int64_t ldc;
    const float* add;
    int64_t rows, in;
    float* r_in;
    int64_t ld;
    const float* sa;
    const float* sb;
    const float* ss;
    float* r_b;
    int rule;
    float eps;
};

__global__ void __launch_bounds__(kThreads) rule_combine_kernel(const CombineArgs a) {
    const int64_t total = a.rows * a.in;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t m = idx / a.in, i = idx - m * a.in;
        const float x = a.x[m * a.ldx + i];
        const float c0 = a.c[m * a.ldc + i], c1 = a.c[m * a.ldc + a.in + i];
        float v;
        if (a.rule == PXK_RULE_ZBOX) {
            v = x * c0 - c1;
        } else {
            const float xp = pos_part(x), xn = x - xp;
            v = xp * c0 + xn * c1;
        }
        const int64_t o = m * a.ld + i;
        if (a.add) v = a.add[o] + v;
        if (a.ss) {  // the residual split of the sum this relevance belongs to
            const float den = stab(a.ss[o], a.eps);
            a.r_in[o] = (a.sa[o] / den) * v;
            a.r_b[o] = (a.sb[o] / den) * v;
        } else {
            a.r_in[o] = v;
        }
    }
}

bool known_rule(int rule) { return rule == PXK_RULE_GAMMA || rule == PXK_RULE_ALPHA_BETA || rule == PXK_RULE_ZBOX; }

}  // namespace
}  // namespace pxk

using namespace pxk;

extern "C" int pxk_lrp_rule_weights(const pxk_rule_params* p, const pxk_rule_block* blocks, int nblocks, int64_t in,
                                    float* w2, float* b2, void* stream) {
    if (!p || !known_rule(p->rule)) return fail(PXK_ERR_INVALID, "pxk_lrp_rule_weights: unknown rule");
    if (!blocks || nblocks <= 0 || in <= 0 || !w2 || !b2)
        return fail(PXK_ERR_INVALID, "pxk_lrp_rule_weights: needs blocks, in > 0 and both outputs");
    int64_t out = 0;
    for (int b = 0; b < nblocks; ++b) {
        const pxk_rule_block& k = blocks[b];
        if (!k.w || k.cols <= 0 || k.ld < (k.trans ? in : k.cols))
            return fail(PXK_ERR_INVALID, "pxk_lrp_rule_weights: block %d needs weights, cols > 0 and a row stride "
                                         "holding its row", b);
        if (k.cols > (int64_t{1} << 24) * 32 || in > 65535 * 32)
            return fail(PXK_ERR_INVALID, "pxk_lrp_rule_weights: block %d is too large", b);
        out += k.cols;
    }
    int64_t col0 = 0;
    for (int b = 0; b < nblocks; ++b) {
        const pxk_rule_block& k = blocks[b];
        const WeightArgs wa{k.w, k.ld, in, k.cols, col0, out, p->rule, p->gamma, p->low, p->high, w2};
        const dim3 grid(static_cast<unsigned>(cdiv(k.cols, 32)), static_cast<unsigned>(cdiv(in, 32)));
        if (k.trans)
            PXK_LAUNCH(rule_weights_kernel<true>, grid, dim3(kThreads), 0, S(stream), wa);
        else
            PXK_LAUNCH(rule_weights_kernel<false>, grid, dim3(kThreads), 0, S(stream), wa);
        const BiasArgs ba{k.w, k.ld, k.trans, k.bias, in, k.cols, col0, out, p->rule, p->gamma, p->low, p->high, b2};
        PXK_LAUNCH(rule_bias_kernel, dim3(static_cast<unsigned>(cdiv(k.cols, kThreads))), dim3(kThreads), 0,
                           S(stream), ba);
        if (const int rc = launched("pxk_lrp_rule_weights")) return rc;
        col0 += k.cols;
    }
    return PXK_OK;
}

extern "C" int pxk_lrp_sign_split(const float* x, int64_t ldx, int64_t rows, int64_t in, float* out, void* stream) {
    if (rows < 0 || in < 0 || ldx < in) return fail(PXK_ERR_INVALID, "pxk_lrp_sign_split: bad sizes");
    if (rows == 0 || in == 0) return PXK_OK;
    if (!x || !out) return fail(PXK_ERR_INVALID, "pxk_lrp_sign_split: NULL operand");
    PXK_LAUNCH(sign_split_kernel, dim3(grid_for(rows * in, kThreads)), dim3(kThreads), 0, S(stream), x, ldx,
                       rows, in, out);
    return launched("pxk_lrp_sign_split");
}

extern "C" int pxk_lrp_rule_divide(const pxk_rule_params* p, const float* r, int64_t ldr, int64_t r_cols,
                                   const float* den, int64_t ld_den, const float* z, int64_t ldz, const float* bias,
                                   const float* b2, int64_t rows, int64_t out, float* g, int64_t ldg, void* stream) {
    if (!p || !known_rule(p->rule)) return fail(PXK_ERR_INVALID, "pxk_lrp_rule_divide: unknown rule");
    const bool zbox = p->rule == PXK_RULE_ZBOX;
    const int64_t width = zbox ? out : 2 * out;
    if (rows < 0 || out < 0 || r_cols <= 0 || r_cols > out || ldr < r_cols || ldg < width ||
        (!zbox && ld_den < width) || ((zbox || p->rule == PXK_RULE_GAMMA) && ldz < out))
        return fail(PXK_ERR_INVALID, "pxk_lrp_rule_divide: bad sizes or row strides");
    if (rows == 0 || out == 0) return PXK_OK;
    if (!r || !b2 || !g || (!zbox && !den) || ((zbox || p->rule == PXK_RULE_GAMMA) && !z))
        return fail(PXK_ERR_INVALID, "pxk_lrp_rule_divide: a required operand is NULL");
    const DivideArgs a{r, ldr, r_cols, den, ld_den, z, ldz, bias, b2, rows, out, g, ldg, p->rule, p->eps, p->alpha,
                       p->beta};
    PXK_LAUNCH(rule_divide_kernel, dim3(grid_for(rows * out, kThreads)), dim3(kThreads), 0, S(stream), a);
    return launched("pxk_lrp_rule_divide");
}

extern "C" int pxk_lrp_rule_combine(int rule, const float* x, int64_t ldx, const float* c, int64_t ldc,
                                    const float* add, int64_t rows, int64_t in, float* r_in, int64_t ld,
                                    const float* split_a, const float* split_b, const float* split_sum, float* r_b,
                                    float eps, void* stream) {
    if (!known_rule(rule)) return fail(PXK_ERR_INVALID, "pxk_lrp_rule_combine: unknown rule");
    if (rows < 0 || in < 0 || ldx < in || ldc < 2 * in || ld < in)
        return fail(PXK_ERR_INVALID, "pxk_lrp_rule_combine: bad sizes or row strides");
    if (rows == 0 || in == 0) return PXK_OK;
    if (!x || !c || !r_in || (split_sum && (!split_a || !split_b || !r_b)))
        return fail(PXK_ERR_INVALID, "pxk_lrp_rule_combine: a required operand is NULL");
    const CombineArgs a{x, ldx, c, ldc, add, rows, in, r_in, ld, split_a, split_b, split_sum, r_b, rule, eps};
    PXK_LAUNCH(rule_combine_kernel, dim3(grid_for(rows * in, kThreads)), dim3(kThreads), 0, S(stream), a);
    return launched("pxk_lrp_rule_combine");
}
