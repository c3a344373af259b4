// gemm_impl.hpp -- device side of the fused fp32 MFMA GEMM for gfx950 (pxk_gemm, include/pxk.h):
// the argument and table types every GEMM translation unit shares, the kernel templates, and the
// macros that instantiate them. gemm_tab_*.hip instantiate the (transpose, prologue, epilogue)
// table in parts that compile in parallel; gemm.hip plans and launches.
//
//
// Tiling. A workgroup of 256 threads (four wave64s) owns a BM x BN output tile. K advances in
// stages of BK staged through LDS, double-buffered: the next stage's global loads are in flight
// while the MFMA pipe works on the current one, and one barrier per stage separates them.
//   128x128 and 64x64: the waves form a 2x2 grid of 64x64 / 32x32 wave tiles, BK = 32.
//   32x64 and 32x32: every wave owns the whole tile and a quarter of a BK = 64 stage; the four
//   partial tiles are summed in LDS in wave order at the end. This keeps four waves busy on tiles
//   small enough that a 512-token GEMM still spreads over all 256 CUs without split-K.
//
// LDS layout. Each operand is kept in the contiguity it has in HBM, so every global->LDS move is
// a 128-bit load and a 128-bit ds_write. A K-contiguous operand sits as [rows][BK + 4] and a lane
// fetches its fragment for a 16-wide K chunk with one ds_read_b128; an M- or N-contiguous operand
// sits as [BK][cols + 4] and a lane fetches its four K values with four ds_read_b32 that the
// 4-float row padding keeps free of bank conflicts.
//
// MFMA mapping. v_mfma_f32_16x16x4_f32 multiplies a 16x4 by a 4x16 fragment; lane l supplies
// A[l%16][kk] and B[kk][l%16] with kk = l/16, and holds D[4*(l/16)+r][l%16] in its r-th result
// register. Lane group g = l/16 is given K indices 16c + 4g + s (chunk c, MFMA step s), so a
// K-contiguous fragment for all four steps is one float4.
//
// Grid. One-dimensional, M-tile fastest, then N-tile, then (batch, split). When the tile count is
// a multiple of 8 the block index is regrouped so that each of the 8 XCDs receives one contiguous
// run of tiles: the M-tiles sharing one B panel then run together on the XCD whose L2 holds it.
//
// Epilogue. The accumulator tile is staged through LDS and walked row-major in float4 columns by
// the whole workgroup, so global writes (and the reads of epilogue operands) are 128-bit and
// coalesced, and an element can see its RoPE pair partner. Split-K writes raw partials to a
// workspace instead; a second kernel sums them in split order (deterministic, no atomics) over
// row slabs and runs the same epilogue.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <utility>

#include "common.hpp"

namespace pxk {
namespace gemm {  // shared by every GEMM translation unit

typedef float f4 __attribute__((ext_vector_type(4)));

struct Op {
    const float* p;
    int64_t ld, so, si, div, sg;
};

struct Args {
    int64_t M, N, K, batch, inner, kgroups;
    int causal, splits;
    float beta, eps;
    Op a, b, c, z, zb, c2, c3, x, y, w, z2, z3, eb, eb2;
    Op c2d, c2db;  // MUL_X_SPLIT: C2's denominator and its bias over n (nullable)
    const float* xr;  // MUL_X, MUL_X_SPLIT: X is an RMSNorm's input, normalised by rms xr[m] and gamma xg[n]
    const float* xg;
    float* row_rms;  // PXK_PRO_RMS: each row's rms (nullable)
    float norm_eps;
    const float* cos_t;
    const float* sin_t;
    int64_t head_dim, rope_cols;
    int rope_half, gate_act;
    int vec_a, vec_b, vec_e;  // 128-bit global access allowed: A (and Z), B, epilogue operands
    int tiles_m, tiles_n, bm;
    int remap;    // XCD-grouped block order
    int group_m;  // M-tiles per group of the tile order (divides tiles_m; tiles_m: M fastest)
    float* ws;
    int64_t kc;  // skinny path: K rows per split
};

using KernelFn = void (*)(const Args);

constexpr int kTiles = 8;  // PXK_TILE_128x128 .. PXK_TILE_32x32_DIRECT, PXK_TILE_32x48_DIRECT, PXK_TILE_32x48

// One (transpose, prologue, epilogue) combination: its kernel on every tile shape, without and
// with a prologue bias over k, and the split-K reduce for each tile width.
struct Entry {
    int ta, tb, pro, epi;
    KernelFn k[2][kTiles];  // [prologue bias over k present][tile]
    KernelFn r[kTiles];
};

// The skinny kernels built: B layout, epilogue, kernels for up to 4, 8 and 16 rows (NN: with 64-,
// 32- and 16-column tiles), and the split reductions of the NN ones.
struct SkinnyEntry {
    int tb, epi;
    KernelFn k[3][3];  // [rows 4, 8, 16][NN: 64, 32, 16 columns; NT: 64]
    KernelFn r[3];
};

struct Table {
    const Entry* e;
    int n;
};

extern const Entry kTable0[];
extern const int kTable0Size;
extern const Entry kTable1[];
extern const int kTable1Size;
extern const Entry kTable2[];
extern const int kTable2Size;
extern const Entry kTable3[];
extern const int kTable3Size;
extern const Entry kTable4[];
extern const int kTable4Size;
extern const Entry kTable5[];
extern const int kTable5Size;
extern const SkinnyEntry kSkinny[];
extern const int kSkinnySize;

}  // namespace gemm
namespace {
using namespace gemm;

// Batch and group counts fit 32 bits (the host checks the grid), so the index splits use 32-bit
// division; batch 0 of group 0 (every unbatched GEMM) needs none.
__device__ __forceinline__ const float* obase(const Op& o, int64_t b, int64_t inner, int64_t s) {
    if (b == 0) return o.p + s * o.sg;
    const uint32_t bb = static_cast<uint32_t>(b), in = static_cast<uint32_t>(inner);
    const uint32_t bo = bb / in, bi = bb - bo * in;
    const uint32_t d = o.div > 1 ? static_cast<uint32_t>(o.div) : 1u;
    return o.p + static_cast<int64_t>(bo) * o.so + static_cast<int64_t>(bi / d) * o.si + s * o.sg;
}
__device__ __forceinline__ float* obase_w(const Op& o, int64_t b, int64_t inner) {
    return const_cast<float*>(obase(o, b, inner, 0));
}

constexpr int NT = 256;
// Kernel-side prologue variants: PXK_PRO_NONE, PXK_PRO_DIV_STAB without a bias over k, with one
// (kProStabBias), and PXK_PRO_RMS (the rows' sums of squares of A kept; gamma is in B).
constexpr int kProStabBias = 3;
static_assert(kProStabBias != PXK_PRO_NONE && kProStabBias != PXK_PRO_DIV_STAB && kProStabBias != PXK_PRO_RMS,
              "internal prologue id collides with a public one");

// The rms of an RMSNorm row from its sum of squares over K, as the row kernel computes it
// (rms_norm_vec_kernel: sqrtf(ss / cols + eps)); the K-slice partials are added in slice order.
__device__ __forceinline__ float rms_of(const float* rss, int parts, int stride, int row, int64_t K, float eps) {
    float t = 0.0f;
    for (int q = 0; q < parts; ++q) t += rss[q * stride + row];
    return sqrtf(t / static_cast<float>(K) + eps);
}

// y of an RMSNorm rebuilt from its input x, gamma over the row and the row's rms, with the row
// kernel's expression (gamma * x / rms): relevance epilogues read the norm's input this way.
__device__ __forceinline__ f4 norm_x(f4 x, f4 gamma, float rms) {
    f4 y;
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = gamma[j] * x[j] / rms;
    return y;
}

// NS_: register sets of prefetched stages. Stage t + 1 .. t + NS are in flight while stage t is
// on the MFMA pipe, so the short stages of the small tiles still cover a global load's latency.
template <int BM_, int BN_, int WM_, int WN_, int KS_, int NS_>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, KS = KS_, NS = NS_;
    static constexpr int NT = 64 * WM * WN * KS;  // threads: four or eight wave64s
    static_assert(NT == 256 || NT == 512, "four or eight waves per workgroup");
    static constexpr int TM = BM / WM / 16, TN = BN / WN / 16;  // 16x16 MFMA tiles per wave
    static constexpr int CH = KS == 1 ? 2 : 1;                   // 16-wide K chunks per wave per stage
    static constexpr int BK = 16 * KS * CH;
    static constexpr int LDC = BN + 4;
};

using C128 = Cfg<128, 128, 2, 2, 1, 1>;
using C64 = Cfg<64, 64, 2, 2, 1, 3>;
using C32x64 = Cfg<32, 64, 1, 1, 4, 2>;
using C32 = Cfg<32, 32, 1, 1, 4, 3>;
using C32x48 = Cfg<32, 48, 1, 1, 4, 2>;  // 192 workgroups over 512 x 576

template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>): register arrays indexed by
// the constant stay in registers.
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS footprint of one operand panel: R rows of M (or N) by BK of K, moved by T threads.
template <int R, int BK, bool KC, int T>
struct Panel {
    static constexpr int LD = KC ? BK + 4 : R + 4;
    static constexpr int SIZE = KC ? R * LD : BK * LD;
    static constexpr int NV = R * BK / 4 / T;  // float4 moved per thread per stage
    static_assert(NV >= 1 && R * BK % (4 * T) == 0, "panel must split evenly over the workgroup");
};

template <class C, bool TA, bool TB>
struct Layout {
    using PA = Panel<C::BM, C::BK, !TA, C::NT>;
    using PB = Panel<C::BN, C::BK, TB, C::NT>;
    static constexpr int STAGE = PA::SIZE + PB::SIZE;
    static constexpr int PART = C::BM * C::LDC;
    static constexpr int SIZE = 2 * STAGE > C::KS * PART ? 2 * STAGE : C::KS * PART;
};

// ---- 128-bit epilogue access with a scalar tail ------------------------------------------------------
__device__ __forceinline__ f4 ld4(const float* p, bool vec, int cnt) {
    if (vec) return *reinterpret_cast<const f4*>(p);
    f4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (j < cnt) v[j] = p[j];
    return v;
}
// Tile outputs are stored non-temporally: the next launch reads them after the kernel boundary's
// L2 invalidation anyway, and lines that do not stay dirty in L2 leave less to write back when the
// kernel ends (measured per launch on the 512-row projections: 0.1-1.0 us less, none slower).
__device__ __forceinline__ void st4(float* p, f4 v, bool vec, int cnt) {
    if (vec) {
        __builtin_nontemporal_store(v, reinterpret_cast<f4*>(p));
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (j < cnt) p[j] = v[j];
}
// Split-K partials, which the reduce launch reads next, are stored as ordinary lines.
__device__ __forceinline__ void st4_keep(float* p, f4 v, bool vec, int cnt) {
    if (vec) {
        *reinterpret_cast<f4*>(p) = v;
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (j < cnt) p[j] = v[j];
}

// MUL_X_SPLIT's second share divided by the stabilised denominator of the relevance GEMM that reads
// it next (that GEMM then needs no DIV_STAB prologue): r / stab(den + bias[n]).
__device__ __forceinline__ f4 split_den(f4 r, const float* den, const float* bias, float eps, bool vec, int cnt) {
    const f4 z = ld4(den, vec, cnt);
    const f4 bz = bias ? ld4(bias, vec, cnt) : f4{0.f, 0.f, 0.f, 0.f};
    f4 out;
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = r[j] / stab(bias ? z[j] + bz[j] : z[j], eps);
    return out;
}

// ---- tile epilogue: ROWS x BN accumulator rows in LDS (Cs[ROWS][ldc]) -> outputs -----------------------
template <int ROWS, int BN, int EPI, int T>
__device__ void epilogue_rows(const float* Cs, int ldc, int64_t m0, int64_t n0, int64_t b, const Args& g) {
    constexpr int CPR = BN / 4;  // float4 columns per row
    const int tid = threadIdx.x;
    const int64_t inner = g.inner;
    float* C = g.c.p ? obase_w(g.c, b, inner) : nullptr;
    float* C2 = g.c2.p ? obase_w(g.c2, b, inner) : nullptr;
    float* C3 = g.c3.p ? obase_w(g.c3, b, inner) : nullptr;
    const float* X = g.x.p ? obase(g.x, b, inner, 0) : nullptr;
    const float* Y = g.y.p ? obase(g.y, b, inner, 0) : nullptr;
    const float* W = g.w.p ? obase(g.w, b, inner, 0) : nullptr;
    const float* Z = g.z.p ? obase(g.z, b, inner, 0) : nullptr;
    const float* Z2 = g.z2.p ? obase(g.z2, b, inner, 0) : nullptr;
    const float* Z3 = g.z3.p ? obase(g.z3, b, inner, 0) : nullptr;
    const float* EB = g.eb.p ? obase(g.eb, b, inner, 0) : nullptr;
    const float* EB2 = g.eb2.p ? obase(g.eb2, b, inner, 0) : nullptr;
    const float* C2D = EPI == PXK_EPI_MUL_X_SPLIT && g.c2d.p ? obase(g.c2d, b, inner, 0) : nullptr;
    const float* C2DB = EPI == PXK_EPI_MUL_X_SPLIT && g.c2db.p ? obase(g.c2db, b, inner, 0) : nullptr;
    const float eps = g.eps;
#pragma unroll 2
    for (int it = tid; it < ROWS * CPR; it += T) {
        const int row = it / CPR, col = 4 * (it % CPR);
        const int64_t m = m0 + row, n = n0 + col;
        if (m >= g.M || n >= g.N) continue;
        const int cnt = g.N - n < 4 ? static_cast<int>(g.N - n) : 4;
        const bool vec = g.vec_e && cnt == 4;
        const f4 acc = *reinterpret_cast<const f4*>(Cs + row * ldc + col);
        if constexpr (EPI == PXK_EPI_STORE) {
            float* dst = C + m * g.c.ld + n;
            f4 v = acc;
            if (g.beta != 0.0f) {
                const f4 old = ld4(dst, vec, cnt);
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = g.beta * old[j] + acc[j];
            }
            st4(dst, v, vec, cnt);
        } else if constexpr (EPI == PXK_EPI_STORE_BIAS) {
            st4(C + m * g.c.ld + n, acc, vec, cnt);
            if (EB) st4(C2 + m * g.c2.ld + n, acc + ld4(EB + n, vec, cnt), vec, cnt);
        } else if constexpr (EPI == PXK_EPI_ADD_RESID) {
            st4(C + m * g.c.ld + n, acc, vec, cnt);
            f4 y = acc;
            if (EB) {
                y = acc + ld4(EB + n, vec, cnt);
                st4(C2 + m * g.c2.ld + n, y, vec, cnt);
            }
            st4(C3 + m * g.c3.ld + n, ld4(X + m * g.x.ld + n, vec, cnt) + y, vec, cnt);
        } else if constexpr (EPI == PXK_EPI_MUL_X) {
            f4 xv = ld4(X + m * g.x.ld + n, vec, cnt);
            if (g.xr) xv = norm_x(xv, ld4(g.xg + n, vec, cnt), g.xr[m]);
            f4 v = xv * acc;
            if (Y) v = ld4(Y + m * g.y.ld + n, vec, cnt) + v;
            st4(C + m * g.c.ld + n, v, vec, cnt);
        } else if constexpr (EPI == PXK_EPI_SWIGLU_FWD) {
            // Columns alternate 32-wide gate and up blocks; the gate block's threads do both.
            if ((n & 63) >= 32) continue;
            const int64_t F = g.N / 2, j = (n >> 6) * 32 + (n & 63);
            const f4 up = *reinterpret_cast<const f4*>(Cs + row * ldc + col + 32);
            st4(C + m * g.c.ld + j, acc, vec, cnt);
            st4(C + m * g.c.ld + F + j, up, vec, cnt);
            f4 gp, hid;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                gp[r] = gate_activation(acc[r], g.gate_act);
                hid[r] = gp[r] * up[r];
            }
            st4(C3 + m * g.c3.ld + j, gp, vec, cnt);
            st4(C2 + m * g.c2.ld + j, hid, vec, cnt);
        } else if constexpr (EPI == PXK_EPI_ROPE_FWD) {
            // z, y = z + bias, and the rotated y of the q / k heads; a head's pair partner is in
            // this tile (whole heads per tile).
            st4(C + m * g.c.ld + n, acc, vec, cnt);
            if (EB) st4(C2 + m * g.c2.ld + n, acc + ld4(EB + n, vec, cnt), vec, cnt);
            if (n < g.rope_cols) {
                // head_dim is even and n a multiple of 4: one modulo places the four columns.
                const int D = static_cast<int>(g.head_dim), half = D / 2;
                const int dn = static_cast<int>(n % D);
                f4 out = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (j >= cnt) continue;
                    const int64_t nj = n + j;
                    int d = dn + j;
                    int64_t hb = n - dn;
                    if (d >= D) {  // head_dim not a multiple of 4: the next head
                        d -= D;
                        hb += D;
                    }
                    const int i = g.rope_half ? (d < half ? d : d - half) : d / 2;
                    const int64_t lo = hb + (g.rope_half ? i : 2 * i), hi = hb + (g.rope_half ? i + half : 2 * i + 1);
                    float x0 = Cs[row * ldc + static_cast<int>(lo - n0)];
                    float x1 = Cs[row * ldc + static_cast<int>(hi - n0)];
                    if (EB) {
                        x0 = x0 + EB[lo];
                        x1 = x1 + EB[hi];
                    }
                    const float c = g.cos_t[m * half + i], sn = g.sin_t[m * half + i];
                    out[j] = nj == lo ? x0 * c - x1 * sn : x0 * sn + x1 * c;  // row_math.hpp:93-110
                }
                st4(C3 + m * g.c3.ld + n, out, vec, cnt);
            }
        } else if constexpr (EPI == PXK_EPI_MUL_X_SPLIT) {
            f4 xv = ld4(X + m * g.x.ld + n, vec, cnt);
            if (g.xr) xv = norm_x(xv, ld4(g.xg + n, vec, cnt), g.xr[m]);
            f4 v = xv * acc;
            if (Y) v = ld4(Y + m * g.y.ld + n, vec, cnt) + v;
            const f4 sa = ld4(Z2 + m * g.z2.ld + n, vec, cnt), sb = ld4(Z3 + m * g.z3.ld + n, vec, cnt);
            const f4 sum = ld4(W + m * g.w.ld + n, vec, cnt);
            f4 ra, rb;
#pragma unroll
            for (int j = 0; j < 4; ++j) {  // ResidualSplitF's expression, with the stored sum
                const float denom = stab(sum[j], eps);
                ra[j] = (sa[j] / denom) * v[j];
                rb[j] = (sb[j] / denom) * v[j];
            }
            if (C2D) rb = split_den(rb, C2D + m * g.c2d.ld + n, C2DB ? C2DB + n : nullptr, eps, vec, cnt);
            st4(C + m * g.c.ld + n, ra, vec, cnt);
            st4(C2 + m * g.c2.ld + n, rb, vec, cnt);
        } else if constexpr (EPI == PXK_EPI_SPV) {
            const f4 o = ld4(X + m * g.x.ld + n, vec, cnt);
            f4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float r = o[j] * acc[j];
                v[j] = r / (2.0f * o[j] + eps * ((o[j] >= 0.0f) ? 1.0f : -1.0f));
            }
            st4(C + m * g.c.ld + n, v, vec, cnt);
        } else if constexpr (EPI == PXK_EPI_ROPE_REL) {
            // Pair (lo, hi) inside the head block holding n; the tile spans whole heads.
            const int64_t D = g.head_dim, half = D / 2;
            const f4 xv = ld4(X + m * g.x.ld + n, vec, cnt);
            const f4 zv = ld4(Z + m * g.z.ld + n, vec, cnt);
            const f4 bv = EB ? ld4(EB + n, vec, cnt) : f4{0.f, 0.f, 0.f, 0.f};
            f4 rin, rz;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (j >= cnt) {  // past the last column: nothing stored
                    rin[j] = rz[j] = 0.0f;
                    continue;
                }
                const int64_t nj = n + j;
                const int64_t d = nj % D, hb = nj - d;
                const int64_t i = g.rope_half ? (d < half ? d : d - half) : d / 2;
                const int64_t lo = hb + (g.rope_half ? i : 2 * i), hi = hb + (g.rope_half ? i + half : 2 * i + 1);
                const float acc_lo = Cs[row * ldc + static_cast<int>(lo - n0)];
                const float acc_hi = Cs[row * ldc + static_cast<int>(hi - n0)];
                const float y_lo = Y[m * g.y.ld + lo], y_hi = Y[m * g.y.ld + hi];
                const float r_lo = y_lo * acc_lo, r_hi = y_hi * acc_hi;  // bilinear share: Q (or K) * (S @ K)
                const float c = g.cos_t[m * half + i], s = g.sin_t[m * half + i];
                const float d0 = stab(y_lo, eps), d1 = stab(y_hi, eps);
                float r_in = 0.0f;
                if (nj == lo) {
                    r_in += (xv[j] * c / d0) * r_lo;
                    r_in += (xv[j] * s / d1) * r_hi;
                } else {
                    r_in += (xv[j] * -s / d0) * r_lo;
                    r_in += (xv[j] * c / d1) * r_hi;
                }
                rin[j] = r_in;
                const float zb = EB ? zv[j] + bv[j] : zv[j];
                rz[j] = r_in / stab(zb, eps);
            }
            if (C) st4(C + m * g.c.ld + n, rin, vec, cnt);
            st4(C2 + m * g.c2.ld + n, rz, vec, cnt);
        } else if constexpr (EPI == PXK_EPI_VALUE_REL) {
            const f4 r = ld4(Y + m * g.y.ld + n, vec, cnt) * acc;
            if (C) st4(C + m * g.c.ld + n, r, vec, cnt);
            const f4 zv = ld4(Z + m * g.z.ld + n, vec, cnt);
            const f4 bv = EB ? ld4(EB + n, vec, cnt) : f4{0.f, 0.f, 0.f, 0.f};
            f4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = r[j] / stab(EB ? zv[j] + bv[j] : zv[j], eps);
            st4(C2 + m * g.c2.ld + n, v, vec, cnt);
        } else if constexpr (EPI == PXK_EPI_SWIGLU_REL) {
            const f4 zg = ld4(Z2 + m * g.z2.ld + n, vec, cnt), zu = ld4(Z3 + m * g.z3.ld + n, vec, cnt);
            f4 rh, a, bb;
            if (X) {
                rh = ld4(X + m * g.x.ld + n, vec, cnt) * acc;  // hidden * (g_down @ W_down^T)
                a = ld4(Y + m * g.y.ld + n, vec, cnt);
                bb = ld4(W + m * g.w.ld + n, vec, cnt);
            } else {  // without biases: gate_post = act(z_gate), up = z_up, hidden = gate_post * up
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    a[j] = gate_activation(zg[j], g.gate_act);
                    bb[j] = zu[j];
                    rh[j] = (a[j] * bb[j]) * acc[j];
                }
            }
            const f4 bg = EB ? ld4(EB + n, vec, cnt) : f4{0.f, 0.f, 0.f, 0.f};
            const f4 bu = EB2 ? ld4(EB2 + n, vec, cnt) : f4{0.f, 0.f, 0.f, 0.f};
            f4 o1, o2;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float cc = a[j] * bb[j];
                const float denom = 2.0f * cc + eps * ((cc >= 0.0f) ? 1.0f : -1.0f);
                const float rg = (a[j] * bb[j] / denom) * rh[j];  // lrp_math.hpp:41-45
                o1[j] = rg / stab(EB ? zg[j] + bg[j] : zg[j], eps);
                o2[j] = rg / stab(EB2 ? zu[j] + bu[j] : zu[j], eps);
            }
            st4(C + m * g.c.ld + n, o1, vec, cnt);
            st4(C2 + m * g.c2.ld + n, o2, vec, cnt);
        }
    }
}

// ---- global -> registers -> LDS for one operand panel ------------------------------------------------
// KC: the operand is stored K-contiguous ((rows of M or N) x K); else (K x (M or N)). `mn` is the
// stored extent along M (or N). issue() only starts the global loads; commit() waits for them,
// applies the DIV_STAB prologue (operand A only) and writes LDS, so the loads of a stage overlap
// the MFMAs of the stages before it.
template <int R, int BK, bool KC, int PRO, int T>
struct PanelLoader {
    using P = Panel<R, BK, KC, T>;
    static constexpr bool RMS = PRO == PXK_PRO_RMS;  // A only, K-contiguous
    static constexpr bool DS = PRO == PXK_PRO_DIV_STAB || PRO == kProStabBias;
    static constexpr bool HB = PRO == kProStabBias;
    f4 v[P::NV];
    f4 z[DS ? P::NV : 1];   // prologue denominators
    f4 zb[HB ? P::NV : 1];  // prologue bias over k
    float ss[RMS ? P::NV : 1] = {};  // RMS: the sums of squares of this thread's share of its rows

    __device__ __forceinline__ static void coords(int idx, int64_t r0, int64_t k0, int64_t& r, int64_t& c) {
        if constexpr (KC) {
            r = r0 + idx / (BK / 4);
            c = k0 + 4 * (idx % (BK / 4));
        } else {
            r = k0 + idx / (R / 4);
            c = r0 + 4 * (idx % (R / 4));
        }
    }

    // The panel lies inside the matrix and every access is 16-byte aligned: straight-line 128-bit
    // loads, so the compiler can wait for exactly the oldest register set at commit().
    __device__ __forceinline__ void issue_fast(const float* A, int64_t lda, const float* Z, int64_t ldz,
                                               const float* ZB, int64_t r0, int64_t k0) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < P::NV; ++i) {
            int64_t r, c;
            coords(tid + i * T, r0, k0, r, c);
            v[i] = *reinterpret_cast<const f4*>(A + r * lda + c);
            if constexpr (DS) z[i] = *reinterpret_cast<const f4*>(Z + r * ldz + c);
            if constexpr (HB) {
                if constexpr (KC)
                    zb[i] = *reinterpret_cast<const f4*>(ZB + c);
                else
                    zb[i] = f4{ZB[r], ZB[r], ZB[r], ZB[r]};
            }
        }
    }

    // Byte offsets of this thread's 16-byte pieces from the panel's first element, the same for
    // every stage: the loop then loads through a buffer resource at the panel's first element
    // (scalar registers) plus these fixed lane offsets, with no per-stage vector address
    // arithmetic. Requires R * ld < 2^29 (checked by the caller).
    __device__ __forceinline__ static void lane_offsets(int64_t ld, unsigned (&off)[P::NV]) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < P::NV; ++i) {
            int64_t r, c;
            coords(tid + i * T, 0, 0, r, c);
            off[i] = 4u * static_cast<unsigned>(r * ld + c);
        }
    }

    // issue_fast without a prologue operand: the panel at `base` (its first element), as a buffer
    // resource built with scalar instructions and the lanes' fixed offsets (every piece lies inside
    // the matrix on this path; the range only has to cover the panel).
    __device__ __forceinline__ void issue_base(const float* base, const unsigned (&off)[P::NV]) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7FFFFFFF, 0x00020000);
#pragma unroll
        for (int i = 0; i < P::NV; ++i)
            v[i] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off[i]), 0, 0));
    }

    // Any panel: element-wise bounds checks, zeros outside the matrix.
    __device__ __forceinline__ void issue(const Args& g, const float* A, int64_t lda, const float* Z, int64_t ldz,
                                          const float* ZB, int64_t mn, int64_t r0, int64_t k0) {
        const int tid = threadIdx.x;
        const int64_t rows = KC ? mn : g.K, cols = KC ? g.K : mn;
#pragma unroll
        for (int i = 0; i < P::NV; ++i) {
            int64_t r, c;
            coords(tid + i * T, r0, k0, r, c);
            f4 a = {0.f, 0.f, 0.f, 0.f};
            f4 zz = {1.f, 1.f, 1.f, 1.f};
            f4 bb = {0.f, 0.f, 0.f, 0.f};
            if (r < rows) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (c + j < cols) {
                        a[j] = A[r * lda + c + j];
                        if constexpr (DS) zz[j] = Z[r * ldz + c + j];
                        if constexpr (HB) bb[j] = ZB[KC ? c + j : r];
                    }
            }
            v[i] = a;
            if constexpr (DS) z[i] = zz;
            if constexpr (HB) zb[i] = bb;
        }
    }

    __device__ __forceinline__ void commit(float* lds, float eps) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < P::NV; ++i) {
            const int idx = tid + i * T;
            f4 a = v[i];
            // A element a is divided once per N tile that reads it, so the prologue multiplies by
            // v_rcp_f32 (within 1 ulp of 1/x) instead of the IEEE division sequence; |stab(z)| >= eps
            // keeps the operand normal.
            if constexpr (RMS) {
                ss[i] += a[0] * a[0] + a[1] * a[1] + a[2] * a[2] + a[3] * a[3];
            } else if constexpr (HB) {
#pragma unroll
                for (int j = 0; j < 4; ++j) a[j] = a[j] * __builtin_amdgcn_rcpf(stab(z[i][j] + zb[i][j], eps));
            } else if constexpr (DS) {
#pragma unroll
                for (int j = 0; j < 4; ++j) a[j] = a[j] * __builtin_amdgcn_rcpf(stab(z[i][j], eps));
            }
            if constexpr (KC)
                *reinterpret_cast<f4*>(lds + (idx / (BK / 4)) * P::LD + 4 * (idx % (BK / 4))) = a;
            else
                *reinterpret_cast<f4*>(lds + (idx / (R / 4)) * P::LD + 4 * (idx % (R / 4))) = a;
        }
    }
};

// MFMA operand fragment of a 16-row (or 16-column) block at `off` for K chunk `c`: element s is
// the value at K index 16c + 4g + s, g = lane / 16.
template <int BK, bool KC, int LD>
__device__ __forceinline__ f4 fragment(const float* lds, int off, int c, int lane) {
    if constexpr (KC) {
        return *reinterpret_cast<const f4*>(lds + (off + (lane & 15)) * LD + 16 * c + 4 * (lane >> 4));
    } else {
        const float* p = lds + (16 * c + 4 * (lane >> 4)) * LD + off + (lane & 15);
        return f4{p[0], p[LD], p[2 * LD], p[3 * LD]};
    }
}

// K range a tile sums over: K_LE_M stops after the tile's last row, K_GE_M starts at its first.
__device__ __forceinline__ int64_t k_first(const Args& g, int64_t m0) {
    return g.causal == PXK_CAUSAL_K_GE_M ? (m0 < g.K ? m0 : g.K) : 0;
}
__device__ __forceinline__ int64_t k_end(const Args& g, int64_t m0, int64_t bm) {
    return g.causal == PXK_CAUSAL_K_LE_M ? (m0 + bm < g.K ? m0 + bm : g.K) : g.K;
}

// Block index -> (M tile, N tile, batch * splits + split).
// Tile order within one (batch, split) slice: groups of group_m M-tiles, M fastest within a group,
// then the N-tiles, then the next group. With the XCD regrouping each XCD's contiguous run of tiles
// is then a group_m x (run / group_m) block, so fewer XCDs fetch each A and B panel into their L2.
__device__ __forceinline__ void tile_of(const Args& g, int& tm, int& tn, int& tz) {
    int id = static_cast<int>(blockIdx.x);
    if (g.remap) {
        const int per = static_cast<int>(gridDim.x) / 8;
        id = (id % 8) * per + id / 8;
    }
    const int slice = g.tiles_m * g.tiles_n;
    tz = id / slice;
    int r = id - tz * slice;
    const int span = g.group_m * g.tiles_n;
    const int sr = r / span;
    r -= sr * span;
    tm = sr * g.group_m + r % g.group_m;
    tn = r / g.group_m;
}

// Each wave's accumulators (one partial tile per K slice) -> LDS, summed in slice order; then the
// split-K partial store or the tile epilogue. smem holds KS * BM * (BN + 4) floats and no wave
// still reads it.
// With `rss` (PXK_PRO_RMS: `parts` partial sums of squares per tile row, `parts` x BM floats in LDS,
// written before the call), every accumulator row is divided by its rms and the tile in the first
// N column writes the rows' rms to g.row_rms.
template <class C, int EPI>
__device__ __forceinline__ void finish_tile(f4 (&acc)[C::TM][C::TN], float* smem, int ks, int wm, int wn, int lane,
                                            int tid, int64_t m0, int64_t n0, int64_t split, int64_t b, const Args& g,
                                            const float* rss = nullptr, int parts = 0) {
    constexpr int BM = C::BM, BN = C::BN, TM = C::TM, TN = C::TN, LDC = C::LDC, PART = BM * LDC;
    float* Cp = smem + ks * PART;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                Cp[(wm + 16 * i + 4 * (lane >> 4) + r) * LDC + wn + 16 * j + (lane & 15)] = acc[i][j][r];
    __syncthreads();
    if (C::KS > 1 || rss) {  // sum the K-slice partials in slice order; under PXK_PRO_RMS divide by the rms
        for (int it = tid; it < BM * (BN / 4); it += C::NT) {
            const int row = it / (BN / 4), off = row * LDC + 4 * (it % (BN / 4));
            f4 v = *reinterpret_cast<const f4*>(smem + off);
#pragma unroll
            for (int q = 1; q < C::KS; ++q) v += *reinterpret_cast<const f4*>(smem + q * PART + off);
            if (rss) {
                const float r = rms_of(rss, parts, BM, row, g.K, g.norm_eps);
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = v[j] / r;
            }
            *reinterpret_cast<f4*>(smem + off) = v;
        }
        if (rss && n0 == 0 && g.row_rms && tid < BM && m0 + tid < g.M)
            g.row_rms[b * g.M + m0 + tid] = rms_of(rss, parts, BM, tid, g.K, g.norm_eps);
        __syncthreads();
    }
    if (g.splits > 1) {  // raw partial tile -> workspace [split][batch][M][N]
        float* P = g.ws + ((split * g.batch + b) * g.M) * g.N;
        const bool vec = (g.N % 4) == 0;
        for (int it = tid; it < BM * (BN / 4); it += C::NT) {
            const int row = it / (BN / 4), col = 4 * (it % (BN / 4));
            const int64_t m = m0 + row, n = n0 + col;
            if (m >= g.M || n >= g.N) continue;
            const int cnt = g.N - n < 4 ? static_cast<int>(g.N - n) : 4;
            st4_keep(P + m * g.N + n, *reinterpret_cast<const f4*>(smem + row * LDC + col), vec && cnt == 4, cnt);
        }
        return;
    }
    epilogue_rows<BM, BN, EPI, C::NT>(smem, LDC, m0, n0, b, g);
}

template <class C, bool TA, bool TB, int PRO, int EPI>
__global__ void __launch_bounds__(C::NT) gemm_kernel(const Args g) {
    constexpr int BM = C::BM, BN = C::BN, BK = C::BK, TM = C::TM, TN = C::TN;
    using L = Layout<C, TA, TB>;
    using PA = typename L::PA;
    using PB = typename L::PB;
    __shared__ __attribute__((aligned(16))) float smem[L::SIZE];
    __shared__ float s_rss[PRO == PXK_PRO_RMS ? BM : 1];  // PXK_PRO_RMS: each tile row's sum of squares

    int tm, tn, tz;
    tile_of(g, tm, tn, tz);
    const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
    const int64_t split = tz % g.splits, b = tz / g.splits;  // 32-bit operands
    if (g.causal == PXK_CAUSAL_TRI && n0 > m0 + BM - 1) return;  // tile strictly above the diagonal

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ks = wave / (C::WM * C::WN), wmn = wave % (C::WM * C::WN);
    const int wm = (wmn / C::WN) * (BM / C::WM), wn = (wmn % C::WN) * (BN / C::WN);

    const int64_t k_lo = k_first(g, m0), k_hi = k_end(g, m0, BM);
    // Stage counts fit 32 bits (K / BK * kgroups < 2^31, checked on the host).
    const int nkb = k_hi > k_lo ? static_cast<int>((k_hi - k_lo + BK - 1) / BK) : 0;
    const int total = nkb * static_cast<int>(g.kgroups);
    const int per = (total + g.splits - 1) / g.splits;
    const int t0 = static_cast<int>(split) * per < total ? static_cast<int>(split) * per : total;
    const int t1 = t0 + per < total ? t0 + per : total;
    const int nt = t1 - t0;  // stage counters in 32 bits: compared and advanced on the scalar unit

    f4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    constexpr int NS = C::NS;
    PanelLoader<BM, BK, !TA, PRO, C::NT> la[NS];
    PanelLoader<BN, BK, TB, PXK_PRO_NONE, C::NT> lb[NS];
    // Load cursor: stage `lt` of the flattened (k-group, K stage) range, at (grp, kb).
    int lt = 0, grp = nkb > 0 ? t0 / nkb : 0, kb = nkb > 0 ? t0 % nkb : 0;  // 32-bit division
    const float* A = obase(g.a, b, g.inner, grp);
    const float* B = obase(g.b, b, g.inner, grp);
    constexpr bool kZ = PRO == PXK_PRO_DIV_STAB || PRO == kProStabBias, kZB = PRO == kProStabBias;
    const float* Z = kZ ? obase(g.z, b, g.inner, grp) : nullptr;
    const float* ZB = kZB ? obase(g.zb, b, g.inner, grp) : nullptr;
    auto advance = [&]() {
        ++lt;
        if (++kb == nkb) {  // next k-group: rebase the operands
            kb = 0;
            ++grp;
            A = obase(g.a, b, g.inner, grp);
            B = obase(g.b, b, g.inner, grp);
            if constexpr (kZ) Z = obase(g.z, b, g.inner, grp);
            if constexpr (kZB) ZB = obase(g.zb, b, g.inner, grp);
        }
    };
    auto commit = [&](auto S, int t) {  // register set S holds stage t -> LDS buffer t % 2
        float* dst = smem + (t & 1) * L::STAGE;
        la[S.value].commit(dst, g.eps);
        lb[S.value].commit(dst + PA::SIZE, g.eps);
    };
    auto compute = [&](int t) {
        const float* As = smem + (t & 1) * L::STAGE;
        const float* Bs = As + PA::SIZE;
#pragma unroll
        for (int cc = 0; cc < C::CH; ++cc) {
            const int c = ks * C::CH + cc;
            f4 af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = fragment<BK, !TA, PA::LD>(As, wm + 16 * i, c, lane);
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = fragment<BK, TB, PB::LD>(Bs, wn + 16 * j, c, lane);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
        }
    };

    // Fast path: every stage of this tile lies inside both matrices and is 16-byte aligned, and
    // there are more stages than register sets. Stage s lives in register set s % NS; before
    // iteration t, stages t + 1 .. t + NS are in flight. Loads are issued unconditionally (past the
    // last stage the cursor stays put and the last stage is loaded again, into a set nobody
    // commits), so the loop body has no branches around vector loads.
    const bool k_inside = k_lo + nkb * BK <= g.K;
    const bool fast = nt >= NS + 1 && k_inside && g.vec_a && g.vec_b && m0 + BM <= g.M && n0 + BN <= g.N;
    // Panels addressed as a uniform base plus fixed 32-bit lane offsets (no prologue operand, and
    // every panel's extent under 2^29 bytes: 128 rows of strides below 2^20 floats).
    const bool based = g.a.ld < (int64_t{1} << 20) && g.b.ld < (int64_t{1} << 20);
    unsigned offa[PA::NV], offb[PB::NV];
    PanelLoader<BM, BK, !TA, PRO, C::NT>::lane_offsets(g.a.ld, offa);
    PanelLoader<BN, BK, TB, PXK_PRO_NONE, C::NT>::lane_offsets(g.b.ld, offb);
    // The fast loop, with its loads through per-stage panel resources (BASED) or from full
    // addresses: both are compiled, each launch runs one, and neither has a branch around its loads.
    auto run_fast = [&](auto BASED) {
        auto issue = [&](auto S) {
            const int64_t k0 = k_lo + kb * BK;
            if constexpr (BASED.value) {
                la[S.value].issue_base(!TA ? A + m0 * g.a.ld + k0 : A + k0 * g.a.ld + m0, offa);
                lb[S.value].issue_base(TB ? B + n0 * g.b.ld + k0 : B + k0 * g.b.ld + n0, offb);
            } else {
                la[S.value].issue_fast(A, g.a.ld, Z, g.z.ld, ZB, m0, k0);
                lb[S.value].issue_fast(B, g.b.ld, nullptr, 0, nullptr, n0, k0);
            }
            if (lt + 1 < nt) advance();
        };
        issue(std::integral_constant<int, 0>{});
        commit(std::integral_constant<int, 0>{}, 0);
        static_for<NS>([&](auto U) { issue(std::integral_constant<int, (U.value + 1) % NS>{}); });
        __syncthreads();
        const int main_iters = (nt - 2) / NS * NS;  // a multiple of NS, >= nt - NS - 1
        for (int tb = 0; tb < main_iters; tb += NS) {
            static_for<NS>([&](auto U) {
                constexpr int nxt = (U.value + 1) % NS;
                const int t = tb + U.value;
                // Buffer (t + 1) % 2 was last read by stage t - 1, before the previous barrier, so
                // stage t + 1 goes to LDS first and its writes overlap this stage's MFMAs.
                commit(std::integral_constant<int, nxt>{}, t + 1);
                compute(t);
                __syncthreads();
                issue(std::integral_constant<int, nxt>{});  // stage t + 1 + NS (or the last one again)
            });
        }
        static_for<NS + 1>([&](auto U) {  // the last 2 .. NS + 1 stages: already in flight
            constexpr int nxt = (U.value + 1) % NS;
            const int t = main_iters + U.value;
            if (t < nt) {
                if (t + 1 < nt) commit(std::integral_constant<int, nxt>{}, t + 1);
                compute(t);
                __syncthreads();
            }
        });
    };
    if (fast && based && !kZ) {
        run_fast(std::true_type{});
    } else if (fast) {
        run_fast(std::false_type{});
    } else if (nt > 0) {
        // Edge tiles and short K ranges: bounds-checked loads, one stage ahead.
        auto issue = [&]() {
            const int64_t k0 = k_lo + kb * BK;
            la[0].issue(g, A, g.a.ld, Z, g.z.ld, ZB, g.M, m0, k0);
            lb[0].issue(g, B, g.b.ld, nullptr, 0, nullptr, g.N, n0, k0);
            advance();
        };
        issue();
        commit(std::integral_constant<int, 0>{}, 0);
        __syncthreads();
        for (int t = 0; t < nt; ++t) {
            const bool more = t + 1 < nt;
            if (more) issue();
            compute(t);
            if (more) commit(std::integral_constant<int, 0>{}, t + 1);
            __syncthreads();
        }
    }

    if constexpr (PRO == PXK_PRO_RMS) {
        // Each A element was committed once, by the thread that loaded it; the BK / 4 consecutive
        // threads that share a row add their sums (lanes of one wave), one of them writes it.
        static_for<PA::NV>([&](auto I) {
            float v = 0.0f;
            static_for<NS>([&](auto S) { v += la[S.value].ss[I.value]; });
#pragma unroll
            for (int o = 1; o < BK / 4; o <<= 1) v += __shfl_xor(v, o, 64);
            const int idx = tid + I.value * C::NT;
            if (idx % (BK / 4) == 0) s_rss[idx / (BK / 4)] = v;
        });
    }
    // The loop ended on a barrier: LDS is free for the partial tiles.
    finish_tile<C, EPI>(acc, smem, ks, wm, wn, lane, tid, m0, n0, split, b, g, PRO == PXK_PRO_RMS ? s_rss : nullptr, 1);
}

// ---- direct-load variant of the K-sliced tiles ---------------------------------------------------
// In the 32x64 and 32x32 tiles the four waves own disjoint K slices and share no operand data, so
// LDS staging is only a layout step costing a write, a read and a barrier per stage. Here every
// wave streams its own 16-deep K chunks straight from L2 into MFMA operand registers: a
// K-contiguous operand is one float4 per 16x16 fragment, an M- or N-contiguous one four dwords.
// PF register sets keep that many chunks in flight; past the wave's last chunk the last one is
// reloaded (unused), so no branch surrounds a load. LDS is used once, to merge the four slices.
template <class C, bool TA, bool TB, int PRO>
struct DirectChunk {
    static constexpr bool RMS = PRO == PXK_PRO_RMS;
    static constexpr bool DS = PRO == PXK_PRO_DIV_STAB || PRO == kProStabBias, HB = PRO == kProStabBias;
    f4 a[C::TM], b[C::TN];
    f4 z[DS ? C::TM : 1];
    f4 zb;  // bias over k, the same for every A row

    // An interior chunk (the whole 16-deep chunk of the tile lies inside both matrices) at K offset
    // kc: unconditional loads.
    __device__ __forceinline__ void load(const Args& g, const float* A, const float* Z, const float* ZB, const float* B,
                                         int64_t m0, int64_t n0, int64_t kc, int lane) {
        const int c = lane & 15, g4 = 4 * (lane >> 4);
#pragma unroll
        for (int i = 0; i < C::TM; ++i) {
            const int64_t m = m0 + 16 * i + c;
            if constexpr (!TA) {
                a[i] = *reinterpret_cast<const f4*>(A + m * g.a.ld + kc + g4);
                if constexpr (DS) z[i] = *reinterpret_cast<const f4*>(Z + m * g.z.ld + kc + g4);
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    a[i][s] = A[(kc + g4 + s) * g.a.ld + m];
                    if constexpr (DS) z[i][s] = Z[(kc + g4 + s) * g.z.ld + m];
                }
            }
        }
        if constexpr (HB) zb = *reinterpret_cast<const f4*>(ZB + kc + g4);
#pragma unroll
        for (int j = 0; j < C::TN; ++j) {
            const int64_t n = n0 + 16 * j + c;
            if constexpr (TB) {
                b[j] = *reinterpret_cast<const f4*>(B + n * g.b.ld + kc + g4);
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) b[j][s] = B[(kc + g4 + s) * g.b.ld + n];
            }
        }
    }

    // Any chunk: element-wise bounds checks on M, N and K, zeros outside the matrix.
    __device__ __forceinline__ void load_guarded(const Args& g, const float* A, const float* Z, const float* ZB,
                                                 const float* B, int64_t m0, int64_t n0, int64_t kc, int lane) {
        const int c = lane & 15, g4 = 4 * (lane >> 4);
#pragma unroll
        for (int i = 0; i < C::TM; ++i) {
            const int64_t m = m0 + 16 * i + c;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int64_t k = kc + g4 + s;
                const bool in = m < g.M && k < g.K;
                a[i][s] = in ? (TA ? A[k * g.a.ld + m] : A[m * g.a.ld + k]) : 0.0f;
                if constexpr (DS) z[i][s] = in ? (TA ? Z[k * g.z.ld + m] : Z[m * g.z.ld + k]) : 1.0f;
            }
        }
        if constexpr (HB) {
#pragma unroll
            for (int s = 0; s < 4; ++s) zb[s] = kc + g4 + s < g.K ? ZB[kc + g4 + s] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < C::TN; ++j) {
            const int64_t n = n0 + 16 * j + c;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int64_t k = kc + g4 + s;
                b[j][s] = (n < g.N && k < g.K) ? (TB ? B[n * g.b.ld + k] : B[k * g.b.ld + n]) : 0.0f;
            }
        }
    }

    __device__ __forceinline__ void mma(f4 (&acc)[C::TM][C::TN], float eps, float (&ss)[C::TM]) {
        if constexpr (RMS) {
#pragma unroll
            for (int i = 0; i < C::TM; ++i)
#pragma unroll
                for (int s = 0; s < 4; ++s) ss[i] += a[i][s] * a[i][s];
        } else if constexpr (DS) {
#pragma unroll
            for (int i = 0; i < C::TM; ++i)
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const float zz = HB ? z[i][s] + zb[s] : z[i][s];
                    a[i][s] = a[i][s] * __builtin_amdgcn_rcpf(stab(zz, eps));
                }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < C::TM; ++i)
#pragma unroll
                for (int j = 0; j < C::TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
    }
};

template <class C, bool TA, bool TB, int PRO, int EPI>
__global__ void __launch_bounds__(C::NT) gemm_direct_kernel(const Args g) {
    static_assert(C::WM == 1 && C::WN == 1, "direct loads: every wave owns the whole tile");
    constexpr int BM = C::BM, BN = C::BN, TM = C::TM, TN = C::TN, KS = C::KS, PF = 3;
    __shared__ __attribute__((aligned(16))) float smem[KS * BM * C::LDC];
    __shared__ float s_rss[PRO == PXK_PRO_RMS ? KS * BM : 1];  // PXK_PRO_RMS: per K slice, each row's sum of squares

    int tm, tn, tz;
    tile_of(g, tm, tn, tz);
    const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
    const int64_t split = tz % g.splits, b = tz / g.splits;
    if (g.causal == PXK_CAUSAL_TRI && n0 > m0 + BM - 1) return;

    const int tid = threadIdx.x, lane = tid & 63;
    const int ks = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t k_lo = k_first(g, m0), k_hi = k_end(g, m0, BM);
    const int nch = k_hi > k_lo ? static_cast<int>((k_hi - k_lo + 15) / 16) : 0;  // 16-deep chunks
    const int total = nch * static_cast<int>(g.kgroups);
    const int per = (total + g.splits - 1) / g.splits;
    const int t0 = static_cast<int>(split) * per < total ? static_cast<int>(split) * per : total;
    const int t1 = t0 + per < total ? t0 + per : total;
    const int first = t0 + ks;                                       // this wave: t0 + ks, + KS, ...
    const int nw = first < t1 ? (t1 - first + KS - 1) / KS : 0;

    f4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    float ss[TM] = {};  // PXK_PRO_RMS: this lane's sums of squares of rows 16 i + lane % 16

    // Cursor over this wave's chunks: (grp, kk) of flattened chunk `first + KS * u`.
    int grp = nch > 0 ? first / nch : 0, kk = nch > 0 ? first % nch : 0, lu = 0;
    const float* A = obase(g.a, b, g.inner, grp);
    const float* B = obase(g.b, b, g.inner, grp);
    constexpr bool kZ = PRO == PXK_PRO_DIV_STAB || PRO == kProStabBias, kZB = PRO == kProStabBias;
    const float* Z = kZ ? obase(g.z, b, g.inner, grp) : nullptr;
    const float* ZB = kZB ? obase(g.zb, b, g.inner, grp) : nullptr;
    auto advance = [&]() {  // to this wave's next chunk
        ++lu;
        kk += KS;
        bool moved = false;
        while (kk >= nch) {
            kk -= nch;
            ++grp;
            moved = true;
        }
        if (moved) {
            A = obase(g.a, b, g.inner, grp);
            B = obase(g.b, b, g.inner, grp);
            if constexpr (kZ) Z = obase(g.z, b, g.inner, grp);
            if constexpr (kZB) ZB = obase(g.zb, b, g.inner, grp);
        }
    };
    const bool interior = m0 + BM <= g.M && n0 + BN <= g.N && k_lo + 16 * static_cast<int64_t>(nch) <= g.K &&
                          g.vec_a && g.vec_b;
    if (nw > 0) {
        if (interior) {
            DirectChunk<C, TA, TB, PRO> ch[PF];
            auto load = [&](auto S) {  // the cursor's chunk -> set S; the cursor stops at the last one
                ch[S.value].load(g, A, Z, ZB, B, m0, n0, k_lo + 16 * kk, lane);
                if (lu + 1 < nw) advance();
            };
            static_for<PF>([&](auto U) { load(U); });
            for (int u0 = 0; u0 < nw; u0 += PF) {
                static_for<PF>([&](auto U) {
                    if (u0 + U.value < nw) ch[U.value].mma(acc, g.eps, ss);
                    load(U);  // chunk u0 + U + PF (or the last one again)
                });
            }
        } else {
            DirectChunk<C, TA, TB, PRO> ch;
            for (int u = 0; u < nw; ++u) {
                ch.load_guarded(g, A, Z, ZB, B, m0, n0, k_lo + 16 * kk, lane);
                ch.mma(acc, g.eps, ss);
                if (u + 1 < nw) advance();
            }
        }
    }
    if constexpr (PRO == PXK_PRO_RMS) {
        // Lane (c, g) summed rows 16 i + c over its K values; the four lane groups, then (in
        // finish_tile) the K slices in slice order.
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            float v = ss[i];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (lane < 16) s_rss[ks * BM + 16 * i + lane] = v;
        }
    }
    finish_tile<C, EPI>(acc, smem, ks, 0, 0, lane, tid, m0, n0, split, b, g, PRO == PXK_PRO_RMS ? s_rss : nullptr, KS);
}

// The split partials of one 4-column group, added in split order. Eight loads are in flight at a
// time, all issued before any is added (the split indices past the count read the last partial
// again and are not added), so fewer than eight splits cost one memory round trip, not one each.
__device__ __forceinline__ f4 sum_partials(const float* P, int64_t plane, int splits, bool vec, int cnt) {
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < splits; k += 8) {
        f4 t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = ld4(P + min(k + u, splits - 1) * plane, vec, cnt);
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (k + u < splits) acc += t[u];
    }
    return acc;
}

// Sums the split partials of a slab of rows in split order and runs the tile epilogue. One
// workgroup per RS x BN slab, one float4 column per thread (threads past RS rows idle when BN / 4
// does not divide the workgroup).
template <int BN, int EPI>
__global__ void __launch_bounds__(NT) splitk_reduce_kernel(const Args g) {
    constexpr int RS = 4 * NT / BN, LDC = BN + 4;
    __shared__ __attribute__((aligned(16))) float Cs[RS * LDC];
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN, m0 = static_cast<int64_t>(blockIdx.y) * RS;
    const int64_t b = blockIdx.z;
    if (g.causal == PXK_CAUSAL_TRI && n0 > (m0 / g.bm) * g.bm + g.bm - 1) return;  // tile never computed
    const int row = threadIdx.x / (BN / 4), col = 4 * (threadIdx.x % (BN / 4));
    const int64_t m = m0 + row, n = n0 + col;
    const bool mine = row < RS;
    if constexpr (EPI == PXK_EPI_MUL_X_SPLIT) {
        // Elementwise epilogue: the thread's epilogue operands are loaded with its partials, so
        // both wait on memory once, and the result goes straight out (no LDS pass). The same
        // expressions, in the same order, as epilogue_rows.
        if (!mine || m >= g.M || n >= g.N) return;
        const int cnt = g.N - n < 4 ? static_cast<int>(g.N - n) : 4;
        const bool vp = (g.N % 4) == 0 && cnt == 4, ve = g.vec_e && cnt == 4;
        const int64_t inner = g.inner;
        const float* Y = g.y.p ? obase(g.y, b, inner, 0) + m * g.y.ld + n : nullptr;
        f4 x = ld4(obase(g.x, b, inner, 0) + m * g.x.ld + n, ve, cnt);
        if (g.xr) x = norm_x(x, ld4(g.xg + n, ve, cnt), g.xr[m]);
        const f4 sa = ld4(obase(g.z2, b, inner, 0) + m * g.z2.ld + n, ve, cnt);
        const f4 sb = ld4(obase(g.z3, b, inner, 0) + m * g.z3.ld + n, ve, cnt);
        const f4 sum = ld4(obase(g.w, b, inner, 0) + m * g.w.ld + n, ve, cnt);
        const f4 y = Y ? ld4(Y, ve, cnt) : f4{0.f, 0.f, 0.f, 0.f};
        const int64_t plane = g.batch * g.M * g.N;
        const float* P = g.ws + (b * g.M + m) * g.N + n;
        f4 acc = sum_partials(P, plane, g.splits, vp, cnt);
        f4 v = x * acc;
        if (Y) v = y + v;
        f4 ra, rb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float denom = stab(sum[j], g.eps);
            ra[j] = (sa[j] / denom) * v[j];
            rb[j] = (sb[j] / denom) * v[j];
        }
        if (g.c2d.p)
            rb = split_den(rb, obase(g.c2d, b, inner, 0) + m * g.c2d.ld + n,
                           g.c2db.p ? obase(g.c2db, b, inner, 0) + n : nullptr, g.eps, ve, cnt);
        st4(obase_w(g.c, b, inner) + m * g.c.ld + n, ra, ve, cnt);
        st4(obase_w(g.c2, b, inner) + m * g.c2.ld + n, rb, ve, cnt);
        return;
    }
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if (mine && m < g.M && n < g.N) {
        const int cnt = g.N - n < 4 ? static_cast<int>(g.N - n) : 4;
        const bool vec = (g.N % 4) == 0 && cnt == 4;
        const int64_t plane = g.batch * g.M * g.N;
        const float* P = g.ws + (b * g.M + m) * g.N + n;
        v = sum_partials(P, plane, g.splits, vec, cnt);
    }
    if (mine) *reinterpret_cast<f4*>(Cs + row * LDC + col) = v;
    __syncthreads();
    epilogue_rows<RS, BN, EPI, NT>(Cs, LDC, m0, n0, b, g);
}

// ---- skinny M: up to 16 rows against a wide weight (decode steps, last-row heads) --------------------
// MFMA tiles of 32 or more rows waste most of their work on a handful of rows, and the launch is
// bound by streaming B from HBM anyway, so these kernels stream B with 128-bit loads on the vector
// ALUs and keep the few A rows in LDS. Both end in the tile epilogue.
constexpr int kSkinnyBN = 64;  // NT column tile
constexpr int kSkinnyLDC = kSkinnyBN + 4;

// NN (B is K x N, N-contiguous): a workgroup owns W = 4 TX columns and the K range of one split,
// walked in chunks of CH = TY * R rows (TY = 256 / TX). Thread (ty, tx) = (tid / TX, tid % TX)
// accumulates columns 4 tx .. 4 tx + 3 over rows kb + ty + TY i of each chunk from the chunk's A
// columns in LDS. R is 16 rows for up to eight rows of A (a workgroup then has 64 KiB of B loads in
// flight and one chunk covers K up to 1024 at 16 columns) and 8 for sixteen, where the next
// chunk's loads are in flight while the current one is multiplied. A column's partial
// sums are added first across the lanes of each wave (xor shuffles over the ty bits), then over the
// waves in wave order. One split runs the epilogue; several write their partials to the workspace
// for splitk_reduce_kernel<W, EPI>.
template <int MB, int TX, int EPI, int R>
__global__ void __launch_bounds__(NT) skinny_nn_kernel(const Args g) {
    constexpr int T = NT, TY = T / TX, W = 4 * TX, CH = TY * R, LDC = W + 4, NW = T / kWave;
    constexpr int AU = MB * CH / T;  // A values each thread stages per chunk
    constexpr bool DB = R <= 8;      // register double-buffering of the chunks
    static_assert(AU * T == MB * CH && kWave % TX == 0, "chunk must split evenly");
    __shared__ __attribute__((aligned(16))) float As[MB * CH];
    __shared__ __attribute__((aligned(16))) float Ps[NW * MB * W];
    __shared__ __attribute__((aligned(16))) float Cs[MB * LDC];
    const int tid = threadIdx.x, tx = tid % TX, ty = tid / TX, lane = tid & (kWave - 1), wave = tid / kWave;
    const int64_t tile = blockIdx.x % g.tiles_n, split = blockIdx.x / g.tiles_n;
    const int64_t n0 = tile * W, n = n0 + 4 * tx;
    const int64_t k0 = split * g.kc, k1 = min(g.K, k0 + g.kc);
    const int cnt = n < g.N ? (g.N - n < 4 ? static_cast<int>(g.N - n) : 4) : 0;
    const bool vec = g.vec_b && cnt == 4;
    const float* A = g.a.p;
    const int64_t row_step = TY * g.b.ld;
    auto load = [&](f4* bv, float* av, int64_t kb) {
        const float* bp = g.b.p + (kb + ty) * g.b.ld + n;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t k = kb + ty + TY * r;
            bv[r] = (k < k1 && cnt > 0) ? ld4(bp + r * row_step, vec, cnt) : f4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < AU; ++u) {
            const int i = tid + T * u, m = i / CH;
            const int64_t k = kb + (i - m * CH);
            av[u] = (m < g.M && k < k1) ? A[m * g.a.ld + k] : 0.0f;
        }
    };
    f4 cur[R], nxt[DB ? R : 1];
    float acur[AU], anxt[DB ? AU : 1];
    load(cur, acur, k0);
    float acc[MB][4];
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[m][j] = 0.0f;
    for (int64_t kb = k0; kb < k1; kb += CH) {
        const bool more = kb + CH < k1;
        if constexpr (DB) {
            if (more) load(nxt, anxt, kb + CH);
        }
        __syncthreads();  // the previous chunk's A is consumed
#pragma unroll
        for (int u = 0; u < AU; ++u) As[tid + T * u] = acur[u];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                const float a = As[m * CH + ty + TY * r];
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[m][j] += a * cur[r][j];
            }
        }
        if (more) {
            if constexpr (DB) {
#pragma unroll
                for (int r = 0; r < R; ++r) cur[r] = nxt[r];
#pragma unroll
                for (int u = 0; u < AU; ++u) acur[u] = anxt[u];
            } else {
                load(cur, acur, kb + CH);
            }
        }
    }
    // Across the lanes of a wave that share tx, then over the waves in order.
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v = acc[m][j];
#pragma unroll
            for (int o = TX; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
            acc[m][j] = v;
        }
    if (lane < TX) {
#pragma unroll
        for (int m = 0; m < MB; ++m)
            *reinterpret_cast<f4*>(Ps + (wave * MB + m) * W + 4 * tx) = f4{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
    }
    __syncthreads();
    for (int o = tid; o < MB * W; o += T) {
        const int m = o / W, c = o - m * W;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += Ps[(w * MB + m) * W + c];
        Cs[m * LDC + c] = v;
    }
    __syncthreads();
    if (g.splits == 1) {
        epilogue_rows<MB, W, EPI, T>(Cs, LDC, 0, n0, 0, g);
        return;
    }
    const int64_t plane = g.M * g.N;
    for (int i = tid; i < MB * W; i += T) {
        const int m = i / W, c = i - m * W;
        if (m < g.M && n0 + c < g.N) g.ws[split * plane + m * g.N + n0 + c] = Cs[m * LDC + c];
    }
}

// NT (B is N x K, K-contiguous: a tied head's table): a workgroup owns 64 columns; each 16-lane
// group takes four of them (group + 16 c) and walks K in float4 steps, lane l at 4 l + 64 i, so a
// group streams 256 contiguous bytes of each column's row per step. A (MB x K) sits in LDS.
// The 16 lane sums are combined with xor shuffles inside the group.
template <int MB, int EPI>
__global__ void __launch_bounds__(NT) skinny_nt_kernel(const Args g) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* As = smem;                         // MB x kpad
    float* Cs = smem + MB * g.kc;             // MB x kSkinnyLDC (kc = K rounded up to 64 here)
    const int tid = threadIdx.x, lane = tid & 15, grp = tid >> 4;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kSkinnyBN;
    const int64_t kp = g.kc;
    const int kpi = static_cast<int>(kp);  // at most 16K floats of LDS
    for (int i = tid; i < MB * kpi; i += NT) {
        const int m = i / kpi, k = i - m * kpi;
        As[i] = (m < g.M && k < g.K) ? g.a.p[m * g.a.ld + k] : 0.0f;
    }
    __syncthreads();
    const float* B = g.b.p;
    float acc[4][MB];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int m = 0; m < MB; ++m) acc[c][m] = 0.0f;
    const float* rows[4];
    bool live[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int64_t n = n0 + grp + 16 * c;
        live[c] = n < g.N;
        rows[c] = B + (live[c] ? n : 0) * g.b.ld;
    }
    for (int64_t k = 4 * lane; k < kp; k += 64) {
        const int cnt = g.K - k >= 4 ? 4 : (g.K > k ? static_cast<int>(g.K - k) : 0);
        const bool vec = g.vec_b && cnt == 4;
        f4 bv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) bv[c] = (live[c] && cnt > 0) ? ld4(rows[c] + k, vec, cnt) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            const f4 av = *reinterpret_cast<const f4*>(As + m * kp + k);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                acc[c][m] += av[0] * bv[c][0] + av[1] * bv[c][1] + av[2] * bv[c][2] + av[3] * bv[c][3];
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            float v = acc[c][m];
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
            acc[c][m] = v;
        }
    if (lane == 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int m = 0; m < MB; ++m) Cs[m * kSkinnyLDC + grp + 16 * c] = acc[c][m];
    }
    __syncthreads();
    epilogue_rows<MB, kSkinnyBN, EPI, NT>(Cs, kSkinnyLDC, 0, n0, 0, g);
}

#define PXK_KSET(TA, TB, P, EPI)                                                                    \
    {gemm_kernel<C128, TA, TB, P, EPI>, gemm_kernel<C64, TA, TB, P, EPI>, gemm_kernel<C32x64, TA, TB, P, EPI>, \
     gemm_kernel<C32, TA, TB, P, EPI>, gemm_direct_kernel<C32x64, TA, TB, P, EPI>,                         \
     gemm_direct_kernel<C32, TA, TB, P, EPI>, gemm_direct_kernel<C32x48, TA, TB, P, EPI>,                  \
     gemm_kernel<C32x48, TA, TB, P, EPI>}
#define PXK_GEMM_ENTRY(TA, TB, PRO, EPI)                                                                   \
    Entry {                                                                                                \
        TA, TB, PRO, EPI, {PXK_KSET(TA, TB, PRO, EPI), PXK_KSET(TA, TB, (PRO == PXK_PRO_DIV_STAB ? kProStabBias : PRO), EPI)}, \
            {splitk_reduce_kernel<128, EPI>, splitk_reduce_kernel<64, EPI>, splitk_reduce_kernel<64, EPI>, \
             splitk_reduce_kernel<32, EPI>, splitk_reduce_kernel<64, EPI>, splitk_reduce_kernel<32, EPI>,   \
             splitk_reduce_kernel<48, EPI>, splitk_reduce_kernel<48, EPI>},                                 \
    }

constexpr int skinny_rows(int mb) { return mb == 4 ? 16 : (mb == 8 ? 16 : 8); }
#define PXK_SKINNY_NN_W(MB, EPI)                                                                        \
    {skinny_nn_kernel<MB, 16, EPI, skinny_rows(MB)>, skinny_nn_kernel<MB, 8, EPI, skinny_rows(MB)>, \
     skinny_nn_kernel<MB, 4, EPI, skinny_rows(MB)>}
#define PXK_SKINNY_NN(EPI)                                                                                        \
    SkinnyEntry {                                                                                                 \
        0, EPI, {PXK_SKINNY_NN_W(4, EPI), PXK_SKINNY_NN_W(8, EPI), PXK_SKINNY_NN_W(16, EPI)},                    \
            {splitk_reduce_kernel<64, EPI>, splitk_reduce_kernel<32, EPI>, splitk_reduce_kernel<16, EPI>}         \
    }

}  // namespace
}  // namespace pxk
