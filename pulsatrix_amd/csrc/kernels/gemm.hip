// gemm.hip -- the fused fp32 MFMA GEMM for gfx950 (pxk_gemm, include/pxk.h).
//
// Tiling. A workgroup of 256 threads (4 wave64s in a 2x2 grid) owns a BM x BN output tile
// (64x64 or 128x128). K advances in blocks of 16 staged through LDS, double-buffered: the next
// block's global loads are in flight while the MFMA pipe works on the current one. LDS holds A as
// [BM][16+4] and B as [BN][16+4], both K-contiguous, so each lane fetches its MFMA operands for a
// whole K block with one 128-bit ds_read per 16x16 sub-tile.
//
// MFMA mapping. v_mfma_f32_16x16x4_f32 multiplies a 16x4 by a 4x16 fragment; lane l supplies
// A[l%16][kk] and B[kk][l%16] with kk = l/16, and holds D[4*(l/16)+r][l%16] in its r-th result
// register. Lane group g = l/16 is given K indices 4g..4g+3 of the block, one per MFMA step, so
// four steps cover the 16-wide block with operands read as float4 from LDS.
//
// Epilogue. The accumulator tile is staged through LDS and then walked row-major by the whole
// workgroup, so global writes (and the reads of epilogue operands) are coalesced and an element
// can see its RoPE pair partner. Split-K writes raw partials to a workspace instead; a second
// kernel sums them in split order (deterministic, no atomics) and runs the same tile epilogue.
#include <cstring>

#include "common.hpp"

namespace pxk {
namespace {

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
    const float* cos_t;
    const float* sin_t;
    int64_t head_dim;
    int rope_half;
    int vec_a, vec_b;
    float* ws;
};

__device__ __forceinline__ const float* obase(const Op& o, int64_t b, int64_t inner, int64_t s) {
    const int64_t bo = b / inner, bi = b % inner;
    const int64_t d = o.div > 1 ? o.div : 1;
    return o.p + bo * o.so + (bi / d) * o.si + s * o.sg;
}
__device__ __forceinline__ float* obase_w(const Op& o, int64_t b, int64_t inner) {
    return const_cast<float*>(obase(o, b, inner, 0));
}

constexpr int BK = 16;
constexpr int LDK = BK + 4;
constexpr int NT = 256;

template <int BM, int BN>
struct Smem {
    static constexpr int AB = 2 * (BM + BN) * LDK;
    static constexpr int LDC = BN + 4;
    static constexpr int C = BM * LDC;
    static constexpr int SIZE = AB > C ? AB : C;
};

// ---- tile epilogue: acc tile in LDS (Cs[BM][LDC]) -> outputs --------------------------------------
template <int BM, int BN, int EPI>
__device__ void epilogue_tile(const float* Cs, int64_t m0, int64_t n0, int64_t b, const Args& g) {
    constexpr int LDC = Smem<BM, BN>::LDC;
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
    const float eps = g.eps;
#pragma unroll 4
    for (int e = tid; e < BM * BN; e += NT) {
        const int row = e / BN, col = e % BN;
        const int64_t m = m0 + row, n = n0 + col;
        if (m >= g.M || n >= g.N) continue;
        const float acc = Cs[row * LDC + col];
        if constexpr (EPI == PXK_EPI_STORE) {
            float* dst = C + m * g.c.ld + n;
            *dst = (g.beta == 0.0f) ? acc : g.beta * *dst + acc;
        } else if constexpr (EPI == PXK_EPI_STORE_BIAS) {
            C[m * g.c.ld + n] = acc;
            if (EB) C2[m * g.c2.ld + n] = acc + EB[n];
        } else if constexpr (EPI == PXK_EPI_ADD_RESID) {
            C[m * g.c.ld + n] = acc;
            float y = acc;
            if (EB) {
                y = acc + EB[n];
                C2[m * g.c2.ld + n] = y;
            }
            C3[m * g.c3.ld + n] = X[m * g.x.ld + n] + y;
        } else if constexpr (EPI == PXK_EPI_MUL_X) {
            float v = X[m * g.x.ld + n] * acc;
            if (Y) v = Y[m * g.y.ld + n] + v;
            C[m * g.c.ld + n] = v;
        } else if constexpr (EPI == PXK_EPI_SPV) {
            const float o = X[m * g.x.ld + n];
            const float r = o * acc;
            C[m * g.c.ld + n] = r / (2.0f * o + eps * ((o >= 0.0f) ? 1.0f : -1.0f));
        } else if constexpr (EPI == PXK_EPI_ROPE_REL) {
            // Pair (lo, hi) inside the head block holding n; the tile spans whole heads.
            const int64_t D = g.head_dim, half = D / 2;
            const int64_t d = n % D, hb = n - d;
            const int64_t i = g.rope_half ? (d < half ? d : d - half) : d / 2;
            const int64_t lo = hb + (g.rope_half ? i : 2 * i), hi = hb + (g.rope_half ? i + half : 2 * i + 1);
            const bool is_lo = (n == lo);
            const float acc_lo = Cs[row * LDC + (int)(lo - n0)], acc_hi = Cs[row * LDC + (int)(hi - n0)];
            const float y_lo = Y[m * g.y.ld + lo], y_hi = Y[m * g.y.ld + hi];
            const float r_lo = y_lo * acc_lo, r_hi = y_hi * acc_hi;  // bilinear share: Q (or K) * (S @ K)
            const float c = g.cos_t[m * half + i], s = g.sin_t[m * half + i];
            const float d0 = stab(y_lo, eps), d1 = stab(y_hi, eps);
            const float xv = X[m * g.x.ld + n];
            float r_in = 0.0f;
            if (is_lo) {
                r_in += (xv * c / d0) * r_lo;
                r_in += (xv * s / d1) * r_hi;
            } else {
                r_in += (xv * -s / d0) * r_lo;
                r_in += (xv * c / d1) * r_hi;
            }
            if (C) C[m * g.c.ld + n] = r_in;
            const float zb = EB ? Z[m * g.z.ld + n] + EB[n] : Z[m * g.z.ld + n];
            C2[m * g.c2.ld + n] = r_in / stab(zb, eps);
        } else if constexpr (EPI == PXK_EPI_VALUE_REL) {
            const float r = Y[m * g.y.ld + n] * acc;
            if (C) C[m * g.c.ld + n] = r;
            const float zb = EB ? Z[m * g.z.ld + n] + EB[n] : Z[m * g.z.ld + n];
            C2[m * g.c2.ld + n] = r / stab(zb, eps);
        } else if constexpr (EPI == PXK_EPI_SWIGLU_REL) {
            const float rh = X[m * g.x.ld + n] * acc;  // hidden * (g_down @ W_down^T)
            const float a = Y[m * g.y.ld + n], bb = W[m * g.w.ld + n];
            const float cc = a * bb;
            const float denom = 2.0f * cc + eps * ((cc >= 0.0f) ? 1.0f : -1.0f);
            const float rg = (a * bb / denom) * rh;  // lrp_math.hpp:41-45
            const float zg = EB ? Z2[m * g.z2.ld + n] + EB[n] : Z2[m * g.z2.ld + n];
            const float zu = EB2 ? Z3[m * g.z3.ld + n] + EB2[n] : Z3[m * g.z3.ld + n];
            C[m * g.c.ld + n] = rg / stab(zg, eps);
            C2[m * g.c2.ld + n] = rg / stab(zu, eps);
        }
    }
}

// ---- global -> register loads of one K block --------------------------------------------------------
template <int BM, int BN, bool TA, bool TB, int PRO>
struct Loader {
    static constexpr int AF = BM * BK / 4 / NT;  // float4 slots per thread (A)
    static constexpr int BF = BN * BK / 4 / NT;
    f4 ra[AF];
    f4 rb[BF];

    __device__ __forceinline__ void load(const Args& g, const float* A, const float* Z, const float* ZB,
                                         const float* B, int64_t m0, int64_t n0, int64_t k0) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < AF; ++i) {
            const int idx = tid + i * NT;
            int64_t r, c;  // stored coordinates: (row, first of 4 contiguous)
            if constexpr (!TA) {
                r = m0 + idx / (BK / 4);
                c = k0 + 4 * (idx % (BK / 4));
            } else {
                r = k0 + idx / (BM / 4);
                c = m0 + 4 * (idx % (BM / 4));
            }
            const int64_t rows = TA ? g.K : g.M, cols = TA ? g.M : g.K;
            f4 v = {0.f, 0.f, 0.f, 0.f};
            f4 zv = {0.f, 0.f, 0.f, 0.f};
            if (r < rows) {
                if (g.vec_a && c + 3 < cols) {
                    v = *reinterpret_cast<const f4*>(A + r * g.a.ld + c);
                    if constexpr (PRO == PXK_PRO_DIV_STAB) zv = *reinterpret_cast<const f4*>(Z + r * g.z.ld + c);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (c + j < cols) {
                            v[j] = A[r * g.a.ld + c + j];
                            if constexpr (PRO == PXK_PRO_DIV_STAB) zv[j] = Z[r * g.z.ld + c + j];
                        }
                }
                if constexpr (PRO == PXK_PRO_DIV_STAB) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int64_t kk = TA ? r : c + j;  // K index of this element
                        const bool in = TA ? true : (c + j < cols);
                        if (in) {
                            const float zz = ZB ? zv[j] + ZB[kk] : zv[j];
                            v[j] = v[j] / stab(zz, g.eps);
                        }
                    }
                }
            }
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < BF; ++i) {
            const int idx = tid + i * NT;
            int64_t r, c;
            if constexpr (TB) {
                r = n0 + idx / (BK / 4);
                c = k0 + 4 * (idx % (BK / 4));
            } else {
                r = k0 + idx / (BN / 4);
                c = n0 + 4 * (idx % (BN / 4));
            }
            const int64_t rows = TB ? g.N : g.K, cols = TB ? g.K : g.N;
            f4 v = {0.f, 0.f, 0.f, 0.f};
            if (r < rows) {
                if (g.vec_b && c + 3 < cols) {
                    v = *reinterpret_cast<const f4*>(B + r * g.b.ld + c);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (c + j < cols) v[j] = B[r * g.b.ld + c + j];
                }
            }
            rb[i] = v;
        }
    }

    // Registers -> LDS buffer (As [BM][LDK], Bs [BN][LDK], K contiguous).
    __device__ __forceinline__ void store(float* As, float* Bs) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < AF; ++i) {
            const int idx = tid + i * NT;
            if constexpr (!TA) {
                *reinterpret_cast<f4*>(As + (idx / (BK / 4)) * LDK + 4 * (idx % (BK / 4))) = ra[i];
            } else {
                const int kr = idx / (BM / 4), mc = 4 * (idx % (BM / 4));
#pragma unroll
                for (int j = 0; j < 4; ++j) As[(mc + j) * LDK + kr] = ra[i][j];
            }
        }
#pragma unroll
        for (int i = 0; i < BF; ++i) {
            const int idx = tid + i * NT;
            if constexpr (TB) {
                *reinterpret_cast<f4*>(Bs + (idx / (BK / 4)) * LDK + 4 * (idx % (BK / 4))) = rb[i];
            } else {
                const int kr = idx / (BN / 4), nc = 4 * (idx % (BN / 4));
#pragma unroll
                for (int j = 0; j < 4; ++j) Bs[(nc + j) * LDK + kr] = rb[i][j];
            }
        }
    }
};

__device__ __forceinline__ void tile_range(const Args& g, int64_t m0, int64_t bm, int64_t& k_lo, int64_t& k_hi) {
    k_lo = 0;
    k_hi = g.K;
    if (g.causal == PXK_CAUSAL_K_LE_M) k_hi = (m0 + bm < g.K) ? m0 + bm : g.K;
    if (g.causal == PXK_CAUSAL_K_GE_M) k_lo = (m0 / BK) * BK;
}

template <int BM, int BN, bool TA, bool TB, int PRO, int EPI>
__global__ void __launch_bounds__(NT) gemm_kernel(const Args g) {
    constexpr int TM = BM / 32, TN = BN / 32;  // 16x16 MFMA tiles per wave along M, N
    __shared__ __attribute__((aligned(16))) float smem[Smem<BM, BN>::SIZE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN, m0 = static_cast<int64_t>(blockIdx.y) * BM;
    const int64_t split = blockIdx.z % g.splits, b = blockIdx.z / g.splits;
    if (g.causal == PXK_CAUSAL_TRI && n0 > m0 + BM - 1) return;  // tile strictly above the diagonal

    int64_t k_lo, k_hi;
    tile_range(g, m0, BM, k_lo, k_hi);
    const int64_t nkb = k_hi > k_lo ? (k_hi - k_lo + BK - 1) / BK : 0;
    const int64_t per = (nkb + g.splits - 1) / g.splits;
    const int64_t kb0 = split * per, kb1 = (kb0 + per < nkb) ? kb0 + per : nkb;
    const int64_t nk = kb1 > kb0 ? kb1 - kb0 : 0;
    const int64_t total = nk * g.kgroups;

    f4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    Loader<BM, BN, TA, TB, PRO> ld;
    auto issue = [&](int64_t t) {
        const int64_t s = t / nk, kb = kb0 + t % nk;
        const float* A = obase(g.a, b, g.inner, s);
        const float* B = obase(g.b, b, g.inner, s);
        const float* Z = PRO ? obase(g.z, b, g.inner, s) : nullptr;
        const float* ZB = (PRO && g.zb.p) ? obase(g.zb, b, g.inner, s) : nullptr;
        ld.load(g, A, Z, ZB, B, m0, n0, k_lo + kb * BK);
    };

    float* As0 = smem;
    float* Bs0 = smem + BM * LDK;
    float* As1 = smem + (BM + BN) * LDK;
    float* Bs1 = As1 + BM * LDK;

    if (total > 0) {
        issue(0);
        ld.store(As0, Bs0);
        __syncthreads();
    }
    for (int64_t t = 0; t < total; ++t) {
        const bool cur0 = (t & 1) == 0;
        const float* As = cur0 ? As0 : As1;
        const float* Bs = cur0 ? Bs0 : Bs1;
        if (t + 1 < total) issue(t + 1);
        f4 af[TM], bf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            af[i] = *reinterpret_cast<const f4*>(As + (wm + i * 16 + (lane & 15)) * LDK + 4 * (lane >> 4));
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bf[j] = *reinterpret_cast<const f4*>(Bs + (wn + j * 16 + (lane & 15)) * LDK + 4 * (lane >> 4));
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
        if (t + 1 < total) {
            ld.store(cur0 ? As1 : As0, cur0 ? Bs1 : Bs0);
        }
        __syncthreads();
    }

    if (g.splits > 1) {  // raw partial tile -> workspace [split][batch][M][N]
        float* P = g.ws + ((split * g.batch + b) * g.M) * g.N;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t m = m0 + wm + i * 16 + 4 * (lane >> 4) + r, n = n0 + wn + j * 16 + (lane & 15);
                    if (m < g.M && n < g.N) P[m * g.N + n] = acc[i][j][r];
                }
        return;
    }
    constexpr int LDC = Smem<BM, BN>::LDC;
    float* Cs = smem;  // the loop ended on a barrier: LDS is free
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                Cs[(wm + i * 16 + 4 * (lane >> 4) + r) * LDC + wn + j * 16 + (lane & 15)] = acc[i][j][r];
    __syncthreads();
    epilogue_tile<BM, BN, EPI>(Cs, m0, n0, b, g);
}

// Sums the split partials of one tile in split order and runs the tile epilogue.
template <int BM, int BN, int EPI>
__global__ void __launch_bounds__(NT) splitk_reduce_kernel(const Args g) {
    constexpr int LDC = Smem<BM, BN>::LDC;
    __shared__ float Cs[BM * LDC];
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN, m0 = static_cast<int64_t>(blockIdx.y) * BM;
    const int64_t b = blockIdx.z;
    if (g.causal == PXK_CAUSAL_TRI && n0 > m0 + BM - 1) return;
    const int64_t plane = g.batch * g.M * g.N;
    for (int e = threadIdx.x; e < BM * BN; e += NT) {
        const int row = e / BN, col = e % BN;
        const int64_t m = m0 + row, n = n0 + col;
        float s = 0.0f;
        if (m < g.M && n < g.N) {
            const float* P = g.ws + (b * g.M + m) * g.N + n;
            for (int k = 0; k < g.splits; ++k) s += P[k * plane];
        }
        Cs[row * LDC + col] = s;
    }
    __syncthreads();
    epilogue_tile<BM, BN, EPI>(Cs, m0, n0, b, g);
}

// ---- host side --------------------------------------------------------------------------------

using KernelFn = void (*)(const Args);

struct Entry {
    int ta, tb, pro, epi;
    KernelFn k64, k128, r64, r128;
};

#define PXK_GEMM_ENTRY(TA, TB, PRO, EPI)                                                                     \
    Entry {                                                                                                  \
        TA, TB, PRO, EPI, gemm_kernel<64, 64, TA, TB, PRO, EPI>, gemm_kernel<128, 128, TA, TB, PRO, EPI>,    \
            splitk_reduce_kernel<64, 64, EPI>, splitk_reduce_kernel<128, 128, EPI>                           \
    }

const Entry kTable[] = {
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_STORE),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_NONE, PXK_EPI_STORE),
    PXK_GEMM_ENTRY(1, 0, PXK_PRO_NONE, PXK_EPI_STORE),
    PXK_GEMM_ENTRY(1, 1, PXK_PRO_NONE, PXK_EPI_STORE),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_STORE_BIAS),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_ADD_RESID),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_MUL_X),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_NONE, PXK_EPI_MUL_X),
    PXK_GEMM_ENTRY(1, 0, PXK_PRO_NONE, PXK_EPI_MUL_X),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_DIV_STAB, PXK_EPI_MUL_X),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_DIV_STAB, PXK_EPI_MUL_X),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_DIV_STAB, PXK_EPI_SPV),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_ROPE_REL),
    PXK_GEMM_ENTRY(1, 0, PXK_PRO_NONE, PXK_EPI_ROPE_REL),
    PXK_GEMM_ENTRY(0, 0, PXK_PRO_NONE, PXK_EPI_VALUE_REL),
    PXK_GEMM_ENTRY(1, 0, PXK_PRO_NONE, PXK_EPI_VALUE_REL),
    PXK_GEMM_ENTRY(0, 1, PXK_PRO_DIV_STAB, PXK_EPI_SWIGLU_REL),
};

const Entry* find_entry(int ta, int tb, int pro, int epi) {
    for (const Entry& e : kTable)
        if (e.ta == ta && e.tb == tb && e.pro == pro && e.epi == epi) return &e;
    return nullptr;
}

Op to_op(const pxk_operand& o) {
    return Op{o.ptr, o.ld, o.batch_stride, o.inner_stride, o.inner_div, o.group_stride};
}

bool vec_ok(const pxk_operand& o, int64_t contiguous_extent) {
    if (o.ptr == nullptr) return true;
    return aligned16(o.ptr) && o.ld % 4 == 0 && o.batch_stride % 4 == 0 && o.inner_stride % 4 == 0 &&
           o.group_stride % 4 == 0 && contiguous_extent % 4 == 0;
}

struct Plan {
    const Entry* e;
    int bm, bn, splits;
    int64_t tiles_m, tiles_n;
};

int plan(const pxk_gemm_desc* d, Plan* p) {
    if (d->m <= 0 || d->n <= 0 || d->batch <= 0) return fail(PXK_ERR_INVALID, "pxk_gemm: m, n and batch must be positive");
    if (d->k < 0 || d->inner <= 0 || d->kgroups <= 0 || d->batch % d->inner != 0)
        return fail(PXK_ERR_INVALID, "pxk_gemm: bad k, inner or kgroups (batch must be a multiple of inner)");
    if (d->causal < 0 || d->causal > 3) return fail(PXK_ERR_INVALID, "pxk_gemm: unknown causal mode %d", d->causal);
    p->e = find_entry(d->trans_a != 0, d->trans_b != 0, d->prologue, d->epilogue);
    if (!p->e)
        return fail(PXK_ERR_INVALID, "pxk_gemm: combination trans_a=%d trans_b=%d prologue=%d epilogue=%d is not built",
                    d->trans_a, d->trans_b, d->prologue, d->epilogue);
    if (d->a.ptr == nullptr || d->b.ptr == nullptr) return fail(PXK_ERR_INVALID, "pxk_gemm: A and B are required");
    // Outputs and inputs each epilogue needs.
    const int epi = d->epilogue;
    const bool need_c = !(epi == PXK_EPI_ROPE_REL || epi == PXK_EPI_VALUE_REL);
    if (need_c && d->c.ptr == nullptr) return fail(PXK_ERR_INVALID, "pxk_gemm: output C is required");
    if ((epi == PXK_EPI_ADD_RESID) && (d->c3.ptr == nullptr || d->x.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: ADD_RESID needs C3 and X");
    if ((epi == PXK_EPI_ADD_RESID || epi == PXK_EPI_STORE_BIAS) && d->e_bias.ptr && d->c2.ptr == nullptr)
        return fail(PXK_ERR_INVALID, "pxk_gemm: a bias needs output C2");
    if ((epi == PXK_EPI_MUL_X || epi == PXK_EPI_SPV || epi == PXK_EPI_SWIGLU_REL || epi == PXK_EPI_ROPE_REL) &&
        d->x.ptr == nullptr)
        return fail(PXK_ERR_INVALID, "pxk_gemm: epilogue %d needs X", epi);
    if ((epi == PXK_EPI_ROPE_REL || epi == PXK_EPI_VALUE_REL) &&
        (d->y.ptr == nullptr || d->z.ptr == nullptr || d->c2.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: epilogue %d needs Y, Z and C2", epi);
    if (epi == PXK_EPI_SWIGLU_REL && (d->y.ptr == nullptr || d->c2.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: SWIGLU_REL needs Y and C2");
    if (epi == PXK_EPI_SWIGLU_REL && (d->w.ptr == nullptr || d->z2.ptr == nullptr || d->z3.ptr == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_gemm: SWIGLU_REL needs W, Z2 and Z3");
    if (d->prologue == PXK_PRO_DIV_STAB && d->z.ptr == nullptr)
        return fail(PXK_ERR_INVALID, "pxk_gemm: the DIV_STAB prologue needs Z");
    if (d->prologue == PXK_PRO_DIV_STAB && (epi == PXK_EPI_ROPE_REL || epi == PXK_EPI_VALUE_REL))
        return fail(PXK_ERR_INVALID, "pxk_gemm: epilogue %d reads Z, which the DIV_STAB prologue owns", epi);
    if (epi == PXK_EPI_ROPE_REL) {
        const int64_t D = d->head_dim;
        if (D <= 0 || D % 2 != 0 || d->cos_t == nullptr || d->sin_t == nullptr)
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_REL needs an even head_dim and cos/sin tables");
        if (!(d->n <= 64 || (64 % D == 0 && d->n % D == 0)))
            return fail(PXK_ERR_INVALID, "pxk_gemm: ROPE_REL needs whole heads inside a 64-wide tile");
    }
    // Tile size: big tiles when they still give the chip a few waves of workgroups.
    const double tri = d->causal == PXK_CAUSAL_TRI ? 0.5 : 1.0;
    const int64_t t128 = cdiv(d->m, 128) * cdiv(d->n, 128) * d->batch;
    const bool big = (epi != PXK_EPI_ROPE_REL) && t128 * tri >= 512 && d->m >= 128 && d->n >= 128;
    p->bm = p->bn = big ? 128 : 64;
    p->tiles_m = cdiv(d->m, p->bm);
    p->tiles_n = cdiv(d->n, p->bn);
    // Split-K when the tiles alone leave most CUs idle and K is long.
    int splits = d->splits;
    if (splits <= 0) {
        const double tiles = static_cast<double>(p->tiles_m * p->tiles_n * d->batch) * tri;
        const int64_t kwork = d->k * d->kgroups;
        splits = 1;
        while (tiles * splits < 384 && kwork / (splits * 2) >= 256 && splits < 64) splits *= 2;
    }
    if (splits > 1 && d->beta != 0.0f) splits = 1;  // beta reads C: keep it single-pass
    p->splits = splits;
    return PXK_OK;
}

}  // namespace
}  // namespace pxk

using namespace pxk;

extern "C" int pxk_gemm_supported(int ta, int tb, int pro, int epi) { return find_entry(ta != 0, tb != 0, pro, epi) != nullptr; }

extern "C" size_t pxk_gemm_workspace(const pxk_gemm_desc* d) {
    Plan p;
    if (plan(d, &p) != PXK_OK || p.splits <= 1) return 0;
    return static_cast<size_t>(p.splits) * d->batch * d->m * d->n * sizeof(float);
}

extern "C" int pxk_gemm(const pxk_gemm_desc* d, void* stream) {
    if (d->m == 0 || d->n == 0 || d->batch == 0) return PXK_OK;
    Plan p;
    if (const int rc = plan(d, &p)) return rc;
    if (p.splits > 1) {
        const size_t need = static_cast<size_t>(p.splits) * d->batch * d->m * d->n * sizeof(float);
        if (d->workspace == nullptr || d->workspace_bytes < need) {
            if (d->splits > 1)
                return fail(PXK_ERR_WORKSPACE, "pxk_gemm: split-K %d needs %zu workspace bytes", p.splits, need);
            p.splits = 1;  // library-chosen split without a workspace: run single-pass
        }
    }
    Args g{};
    g.M = d->m;
    g.N = d->n;
    g.K = d->k;
    g.batch = d->batch;
    g.inner = d->inner;
    g.kgroups = d->kgroups;
    g.causal = d->causal;
    g.splits = p.splits;
    g.beta = d->beta;
    g.eps = d->eps;
    g.a = to_op(d->a);
    g.b = to_op(d->b);
    g.c = to_op(d->c);
    g.z = to_op(d->z);
    g.zb = to_op(d->z_bias);
    g.c2 = to_op(d->c2);
    g.c3 = to_op(d->c3);
    g.x = to_op(d->x);
    g.y = to_op(d->y);
    g.w = to_op(d->w);
    g.z2 = to_op(d->z2);
    g.z3 = to_op(d->z3);
    g.eb = to_op(d->e_bias);
    g.eb2 = to_op(d->e_bias2);
    g.cos_t = d->cos_t;
    g.sin_t = d->sin_t;
    g.head_dim = d->head_dim;
    g.rope_half = d->rope_half;
    g.ws = d->workspace;
    // 128-bit loads when every base, stride and the contiguous extent allow them.
    const int64_t a_ext = d->trans_a ? d->m : d->k, b_ext = d->trans_b ? d->k : d->n;
    g.vec_a = vec_ok(d->a, a_ext) && (d->prologue == PXK_PRO_NONE || vec_ok(d->z, a_ext));
    g.vec_b = vec_ok(d->b, b_ext);
    const dim3 grid(static_cast<unsigned>(p.tiles_n), static_cast<unsigned>(p.tiles_m),
                    static_cast<unsigned>(d->batch * p.splits));
    if (grid.y > 65535 || grid.z > 65535) return fail(PXK_ERR_INVALID, "pxk_gemm: grid too large");
    KernelFn k = p.bm == 128 ? p.e->k128 : p.e->k64;
    hipLaunchKernelGGL(k, grid, dim3(NT), 0, S(stream), g);
    if (const int rc = launched("pxk_gemm")) return rc;
    if (p.splits > 1) {
        const dim3 rgrid(static_cast<unsigned>(p.tiles_n), static_cast<unsigned>(p.tiles_m),
                         static_cast<unsigned>(d->batch));
        KernelFn r = p.bm == 128 ? p.e->r128 : p.e->r64;
        hipLaunchKernelGGL(r, rgrid, dim3(NT), 0, S(stream), g);
        return launched("pxk_gemm split-K reduce");
    }
    return PXK_OK;
}

extern "C" int pxk_gemm_ex(const float* a, int ta, const float* b, int tb, float* out, int64_t m, int64_t k, int64_t n,
                           float beta, float* workspace, size_t workspace_bytes, void* stream) {
    if (m == 0 || n == 0) return PXK_OK;
    pxk_gemm_desc d;
    std::memset(&d, 0, sizeof(d));
    d.m = m;
    d.n = n;
    d.k = k;
    d.batch = d.inner = d.kgroups = 1;
    d.trans_a = ta;
    d.trans_b = tb;
    d.epilogue = PXK_EPI_STORE;
    d.beta = beta;
    d.a = pxk_operand{a, ta ? m : k, 0, 0, 0, 0};
    d.b = pxk_operand{b, tb ? k : n, 0, 0, 0, 0};
    d.c = pxk_operand{out, n, 0, 0, 0, 0};
    d.workspace = workspace;
    d.workspace_bytes = workspace_bytes;
    return pxk_gemm(&d, stream);
}
