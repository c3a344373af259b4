// attention.hip -- fused causal GQA attention for gfx950 (include/pxk.h): scores, mask, softmax
// and P V in one launch, keeping what the AttnLRP pass reads (raw scores and P).
//
// Tiling. One workgroup owns 16 query rows of one query head; its four wave64s take the visible
// keys in 16-key tiles, round-robin. Scores are formed transposed, S^T = K Q^T, on
// v_mfma_f32_16x16x4_f32: lane l then holds S[row = l % 16][key = 4 (l / 16) + r] in its r-th
// result register, which is exactly the B-operand layout of ctx^T = V^T P^T. P therefore never
// leaves registers between the two products; a row's max and sum are in-lane reductions plus two
// wavefront shuffles (lanes l, l ^ 16, l ^ 32, l ^ 48 share a row). K and V are streamed from L2
// (the 16-row workgroups of one KV head re-read the same 2 x L x D floats) two tiles ahead, with
// no LDS staging and no barrier in the key loop.
//
// Softmax. Each wave runs an online softmax over its tiles (running max, rescaled sum and
// context); the four waves are merged in LDS in wave order at the end (deterministic). The raw
// scores of the workgroup's 16 rows wait in LDS meanwhile (16 x L floats), so the last pass
// writes raw and the normalized P = exp(scale * raw - max) / sum (DeviceBackend::softmax_rows,
// cpu_backend.cpp:292-310; the hardware exponential __expf on arguments <= 0, and one reciprocal
// per row) as whole contiguous row segments, 16 threads per row, reading nothing back from HBM. P is written over whole rows, zeros past the
// visible keys: the relevance pass reads it as a dense operand.
//
// Relevance (pxk_attention_relevance_q). The same workgroup tiling runs the AttnLRP steps of one
// query head that need whole score rows: the P V bilinear share r_attn = P * (s_pv V^T), formed
// as (V s_pv^T)^T so it lands in the score layout; the softmax rule and the Q K^T bilinear
// denominator, s = (scale raw)(r_attn - P sum r_attn) / (2 raw + eps sign raw); and the query
// share (s K), whose transposed product takes s straight from registers as its B operand, with
// the RoPE epsilon rule and q_proj's denominator applied per pair at the end. r_attn, then s, wait
// in LDS for the row sums and for the contiguous store of s (the key share reads it).
#include <algorithm>
#include <cmath>

#include "common.hpp"

namespace pxk {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kWaves = 4;

struct FwdArgs {
    const float* q;
    const float* k;
    const float* v;
    float* raw;
    float* p;
    float* ctx;
    int64_t ldq, ldk, ldv, ldctx;
    int n, l, heads, kv_heads, D;
    float scale;
    int causal;
    int lds_ld;    // row stride of the LDS score block
    float* stats;  // nullable: (n, heads, l, 2) the rows' softmax max of scale * raw and 1 / sum
    int keep;      // raw or P is written: the raw scores wait in LDS for the last pass
};

// Lane l's value and lane (l ^ 16)'s, or (l ^ 32)'s, one in each half of the pair: v_permlane16_swap
// (odd 16-lane rows of the first operand with even rows of the second) and v_permlane32_swap (upper
// half with lower half) on two copies of v. They are VALU operations, where a shuffle is an LDS
// permute and a wait on it. Every lane of the wave must be active.
__device__ __forceinline__ void pair16(float v, float& x, float& y) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    x = __uint_as_float(r[0]);
    y = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair32(float v, float& x, float& y) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    x = __uint_as_float(r[0]);
    y = __uint_as_float(r[1]);
}
// Over the four lanes c, c + 16, c + 32, c + 48 (one score row), pairs at distance 16 first.
__device__ __forceinline__ float row_max4(float v) {
    float x, y;
    pair16(v, x, y);
    pair32(fmaxf(x, y), x, y);
    return fmaxf(x, y);
}
__device__ __forceinline__ float row_sum4(float v) {
    float x, y;
    pair16(v, x, y);
    pair32(x + y, x, y);
    return x + y;
}

// Byte range of the forward's K or V tile resource, counted from the tile's first row (key0) of one
// head's column segment in a row-major (rows, ldr) operand: it ends with the head's D values of the
// sequence's last row (l - 1). One definition for the kernel and for pxk_attention_kv_tile_records,
// which checks it on the host.
__host__ __device__ inline int kv_tile_records(int l, int key0, int ldr, int D) {
    return ((l - 1 - key0) * ldr + D) * 4;
}

// DT: head_dim in 16-wide tiles (D <= 16 DT, D % 4 == 0). VEC: l % 4 == 0 (128-bit row stores).
template <int DT, bool VEC>
__global__ void __launch_bounds__(kThreads) attn_fwd_kernel(const FwdArgs a) {
    extern __shared__ __attribute__((aligned(16))) float sc[];  // [16][lds_ld] raw scores of the block's rows
    __shared__ float s_m[kWaves][16], s_s[kWaves][16];
    __shared__ __attribute__((aligned(16))) float s_ctx[kWaves][16][16 * DT + 4];
    __shared__ float f_m[16], f_s[16];

    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: the tile loop is scalar
    const int l = a.l, D = a.D, ld = a.lds_ld;
    const int nrb = (l + 15) / 16;
    // Long causal rows first, heads fastest: the heaviest blocks start first and spread over the CUs.
    const int nbh = a.n * a.heads;
    const int rb = nrb - 1 - static_cast<int>(blockIdx.x) / nbh, bh = static_cast<int>(blockIdx.x) % nbh;
    const int h = bh % a.heads, b = bh / a.heads;
    const int hk = h / (a.heads / a.kv_heads);
    const int i0 = rb * 16, row = i0 + c;
    const bool row_ok = row < l;

    // Q^T fragments: qf[t][s] = Q[row][16 t + 4 g + s].
    f4 qf[DT];
    {
        const float* qp = a.q + (static_cast<int64_t>(b) * l + (row_ok ? row : l - 1)) * a.ldq + h * D;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            // Unconditional loads (clamped column), then a zero factor for columns past head_dim:
            // no branch around the loads, so the key loop inherits no pending-load state.
            const int d0 = 16 * t + 4 * g;
            qf[t] = *reinterpret_cast<const f4*>(qp + min(d0, D - 4)) * (d0 < D ? 1.0f : 0.0f);
        }
    }
    const float* kbase = a.k + static_cast<int64_t>(b) * l * a.ldk + hk * D;
    const float* vbase = a.v + static_cast<int64_t>(b) * l * a.ldv + hk * D;
    const int vis_end = a.causal ? min(i0 + 16, l) : l;
    const int ntile = (vis_end + 15) / 16;
    const int last_key = a.causal ? min(row, l - 1) : l - 1;  // the lane's row sees keys 0 .. last_key

    float m = -INFINITY, ssum = 0.0f;
    f4 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};

    // Operands of one 16-key tile: kf[t][s] = K[key0 + c][16 t + 4 g + s] (A of S^T) and
    // vf[t][s] = V[key0 + 4 g + s][16 t + c] (A of ctx^T). Two register sets per wave: while one
    // tile is on the MFMA pipe the next one's K and V are in flight. A set is reloaded right after
    // its last read (K after the score MFMAs, V after the context MFMAs), so old and new values
    // never live at once and the loop needs no register copies (a copy of a register with a load
    // pending would wait for that load).
    //
    // The loads are buffer loads: a tile's rows start at a scalar base (the buffer resource, built
    // per tile with scalar instructions) and each lane's offsets are fixed for the whole loop, with
    // the head-dimension step in the instruction's immediate offset, so a tile costs no vector
    // address arithmetic. The resource's range (kv_tile_records) ends with the head's D values of
    // the sequence's last row: rows past the sequence, and columns past head_dim on that last row,
    // fall outside it and read 0 (a V row there meets a zero probability anyway), so no load ever
    // leaves the operand. Columns past head_dim on earlier rows read finite neighbouring data of the
    // same matrix (a K column there meets a zero Q fragment, a ctx row there is never stored).
    f4 kf[2][DT], vf[2][DT];
    const int ldk = static_cast<int>(a.ldk), ldv = static_cast<int>(a.ldv);
    const int koff = (c * ldk + 4 * g) * 4, voff = ((4 * g) * ldv + c) * 4;
    auto rsrc = [&](const float* base, int key0, int ldr) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base + key0 * ldr), 0,
                                                 kv_tile_records(l, key0, ldr, D), 0x00020000);
    };
    auto load_k = [&](int set, int kt) {
        const int key0 = 16 * min(kt, ntile - 1);  // past the last tile: the last one again, unused
        const __amdgpu_buffer_rsrc_t r = rsrc(kbase, key0, ldk);
#pragma unroll
        for (int t = 0; t < DT; ++t)
            kf[set][t] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, koff + 64 * t, 0, 0));
    };
    auto load_v = [&](int set, int kt) {
        const int key0 = 16 * min(kt, ntile - 1);
        const __amdgpu_buffer_rsrc_t r = rsrc(vbase, key0, ldv);
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int t = 0; t < DT; ++t)
                vf[set][t][st] =
                    __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff + st * ldv * 4 + 64 * t, 0, 0));
    };
    auto tile = [&](int set, int kt) {
        const int key0 = 16 * kt;
        // S^T tile = K[key0 .. key0 + 15] Q^T over the head dimension.
        f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int st = 0; st < 4; ++st) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[set][t][st], qf[t][st], s, 0, 0, 0);
        // The reloads stay where they are written: the scheduler would otherwise sink them to the
        // end of the loop body and the next tile would wait for them.
        __builtin_amdgcn_sched_barrier(0);
        load_k(set, kt + 2 * kWaves);
        __builtin_amdgcn_sched_barrier(0);
        // s[r] = raw score of (row, key0 + 4 g + r), kept in LDS for the last pass.
        const int kk0 = key0 + 4 * g;
        // A tile past the last one (the second of a pair) lands on column block ntile, inside the
        // LDS row and past every visible key of this block: written, never read.
        if (a.keep) *reinterpret_cast<f4*>(sc + c * ld + 16 * min(kt, ntile) + 4 * g) = s;
        float x[4];
        bool valid[4];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            valid[r] = kk0 + r <= last_key;
            x[r] = a.scale * s[r];
            mt = fmaxf(mt, valid[r] ? x[r] : -INFINITY);
        }
        mt = row_max4(mt);
        const float m_new = fmaxf(m, mt);
        const float alpha = m_new == -INFINITY ? 1.0f : __expf(m - m_new);
        float e[4];
        float part = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            e[r] = valid[r] ? __expf(x[r] - m_new) : 0.0f;
            part += e[r];
        }
        ssum = ssum * alpha + part;
        m = m_new;
        // ctx^T (D x rows) += V^T (D x keys) P^T (keys x rows); the rescale is per row = per lane.
        // The rescale is skipped (wave-uniformly) once no row's running max moved, which is most
        // tiles after the first few; it multiplies by exactly 1 otherwise.
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int t = 0; t < DT; ++t) acc[t] *= alpha;
        }
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int st = 0; st < 4; ++st)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[set][t][st], e[st], acc[t], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_v(set, kt + 2 * kWaves);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Tiles go in pairs, the second one unconditionally: past the last tile every key of it is
    // masked (keys >= 16 ntile are past the diagonal, or past l), so it leaves m, the sum and the
    // context unchanged. No branch splits the load stream.
    load_k(0, wave);
    load_v(0, wave);
    // The first set and Q have landed before the second set is requested: it overlaps the first
    // tile, and the loop head's wait covers only the loop's own reloads (two tiles ahead).
    __builtin_amdgcn_s_waitcnt(0);
    load_k(1, wave + kWaves);
    load_v(1, wave + kWaves);
    for (int kt = wave; kt < ntile; kt += 2 * kWaves) {
        tile(0, kt);
        tile(1, kt + kWaves);
    }

    // Merge the four waves: acc[t][r] = ctx^T[16 t + 4 g + r][row c] of this wave.
    ssum = row_sum4(ssum);
    if (g == 0) {
        s_m[wave][c] = m;
        s_s[wave][c] = ssum;
    }
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_ctx[wave][c][16 * t + 4 * g + r] = acc[t][r];
    __syncthreads();
    const int rr = threadIdx.x >> 4, cc = threadIdx.x & 15;  // 16 rows x 16 threads
    const int orow = i0 + rr;
    {
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][rr]);
        float wsc[kWaves];
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            wsc[w] = s_m[w][rr] == -INFINITY ? 0.0f : __expf(s_m[w][rr] - mx);
            tot += s_s[w][rr] * wsc[w];
        }
        if (cc == 0) {
            f_m[rr] = mx;
            f_s[rr] = tot;
            if (a.stats && orow < l) {
                float* st = a.stats + 2 * (((static_cast<int64_t>(b) * a.heads + h) * l) + orow);
                st[0] = mx;
                st[1] = 1.0f / tot;
            }
        }
        if (orow < l) {
            float* cp = a.ctx + (static_cast<int64_t>(b) * l + orow) * a.ldctx + h * D;
            for (int d = cc; d < D; d += 16) {
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) v += s_ctx[w][rr][d] * wsc[w];
                cp[d] = v / tot;
            }
        }
    }
    if (!a.keep) return;  // uniform: the statistics form writes no score rows
    __syncthreads();

    // raw (visible keys) and P (every key, zeros past the visible ones) as contiguous row segments.
    if (orow < l) {
        const float mx = f_m[rr], inv = 1.0f / f_s[rr];
        const int vis = a.causal ? orow + 1 : l;
        const int64_t off = ((static_cast<int64_t>(b) * a.heads + h) * l + orow) * l;
        float* prow = a.p ? a.p + off : nullptr;
        float* rrow = a.raw ? a.raw + off : nullptr;
        const float* srow = sc + rr * ld;
        if constexpr (VEC) {
            for (int k0 = 4 * cc; k0 < l; k0 += 64) {
                f4 out = {0.f, 0.f, 0.f, 0.f};
                if (k0 < vis) {
                    const f4 x = *reinterpret_cast<const f4*>(srow + k0);
                    if (!a.raw) {
                    } else if (k0 + 3 < vis) {
                        *reinterpret_cast<f4*>(rrow + k0) = x;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (k0 + r < vis) rrow[k0 + r] = x[r];
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) out[r] = k0 + r < vis ? __expf(a.scale * x[r] - mx) * inv : 0.0f;
                }
                if (a.p) *reinterpret_cast<f4*>(prow + k0) = out;
            }
        } else {
            for (int k = cc; k < l; k += 16) {
                float out = 0.0f;
                if (k < vis) {
                    const float x = srow[k];
                    if (a.raw) rrow[k] = x;
                    out = __expf(a.scale * x - mx) * inv;
                }
                if (a.p) prow[k] = out;
            }
        }
    }
}

// GQA-shared forward (statistics form), for grids many times the chip's size: one workgroup per
// (sequence, KV head, 16-row block) and one wave per query head of the KV head's group, each wave
// over all of the block's key tiles with its own online softmax, so no merge. Every K / V tile
// comes from memory once per workgroup into LDS (two buffers: the next tile's loads are in flight
// while the current one is on the MFMAs) and feeds the G waves, where attn_fwd_kernel reads it once
// per query head through the vector memory path. Per wave the arithmetic is attn_fwd_kernel's, tile
// after tile.
template <int DT, int G>
__global__ void __launch_bounds__(G * kWave) attn_fwd_gqa_kernel(const FwdArgs a) {
    constexpr int NT = G * kWave, LD = 16 * DT + 4;
    constexpr int PER = (16 * 4 * DT + NT - 1) / NT;                      // float4 per thread per tile operand
    __shared__ __attribute__((aligned(16))) float kv_lds[2][2][16][LD];  // [buffer][K, V][key][dim]

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the query head
    const int l = a.l, D = a.D;
    const int nrb = (l + 15) / 16;
    // Long causal rows first, KV heads fastest.
    const int nbk = a.n * a.kv_heads;
    const int rb = nrb - 1 - static_cast<int>(blockIdx.x) / nbk, bk = static_cast<int>(blockIdx.x) % nbk;
    const int hk = bk % a.kv_heads, b = bk / a.kv_heads;
    const int h = hk * G + wave;
    const int i0 = rb * 16, row = i0 + c;
    const int last_key = a.causal ? min(row, l - 1) : l - 1;  // the lane's row sees keys 0 .. last_key
    const bool row_ok = row < l;

    // Q^T fragments: qf[t][s] = Q[row][16 t + 4 g + s], zero past head_dim.
    f4 qf[DT];
    {
        const float* qp = a.q + (static_cast<int64_t>(b) * l + (row_ok ? row : l - 1)) * a.ldq + h * D;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const int d0 = 16 * t + 4 * g;
            qf[t] = *reinterpret_cast<const f4*>(qp + min(d0, D - 4)) * (d0 < D ? 1.0f : 0.0f);
        }
    }
    const float* kbase = a.k + static_cast<int64_t>(b) * l * a.ldk + hk * D;
    const float* vbase = a.v + static_cast<int64_t>(b) * l * a.ldv + hk * D;
    const int vis_end = a.causal ? min(i0 + 16, l) : l;
    const int ntile = (vis_end + 15) / 16;
    const int q4 = D / 4;

    // Columns past head_dim stay zero in both buffers: K's meet zero Q fragments, V's feed context
    // dims that are never stored.
    for (int i = tid; i < 2 * 2 * 16 * (16 * DT - D); i += NT) {
        const int w = 16 * DT - D, r = i / w, col = D + i - r * w;
        (&kv_lds[0][0][0][0])[r * LD + col] = 0.0f;
    }
    // A tile's 16 K rows and 16 V rows as float4 pieces over the workgroup, through per-tile buffer
    // resources (kv_tile_records, as in attn_fwd_kernel) and each thread's byte offsets, fixed for
    // the loop: rows past the sequence read 0 (their keys are masked and meet zero probabilities).
    f4 sk[PER], sv[PER];
    int koff[PER], voff[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int i = min(tid + NT * j, 16 * q4 - 1);
        const int r = i / q4, c4 = 4 * (i - r * q4);
        koff[j] = (r * static_cast<int>(a.ldk) + c4) * 4;
        voff[j] = (r * static_cast<int>(a.ldv) + c4) * 4;
    }
    auto fetch = [&](int kt) {
        const int key0 = 16 * kt;
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(kbase + key0 * a.ldk), 0, kv_tile_records(l, key0, static_cast<int>(a.ldk), D), 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(vbase + key0 * a.ldv), 0, kv_tile_records(l, key0, static_cast<int>(a.ldv), D), 0x00020000);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            sk[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff[j], 0, 0));
            sv[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff[j], 0, 0));
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = tid + NT * j;
            if (i < 16 * q4) {
                const int r = i / q4, c4 = 4 * (i - r * q4);
                *reinterpret_cast<f4*>(&kv_lds[buf][0][r][c4]) = sk[j];
                *reinterpret_cast<f4*>(&kv_lds[buf][1][r][c4]) = sv[j];
            }
        }
    };

    float m = -INFINITY, ssum = 0.0f;
    f4 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    fetch(0);
    stash(0);
    __syncthreads();
    for (int kt = 0; kt < ntile; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ntile) fetch(kt + 1);  // uniform
        // S^T tile = K[16 kt .. 16 kt + 15] Q^T over the head dimension.
        f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const f4 kf = *reinterpret_cast<const f4*>(&kv_lds[buf][0][c][16 * t + 4 * g]);
#pragma unroll
            for (int st = 0; st < 4; ++st) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[st], qf[t][st], s, 0, 0, 0);
        }
        // s[r] = raw score of (row, 16 kt + 4 g + r); the online softmax step of attn_fwd_kernel.
        const int kk0 = 16 * kt + 4 * g;
        float x[4];
        bool valid[4];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            valid[r] = kk0 + r <= last_key;
            x[r] = a.scale * s[r];
            mt = fmaxf(mt, valid[r] ? x[r] : -INFINITY);
        }
        mt = row_max4(mt);
        const float m_new = fmaxf(m, mt);
        const float alpha = m_new == -INFINITY ? 1.0f : __expf(m - m_new);
        float e[4];
        float part = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            e[r] = valid[r] ? __expf(x[r] - m_new) : 0.0f;
            part += e[r];
        }
        ssum = ssum * alpha + part;
        m = m_new;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int t = 0; t < DT; ++t) acc[t] *= alpha;
        }
        // ctx^T (D x rows) += V^T (D x keys) P^T (keys x rows): vf = V[16 kt + 4 g + st][16 t + c].
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int st = 0; st < 4; ++st)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv_lds[buf][1][4 * g + st][16 * t + c], e[st], acc[t], 0, 0, 0);
        }
        // The other buffer was last read in the previous iteration, before its barrier.
        if (kt + 1 < ntile) stash(buf ^ 1);
        __syncthreads();
    }
    // acc[t][r] = ctx^T[16 t + 4 g + r][row c] of head h; the row's sum over its four lanes.
    ssum = row_sum4(ssum);
    if (row_ok) {
        float* cp = a.ctx + (static_cast<int64_t>(b) * l + row) * a.ldctx + h * D;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = 16 * t + 4 * g + r;
                if (d < D) cp[d] = acc[t][r] / ssum;
            }
        if (g == 0) {
            float* st = a.stats + 2 * (((static_cast<int64_t>(b) * a.heads + h) * l) + row);
            st[0] = m;
            st[1] = 1.0f / ssum;
        }
    }
}

struct RelArgs {
    const float* spv;
    const float* v;
    const float* k;
    const float* p;
    const float* raw;
    float* s;
    const float* q;
    const float* q_pre;
    const float* z;
    const float* bias;
    const float* cos_t;
    const float* sin_t;
    float* g;
    int ld_spv, ld_v, ld_k, ld_q, ld_q_pre, ld_z, ld_g;
    int n, l, heads, kv_heads, D;
    float scale, eps;
    int causal, rope, rope_half;
    int lds_ld;
    int rel_only;  // g receives the relevance itself (no projection denominator)
    const float* ctx;    // the attention output, head-packed (recomputing form)
    int ld_ctx;
    const float* stats;  // the forward's row statistics (recomputing form), or null
    float* row_sum;      // nullable (recomputing form): receives s_pv . ctx per row
    float* p_out;        // nullable (recomputing form): receives P on the visible keys
};

template <int DT, bool VEC>
__global__ void __launch_bounds__(kThreads) attn_rel_q_kernel(const RelArgs a) {
    extern __shared__ __attribute__((aligned(16))) float ra[];  // [16][lds_ld]: r_attn, then s
    __shared__ float s_sum[kWaves][16], f_sum[16];
    __shared__ __attribute__((aligned(16))) float s_acc[kWaves][16][16 * DT + 4];
    __shared__ __attribute__((aligned(16))) float m_acc[16][16 * DT + 4];

    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: the tile loops are scalar
    const int l = a.l, D = a.D, ld = a.lds_ld;
    const int nrb = (l + 15) / 16;
    // Long causal rows first, heads fastest: the heaviest blocks start first and spread over the CUs.
    const int nbh = a.n * a.heads;
    const int rb = nrb - 1 - static_cast<int>(blockIdx.x) / nbh, bh = static_cast<int>(blockIdx.x) % nbh;
    const int h = bh % a.heads, b = bh / a.heads;
    const int hk = h / (a.heads / a.kv_heads);
    const int i0 = rb * 16, row = i0 + c;
    const bool row_ok = row < l;
    const int64_t slab = (static_cast<int64_t>(b) * a.heads + h) * l * l;  // P, raw, s (N, H, L, L)
    const float* prow = a.p + slab + static_cast<int64_t>(row_ok ? row : l - 1) * l;
    const float* rrow = a.raw + slab + static_cast<int64_t>(row_ok ? row : l - 1) * l;

    // s_pv^T fragments (B operand): bf[t][s] = s_pv[row][16 t + 4 g + s].
    f4 bf[DT];
    {
        const float* sp = a.spv + (static_cast<int64_t>(b) * l + (row_ok ? row : l - 1)) * a.ld_spv + h * D;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const int d0 = 16 * t + 4 * g;
            bf[t] = *reinterpret_cast<const f4*>(sp + min(d0, D - 4)) * (d0 < D ? 1.0f : 0.0f);
        }
    }
    const float* vbase = a.v + static_cast<int64_t>(b) * l * a.ld_v + hk * D;
    const float* kbase = a.k + static_cast<int64_t>(b) * l * a.ld_k + hk * D;
    const int vis_end = a.causal ? min(i0 + 16, l) : l;
    const int ntile = (vis_end + 15) / 16;

    // The query share's operands, loaded before the key loop so the last pass waits on no memory:
    // thread (rr, cc) takes dims d = cc + 16 j of row i0 + rr (rows and dims clamped; the clamped
    // ones are never stored). y_lo / y_hi: the rotated q at the dim's RoPE pair (y at d without
    // RoPE); cs / sn: the pair's angle; xq: q before the rotation; zq, bq: z and the bias.
    const int rr = threadIdx.x >> 4, cc = threadIdx.x & 15;
    const int orow = i0 + rr;
    const int half = D / 2;
    float y_lo[DT], y_hi[DT], cs[DT], sn[DT], xq[DT], zq[DT], bq[DT];
    {
        const int64_t tok = static_cast<int64_t>(b) * l + min(orow, l - 1);
        const float* qr = a.q + tok * a.ld_q + h * D;
#pragma unroll
        for (int j = 0; j < DT; ++j) {
            const int d = min(cc + 16 * j, D - 1);
            if (a.rope) {
                const int i = a.rope_half ? (d < half ? d : d - half) : d / 2;
                const int lo = a.rope_half ? i : 2 * i, hi = a.rope_half ? i + half : 2 * i + 1;
                y_lo[j] = qr[lo];
                y_hi[j] = qr[hi];
                cs[j] = a.cos_t[static_cast<int64_t>(min(orow, l - 1)) * half + i];
                sn[j] = a.sin_t[static_cast<int64_t>(min(orow, l - 1)) * half + i];
                xq[j] = a.q_pre[tok * a.ld_q_pre + h * D + d];
            } else {
                y_lo[j] = qr[d];
                y_hi[j] = cs[j] = sn[j] = xq[j] = 0.0f;
            }
            zq[j] = a.rel_only ? 1.0f : a.z[tok * a.ld_z + h * D + d];
            bq[j] = a.bias ? a.bias[h * D + d] : 0.0f;
        }
    }

    // Both passes walk this wave's tiles two at a time with two register sets: a set is reloaded
    // with the tile after next right after its last read, the second tile of a pair runs even
    // past the last tile (all its keys masked: it adds nothing and stores nothing to LDS), and
    // loads clamp their addresses, so no branch surrounds a load.
    auto p4 = [&](const float* rowp, int kt) -> f4 {  // 4 entries of a score row at tile kt, clamped
        const int kk0 = 16 * min(kt, ntile - 1) + 4 * g;
        if constexpr (VEC) return *reinterpret_cast<const f4*>(rowp + min(kk0, l - 4));
        f4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = rowp[min(kk0 + j, l - 1)];
        return v;
    };
    const int last_key = a.causal ? min(row, l - 1) : l - 1;  // the lane's row sees keys 0 .. last_key
    auto valid_mask = [&](int kk0, bool (&valid)[4]) {
#pragma unroll
        for (int r = 0; r < 4; ++r) valid[r] = kk0 + r <= last_key;
    };

    const int ldv = a.ld_v, ldk = a.ld_k;
    f4 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    {
        // Pass 1: r_attn = P * (s_pv V^T), row sums. A operand: va[t][s] = V[key0 + c][16 t + 4 g + s].
        f4 va[2][DT], pa[2];
        auto load1 = [&](int set, int kt) {
            const float* vp = vbase + min(16 * min(kt, ntile - 1) + c, l - 1) * ldv;
#pragma unroll
            for (int t = 0; t < DT; ++t) va[set][t] = *reinterpret_cast<const f4*>(vp + min(16 * t + 4 * g, D - 4));
            pa[set] = p4(prow, kt);
        };
        float rs = 0.0f;
        auto tile1 = [&](int set, int kt) {
            const int kk0 = 16 * kt + 4 * g;
            f4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int st = 0; st < 4; ++st) u = __builtin_amdgcn_mfma_f32_16x16x4f32(va[set][t][st], bf[t][st], u, 0, 0, 0);
            bool valid[4];
            valid_mask(kk0, valid);
            f4 r4;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                r4[r] = valid[r] ? pa[set][r] * u[r] : 0.0f;
                rs += r4[r];
            }
            *reinterpret_cast<f4*>(ra + c * ld + 16 * min(kt, ntile) + 4 * g) = r4;  // past the end: never read
            // The set is reloaded only after its last read: a copy of a register whose reload is in
            // flight would make the wave wait for that reload.
            __builtin_amdgcn_sched_barrier(0);
            load1(set, kt + 2 * kWaves);
            __builtin_amdgcn_sched_barrier(0);
        };
        load1(0, wave);
        load1(1, wave + kWaves);
        __builtin_amdgcn_s_waitcnt(0);  // enter the loop with nothing in flight (as in attn_fwd_kernel)
        for (int kt = wave; kt < ntile; kt += 2 * kWaves) {
            tile1(0, kt);
            tile1(1, kt + kWaves);
        }
        rs = row_sum4(rs);
        if (g == 0) s_sum[wave][c] = rs;
        __syncthreads();
        if (threadIdx.x < 16) {
            float t = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) t += s_sum[w][threadIdx.x];
            f_sum[threadIdx.x] = t;
        }
        __syncthreads();

        // Pass 2: s = (scale raw)(r_attn - P sum) / (2 raw + eps sign raw); (s K)^T += K^T s^T with
        // A operand kb[t][s] = K[key0 + 4 g + s][16 t + c] and B = this lane's s values.
        const float sum = f_sum[c];
        f4 kb[2][DT], pb[2], rb2[2];
        auto load2 = [&](int set, int kt) {
            const int key0 = 16 * min(kt, ntile - 1);
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const float* kp = kbase + min(key0 + 4 * g + st, l - 1) * ldk;
#pragma unroll
                for (int t = 0; t < DT; ++t) kb[set][t][st] = kp[min(16 * t + c, D - 1)];
            }
            pb[set] = p4(prow, kt);
            rb2[set] = p4(rrow, kt);
        };
        auto tile2 = [&](int set, int kt) {
            const int kk0 = 16 * kt + 4 * g;
            const f4 pv = pb[set], rw = rb2[set];
            const int lcol = 16 * min(kt, ntile) + 4 * g;  // past the end: a masked, never-stored column
            const f4 r4 = *reinterpret_cast<const f4*>(ra + c * ld + lcol);
            bool valid[4];
            valid_mask(kk0, valid);
            f4 s4;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float o = rw[r];
                const float rsc = (a.scale * o) * (r4[r] - pv[r] * sum);
                s4[r] = valid[r] ? rsc / (2.0f * o + a.eps * ((o >= 0.0f) ? 1.0f : -1.0f)) : 0.0f;
            }
            *reinterpret_cast<f4*>(ra + c * ld + lcol) = s4;
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kb[set][t][st], s4[st], acc[t], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            load2(set, kt + 2 * kWaves);
            __builtin_amdgcn_sched_barrier(0);
        };
        load2(0, wave);
        load2(1, wave + kWaves);
        __builtin_amdgcn_s_waitcnt(0);
        for (int kt = wave; kt < ntile; kt += 2 * kWaves) {
            tile2(0, kt);
            tile2(1, kt + kWaves);
        }
    }
    // Merge: acc[t][r] = (s K)^T[16 t + 4 g + r][row c] of this wave.
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_acc[wave][c][16 * t + 4 * g + r] = acc[t][r];
    __syncthreads();
    for (int d = cc; d < D; d += 16) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) v += s_acc[w][rr][d];
        m_acc[rr][d] = v;
    }
    __syncthreads();

    if (orow < l) {
        // s over the whole row (zeros past the visible keys), contiguous.
        const int vis = a.causal ? orow + 1 : l;
        float* srow = a.s + slab + static_cast<int64_t>(orow) * l;
        const float* lrow = ra + rr * ld;
        if constexpr (VEC) {
            for (int k0 = 4 * cc; k0 < l; k0 += 64) {
                f4 out = {0.f, 0.f, 0.f, 0.f};
                if (k0 < vis) {
                    const f4 x = *reinterpret_cast<const f4*>(lrow + k0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) out[r] = k0 + r < vis ? x[r] : 0.0f;
                }
                *reinterpret_cast<f4*>(srow + k0) = out;
            }
        } else {
            for (int k = cc; k < l; k += 16) srow[k] = k < vis ? lrow[k] : 0.0f;
        }
        // Query share: r = Q_rot * (s K), the RoPE epsilon rule (lrp_math.hpp:104-123), then q_proj's
        // denominator: g = r_in / stab(z + bias).
        float* gr = a.g + (static_cast<int64_t>(b) * l + orow) * a.ld_g + h * D;
#pragma unroll
        for (int j = 0; j < DT; ++j) {
            const int d = cc + 16 * j;
            if (d >= D) continue;
            float r_in;
            if (a.rope) {
                const int i = a.rope_half ? (d < half ? d : d - half) : d / 2;
                const int lo = a.rope_half ? i : 2 * i, hi = a.rope_half ? i + half : 2 * i + 1;
                const float r_lo = y_lo[j] * m_acc[rr][lo], r_hi = y_hi[j] * m_acc[rr][hi];
                const float d0 = stab(y_lo[j], a.eps), d1 = stab(y_hi[j], a.eps);
                const float xv = xq[j];
                r_in = 0.0f;
                if (d == lo) {
                    r_in += (xv * cs[j] / d0) * r_lo;
                    r_in += (xv * sn[j] / d1) * r_hi;
                } else {
                    r_in += (xv * -sn[j] / d0) * r_lo;
                    r_in += (xv * cs[j] / d1) * r_hi;
                }
            } else {
                r_in = y_lo[j] * m_acc[rr][d];
            }
            gr[d] = a.rel_only ? r_in : r_in / stab(a.bias ? zq[j] + bq[j] : zq[j], a.eps);
        }
    }
}

// Recomputing form (pxk_attention_relevance_q with stats and ctx): no score rows are read. Per
// 16-key tile the kernel forms raw^T = K Q^T again (the forward's MFMA sequence, so the same
// values), P = exp(scale raw - m) / sum from the row statistics the forward kept, and
// u = s_pv V^T; the softmax rule's row sum of r_attn = P u is s_pv[row] . ctx[row] (the sum over
// the keys of P[row][k] (s_pv[row] . V[k])), a D-long dot product before the loop. Then
// s = (scale raw)(r_attn - P sum) / (2 raw + eps sign raw) and (s K)^T += K^T s^T.
//
// Memory. Everything the block reads outside the key loop (its 16 rows of Q, s_pv, ctx, and of
// q_pre, z, the RoPE angles for the query share, the bias and the row statistics) comes in one
// burst of whole-row 16-byte loads spread over the workgroup, into LDS; the waves take their
// fragments from there. The key loop reads only K and V tiles of the block's KV head (shared by
// all its blocks in L2), as 16 whole rows per tile; the transposed K fragments of (s K)^T come
// from those rows through a per-wave LDS tile rather than a second, gathering load. s and P, when
// asked for, are stored straight from the tile registers over the block's tiles.
template <int DT, bool VEC, int NW>
__global__ void __launch_bounds__(NW * kWave) attn_rel_q2_kernel(const RelArgs a) {
    constexpr int NT = NW * kWave;
    constexpr int RT = NT / 16;                 // threads per row in the last pass
    constexpr int DJ = (16 * DT + RT - 1) / RT;  // head dims per thread in the last pass
    constexpr int RS = 16 * DT + 4;             // LDS row stride of a 16-row operand block
    constexpr int HS = 8 * DT + 4;              // LDS row stride of the RoPE angle blocks
    // A wave's slot holds its K tile during the key loop, then its (s K)^T partial for the merge.
    __shared__ __attribute__((aligned(16))) float wave_lds[NW][16][RS];
    __shared__ __attribute__((aligned(16))) float op_lds[5][16][RS];  // Q, s_pv, ctx, q_pre, z rows
    __shared__ __attribute__((aligned(16))) float ang_lds[2][16][HS];  // cos, sin rows
    __shared__ __attribute__((aligned(16))) float bias_lds[16 * DT];
    __shared__ float stat_lds[16][2];
    __shared__ float m_acc[16][RS];

    const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: the tile loop is scalar
    const int l = a.l, D = a.D;
    const int nrb = (l + 15) / 16;
    // Long causal rows first, heads fastest: the heaviest blocks start first and spread over the CUs.
    const int nbh = a.n * a.heads;
    const int rb = nrb - 1 - static_cast<int>(blockIdx.x) / nbh, bh = static_cast<int>(blockIdx.x) % nbh;
    const int h = bh % a.heads, b = bh / a.heads;
    const int hk = h / (a.heads / a.kv_heads);
    const int i0 = rb * 16, row = i0 + c;
    const int vis_end = a.causal ? min(i0 + 16, l) : l;
    const int ntile = (vis_end + 15) / 16;
    const int vis_row = a.causal ? min(row + 1, l) : l;  // keys visible to the lane's row
    const int half = D / 2;

    // K and V tiles, two sets: kf[t][s] = K[key0 + c][16 t + 4 g + s] (A of raw^T), va[t][s] =
    // V[key0 + c][16 t + 4 g + s] (A of u). A set is reloaded with the tile after next right after
    // its last read; past the last tile the last one again, so no branch surrounds a load. As in
    // attn_fwd_kernel the loads are buffer loads from a per-tile resource built with scalar
    // instructions, each lane's byte offset fixed for the loop, the range (kv_tile_records) ending
    // with the head's D values of the sequence's last row: rows past the sequence read 0 (their keys
    // are masked), columns past head_dim read finite neighbouring data that meets zero Q and s_pv
    // fragments, and their (s K) dims are never stored.
    const float* vbase = a.v + static_cast<int64_t>(b) * l * a.ld_v + hk * D;
    const float* kbase = a.k + static_cast<int64_t>(b) * l * a.ld_k + hk * D;
    const int ldv = a.ld_v, ldk = a.ld_k;
    const int koff = (c * ldk + 4 * g) * 4, voff = (c * ldv + 4 * g) * 4;
    f4 kf[2][DT], va[2][DT];
    auto load = [&](int set, int kt) {
        const int key0 = 16 * min(kt, ntile - 1);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(kbase + key0 * ldk), 0, kv_tile_records(l, key0, ldk, D), 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(vbase + key0 * ldv), 0, kv_tile_records(l, key0, ldv, D), 0x00020000);
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            kf[set][t] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff + 64 * t, 0, 0));
            va[set][t] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff + 64 * t, 0, 0));
        }
    };
    // ---- the burst: the block's row operands into LDS, and the first K / V tile ----
    // Every load is issued before any LDS store (fixed per-thread counts, unrolled), so the burst
    // costs one memory round trip.
    {
        constexpr int F4N = (16 * 4 * DT + NT - 1) / NT;  // 16-byte pieces per thread per operand
        constexpr int SCN = (16 * 16 * DT + NT - 1) / NT;  // scalars per thread per operand
        constexpr int ANN = (16 * 8 * DT + NT - 1) / NT;   // angles per thread per table
        const int q4n = D / 4;
        const int64_t tok0 = static_cast<int64_t>(b) * l;
        f4 lq[F4N], ls[F4N], lc[F4N];
#pragma unroll
        for (int j = 0; j < F4N; ++j) {
            const int i = min(static_cast<int>(threadIdx.x) + NT * j, 16 * q4n - 1);
            const int r = i / q4n, c4 = 4 * (i - r * q4n);
            const int64_t tok = tok0 + min(i0 + r, l - 1);
            const int col = h * D + c4;
            lq[j] = *reinterpret_cast<const f4*>(a.q + tok * a.ld_q + col);
            ls[j] = *reinterpret_cast<const f4*>(a.spv + tok * a.ld_spv + col);
            lc[j] = *reinterpret_cast<const f4*>(a.ctx + tok * a.ld_ctx + col);
        }
        // The query share's operands, read as scalars (their strides need not be multiples of 4).
        float lx[SCN], lz[SCN];
#pragma unroll
        for (int j = 0; j < SCN; ++j) {
            const int i = min(static_cast<int>(threadIdx.x) + NT * j, 16 * D - 1);
            const int r = i / D, d = i - r * D;
            const int64_t tok = tok0 + min(i0 + r, l - 1);
            lx[j] = a.rope ? a.q_pre[tok * a.ld_q_pre + h * D + d] : 0.0f;
            lz[j] = a.rel_only ? 0.0f : a.z[tok * a.ld_z + h * D + d];
        }
        float lcs[ANN], lsn[ANN];
#pragma unroll
        for (int j = 0; j < ANN; ++j) {
            const int i = min(static_cast<int>(threadIdx.x) + NT * j, 16 * max(half, 1) - 1);
            const int r = i / max(half, 1), jj = i - r * max(half, 1);
            const int64_t pos = min(i0 + r, l - 1);
            lcs[j] = a.rope ? a.cos_t[pos * half + jj] : 0.0f;
            lsn[j] = a.rope ? a.sin_t[pos * half + jj] : 0.0f;
        }
        const float lb = (a.bias && static_cast<int>(threadIdx.x) < D) ? a.bias[h * D + threadIdx.x] : 0.0f;
        const int sr_ = min(static_cast<int>(threadIdx.x) >> 1, 15);
        const float lst =
            a.stats[2 * ((static_cast<int64_t>(b) * a.heads + h) * l + min(i0 + sr_, l - 1)) + (threadIdx.x & 1)];
        load(0, wave);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < F4N; ++j) {
            const int i = static_cast<int>(threadIdx.x) + NT * j;
            if (i < 16 * q4n) {
                const int r = i / q4n, c4 = 4 * (i - r * q4n);
                *reinterpret_cast<f4*>(&op_lds[0][r][c4]) = lq[j];
                *reinterpret_cast<f4*>(&op_lds[1][r][c4]) = ls[j];
                *reinterpret_cast<f4*>(&op_lds[2][r][c4]) = lc[j];
            }
        }
#pragma unroll
        for (int j = 0; j < SCN; ++j) {
            const int i = static_cast<int>(threadIdx.x) + NT * j;
            if (i < 16 * D) {
                const int r = i / D, d = i - r * D;
                op_lds[3][r][d] = lx[j];
                op_lds[4][r][d] = lz[j];
            }
        }
#pragma unroll
        for (int j = 0; j < ANN; ++j) {
            const int i = static_cast<int>(threadIdx.x) + NT * j;
            if (i < 16 * half) {
                const int r = i / half, jj = i - r * half;
                ang_lds[0][r][jj] = lcs[j];
                ang_lds[1][r][jj] = lsn[j];
            }
        }
        if (static_cast<int>(threadIdx.x) < D) bias_lds[threadIdx.x] = lb;
        if (threadIdx.x < 32) stat_lds[sr_][threadIdx.x & 1] = lst;
        // Q and s_pv columns past head_dim read as zeros in the fragments below.
        for (int i = threadIdx.x; i < 16 * (16 * DT - D); i += NT) {
            const int r = i / (16 * DT - D), d = D + i - r * (16 * DT - D);
            op_lds[0][r][d] = 0.0f;
            op_lds[1][r][d] = 0.0f;
        }
    }
    __syncthreads();

    // The second tile set is requested once the burst has landed: it overlaps the first tile.
    load(1, wave + NW);

    // Lane (c, g) takes dims 16 t + 4 g .. of row c: Q (B operand of raw^T) and s_pv (B operand of
    // u) are read from LDS per tile (zeros past head_dim); sum = s_pv . ctx of the row (its four
    // lanes l, l ^ 16, l ^ 32, l ^ 48).
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        const int d0 = min(16 * t + 4 * g, D - 4);
        const f4 bv = *reinterpret_cast<const f4*>(&op_lds[1][c][16 * t + 4 * g]);
        const f4 cv = *reinterpret_cast<const f4*>(&op_lds[2][c][d0]);
        sum += bv[0] * cv[0] + bv[1] * cv[1] + bv[2] * cv[2] + bv[3] * cv[3];
    }
    sum = row_sum4(sum);
    const float m_row = stat_lds[c][0], inv_row = stat_lds[c][1];
    if (a.row_sum && g == 0 && row < l) a.row_sum[(static_cast<int64_t>(b) * a.heads + h) * l + row] = sum;

    float* s_row = a.s ? a.s + (static_cast<int64_t>(b) * a.heads + h) * l * l + static_cast<int64_t>(row) * l : nullptr;
    float* p_row = a.p_out ? a.p_out + (static_cast<int64_t>(b) * a.heads + h) * l * l + static_cast<int64_t>(row) * l
                           : nullptr;
    float(*kt_w)[RS] = wave_lds[wave];
    f4 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    auto tile = [&](int set, int kt) {
        const int kk0 = 16 * kt + 4 * g;
        // The K tile's rows into the wave's LDS tile, for the transposed fragments below.
#pragma unroll
        for (int t = 0; t < DT; ++t) *reinterpret_cast<f4*>(&kt_w[c][16 * t + 4 * g]) = kf[set][t];
        __builtin_amdgcn_wave_barrier();
        // raw^T tile, the forward's sequence: lane (c, g) gets raw[row c][key kk0 + r].
        f4 sr = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const f4 qf = *reinterpret_cast<const f4*>(&op_lds[0][c][16 * t + 4 * g]);
#pragma unroll
            for (int st = 0; st < 4; ++st) sr = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[set][t][st], qf[st], sr, 0, 0, 0);
        }
        f4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const f4 bf = *reinterpret_cast<const f4*>(&op_lds[1][c][16 * t + 4 * g]);
#pragma unroll
            for (int st = 0; st < 4; ++st) u = __builtin_amdgcn_mfma_f32_16x16x4f32(va[set][t][st], bf[st], u, 0, 0, 0);
        }
        // kb[t][s] = K[key0 + 4 g + s][16 t + c] (A of (s K)^T)
        f4 kb[DT];
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int st = 0; st < 4; ++st) kb[t][st] = kt_w[4 * g + st][16 * t + c];
        f4 s4, p4v;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool valid = kk0 + r < vis_row;
            const float o = sr[r];
            const float pv = valid ? __expf(a.scale * o - m_row) * inv_row : 0.0f;
            const float rsc = (a.scale * o) * (pv * u[r] - pv * sum);
            // The hardware reciprocal (1 ulp) in place of a full-precision divide.
            s4[r] = valid ? rsc * __builtin_amdgcn_rcpf(2.0f * o + a.eps * ((o >= 0.0f) ? 1.0f : -1.0f)) : 0.0f;
            p4v[r] = pv;
        }
        // s and P over the block's tiles up to its diagonal, zeros at the masked keys within them:
        // the key side reads each row's keys up to the end of its diagonal tile.
        if (row < l && kt < ntile && kk0 < l) {
            if constexpr (VEC) {
                if (s_row) *reinterpret_cast<f4*>(s_row + kk0) = s4;
                if (p_row) *reinterpret_cast<f4*>(p_row + kk0) = p4v;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (kk0 + r < l) {
                        if (s_row) s_row[kk0 + r] = s4[r];
                        if (p_row) p_row[kk0 + r] = p4v[r];
                    }
            }
        }
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int st = 0; st < 4; ++st)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kb[t][st], s4[st], acc[t], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        load(set, kt + 2 * NW);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Tiles in pairs, the second unconditionally: past the last tile every key is masked.
    for (int kt = wave; kt < ntile; kt += 2 * NW) {
        tile(0, kt);
        tile(1, kt + NW);
    }

    // Merge: acc[t][r] = (s K)^T[16 t + 4 g + r][row c] of this wave, summed in wave order.
    __builtin_amdgcn_wave_barrier();  // the wave's last K-tile reads are issued before its slot is rewritten
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) wave_lds[wave][c][16 * t + 4 * g + r] = acc[t][r];
    __syncthreads();
    const int rr = threadIdx.x / RT, cc = threadIdx.x % RT;
    const int orow = i0 + rr;
    for (int d = cc; d < D; d += RT) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += wave_lds[w][rr][d];
        m_acc[rr][d] = v;
    }
    __syncthreads();
    if (orow >= l) return;

    // Query share: r = Q_rot * (s K), the RoPE epsilon rule (lrp_math.hpp:104-123), then q_proj's
    // denominator: g = r_in / stab(z + bias). Thread (rr, cc) takes dims d = cc + RT j of row i0 + rr.
    float* gr = a.g + (static_cast<int64_t>(b) * l + orow) * a.ld_g + h * D;
#pragma unroll
    for (int j = 0; j < DJ; ++j) {
        const int d = cc + RT * j;
        if (d >= D) continue;
        float r_in;
        if (a.rope) {
            const int i = a.rope_half ? (d < half ? d : d - half) : d / 2;
            const int lo = a.rope_half ? i : 2 * i, hi = a.rope_half ? i + half : 2 * i + 1;
            const float y_lo = op_lds[0][rr][lo], y_hi = op_lds[0][rr][hi];
            const float r_lo = y_lo * m_acc[rr][lo], r_hi = y_hi * m_acc[rr][hi];
            const float cs = ang_lds[0][rr][i], sn = ang_lds[1][rr][i];
            const float d0 = stab(y_lo, a.eps), d1 = stab(y_hi, a.eps);
            const float xv = op_lds[3][rr][d];
            r_in = 0.0f;
            if (d == lo) {
                r_in += (xv * cs / d0) * r_lo;
                r_in += (xv * sn / d1) * r_hi;
            } else {
                r_in += (xv * -sn / d0) * r_lo;
                r_in += (xv * cs / d1) * r_hi;
            }
        } else {
            r_in = op_lds[0][rr][d] * m_acc[rr][d];
        }
        if (a.rel_only) {
            gr[d] = r_in;
        } else {
            const float zz = op_lds[4][rr][d];
            gr[d] = r_in / stab(a.bias ? zz + bias_lds[d] : zz, a.eps);
        }
    }
}

// GQA-shared recomputing q side, for grids many times the chip's size: one workgroup per
// (sequence, KV head, 16-row block) and one wave per query head of the KV head's group, each wave
// over all of the block's key tiles, so no merge. Every K / V tile comes from memory into LDS once
// for the group (two buffers, the next tile's loads in flight during the current one) and supplies
// the waves' K, V and transposed K fragments; each wave keeps its head's Q and s_pv fragments in
// registers. Per tile the arithmetic is attn_rel_q2_kernel's, and so is the query share at the end
// (its operands read from memory, once per workgroup).
template <int DT, int G, bool VEC>
__global__ void __launch_bounds__(G * kWave) attn_rel_q2_gqa_kernel(const RelArgs a) {
    constexpr int NT = G * kWave, LD = 16 * DT + 4;
    constexpr int PER = (16 * 4 * DT + NT - 1) / NT;  // float4 per thread per tile operand
    __shared__ __attribute__((aligned(16))) float kv_lds[2][2][16][LD];  // [buffer][K, V][key][dim]
    __shared__ __attribute__((aligned(16))) float m_acc[G][16][LD];      // each head's (s K) rows

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the query head
    const int l = a.l, D = a.D;
    const int nrb = (l + 15) / 16;
    // Long causal rows first, KV heads fastest.
    const int nbk = a.n * a.kv_heads;
    const int rb = nrb - 1 - static_cast<int>(blockIdx.x) / nbk, bk = static_cast<int>(blockIdx.x) % nbk;
    const int hk = bk % a.kv_heads, b = bk / a.kv_heads;
    const int h = hk * G + wave;
    const int i0 = rb * 16, row = i0 + c;
    const int vis_end = a.causal ? min(i0 + 16, l) : l;
    const int ntile = (vis_end + 15) / 16;
    const int vis_row = a.causal ? min(row + 1, l) : l;  // keys visible to the lane's row
    const int64_t tok0 = static_cast<int64_t>(b) * l, tok = tok0 + min(row, l - 1);
    const int q4 = D / 4;

    // Lane (c, g) holds dims 16 t + 4 g .. of row c: Q (B operand of raw^T) and s_pv (B operand of
    // u), zeros past head_dim; sum = s_pv . ctx of the row over its four lanes.
    f4 qf[DT], sf[DT];
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        const int d0 = 16 * t + 4 * g, dc = min(d0, D - 4);
        const float keep = d0 < D ? 1.0f : 0.0f;
        qf[t] = *reinterpret_cast<const f4*>(a.q + tok * a.ld_q + h * D + dc) * keep;
        sf[t] = *reinterpret_cast<const f4*>(a.spv + tok * a.ld_spv + h * D + dc) * keep;
        const f4 cv = *reinterpret_cast<const f4*>(a.ctx + tok * a.ld_ctx + h * D + dc);
        sum += sf[t][0] * cv[0] + sf[t][1] * cv[1] + sf[t][2] * cv[2] + sf[t][3] * cv[3];
    }
    sum = row_sum4(sum);
    const float* strow = a.stats + 2 * ((static_cast<int64_t>(b) * a.heads + h) * l + min(row, l - 1));
    const float m_row = strow[0], inv_row = strow[1];
    if (a.row_sum && g == 0 && row < l) a.row_sum[(static_cast<int64_t>(b) * a.heads + h) * l + row] = sum;
    float* s_row = a.s ? a.s + (static_cast<int64_t>(b) * a.heads + h) * l * l + static_cast<int64_t>(row) * l : nullptr;
    float* p_row = a.p_out ? a.p_out + (static_cast<int64_t>(b) * a.heads + h) * l * l + static_cast<int64_t>(row) * l
                           : nullptr;

    const float* kbase = a.k + tok0 * a.ld_k + hk * D;
    const float* vbase = a.v + tok0 * a.ld_v + hk * D;
    // Columns past head_dim stay zero in both buffers: K's meet zero Q fragments and feed (s K)
    // dims that are never stored, V's meet zero s_pv fragments.
    for (int i = tid; i < 2 * 2 * 16 * (16 * DT - D); i += NT) {
        const int w = 16 * DT - D, r = i / w, col = D + i - r * w;
        (&kv_lds[0][0][0][0])[r * LD + col] = 0.0f;
    }
    // A tile's 16 K rows and 16 V rows as float4 pieces over the workgroup, through per-tile buffer
    // resources (kv_tile_records) and each thread's byte offsets, fixed for the loop: rows past the
    // sequence read 0 (their keys are masked).
    f4 sk[PER], sv[PER];
    int koff[PER], voff[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int i = min(tid + NT * j, 16 * q4 - 1);
        const int r = i / q4, c4 = 4 * (i - r * q4);
        koff[j] = (r * a.ld_k + c4) * 4;
        voff[j] = (r * a.ld_v + c4) * 4;
    }
    auto fetch = [&](int kt) {
        const int key0 = 16 * kt;
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(kbase + key0 * a.ld_k), 0, kv_tile_records(l, key0, a.ld_k, D), 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(vbase + key0 * a.ld_v), 0, kv_tile_records(l, key0, a.ld_v, D), 0x00020000);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            sk[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff[j], 0, 0));
            sv[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff[j], 0, 0));
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = tid + NT * j;
            if (i < 16 * q4) {
                const int r = i / q4, c4 = 4 * (i - r * q4);
                *reinterpret_cast<f4*>(&kv_lds[buf][0][r][c4]) = sk[j];
                *reinterpret_cast<f4*>(&kv_lds[buf][1][r][c4]) = sv[j];
            }
        }
    };

    f4 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    fetch(0);
    stash(0);
    __syncthreads();
    for (int kt = 0; kt < ntile; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ntile) fetch(kt + 1);  // uniform
        const int kk0 = 16 * kt + 4 * g;
        // raw^T tile, the forward's sequence: lane (c, g) gets raw[row c][key kk0 + r]; u[r] =
        // s_pv[row c] . V[key kk0 + r].
        f4 sr = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const f4 kf = *reinterpret_cast<const f4*>(&kv_lds[buf][0][c][16 * t + 4 * g]);
#pragma unroll
            for (int st = 0; st < 4; ++st) sr = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[st], qf[t][st], sr, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            const f4 vf = *reinterpret_cast<const f4*>(&kv_lds[buf][1][c][16 * t + 4 * g]);
#pragma unroll
            for (int st = 0; st < 4; ++st) u = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[st], sf[t][st], u, 0, 0, 0);
        }
        f4 s4, p4v;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool valid = kk0 + r < vis_row;
            const float o = sr[r];
            const float pv = valid ? __expf(a.scale * o - m_row) * inv_row : 0.0f;
            const float rsc = (a.scale * o) * (pv * u[r] - pv * sum);
            // The hardware reciprocal (1 ulp) in place of a full-precision divide.
            s4[r] = valid ? rsc * __builtin_amdgcn_rcpf(2.0f * o + a.eps * ((o >= 0.0f) ? 1.0f : -1.0f)) : 0.0f;
            p4v[r] = pv;
        }
        // s and P over the block's tiles up to its diagonal, zeros at the masked keys within them.
        if (row < l && kk0 < l) {
            if constexpr (VEC) {
                if (s_row) *reinterpret_cast<f4*>(s_row + kk0) = s4;
                if (p_row) *reinterpret_cast<f4*>(p_row + kk0) = p4v;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (kk0 + r < l) {
                        if (s_row) s_row[kk0 + r] = s4[r];
                        if (p_row) p_row[kk0 + r] = p4v[r];
                    }
            }
        }
        // (s K)^T += K^T s^T: A = K[16 kt + 4 g + st][16 t + c].
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int st = 0; st < 4; ++st)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv_lds[buf][0][4 * g + st][16 * t + c], s4[st], acc[t], 0, 0, 0);
        // The other buffer was last read in the previous iteration, before its barrier.
        if (kt + 1 < ntile) stash(buf ^ 1);
        __syncthreads();
    }

    // acc[t][r] = (s K)^T[16 t + 4 g + r][row c] of head h, into the wave's rows.
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) m_acc[wave][c][16 * t + 4 * g + r] = acc[t][r];
    __builtin_amdgcn_wave_barrier();
    // Query share: r = Q_rot * (s K), the RoPE epsilon rule (lrp_math.hpp:104-123), then q_proj's
    // denominator: g = r_in / stab(z + bias). Lane (rr, cc) takes dims cc + 4 j of row i0 + rr.
    const int rr = lane >> 2, cc = lane & 3, orow = i0 + rr;
    if (orow >= l) return;
    const int half = D / 2;
    const int64_t otok = tok0 + orow;
    const float* yq = a.q + otok * a.ld_q + h * D;
    float* gr = a.g + otok * a.ld_g + h * D;
    for (int d = cc; d < D; d += 4) {
        float r_in;
        if (a.rope) {
            const int i = a.rope_half ? (d < half ? d : d - half) : d / 2;
            const int lo = a.rope_half ? i : 2 * i, hi = a.rope_half ? i + half : 2 * i + 1;
            const float y_lo = yq[lo], y_hi = yq[hi];
            const float r_lo = y_lo * m_acc[wave][rr][lo], r_hi = y_hi * m_acc[wave][rr][hi];
            const float cs = a.cos_t[static_cast<int64_t>(orow) * half + i], sn = a.sin_t[static_cast<int64_t>(orow) * half + i];
            const float d0 = stab(y_lo, a.eps), d1 = stab(y_hi, a.eps);
            const float xv = a.q_pre[otok * a.ld_q_pre + h * D + d];
            r_in = 0.0f;
            if (d == lo) {
                r_in += (xv * cs / d0) * r_lo;
                r_in += (xv * sn / d1) * r_hi;
            } else {
                r_in += (xv * -sn / d0) * r_lo;
                r_in += (xv * cs / d1) * r_hi;
            }
        } else {
            r_in = yq[d] * m_acc[wave][rr][d];
        }
        if (a.rel_only) {
            gr[d] = r_in;
        } else {
            const float zz = a.z[otok * a.ld_z + h * D + d];
            gr[d] = r_in / stab(a.bias ? zz + a.bias[h * D + d] : zz, a.eps);
        }
    }
}

}  // namespace
}  // namespace pxk

using namespace pxk;

namespace {

constexpr int kMaxLds = 160 * 1024;  // gfx950 LDS per workgroup

// Row stride of the LDS score block: a multiple of 64 floats plus 20. The 16 columns past the
// rounded length take the branch-free tile past the last one (written, never read). The score-tile
// accesses put 16 rows' 16-byte pieces in one instruction (lane c at row c): 20 c modulo 64 gives
// 16 distinct groups of 4 banks (4 floats apart modulo 64 would too, but leaves no room past the
// end). The last pass reads whole row segments, 16 lanes per row.
int score_lds_ld(int64_t l) { return static_cast<int>((l + 63) / 64 * 64 + 20); }

// When the statistics-form forward runs GQA-shared: at least 16 (sequence, KV head) workgroups per
// 16-row block and 512 workgroups in all, with 2, 3, 4 or 8 query heads per KV head. Per launch at
// head_dim 64: 8 x 1024 tokens with 32 / 8 heads 642 -> 396 us, 4 x 1024 265 -> 198, 2 x 1024
// 133 -> 123; kept on the per-head kernel, where the heaviest blocks' tile chains (all of a block's
// key tiles in one wave) bound the launch: 1 x 1024 (70 against 87 us), 1 x 2048 (222 against 228),
// 1 x 4096 with 16 / 8 heads (393 against 537), 1 x 512 with 9 / 3 (14.5 against 37).
constexpr int64_t kGqaMinGroups = 16, kGqaMinBlocks = 512;

bool gqa_forward(int64_t n, int64_t l, int64_t heads, int64_t kv_heads) {
    if (n <= 0 || l <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0) return false;
    const int64_t grp = heads / kv_heads;
    return (grp == 2 || grp == 3 || grp == 4 || grp == 8) && n * kv_heads >= kGqaMinGroups &&
           n * kv_heads * ((l + 15) / 16) >= kGqaMinBlocks;
}

template <int DT>
int static_lds() {
    return static_cast<int>(sizeof(float) * (2 * kWaves * 16 + kWaves * 16 * (16 * DT + 4) + 2 * 16));
}

int dt_of(int64_t head_dim) { return head_dim <= 16 ? 1 : head_dim <= 32 ? 2 : head_dim <= 64 ? 4 : 8; }

int lds_bytes_needed(int64_t head_dim, int64_t l) {
    const int stat = dt_of(head_dim) == 8 ? static_lds<8>() : static_lds<4>();
    return stat + 16 * score_lds_ld(l) * static_cast<int>(sizeof(float));
}

}  // namespace

extern "C" int64_t pxk_attention_kv_tile_records(int64_t l, int64_t key0, int64_t ld, int64_t head_dim) {
    if (l <= 0 || key0 < 0 || key0 >= l || ld < head_dim || head_dim <= 0 ||
        (l * ld + head_dim) * 4 >= (int64_t{1} << 31)) {
        (void)fail(PXK_ERR_INVALID, "pxk_attention_kv_tile_records: bad arguments");
        return -1;
    }
    return kv_tile_records(static_cast<int>(l), static_cast<int>(key0), static_cast<int>(ld), static_cast<int>(head_dim));
}

extern "C" int pxk_attention_supported(int64_t head_dim, int64_t seq_len, int64_t ldq, int64_t ldk, int64_t ldv) {
    return head_dim > 0 && head_dim <= 128 && head_dim % 4 == 0 && ldq % 4 == 0 && ldk % 4 == 0 && ldv >= head_dim &&
           seq_len >= 0 && seq_len <= 8192 && lds_bytes_needed(head_dim, seq_len) <= kMaxLds;
}

namespace {

int attention_forward(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v, int64_t ldv,
                      float* raw, float* p, float* stats, float* ctx, int64_t ldctx, int64_t n, int64_t l,
                      int64_t heads, int64_t kv_heads, int64_t head_dim, float scale, int causal, void* stream,
                      const char* who) {
    const bool keep = raw || p;
    if (n < 0 || l < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0)
        return fail(PXK_ERR_INVALID, "%s: bad sizes (heads must be a multiple of kv_heads)", who);
    const bool shape_ok = keep ? pxk_attention_supported(head_dim, l, ldq, ldk, ldv) != 0
                               : head_dim > 0 && head_dim <= 128 && head_dim % 4 == 0 && ldq % 4 == 0 &&
                                     ldk % 4 == 0 && ldv >= head_dim && l <= 65536;
    if (!shape_ok || ldq < heads * head_dim || ldk < kv_heads * head_dim || ldv < kv_heads * head_dim ||
        ldctx < heads * head_dim)
        return fail(PXK_ERR_INVALID, "%s: head_dim must be a multiple of 4 up to 128, the sequence's score rows "
                                     "must fit LDS when raw or P is written (about 2000 tokens), and the row "
                                     "strides must hold every head (q and k strides a multiple of 4)", who);
    if (!aligned16(q) || !aligned16(k)) return fail(PXK_ERR_INVALID, "%s: q and k must be 16-byte aligned", who);
    if (n == 0 || l == 0) return PXK_OK;
    const int64_t blocks = n * heads * ((l + 15) / 16);
    // The K / V tile resources count bytes in 32 bits (kv_tile_records).
    if (blocks > (int64_t{1} << 31) - 1 || n * heads * l * l > (int64_t{1} << 40) ||
        (l * ldk + head_dim) * 4 >= (int64_t{1} << 31) || (l * ldv + head_dim) * 4 >= (int64_t{1} << 31))
        return fail(PXK_ERR_INVALID, "%s: problem too large", who);
    const int lds_ld = score_lds_ld(l);
    FwdArgs a{q, k, v, raw, p, ctx, ldq, ldk, ldv, ldctx, static_cast<int>(n), static_cast<int>(l),
              static_cast<int>(heads), static_cast<int>(kv_heads), static_cast<int>(head_dim), scale, causal != 0,
              lds_ld, stats, keep};
    const int dt = dt_of(head_dim);
    const int di = dt == 1 ? 0 : dt == 2 ? 1 : dt == 4 ? 2 : 3;
    // Many workgroups per CU: the GQA-shared kernel (one workgroup per KV head and row block, each
    // K / V tile read once for the group's query heads); fewer: the per-head kernel, whose four
    // waves split each block's key tiles and so shorten the heaviest blocks' chains.
    const int64_t grp = heads / kv_heads, gblocks = n * kv_heads * ((l + 15) / 16);
    const int gi = grp == 2 ? 0 : grp == 3 ? 1 : grp == 4 ? 2 : grp == 8 ? 3 : -1;
    if (!keep && stats && gqa_forward(n, l, heads, kv_heads) && ldv % 4 == 0 && aligned16(v)) {
        using KG = void (*)(const FwdArgs);
        static const KG gqa[4][4] = {
            {attn_fwd_gqa_kernel<1, 2>, attn_fwd_gqa_kernel<2, 2>, attn_fwd_gqa_kernel<4, 2>, attn_fwd_gqa_kernel<8, 2>},
            {attn_fwd_gqa_kernel<1, 3>, attn_fwd_gqa_kernel<2, 3>, attn_fwd_gqa_kernel<4, 3>, attn_fwd_gqa_kernel<8, 3>},
            {attn_fwd_gqa_kernel<1, 4>, attn_fwd_gqa_kernel<2, 4>, attn_fwd_gqa_kernel<4, 4>, attn_fwd_gqa_kernel<8, 4>},
            {attn_fwd_gqa_kernel<1, 8>, attn_fwd_gqa_kernel<2, 8>, attn_fwd_gqa_kernel<4, 8>, attn_fwd_gqa_kernel<8, 8>}};
        PXK_LAUNCH(gqa[gi][di], dim3(static_cast<unsigned>(gblocks)), dim3(static_cast<unsigned>(grp * kWave)), 0,
                   S(stream), a);
        return launched(who);
    }
    const bool vec = l % 4 == 0 && (!raw || aligned16(raw)) && (!p || aligned16(p));
    using K = void (*)(const FwdArgs);
    static const K table[2][4] = {
        {attn_fwd_kernel<1, false>, attn_fwd_kernel<2, false>, attn_fwd_kernel<4, false>, attn_fwd_kernel<8, false>},
        {attn_fwd_kernel<1, true>, attn_fwd_kernel<2, true>, attn_fwd_kernel<4, true>, attn_fwd_kernel<8, true>}};
    const K fn = table[vec ? 1 : 0][di];
    const size_t dyn = keep ? static_cast<size_t>(16) * lds_ld * sizeof(float) : 0;
    if (dyn > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(dyn)) != hipSuccess)
        return fail(PXK_ERR_LAUNCH, "%s: %zu bytes of LDS refused", who, dyn);
    PXK_LAUNCH(fn, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), dyn, S(stream), a);
    return launched(who);
}

}  // namespace

extern "C" int pxk_attention_forward(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                                     int64_t ldv, float* raw, float* p, float* ctx, int64_t ldctx, int64_t n,
                                     int64_t l, int64_t heads, int64_t kv_heads, int64_t head_dim, float scale,
                                     int causal, void* stream) {
    if (!raw || !p) return fail(PXK_ERR_INVALID, "pxk_attention_forward: raw and p are required");
    return attention_forward(q, ldq, k, ldk, v, ldv, raw, p, nullptr, ctx, ldctx, n, l, heads, kv_heads, head_dim,
                             scale, causal, stream, "pxk_attention_forward");
}

extern "C" int pxk_attention_forward_gqa(int64_t n, int64_t l, int64_t heads, int64_t kv_heads) {
    return gqa_forward(n, l, heads, kv_heads) ? 1 : 0;
}

extern "C" int pxk_attention_forward_stats(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                                           int64_t ldv, float* raw, float* p, float* stats, float* ctx, int64_t ldctx,
                                           int64_t n, int64_t l, int64_t heads, int64_t kv_heads, int64_t head_dim,
                                           float scale, int causal, void* stream) {
    if (!stats) return fail(PXK_ERR_INVALID, "pxk_attention_forward_stats: stats is required");
    return attention_forward(q, ldq, k, ldk, v, ldv, raw, p, stats, ctx, ldctx, n, l, heads, kv_heads, head_dim,
                             scale, causal, stream, "pxk_attention_forward_stats");
}

namespace {

template <int DT>
int rel_static_lds() {
    return static_cast<int>(sizeof(float) * (kWaves * 16 + 16 + (kWaves + 1) * 16 * (16 * DT + 4)));
}

// Waves per block of the recomputing q relevance: four, one per SIMD. At 1 x 512 tokens, 9 heads,
// head_dim 64 the launch takes 21.6 us against 24.7 with eight waves, 27.9 with sixteen and 31.0
// with two: fewer waves spend less of the block's prologue on their first K / V tiles, and two
// blocks share a CU instead.
template <int DT>
constexpr int rel_q2_waves() {
    return 4;
}

template <int DT>
int rel2_static_lds() {
    return static_cast<int>(sizeof(float) * ((rel_q2_waves<DT>() + 6) * 16 * (16 * DT + 4) + 2 * 16 * (8 * DT + 4) +
                                             16 * DT + 32));
}

}  // namespace

extern "C" int pxk_attention_relevance_q(const pxk_attn_rel_desc* d, void* stream) {
    const int64_t n = d->n, l = d->l, H = d->heads, Hkv = d->kv_heads, D = d->head_dim;
    const bool rc = d->stats != nullptr;  // the recomputing form
    if (n < 0 || l < 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0)
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_q: bad sizes (heads must be a multiple of kv_heads)");
    if (D <= 0 || D > 128 || D % 4 != 0 || (d->rope && D % 2 != 0))
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_q: head_dim must be a multiple of 4 up to 128");
    if (!d->spv || !d->v || !d->k || !d->q || (!d->z && !d->relevance_only) || !d->g ||
        (rc ? !d->ctx : (!d->p || !d->raw || !d->s)) || (d->rope && (!d->q_pre || !d->cos_t || !d->sin_t)))
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_q: a required operand is NULL");
    if (rc && (d->ld_ctx % 4 || !aligned16(d->ctx) || d->ld_ctx < H * D || d->ld_q % 4 || !aligned16(d->q) ||
               d->ld_k % 4 || !aligned16(d->k)))
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_q: ctx, q and k must be 16-byte aligned with row "
                                     "strides that are a multiple of 4 (ctx's holding every head)");
    if (d->ld_spv % 4 || d->ld_v % 4 || !aligned16(d->spv) || !aligned16(d->v) || d->ld_spv < H * D ||
        d->ld_v < Hkv * D || d->ld_k < Hkv * D || d->ld_q < H * D || d->ld_z < H * D || d->ld_g < H * D ||
        (d->rope && d->ld_q_pre < H * D))
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_q: row strides must hold every head (s_pv and v "
                                     "16-byte aligned with strides a multiple of 4)");
    const int lds_ld = score_lds_ld(l);
    const int dt = dt_of(D);
    const int stat = rc ? (dt == 8 ? rel2_static_lds<8>() : rel2_static_lds<4>())
                        : (dt == 8 ? rel_static_lds<8>() : rel_static_lds<4>());
    // Score rows wait in LDS for s in the two-pass form; the recomputing form keeps none.
    const size_t dyn = rc ? 0 : static_cast<size_t>(16) * lds_ld * sizeof(float);
    if (l > (rc ? 65536 : 8192) || stat + static_cast<int64_t>(dyn) > kMaxLds)
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_q: the sequence's score rows must fit LDS");
    if (n == 0 || l == 0) return PXK_OK;
    const int64_t blocks = n * H * ((l + 15) / 16);
    const int64_t lds_max = std::max({d->ld_spv, d->ld_v, d->ld_k, d->ld_q, d->ld_q_pre, d->ld_z, d->ld_g,
                                      rc ? d->ld_ctx : int64_t{0}});
    // The recomputing form's K / V tile resources count bytes in 32 bits (kv_tile_records), as the
    // forward's do.
    if (blocks > (int64_t{1} << 31) - 1 || n * l * lds_max >= (int64_t{1} << 31) ||
        ((d->s || d->p_out) && n * H * l * l >= (int64_t{1} << 40)) ||
        (rc && ((l * d->ld_k + D) * 4 >= (int64_t{1} << 31) || (l * d->ld_v + D) * 4 >= (int64_t{1} << 31))))
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_q: problem too large");
    RelArgs a{d->spv, d->v, d->k, d->p, d->raw, d->s, d->q, d->q_pre, d->z, d->bias, d->cos_t, d->sin_t, d->g,
              static_cast<int>(d->ld_spv), static_cast<int>(d->ld_v), static_cast<int>(d->ld_k),
              static_cast<int>(d->ld_q), static_cast<int>(d->ld_q_pre), static_cast<int>(d->ld_z),
              static_cast<int>(d->ld_g), static_cast<int>(n), static_cast<int>(l), static_cast<int>(H),
              static_cast<int>(Hkv), static_cast<int>(D), d->scale, d->eps, d->causal != 0, d->rope != 0,
              d->rope_half != 0, lds_ld, d->relevance_only != 0, d->ctx, static_cast<int>(d->ld_ctx), d->stats,
              d->row_sum, rc ? d->p_out : nullptr};
    const bool vec = l % 4 == 0 && (!d->p || aligned16(d->p)) && (!d->raw || aligned16(d->raw)) &&
                     (!d->s || aligned16(d->s)) && (!rc || !d->p_out || aligned16(d->p_out));
    using K = void (*)(const RelArgs);
    static const K two_pass[2][4] = {
        {attn_rel_q_kernel<1, false>, attn_rel_q_kernel<2, false>, attn_rel_q_kernel<4, false>,
         attn_rel_q_kernel<8, false>},
        {attn_rel_q_kernel<1, true>, attn_rel_q_kernel<2, true>, attn_rel_q_kernel<4, true>, attn_rel_q_kernel<8, true>}};
    static const K recompute[2][4] = {
        {attn_rel_q2_kernel<1, false, rel_q2_waves<1>()>, attn_rel_q2_kernel<2, false, rel_q2_waves<2>()>,
         attn_rel_q2_kernel<4, false, rel_q2_waves<4>()>, attn_rel_q2_kernel<8, false, rel_q2_waves<8>()>},
        {attn_rel_q2_kernel<1, true, rel_q2_waves<1>()>, attn_rel_q2_kernel<2, true, rel_q2_waves<2>()>,
         attn_rel_q2_kernel<4, true, rel_q2_waves<4>()>, attn_rel_q2_kernel<8, true, rel_q2_waves<8>()>}};
    const int di = dt == 1 ? 0 : dt == 2 ? 1 : dt == 4 ? 2 : 3;
    if (rc && gqa_forward(n, l, H, Hkv)) {
        // Wide grids: the GQA-shared form, under the forward's rule (the shapes where the
        // statistics-form forward runs GQA-shared).
#define PXK_Q2G(G) {attn_rel_q2_gqa_kernel<1, G, false>, attn_rel_q2_gqa_kernel<2, G, false>, \
                    attn_rel_q2_gqa_kernel<4, G, false>, attn_rel_q2_gqa_kernel<8, G, false>}, \
                   {attn_rel_q2_gqa_kernel<1, G, true>, attn_rel_q2_gqa_kernel<2, G, true>, \
                    attn_rel_q2_gqa_kernel<4, G, true>, attn_rel_q2_gqa_kernel<8, G, true>}
        static const K gqa[4][2][4] = {{PXK_Q2G(2)}, {PXK_Q2G(3)}, {PXK_Q2G(4)}, {PXK_Q2G(8)}};
#undef PXK_Q2G
        const int64_t grp = H / Hkv;
        const int gi = grp == 2 ? 0 : grp == 3 ? 1 : grp == 4 ? 2 : 3;
        PXK_LAUNCH(gqa[gi][vec ? 1 : 0][di], dim3(static_cast<unsigned>(n * Hkv * ((l + 15) / 16))),
                   dim3(static_cast<unsigned>(grp * kWave)), 0, S(stream), a);
        return launched("pxk_attention_relevance_q");
    }
    const K fn = rc ? recompute[vec ? 1 : 0][di] : two_pass[vec ? 1 : 0][di];
    const int threads = rc ? (dt == 8 ? rel_q2_waves<8>() : rel_q2_waves<4>()) * kWave : kThreads;
    if (dyn > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(dyn)) != hipSuccess)
        return fail(PXK_ERR_LAUNCH, "pxk_attention_relevance_q: %zu bytes of LDS refused", dyn);
    PXK_LAUNCH(fn, dim3(static_cast<unsigned>(blocks)), dim3(threads), dyn, S(stream), a);
    return launched("pxk_attention_relevance_q");
}

// ---- key and value shares (pxk_attention_relevance_kv) ------------------------------------------------
//
// One workgroup owns 16 keys of one KV head and DG groups of 16 head dimensions, each group closed
// under the RoPE pairing: dims 8j..8j+7 with their partners 8j+half.. under rotate-half,
// 16j..16j+15 for adjacent pairs or no RoPE. Its products are D[key][dim] = sum over (query head of
// the group, query row) of s[row][key] * Q[row][dim] and P[row][key] * s_pv[row][dim]:
// v_mfma_f32_16x16x4_f32 with A = one 16-key segment of 4 score rows and B = the matching 4 query
// rows' dims, so every operand is a single coalesced float per lane, and each score segment serves
// the DG groups. The (head, 4-row) items go round-robin over the NW waves, each with two accumulator
// pairs per group; the waves merge in LDS in wave order (deterministic). Loads run two register
// sets of U items ahead, with addresses clamped in range and rows past the end masked to 0 in the A
// operand, so the loop has no branch around a load. Each load is a wave-uniform base in scalar
// registers (moved by a few scalar adds per item) plus a per-lane offset fixed for the whole loop:
// per item the loop issues 6 loads, 4 MFMAs and a handful of vector instructions (the address
// arithmetic per item took 33 vector and 35 scalar instructions before; 20.6 -> 18.1 us at 1 x 512
// tokens with 9 / 3 heads, 715 -> 560 us at 8 x 1024 with 32 / 8, bitwise the same results).
// Causal: rows before the block's first key hold
// only masked (zero) entries and are skipped. Workgroups are ordered so each group of eight pairs a
// long causal key block with a short one, and (with a multiple of 8 workgroups) a group shares one
// XCD and its L2.
namespace {


struct RelKvArgs {
    const float* s;
    const float* p;
    const float* q;
    const float* spv;
    const float* k;
    const float* k_pre;
    const float* v;
    const float* z_k;
    const float* z_v;
    const float* bias_k;
    const float* bias_v;
    const float* cos_t;
    const float* sin_t;
    float* key_rel;
    float* value_rel;
    float* g_k;
    float* g_v;
    int ld_q, ld_spv, ld_k, ld_k_pre, ld_v, ld_z, ld_rel, ld_g;
    int n, l, heads, kv_heads, D, ngroups, nkb;
    float eps;
    int causal, rope, rope_half, remap;
    int rel_only;  // g_k / g_v receive the relevances themselves (no projection denominators)
};

// Head dimension held by MFMA column c of dim group dq, or -1.
__device__ __forceinline__ int kv_dim(const RelKvArgs& a, int dq, int c) {
    if (a.rope && a.rope_half) {
        const int half = a.D / 2, i = 8 * dq + (c & 7);
        return i < half ? (c < 8 ? i : i + half) : -1;
    }
    const int d = 16 * dq + c;
    return d < a.D ? d : -1;
}

template <int U, int DG, int KB>
struct KvSet {
    float s[KB][U], p[KB][U], q[DG][U], v[DG][U];
    bool ok[KB][U];  // the lane's row of item u is a real row that sees key block kb
};

// The wave's walk over its (query head j, 4-row chunk qi) items, item = wave + NW step, with the
// bases of the item's first row: s and P rows of head h, q and s_pv rows. A step moves the bases by
// 4 NW rows (a few scalar adds); crossing into the next head repositions them. Past the last item
// the walk stays on the wave's last one (its loads repeat, masked off).
struct KvCursor {
    int item, j, qi;
    const float *sb, *pb, *qb, *vb;
};

__device__ __forceinline__ void kv_seek(KvCursor& cur, const RelKvArgs& a, int b, int hk, int grp, int i_start) {
    const int h = hk * grp + cur.j, r0 = i_start + 4 * cur.qi;
    const int64_t hrow = (static_cast<int64_t>(b) * a.heads + h) * a.l + r0;
    const int64_t trow = static_cast<int64_t>(b) * a.l + r0;
    cur.sb = a.s + hrow * a.l;
    cur.pb = a.p + hrow * a.l;
    cur.qb = a.q + trow * a.ld_q + h * a.D;
    cur.vb = a.spv + trow * a.ld_spv + h * a.D;
}

// float at a byte offset from a wave-uniform base: the base stays in scalar registers and the load
// takes the 32-bit per-lane offset (global_load ... saddr), so a row step costs no vector address
// arithmetic.
__device__ __forceinline__ float ld_at(const float* base, unsigned byte_off) {
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + byte_off);
}

// The lane's byte offsets from an item's bases: row g4 of the chunk at its key column (s, P) and dim
// columns (q, s_pv).
template <int DG, int KB>
struct KvLane {
    int g4, key_c[KB], dim_c[DG];
    unsigned so[KB], qo[DG], vo[DG];
};

template <int NW, int U, int DG, int KB>
__device__ __forceinline__ void kv_load(KvSet<U, DG, KB>& r, const RelKvArgs& a, KvCursor& cur, int b, int hk, int grp,
                                        int total, int nq, int i_start, const int* row_from, const KvLane<DG, KB>& ln,
                                        int64_t step_s, int64_t step_q, int64_t step_v) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const bool it_ok = cur.item < total;  // uniform
        const int r0 = i_start + 4 * cur.qi;  // the item's first row
        const int lim = a.l - 1 - r0;          // rows of the sequence below it
        unsigned so[KB], qo[DG], vo[DG];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) so[kb] = ln.so[kb];
#pragma unroll
        for (int g = 0; g < DG; ++g) {
            qo[g] = ln.qo[g];
            vo[g] = ln.vo[g];
        }
        if (lim < 3) {  // uniform: the last chunk of a length not a multiple of 4 reads its last row again
            const int lr = min(ln.g4, lim);
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) so[kb] = 4u * static_cast<unsigned>(lr * a.l + ln.key_c[kb]);
#pragma unroll
            for (int g = 0; g < DG; ++g) {
                qo[g] = 4u * static_cast<unsigned>(lr * a.ld_q + ln.dim_c[g]);
                vo[g] = 4u * static_cast<unsigned>(lr * a.ld_spv + ln.dim_c[g]);
            }
        }
        const bool row_in = it_ok && ln.g4 <= lim;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            // Key block kb is read only from rows at or past its first row (the q side writes each
            // row's keys up to the end of its diagonal tile); other rows take zeros.
            r.ok[kb][u] = row_in && ln.g4 >= row_from[kb] - r0;
            r.s[kb][u] = ld_at(cur.sb, so[kb]);
            r.p[kb][u] = ld_at(cur.pb, so[kb]);
        }
#pragma unroll
        for (int g = 0; g < DG; ++g) {
            r.q[g][u] = ld_at(cur.qb, qo[g]);
            r.v[g][u] = ld_at(cur.vb, vo[g]);
        }
        if (cur.item + NW < total) {
            cur.qi += NW;
            if (cur.qi < nq) {
                cur.sb += step_s;
                cur.pb += step_s;
                cur.qb += step_q;
                cur.vb += step_v;
            } else {
                do {
                    cur.qi -= nq;
                    ++cur.j;
                } while (cur.qi >= nq);
                kv_seek(cur, a, b, hk, grp, i_start);
            }
        }
        cur.item += NW;
    }
}

template <int U, int DG, int KB>
__device__ __forceinline__ void kv_compute(const KvSet<U, DG, KB>& r, f4 (*acck)[DG][2], f4 (*accv)[DG][2]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const bool ok = r.ok[kb][u];
            const float as = ok ? r.s[kb][u] : 0.0f, ap = ok ? r.p[kb][u] : 0.0f;
#pragma unroll
            for (int g = 0; g < DG; ++g) {
                acck[kb][g][u & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(as, r.q[g][u], acck[kb][g][u & 1], 0, 0, 0);
                accv[kb][g][u & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(ap, r.v[g][u], accv[kb][g][u & 1], 0, 0, 0);
            }
        }
}

// NW waves per workgroup, U items per register set, DG dim groups of 16 and KB consecutive 16-key
// blocks per workgroup: the score rows (s, P) of a key block are read once for DG groups' query
// and s_pv columns, and each query and s_pv row once for KB key blocks.
template <int NW, int U, int DG, int KB>
__global__ void __launch_bounds__(NW * kWave) attn_rel_kv_kernel(const RelKvArgs a) {
    __shared__ float red[2][NW][16][17];  // per-wave k / v partial blocks [key][dim column], one group at a time

    const int lane = threadIdx.x & 63, g4 = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int id = blockIdx.x;
    if (a.remap) id = (id % 8) * (gridDim.x / 8) + id / 8;
    const int ngb = a.ngroups / DG;
    const int dqb = id % ngb;
    const int t = id / ngb;
    const int nkg = (a.nkb + KB - 1) / KB;  // groups of KB key blocks
    const int tkb = t % nkg, bg = t / nkg;
    const int kg = (tkb & 1) ? nkg - 1 - (tkb >> 1) : (tkb >> 1);  // long and short causal blocks alternate
    const int hk = bg % a.kv_heads, b = bg / a.kv_heads;
    const int grp = a.heads / a.kv_heads;
    const int m0 = kg * KB * 16;

    KvLane<DG, KB> ln;
    ln.g4 = g4;
    int row_from[KB];  // the first row reading each key block
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        ln.key_c[kb] = min(m0 + 16 * kb + c, a.l - 1);
        ln.so[kb] = 4u * static_cast<unsigned>(g4 * a.l + ln.key_c[kb]);
        // A key block past the sequence (the last group's second block) is read by no row.
        row_from[kb] = m0 + 16 * kb >= a.l ? a.l : (a.causal ? m0 + 16 * kb : 0);
    }
#pragma unroll
    for (int g = 0; g < DG; ++g) {
        const int dim = kv_dim(a, dqb * DG + g, c);
        ln.dim_c[g] = dim < 0 ? 0 : dim;
        ln.qo[g] = 4u * static_cast<unsigned>(g4 * a.ld_q + ln.dim_c[g]);
        ln.vo[g] = 4u * static_cast<unsigned>(g4 * a.ld_spv + ln.dim_c[g]);
    }
    const int i_start = a.causal ? m0 : 0;
    const int nq = (a.l - i_start + 3) / 4;
    const int total = grp * nq;
    const int mine = total > wave ? (total - wave + NW - 1) / NW : 0;
    const int steps = (mine + U - 1) / U;
    KvCursor cur;
    cur.item = wave;
    cur.j = wave < total ? wave / nq : grp - 1;
    cur.qi = wave < total ? wave % nq : nq - 1;
    kv_seek(cur, a, b, hk, grp, i_start);
    const int64_t step_s = static_cast<int64_t>(4 * NW) * a.l, step_q = static_cast<int64_t>(4 * NW) * a.ld_q,
                  step_v = static_cast<int64_t>(4 * NW) * a.ld_spv;

    f4 acck[KB][DG][2], accv[KB][DG][2];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int g = 0; g < DG; ++g)
#pragma unroll
            for (int h = 0; h < 2; ++h) acck[kb][g][h] = accv[kb][g][h] = f4{0.f, 0.f, 0.f, 0.f};
    KvSet<U, DG, KB> s0, s1;
    kv_load<NW, U, DG, KB>(s0, a, cur, b, hk, grp, total, nq, i_start, row_from, ln, step_s, step_q, step_v);
    kv_load<NW, U, DG, KB>(s1, a, cur, b, hk, grp, total, nq, i_start, row_from, ln, step_s, step_q, step_v);
    __builtin_amdgcn_sched_barrier(0);
    for (int st = 0; st < steps; st += 2) {
        kv_compute(s0, acck, accv);
        kv_load<NW, U, DG, KB>(s0, a, cur, b, hk, grp, total, nq, i_start, row_from, ln, step_s, step_q, step_v);
        __builtin_amdgcn_sched_barrier(0);
        kv_compute(s1, acck, accv);
        kv_load<NW, U, DG, KB>(s1, a, cur, b, hk, grp, total, nq, i_start, row_from, ln, step_s, step_q, step_v);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Epilogue, one key block and dim group at a time: thread -> (key row kl, dim column nn) of its
    // 16 x 16 block.
    const int kl = threadIdx.x >> 4, nn = threadIdx.x & 15;
    const float eps = a.eps;
#pragma unroll
    for (int e = 0; e < KB * DG; ++e) {
        const int kb = e / DG, g = e % DG;
        const int m = m0 + 16 * kb + kl;
        const int row = b * a.l + m;
        const f4 kk = acck[kb][g][0] + acck[kb][g][1], vv = accv[kb][g][0] + accv[kb][g][1];
        if (e > 0) __syncthreads();  // the previous block's epilogue has read red
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            red[0][wave][4 * g4 + r][c] = kk[r];
            red[1][wave][4 * g4 + r][c] = vv[r];
        }
        __syncthreads();
        const int dq = dqb * DG + g;
        const int d = kv_dim(a, dq, nn);
        if (threadIdx.x >= 256 || m >= a.l || d < 0) continue;
        auto sum4 = [&](int which, int col) {
            float v = red[which][0][kl][col];
#pragma unroll
            for (int w = 1; w < NW; ++w) v += red[which][w][kl][col];
            return v;
        };
        const int col = hk * a.D + d;
        float rk;
        if (a.rope) {
            const int D = a.D, half = D / 2;
            const int i = a.rope_half ? (d < half ? d : d - half) : d / 2;
            const int lo = a.rope_half ? i : 2 * i, hi = a.rope_half ? i + half : 2 * i + 1;
            const int n_lo = a.rope_half ? (nn & 7) : (nn & ~1), n_hi = a.rope_half ? (nn | 8) : (nn | 1);
            const float acc_lo = sum4(0, n_lo), acc_hi = sum4(0, n_hi);
            const float* K = a.k + row * a.ld_k + hk * D;
            const float y_lo = K[lo], y_hi = K[hi];
            const float r_lo = y_lo * acc_lo, r_hi = y_hi * acc_hi;
            const float cs = a.cos_t[m * half + i], sn = a.sin_t[m * half + i];
            const float d0 = stab(y_lo, eps), d1 = stab(y_hi, eps);
            const float xv = a.k_pre[row * a.ld_k_pre + col];
            rk = 0.0f;
            if (d == lo) {
                rk += (xv * cs / d0) * r_lo;
                rk += (xv * sn / d1) * r_hi;
            } else {
                rk += (xv * -sn / d0) * r_lo;
                rk += (xv * cs / d1) * r_hi;
            }
        } else {
            rk = a.k[row * a.ld_k + col] * sum4(0, nn);
        }
        if (a.key_rel) a.key_rel[row * a.ld_rel + col] = rk;
        const float rv = a.v[row * a.ld_v + col] * sum4(1, nn);
        if (a.value_rel) a.value_rel[row * a.ld_rel + col] = rv;
        if (a.rel_only) {
            a.g_k[row * a.ld_g + col] = rk;
            a.g_v[row * a.ld_g + col] = rv;
            continue;
        }
        const float zk = a.bias_k ? a.z_k[row * a.ld_z + col] + a.bias_k[col] : a.z_k[row * a.ld_z + col];
        a.g_k[row * a.ld_g + col] = rk / stab(zk, eps);
        const float zv = a.bias_v ? a.z_v[row * a.ld_z + col] + a.bias_v[col] : a.z_v[row * a.ld_z + col];
        a.g_v[row * a.ld_g + col] = rv / stab(zv, eps);
    }
}

}  // namespace

// 16-key blocks per workgroup of the wide-grid key side (four dim groups per workgroup).
constexpr int kKvBlocks = 2;

extern "C" int pxk_attention_relevance_kv(const pxk_attn_rel_kv_desc* d, void* stream) {
    const int64_t n = d->n, l = d->l, H = d->heads, Hkv = d->kv_heads, D = d->head_dim;
    if (n < 0 || l < 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0 || D <= 0 || D > 1024 || (d->rope && D % 2 != 0))
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_kv: bad sizes (heads a multiple of kv_heads, head_dim "
                                     "up to 1024 and even with RoPE)");
    if (!d->s || !d->p || !d->q || !d->spv || !d->k || !d->v || ((!d->z_k || !d->z_v) && !d->relevance_only) ||
        !d->g_k || !d->g_v ||
        (d->rope && (!d->k_pre || !d->cos_t || !d->sin_t)))
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_kv: a required operand is NULL");
    if (d->ld_q < H * D || d->ld_spv < H * D || d->ld_k < Hkv * D || d->ld_v < Hkv * D || d->ld_z < Hkv * D ||
        d->ld_g < Hkv * D || (d->rope && d->ld_k_pre < Hkv * D) ||
        ((d->key_rel || d->value_rel) && d->ld_rel < Hkv * D))
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_kv: row strides must hold every head");
    if (n == 0 || l == 0) return PXK_OK;
    const int64_t ngroups = (d->rope && d->rope_half) ? (D / 2 + 7) / 8 : (D + 15) / 16;
    const int64_t nkb = (l + 15) / 16;
    const int64_t blocks = n * Hkv * nkb * ngroups;
    const int64_t lds_max = std::max({d->ld_q, d->ld_spv, d->ld_k, d->rope ? d->ld_k_pre : 0, d->ld_v, d->ld_z,
                                      d->ld_rel, d->ld_g});
    if (blocks > (int64_t{1} << 31) - 1 || n * H * l * l >= (int64_t{1} << 31) || n * l * lds_max >= (int64_t{1} << 31))
        return fail(PXK_ERR_INVALID, "pxk_attention_relevance_kv: problem too large");
    RelKvArgs a{d->s, d->p, d->q, d->spv, d->k, d->k_pre, d->v, d->z_k, d->z_v, d->bias_k, d->bias_v, d->cos_t,
                d->sin_t, d->key_rel, d->value_rel, d->g_k, d->g_v, static_cast<int>(d->ld_q),
                static_cast<int>(d->ld_spv), static_cast<int>(d->ld_k), static_cast<int>(d->rope ? d->ld_k_pre : 0),
                static_cast<int>(d->ld_v), static_cast<int>(d->ld_z), static_cast<int>(d->ld_rel),
                static_cast<int>(d->ld_g), static_cast<int>(n), static_cast<int>(l), static_cast<int>(H),
                static_cast<int>(Hkv), static_cast<int>(D), static_cast<int>(ngroups), static_cast<int>(nkb), d->eps,
                d->causal != 0, d->rope != 0, d->rope_half != 0, blocks % 8 == 0, d->relevance_only != 0};
    // One item per register set throughout. Four dim groups and two 16-key blocks per workgroup
    // where the dim groups divide evenly and there are at least 512 (KV head, key block, 4 groups)
    // units (wide grids: many sequences, long ones, or head_dim 256), so each score row is read a
    // quarter as often and each query and s_pv row half as often, on eight waves: at 32 / 8 heads
    // of 64, 8 x 1024 tokens 706 us against 1101 with one key block per workgroup (1165 for sixteen
    // waves with two items per set, 1209 for two groups), 2 x 1024 233 against 340 for two groups,
    // 1 x 2048 377 against 625, 1 x 1024 121 against 138; four key blocks per workgroup 739 at
    // 8 x 1024. Otherwise sixteen waves, the widest spread of a long key block's rows, and two dim
    // groups where they divide (the score rows read half as often, 192 workgroups for one 512-token
    // sequence of three KV heads): 20.2 us against 23.2 for one group and two items per set, 34 for
    // four groups (96 workgroups) at 1 x 512, 9 / 3 heads of 64; at 4 x 512 (384 units) 46 against
    // 53 for the wide form.
    // Between the two: four dim groups per workgroup, one 16-key block, sixteen waves, from 128
    // (KV head, key block) pairs (one workgroup each at head_dim 64), where the score rows read once
    // instead of twice beat the wider spread (with the scalar-base loader, at 9 / 3 heads of 64:
    // 2 x 512 26.1 against 30.4 us, 1 x 1024 41.5 against 53.0, 1 x 2048 133.8 against 166.8; 16 / 4
    // heads at 1 x 1024 53.1 against 69.5; 4 x 512 45.3 against 47.0). Below 128 pairs (1 x 512
    // with 3 KV heads: 96) two groups stay ahead, 17.9 against 25.4 us.
    const int64_t pairs = n * Hkv * nkb;
    if (ngroups % 4 == 0 && blocks / 4 >= 512) {
        const int64_t wg = n * Hkv * ((nkb + kKvBlocks - 1) / kKvBlocks) * (ngroups / 4);
        a.remap = wg % 8 == 0;
        PXK_LAUNCH((attn_rel_kv_kernel<8, 1, 4, kKvBlocks>), dim3(static_cast<unsigned>(wg)), dim3(8 * kWave), 0,
                           S(stream), a);
    } else if (ngroups % 4 == 0 && pairs >= 128) {
        a.remap = (blocks / 4) % 8 == 0;
        PXK_LAUNCH((attn_rel_kv_kernel<16, 1, 4, 1>), dim3(static_cast<unsigned>(blocks / 4)), dim3(16 * kWave), 0,
                           S(stream), a);
    } else if (ngroups % 2 == 0) {
        a.remap = (blocks / 2) % 8 == 0;
        PXK_LAUNCH((attn_rel_kv_kernel<16, 1, 2, 1>), dim3(static_cast<unsigned>(blocks / 2)), dim3(16 * kWave), 0,
                           S(stream), a);
    } else {
        PXK_LAUNCH((attn_rel_kv_kernel<16, 1, 1, 1>), dim3(static_cast<unsigned>(blocks)), dim3(16 * kWave), 0,
                           S(stream), a);
    }
    return launched("pxk_attention_relevance_kv");
}
