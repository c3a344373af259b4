// decode.hip -- the position-dependent kernels of a KV-cached decode step (include/pxk.h).
//
// The decode position lives in device memory (`pos`, one int32 shared by the batch), so a whole
// step -- embedding gather, every layer, the LM head and the greedy pick -- launches with the same
// arguments at every position and is captured once into a HIP graph; pxk_decode_advance() moves
// the position at the end of the step. Replaces the per-step host work of
// MakeCachedNextTokenLogits (generation.cpp:189-258): the KVCache appends (kv_cache.cpp:18-39),
// MultiHeadAttentionModule::forward_cached's per-head gemm_ex / softmax / gemm against the cache
// (multihead_attention_module.cpp:501-587), the last hidden row's device-host round trip and the
// host-side argmax.
#include <algorithm>

#include "common.hpp"

namespace pxk {
namespace {

constexpr int kThreads = 256;

struct RopeAppendArgs {
    const float* q;      // (n, H*D) rows, row stride ldq: the step's queries before RoPE
    int64_t ldq;
    const float* k;      // (n, Hkv*D), stride ldk
    int64_t ldk;
    const float* v;      // (n, Hkv*D), stride ldv
    int64_t ldv;
    float* q_out;        // (n, H*D), contiguous
    float* k_cache;      // sequence b at k_cache + b * seq_stride, position p at + p * Hkv*D
    float* v_cache;
    int64_t seq_stride;
    const float* cos_t;  // (positions, D/2)
    const float* sin_t;
    const int32_t* pos;
    int64_t n, H, Hkv, D, positions;  // positions: what the cache and the tables hold
    int rope, rotate_half;
};

// One thread per (row, head, pair) of q and of k, and per (row, element) of v.
__global__ void __launch_bounds__(kThreads) rope_append_kernel(const RopeAppendArgs a) {
    const int64_t p = *a.pos, half = a.D / 2, kvd = a.Hkv * a.D;
    if (p < 0 || p >= a.positions) return;  // past the cache: nothing is written (the host bounds the steps)
    const int64_t nq = a.n * a.H * half, nk = a.n * a.Hkv * half, nv = a.n * kvd;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; t < nq + nk + nv; t += stride) {
        if (t >= nq + nk) {  // value: copied into the cache
            const int64_t u = t - nq - nk, b = u / kvd, c = u - b * kvd;
            a.v_cache[b * a.seq_stride + p * kvd + c] = a.v[b * a.ldv + c];
            continue;
        }
        const bool is_q = t < nq;
        const int64_t u = is_q ? t : t - nq, heads = is_q ? a.H : a.Hkv;
        const int64_t i = u % half, h = (u / half) % heads, b = u / (half * heads);
        const int64_t lo = h * a.D + (a.rotate_half ? i : 2 * i), hi = h * a.D + (a.rotate_half ? i + half : 2 * i + 1);
        const float* src = is_q ? a.q + b * a.ldq : a.k + b * a.ldk;
        float* dst = is_q ? a.q_out + b * a.H * a.D : a.k_cache + b * a.seq_stride + p * kvd;
        const float x0 = src[lo], x1 = src[hi];
        if (a.rope) {  // rope_rotate (row_math.hpp:93-110) at position p
            const float c = a.cos_t[p * half + i], s = a.sin_t[p * half + i];
            dst[lo] = x0 * c - x1 * s;
            dst[hi] = x0 * s + x1 * c;
        } else {
            dst[lo] = x0;
            dst[hi] = x1;
        }
    }
}

struct DecodeAttnArgs {
    const float* q;  // (n, H*D) contiguous, rotated
    const float* k_cache;
    const float* v_cache;
    int64_t seq_stride;
    float* ctx;      // (n, H*D) contiguous
    const int32_t* pos;
    int64_t H, Hkv, D, window, max_keys;
    float scale;
};

// One workgroup per (sequence, query head): the single query's scores against keys
// [lo, pos] of the cache (a sliding layer's window, attention_masked row_math.hpp:117-126), the
// softmax over them (max-subtract, exp, sum, divide: softmax_rows cpu_backend.cpp:292-310) and
// ctx = P V. Scores live in LDS (max_keys floats, dynamic).
__global__ void __launch_bounds__(kThreads) decode_attention_kernel(const DecodeAttnArgs a) {
    extern __shared__ float sm[];
    float* qs = sm;              // D
    float* sc = sm + a.D;        // max_keys
    __shared__ float red[kThreads / kWave];
    const int64_t b = blockIdx.x / a.H, h = blockIdx.x % a.H, hk = h / (a.H / a.Hkv);
    const int64_t kvd = a.Hkv * a.D;
    const int64_t p = min(max(static_cast<int64_t>(*a.pos), int64_t{0}), a.max_keys - 1);  // stays inside the cache
    const int64_t lo = (a.window > 0 && p + 1 > a.window) ? p + 1 - a.window : 0;
    const int64_t nkeys = p + 1 - lo;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    for (int64_t d = tid; d < a.D; d += kThreads) qs[d] = a.q[b * a.H * a.D + h * a.D + d];
    __syncthreads();
    const float* kb = a.k_cache + b * a.seq_stride + hk * a.D;
    for (int64_t j = wave; j < nkeys; j += kThreads / kWave) {
        const float* kr = kb + (lo + j) * kvd;
        float s = 0.0f;
        for (int64_t d = lane; d < a.D; d += kWave) s += qs[d] * kr[d];
        s = wave_sum(s);
        if (lane == 0) sc[j] = a.scale * s;
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int64_t j = tid; j < nkeys; j += kThreads) mx = fmaxf(mx, sc[j]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < kThreads / kWave; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();
    float sum = 0.0f;
    for (int64_t j = tid; j < nkeys; j += kThreads) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    sum = 0.0f;
    for (int w = 0; w < kThreads / kWave; ++w) sum += red[w];
    const float* vb = a.v_cache + b * a.seq_stride + hk * a.D;
    for (int64_t d = tid; d < a.D; d += kThreads) {
        float acc = 0.0f;
        for (int64_t j = 0; j < nkeys; ++j) acc += (sc[j] / sum) * vb[(lo + j) * kvd + d];
        a.ctx[b * a.H * a.D + h * a.D + d] = acc;
    }
}

constexpr int kPickThreads = 1024;

// Greedy pick per sequence (Generate's greedy step: the first maximum of the logits): one
// workgroup scans a row, shares merged larger value first and lower index on ties. The pick is
// written as the sequence's next id (ids[b, pos + 1]), as this step's token (cur[b]) and its logit
// (picked_logit[b * ld_logit + pos + 1], the OutputValue seed an explanation of it uses).
__global__ void __launch_bounds__(kPickThreads) decode_pick_kernel(const float* logits, int64_t ld_logits, int64_t V,
                                                                  float* ids, int64_t ld_ids, float* cur,
                                                                  float* picked_logit, int64_t ld_logit,
                                                                  const int32_t* pos) {
    const int64_t b = blockIdx.x;
    const float* row = logits + b * ld_logits;
    __shared__ float bv[kPickThreads];
    __shared__ int64_t bi[kPickThreads];
    float best = -INFINITY;
    int64_t idx = V;
    for (int64_t j = threadIdx.x; j < V; j += kPickThreads) {
        const float x = row[j];
        if (idx == V || x > best) {
            best = x;
            idx = j;
        }
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = idx;
    __syncthreads();
    for (int s = kPickThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            const float ov = bv[threadIdx.x + s], cv = bv[threadIdx.x];
            const int64_t oi = bi[threadIdx.x + s], ci = bi[threadIdx.x];
            if (ci == V || (oi != V && (ov > cv || (ov == cv && oi < ci)))) {
                bv[threadIdx.x] = ov;
                bi[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int64_t next = static_cast<int64_t>(*pos) + 1;
        const int64_t t = bi[0] < V ? bi[0] : 0;  // a row of NaNs picks id 0 rather than leave the table
        cur[b] = static_cast<float>(t);
        if (next >= 0 && next < ld_ids) ids[b * ld_ids + next] = static_cast<float>(t);
        if (picked_logit && next >= 0 && next < ld_logit) picked_logit[b * ld_logit + next] = bv[0];
    }
}

__global__ void decode_advance_kernel(int32_t* pos) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *pos += 1;
}

// Seed of one row per sequence (the last row of each prefix an explanation runs on): one-hot at the
// target id (targets[b * stride], a float id rounded half away from zero as llround does) with the
// row's logit there (OutputValue) or 1 (unit, OneHot); every other entry of seed (n x V) is 0.
__global__ void __launch_bounds__(kThreads) seed_rows_kernel(const float* logits, int64_t ld_logits,
                                                            const float* targets, int64_t stride, int64_t V, float* seed,
                                                            int64_t* targets_out, int unit) {
    const int64_t b = blockIdx.y;
    const int64_t t = static_cast<int64_t>(llroundf(targets[b * stride]));
    const int64_t tt = (t >= 0 && t < V) ? t : 0;
    const float value = unit ? 1.0f : logits[b * ld_logits + tt];
    for (int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; j < V;
         j += static_cast<int64_t>(gridDim.x) * kThreads)
        seed[b * V + j] = j == tt ? value : 0.0f;
    if (blockIdx.x == 0 && threadIdx.x == 0 && targets_out) targets_out[b] = tt;
}

}  // namespace
}  // namespace pxk

using namespace pxk;

extern "C" int pxk_decode_rope_append(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                                      int64_t ldv, float* q_out, float* k_cache, float* v_cache, int64_t seq_stride,
                                      int64_t positions, const float* cos_t, const float* sin_t, const int32_t* pos,
                                      int64_t n, int64_t heads, int64_t kv_heads, int64_t head_dim, int rope,
                                      int rotate_half, void* stream) {
    const int64_t qd = heads * head_dim, kvd = kv_heads * head_dim;
    if (n < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || head_dim <= 0 || head_dim % 2 != 0 ||
        ldq < qd || ldk < kvd || ldv < kvd || positions <= 0 || seq_stride < positions * kvd)
        return fail(PXK_ERR_INVALID, "pxk_decode_rope_append: bad sizes or strides (the cache must hold `positions`)");
    if (n == 0) return PXK_OK;
    if (!q || !k || !v || !q_out || !k_cache || !v_cache || !pos || (rope && (!cos_t || !sin_t)))
        return fail(PXK_ERR_INVALID, "pxk_decode_rope_append: a required operand is NULL");
    const RopeAppendArgs a{q, ldq, k, ldk, v, ldv, q_out, k_cache, v_cache, seq_stride, cos_t, sin_t, pos,
                           n, heads, kv_heads, head_dim, positions, rope, rotate_half};
    const int64_t work = n * (heads + kv_heads) * (head_dim / 2) + n * kvd;
    hipLaunchKernelGGL(rope_append_kernel, dim3(grid_for(work, kThreads)), dim3(kThreads), 0, S(stream), a);
    return launched("pxk_decode_rope_append");
}

extern "C" int pxk_decode_attention(const float* q, const float* k_cache, const float* v_cache, int64_t seq_stride,
                                    float* ctx, const int32_t* pos, int64_t n, int64_t heads, int64_t kv_heads,
                                    int64_t head_dim, int64_t window, int64_t max_keys, float scale, void* stream) {
    if (n < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || head_dim <= 0 || window < 0 ||
        max_keys <= 0 || seq_stride < max_keys * kv_heads * head_dim)
        return fail(PXK_ERR_INVALID, "pxk_decode_attention: bad sizes (the cache must hold max_keys positions)");
    const size_t lds = static_cast<size_t>(head_dim + max_keys) * sizeof(float);
    if (lds > 60 * 1024)
        return fail(PXK_ERR_INVALID, "pxk_decode_attention: head_dim + max_keys must fit 60 KiB of LDS");
    if (n == 0) return PXK_OK;
    if (!q || !k_cache || !v_cache || !ctx || !pos) return fail(PXK_ERR_INVALID, "pxk_decode_attention: NULL operand");
    const DecodeAttnArgs a{q, k_cache, v_cache, seq_stride, ctx, pos, heads, kv_heads, head_dim, window, max_keys, scale};
    hipLaunchKernelGGL(decode_attention_kernel, dim3(static_cast<unsigned>(n * heads)), dim3(kThreads), lds, S(stream),
                       a);
    return launched("pxk_decode_attention");
}

extern "C" int pxk_decode_pick(const float* logits, int64_t ld_logits, int64_t n, int64_t vocab, float* ids,
                               int64_t ld_ids, float* cur, float* picked_logit, int64_t ld_logit, const int32_t* pos,
                               void* stream) {
    if (n < 0 || vocab <= 0 || ld_logits < vocab || ld_ids < 1 || (picked_logit && ld_logit < 1))
        return fail(PXK_ERR_INVALID, "pxk_decode_pick: bad sizes");
    if (n == 0) return PXK_OK;
    if (!logits || !ids || !cur || !pos) return fail(PXK_ERR_INVALID, "pxk_decode_pick: NULL operand");
    hipLaunchKernelGGL(decode_pick_kernel, dim3(static_cast<unsigned>(n)), dim3(kPickThreads), 0, S(stream), logits,
                       ld_logits, vocab, ids, ld_ids, cur, picked_logit, ld_logit, pos);
    return launched("pxk_decode_pick");
}

extern "C" int pxk_decode_advance(int32_t* pos, void* stream) {
    if (!pos) return fail(PXK_ERR_INVALID, "pxk_decode_advance: NULL position");
    hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(kWave), 0, S(stream), pos);
    return launched("pxk_decode_advance");
}

extern "C" int pxk_seed_rows(const float* logits, int64_t ld_logits, const float* targets, int64_t stride, int64_t n,
                             int64_t vocab, float* seed, int64_t* targets_out, int unit, void* stream) {
    if (n < 0 || vocab <= 0 || stride < 0 || n > 65535 || ld_logits < vocab)
        return fail(PXK_ERR_INVALID, "pxk_seed_rows: bad sizes");
    if (n == 0) return PXK_OK;
    if (!targets || !seed || (!unit && !logits)) return fail(PXK_ERR_INVALID, "pxk_seed_rows: NULL operand");
    const unsigned gx = static_cast<unsigned>(std::min<int64_t>(cdiv(vocab, kThreads), 1024));
    hipLaunchKernelGGL(seed_rows_kernel, dim3(gx, static_cast<unsigned>(n)), dim3(kThreads), 0, S(stream), logits,
                       ld_logits, targets, stride, vocab, seed, targets_out, unit);
    return launched("pxk_seed_rows");
}
