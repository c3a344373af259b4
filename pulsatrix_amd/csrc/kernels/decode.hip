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
    const float* q_gamma;  // QK-Norm's scales (both or neither)
    const float* k_gamma;
    float norm_eps;
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

// With QK-Norm: one workgroup per (sequence, query or key head). The head's D values are staged in
// LDS, normalised (RMSNorm over the head, as pxk_rms_norm_heads computes it: the wave sums of squares
// added in wave order), rotated at the position and written; a key head's workgroup also copies its
// value head into the cache.
__global__ void __launch_bounds__(kThreads) rope_append_norm_kernel(const RopeAppendArgs a) {
    extern __shared__ float row[];  // D
    __shared__ float part[kThreads / kWave];
    const int64_t p = *a.pos, half = a.D / 2, kvd = a.Hkv * a.D;
    if (p < 0 || p >= a.positions) return;  // past the cache: nothing is written (the host bounds the steps)
    const int64_t blk = blockIdx.x, hs = a.H + a.Hkv, b = blk / hs, hh = blk - b * hs;
    const bool is_q = hh < a.H;
    const int64_t h = is_q ? hh : hh - a.H;
    const float* src = is_q ? a.q + b * a.ldq + h * a.D : a.k + b * a.ldk + h * a.D;
    const float* gamma = is_q ? a.q_gamma : a.k_gamma;
    const int tid = threadIdx.x;
    float ss = 0.0f;
    for (int64_t d = tid; d < a.D; d += kThreads) {
        const float x = src[d];
        row[d] = x;
        ss += x * x;
    }
    ss = wave_sum(ss);
    if ((tid & (kWave - 1)) == 0) part[tid / kWave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) tot += part[w];
    const float rms = sqrtf(tot / static_cast<float>(a.D) + a.norm_eps);
    for (int64_t d = tid; d < a.D; d += kThreads) row[d] = gamma[d] * row[d] / rms;
    __syncthreads();
    float* dst = is_q ? a.q_out + b * a.H * a.D + h * a.D : a.k_cache + b * a.seq_stride + p * kvd + h * a.D;
    for (int64_t i = tid; i < half; i += kThreads) {
        const int64_t lo = a.rotate_half ? i : 2 * i, hi = a.rotate_half ? i + half : 2 * i + 1;
        const float x0 = row[lo], x1 = row[hi];
        if (a.rope) {  // rope_rotate (row_math.hpp:93-110) at position p
            const float c = a.cos_t[p * half + i], s = a.sin_t[p * half + i];
            dst[lo] = x0 * c - x1 * s;
            dst[hi] = x0 * s + x1 * c;
        } else {
            dst[lo] = x0;
            dst[hi] = x1;
        }
    }
    if (!is_q) {
        const float* vs = a.v + b * a.ldv + h * a.D;
        float* vd = a.v_cache + b * a.seq_stride + p * kvd + h * a.D;
        for (int64_t d = tid; d < a.D; d += kThreads) vd[d] = vs[d];
    }
}

struct DecodeAttnArgs {
    const float* q;  // (n, H*D) contiguous, rotated
    const float* k_cache;
    const float* v_cache;
    int64_t seq_stride;
    float* ctx;      // (n, H*D) contiguous
    float* part;     // per (sequence, head, chunk): max, exp-sum, 2 pad, D partial context values
    const int32_t* pos;
    int64_t H, Hkv, D, window, max_keys, chunks;
    float scale;
    int vec;  // 128-bit key loads (head_dim, the strides and the bases multiples of 4 floats)
};

constexpr int kKeyChunk = 64;  // keys per workgroup of the first pass
constexpr int kPartHead = 4;   // a chunk's partial: max, exp-sum, two pad floats, then D context values
static_assert(kKeyChunk == kWave && kThreads == 4 * kKeyChunk, "a lane per key in the softmax, four threads per key");
typedef float f4 __attribute__((ext_vector_type(4)));

// The keys [j0, j1) of 64-key `chunk` that a query at cache position *pos sees: the position is
// clamped to the cache, a sliding layer's window starts at p + 1 - window (attention_masked,
// row_math.hpp:117-126), and a chunk wholly outside [lo, p] gets j1 <= j0. One definition for the
// kernel and for pxk_decode_chunk_keys, which checks it on the host.
__host__ __device__ inline void chunk_keys(int64_t pos, int64_t max_keys, int64_t window, int64_t chunk, int64_t* j0,
                                           int64_t* j1) {
    const int64_t p = pos < 0 ? 0 : (pos > max_keys - 1 ? max_keys - 1 : pos);
    const int64_t lo = (window > 0 && p + 1 > window) ? p + 1 - window : 0;
    const int64_t c0 = chunk * kKeyChunk, c1 = c0 + kKeyChunk;
    *j0 = c0 > lo ? c0 : lo;
    *j1 = c1 < p + 1 ? c1 : p + 1;
}

// First pass, one workgroup per (sequence, query head, 64-key chunk): the chunk's visible keys
// (within [lo, pos], a sliding layer's window per attention_masked, row_math.hpp:117-126) scored
// against the query by four threads per key (each on every fourth float4 of head_dim, summed with
// two shuffles), their max, exp-sum and exp-weighted values. Chunks past the position write an
// empty partial; the grid is the same at every position, so a step stays capturable.
__global__ void __launch_bounds__(kThreads) decode_attention_part_kernel(const DecodeAttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float* qs = sm;        // D
    float* sc = sm + a.D;  // kKeyChunk
    const int64_t bh = blockIdx.x / a.chunks, chunk = blockIdx.x - bh * a.chunks;
    const int64_t b = bh / a.H, h = bh - b * a.H, hk = h / (a.H / a.Hkv);
    const int64_t kvd = a.Hkv * a.D;
    int64_t j0, j1;
    chunk_keys(static_cast<int64_t>(*a.pos), a.max_keys, a.window, chunk, &j0, &j1);
    const int nk = j1 > j0 ? static_cast<int>(j1 - j0) : 0;
    float* out = a.part + (bh * a.chunks + chunk) * (a.D + kPartHead);
    const int tid = threadIdx.x;
    if (nk == 0) {  // nothing visible here
        for (int64_t d = tid; d < a.D + kPartHead; d += kThreads) out[d] = d == 0 ? -INFINITY : 0.0f;
        return;
    }
    for (int64_t d = tid; d < a.D; d += kThreads) qs[d] = a.q[b * a.H * a.D + h * a.D + d];
    __syncthreads();
    const int key = tid >> 2, quarter = tid & 3;
    float s = 0.0f;
    if (key < nk) {
        const float* kr = a.k_cache + b * a.seq_stride + (j0 + key) * kvd + hk * a.D;
        if (a.vec) {
            const int64_t nv = a.D / 4;
            for (int64_t f = quarter; f < nv; f += 4) {
                const f4 kv = *reinterpret_cast<const f4*>(kr + 4 * f);
                const f4 qv = *reinterpret_cast<const f4*>(qs + 4 * f);
                s += qv[0] * kv[0] + qv[1] * kv[1] + qv[2] * kv[2] + qv[3] * kv[3];
            }
        } else {
            for (int64_t d = quarter; d < a.D; d += 4) s += qs[d] * kr[d];
        }
    }
    s += __shfl_xor(s, 1, kWave);
    s += __shfl_xor(s, 2, kWave);
    if (key < nk && quarter == 0) sc[key] = a.scale * s;
    __syncthreads();
    if (tid < kWave) {  // kKeyChunk == kWave: one key per lane of the first wave
        const float v = tid < nk ? sc[tid] : -INFINITY;
        const float mx = wave_max(v);
        const float e = tid < nk ? expf(v - mx) : 0.0f;
        const float sum = wave_sum(e);
        if (tid < nk) sc[tid] = e;
        if (tid == 0) {
            out[0] = mx;
            out[1] = sum;
        }
    }
    __syncthreads();
    const float* vb = a.v_cache + b * a.seq_stride + j0 * kvd + hk * a.D;
    const int64_t nd4 = a.D / 4;
    if (a.vec && nd4 <= kThreads) {
        // Key groups of kThreads / nd4 threads: thread (kg, c) sums the float4 column c over keys
        // kg, kg + G, ...; the groups are added in order.
        f4* red = reinterpret_cast<f4*>(qs);  // the query is no longer needed; LDS holds D + 64 floats
        const int G = static_cast<int>(kThreads / nd4), c = static_cast<int>(tid % nd4), kg = static_cast<int>(tid / nd4);
        f4 acc = {0.f, 0.f, 0.f, 0.f};
        if (kg < G) {
#pragma unroll 4
            for (int j = kg; j < nk; j += G) acc += sc[j] * *reinterpret_cast<const f4*>(vb + j * kvd + 4 * c);
        }
        __syncthreads();  // every score read of the query row is done before it is overwritten
        for (int g = 0; g < G; ++g) {
            if (kg == g) red[c] = g == 0 ? acc : red[c] + acc;
            __syncthreads();
        }
        if (tid < nd4) *reinterpret_cast<f4*>(out + kPartHead + 4 * tid) = red[tid];
        return;
    }
    for (int64_t d = tid; d < a.D; d += kThreads) {
        float acc = 0.0f;
#pragma unroll 8
        for (int j = 0; j < nk; ++j) acc += sc[j] * vb[j * kvd + d];
        out[kPartHead + d] = acc;
    }
}

// Second pass, one workgroup per (sequence, query head): the chunks' partials merged with their
// maxima, ctx = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c.
__global__ void __launch_bounds__(kThreads) decode_attention_merge_kernel(const DecodeAttnArgs a) {
    const int64_t bh = blockIdx.x;
    const int64_t ps = a.D + kPartHead;
    const float* part = a.part + bh * a.chunks * ps;
    float M = -INFINITY;
    for (int64_t c = 0; c < a.chunks; ++c) M = fmaxf(M, part[c * ps]);
    float l = 0.0f;
    for (int64_t c = 0; c < a.chunks; ++c) {
        const float m = part[c * ps];
        if (m != -INFINITY) l += expf(m - M) * part[c * ps + 1];
    }
    for (int64_t d = threadIdx.x; d < a.D; d += kThreads) {
        float acc = 0.0f;
        for (int64_t c = 0; c < a.chunks; ++c) {
            const float m = part[c * ps];
            if (m != -INFINITY) acc += expf(m - M) * part[c * ps + kPartHead + d];
        }
        a.ctx[bh * a.D + d] = acc / l;
    }
}

constexpr int kPickThreads = 256;
constexpr int kPickSlices = 64;  // workgroups per sequence in the first pass

// The first maximum of a range of a row (ties to the lower index), 8 loads in flight per thread,
// merged across the workgroup in LDS; `none` is index V.
__device__ void argmax_range(const float* row, int64_t j0, int64_t j1, int64_t V, float& best, int64_t& idx) {
    __shared__ float bv[kPickThreads];
    __shared__ int64_t bi[kPickThreads];
    best = -INFINITY;
    idx = V;
    constexpr int kAhead = 8;
    for (int64_t base = j0 + threadIdx.x; base < j1; base += static_cast<int64_t>(kAhead) * kPickThreads) {
        float v[kAhead];
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            const int64_t j = base + static_cast<int64_t>(u) * kPickThreads;
            v[u] = row[j < j1 ? j : j1 - 1];
        }
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {  // j ascends within a thread: ties keep the first
            const int64_t j = base + static_cast<int64_t>(u) * kPickThreads;
            if (j < j1 && (idx == V || v[u] > best)) {
                best = v[u];
                idx = j;
            }
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
    best = bv[0];
    idx = bi[0];
}

struct PickArgs {
    const float* logits;
    int64_t ld_logits, V;
    float* ids;
    int64_t ld_ids;
    float* cur;
    float* picked_logit;
    int64_t ld_logit;
    const int32_t* pos;
    float* part_v;  // (n, kPickSlices) slice maxima and their indices
    int64_t* part_i;
};

// Greedy pick (Generate's greedy step: the first maximum of the logits), first pass: one slice of
// a row per workgroup.
__global__ void __launch_bounds__(kPickThreads) decode_pick_part_kernel(const PickArgs a) {
    const int64_t b = blockIdx.y, slice = blockIdx.x;
    const int64_t len = (a.V + kPickSlices - 1) / kPickSlices;
    const int64_t j0 = slice * len, j1 = min(a.V, j0 + len);
    float best;
    int64_t idx;
    argmax_range(a.logits + b * a.ld_logits, j0, j1 > j0 ? j1 : j0, a.V, best, idx);
    if (threadIdx.x == 0) {
        a.part_v[b * kPickSlices + slice] = best;
        a.part_i[b * kPickSlices + slice] = idx;
    }
}

// Second pass: the slices merged in index order (larger value first, the lower index on ties); the
// pick is written as the sequence's next id (ids[b, pos + 1]), as the next step's token (cur[b]) and
// with its logit (picked_logit[b, pos + 1], the OutputValue seed an explanation of it uses).
__global__ void __launch_bounds__(kWave) decode_pick_merge_kernel(const PickArgs a) {
    const int64_t b = blockIdx.x;
    if (threadIdx.x != 0) return;
    float best = -INFINITY;
    int64_t idx = a.V;
    for (int s = 0; s < kPickSlices; ++s) {
        const float v = a.part_v[b * kPickSlices + s];
        const int64_t i = a.part_i[b * kPickSlices + s];
        if (i != a.V && (idx == a.V || v > best)) {
            best = v;
            idx = i;
        }
    }
    const int64_t next = static_cast<int64_t>(*a.pos) + 1;
    const int64_t t = idx < a.V ? idx : 0;  // a row of NaNs picks id 0 rather than leave the table
    a.cur[b] = static_cast<float>(t);
    if (next >= 0 && next < a.ld_ids) a.ids[b * a.ld_ids + next] = static_cast<float>(t);
    if (a.picked_logit && next >= 0 && next < a.ld_logit) a.picked_logit[b * a.ld_logit + next] = best;
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
                                      int rotate_half, const float* q_gamma, const float* k_gamma, float norm_eps,
                                      void* stream) {
    const int64_t qd = heads * head_dim, kvd = kv_heads * head_dim;
    if (n < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || head_dim <= 0 || head_dim % 2 != 0 ||
        ldq < qd || ldk < kvd || ldv < kvd || positions <= 0 || seq_stride < positions * kvd)
        return fail(PXK_ERR_INVALID, "pxk_decode_rope_append: bad sizes or strides (the cache must hold `positions`)");
    if (n == 0) return PXK_OK;
    if (!q || !k || !v || !q_out || !k_cache || !v_cache || !pos || (rope && (!cos_t || !sin_t)))
        return fail(PXK_ERR_INVALID, "pxk_decode_rope_append: a required operand is NULL");
    if ((q_gamma == nullptr) != (k_gamma == nullptr))
        return fail(PXK_ERR_INVALID, "pxk_decode_rope_append: QK-Norm needs both q_gamma and k_gamma");
    const RopeAppendArgs a{q,        ldq,     k,       ldk,   v,       ldv,       q_out,    k_cache,
                           v_cache,  seq_stride, cos_t, sin_t, pos,   n,         heads,    kv_heads,
                           head_dim, positions,  rope,  rotate_half, q_gamma, k_gamma, norm_eps};
    if (q_gamma) {
        const size_t lds = static_cast<size_t>(head_dim) * sizeof(float);
        if (lds > 60 * 1024 || n * (heads + kv_heads) > (int64_t{1} << 31) - 1)
            return fail(PXK_ERR_INVALID, "pxk_decode_rope_append: head_dim must fit LDS");
        PXK_LAUNCH(rope_append_norm_kernel, dim3(static_cast<unsigned>(n * (heads + kv_heads))), dim3(kThreads),
                           lds, S(stream), a);
        return launched("pxk_decode_rope_append (QK-Norm)");
    }
    const int64_t work = n * (heads + kv_heads) * (head_dim / 2) + n * kvd;
    PXK_LAUNCH(rope_append_kernel, dim3(grid_for(work, kThreads)), dim3(kThreads), 0, S(stream), a);
    return launched("pxk_decode_rope_append");
}

extern "C" size_t pxk_decode_attention_workspace(int64_t n, int64_t heads, int64_t head_dim, int64_t max_keys) {
    if (n <= 0 || heads <= 0 || head_dim <= 0 || max_keys <= 0) return 0;
    return static_cast<size_t>(n * heads * cdiv(max_keys, kKeyChunk) * (head_dim + kPartHead)) * sizeof(float);
}

extern "C" int pxk_decode_attention(const float* q, const float* k_cache, const float* v_cache, int64_t seq_stride,
                                    float* ctx, const int32_t* pos, int64_t n, int64_t heads, int64_t kv_heads,
                                    int64_t head_dim, int64_t window, int64_t max_keys, float scale, float* workspace,
                                    size_t workspace_bytes, void* stream) {
    if (n < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || head_dim <= 0 || window < 0 ||
        max_keys <= 0 || seq_stride < max_keys * kv_heads * head_dim)
        return fail(PXK_ERR_INVALID, "pxk_decode_attention: bad sizes (the cache must hold max_keys positions)");
    const size_t lds = static_cast<size_t>(head_dim + kKeyChunk) * sizeof(float);
    if (lds > 60 * 1024) return fail(PXK_ERR_INVALID, "pxk_decode_attention: head_dim must fit LDS");
    if (n == 0) return PXK_OK;
    if (!q || !k_cache || !v_cache || !ctx || !pos) return fail(PXK_ERR_INVALID, "pxk_decode_attention: NULL operand");
    const size_t need = pxk_decode_attention_workspace(n, heads, head_dim, max_keys);
    if (!workspace || workspace_bytes < need)
        return fail(PXK_ERR_WORKSPACE, "pxk_decode_attention: needs %zu workspace bytes", need);
    const int64_t chunks = cdiv(max_keys, kKeyChunk);
    if (n * heads * chunks > (int64_t{1} << 31) - 1) return fail(PXK_ERR_INVALID, "pxk_decode_attention: too large");
    const int vec = head_dim % 4 == 0 && seq_stride % 4 == 0 && aligned16(k_cache) && aligned16(v_cache) &&
                    aligned16(workspace);
    const DecodeAttnArgs a{q,        k_cache, v_cache,  seq_stride, ctx,   workspace, pos, heads,
                           kv_heads, head_dim, window, max_keys, chunks, scale, vec};
    PXK_LAUNCH(decode_attention_part_kernel, dim3(static_cast<unsigned>(n * heads * chunks)), dim3(kThreads),
                       lds, S(stream), a);
    if (const int rc = launched("pxk_decode_attention")) return rc;
    PXK_LAUNCH(decode_attention_merge_kernel, dim3(static_cast<unsigned>(n * heads)), dim3(kThreads), 0,
                       S(stream), a);
    return launched("pxk_decode_attention (merge)");
}

extern "C" int pxk_decode_chunk_keys(int64_t pos, int64_t max_keys, int64_t window, int64_t chunk, int64_t* j0,
                                     int64_t* j1) {
    if (max_keys <= 0 || window < 0 || chunk < 0 || !j0 || !j1)
        return fail(PXK_ERR_INVALID, "pxk_decode_chunk_keys: bad arguments");
    chunk_keys(pos, max_keys, window, chunk, j0, j1);
    return PXK_OK;
}

extern "C" size_t pxk_decode_pick_workspace(int64_t n) {
    return n > 0 ? static_cast<size_t>(n * kPickSlices) * (sizeof(float) + sizeof(int64_t)) : 0;
}

extern "C" int pxk_decode_pick(const float* logits, int64_t ld_logits, int64_t n, int64_t vocab, float* ids,
                               int64_t ld_ids, float* cur, float* picked_logit, int64_t ld_logit, const int32_t* pos,
                               void* workspace, size_t workspace_bytes, void* stream) {
    if (n < 0 || vocab <= 0 || ld_logits < vocab || ld_ids < 1 || (picked_logit && ld_logit < 1) || n > 65535)
        return fail(PXK_ERR_INVALID, "pxk_decode_pick: bad sizes");
    if (n == 0) return PXK_OK;
    if (!logits || !ids || !cur || !pos) return fail(PXK_ERR_INVALID, "pxk_decode_pick: NULL operand");
    if (!workspace || workspace_bytes < pxk_decode_pick_workspace(n) || !aligned16(workspace))
        return fail(PXK_ERR_WORKSPACE, "pxk_decode_pick: needs %zu workspace bytes (16-byte aligned)",
                    pxk_decode_pick_workspace(n));
    auto* pi = static_cast<int64_t*>(workspace);
    auto* pv = reinterpret_cast<float*>(pi + n * kPickSlices);
    const PickArgs a{logits, ld_logits, vocab, ids, ld_ids, cur, picked_logit, ld_logit, pos, pv, pi};
    PXK_LAUNCH(decode_pick_part_kernel, dim3(kPickSlices, static_cast<unsigned>(n)), dim3(kPickThreads), 0,
                       S(stream), a);
    if (const int rc = launched("pxk_decode_pick")) return rc;
    PXK_LAUNCH(decode_pick_merge_kernel, dim3(static_cast<unsigned>(n)), dim3(kWave), 0, S(stream), a);
    return launched("pxk_decode_pick (merge)");
}

extern "C" int pxk_decode_advance(int32_t* pos, void* stream) {
    if (!pos) return fail(PXK_ERR_INVALID, "pxk_decode_advance: NULL position");
    PXK_LAUNCH(decode_advance_kernel, dim3(1), dim3(kWave), 0, S(stream), pos);
    return launched("pxk_decode_advance");
}

extern "C" int pxk_seed_rows(const float* logits, int64_t ld_logits, const float* targets, int64_t stride, int64_t n,
                             int64_t vocab, float* seed, int64_t* targets_out, int unit, void* stream) {
    if (n < 0 || vocab <= 0 || stride < 0 || n > 65535 || ld_logits < vocab)
        return fail(PXK_ERR_INVALID, "pxk_seed_rows: bad sizes");
    if (n == 0) return PXK_OK;
    if (!targets || !seed || (!unit && !logits)) return fail(PXK_ERR_INVALID, "pxk_seed_rows: NULL operand");
    const unsigned gx = static_cast<unsigned>(std::min<int64_t>(cdiv(vocab, kThreads), 1024));
    PXK_LAUNCH(seed_rows_kernel, dim3(gx, static_cast<unsigned>(n)), dim3(kThreads), 0, S(stream), logits,
                       ld_logits, targets, stride, vocab, seed, targets_out, unit);
    return launched("pxk_seed_rows");
}
