/*
 * pxk.h -- C ABI of the gfx950 kernel library (libpxk_gfx950.so).
 *
 * Hand-written HIP kernels for MI355X (CDNA4, wave64, fp32 MFMA) behind plain C entry points:
 * device pointers, sizes, scalars and a hipStream_t passed as void*. No C++ types cross this
 * boundary. Every entry point is asynchronous on `stream` (NULL = the default stream), returns
 * PXK_OK or an error code, and leaves a message for pxk_last_error(). Sizes are validated on the
 * host before any launch; n == 0 is a no-op (src/hip_backend.hip:142-147 contract).
 *
 * Each entry point names the reference interface it replaces: the DeviceBackend virtual in
 * include/pulsatrix/device_backend.hpp (file:line) and, where Pulsatrix's HIP backend ran it
 * through hipBLAS or a one-thread-per-output kernel, that implementation. Aliasing follows the
 * virtual's contract.
 */
#ifndef PXK_H
#define PXK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    PXK_OK = 0,
    PXK_ERR_INVALID = 1,  /* bad size, layout or mode: nothing was launched */
    PXK_ERR_LAUNCH = 2,   /* the HIP runtime refused the launch */
    PXK_ERR_WORKSPACE = 3 /* a split-K GEMM, decode attention or pick was given too small a workspace */
};

const char* pxk_last_error(void);
/* Library and device identification, for the test that the library loads on the GPU box. */
const char* pxk_version(void);

/* Per-dispatch timing, a profiling aid with no reference counterpart. Between pxk_timing_begin
 * and pxk_timing_end on one host thread, each kernel that thread launches (up to `capacity`)
 * records its own start and end events (hipExtLaunchKernelGGL); pxk_timing_count() is the number
 * of launches recorded so far, and pxk_timing_end waits for them and writes their durations in
 * milliseconds, in launch order. Launches under HIP graph capture must not run inside a window. */
int pxk_timing_begin(int capacity);
int pxk_timing_count(void);
int pxk_timing_end(float* ms, int capacity);

/* ---- the fused fp32 MFMA GEMM ------------------------------------------------------------------
 * C[b] = op(Aeff[b]) * op(B[b]) over a batch of independent products, fp32 in, fp32 MFMA
 * (v_mfma_f32_16x16x4_f32) with fp32 accumulation, LDS-staged double-buffered tiles of 128x128,
 * 64x64, 32x64 or 32x32 (the small ones split each K stage over their four waves), optional
 * deterministic split-K (fixed-order reduction, no atomics in the sum).
 *
 * Batch addressing, per operand: batch index b = outer * inner + i (inner = desc.inner), and
 *   base(b, s) = ptr + outer * batch_stride + (i / inner_div) * inner_stride + s * group_stride
 * where s runs over desc.kgroups sub-products accumulated into the same output (a GQA key/value
 * head summing its query heads). inner_div maps a query head to its KV head.
 *
 * Replaces: DeviceBackend::gemm (device_backend.hpp:303), gemm_ex (:361), gemm_strided_batched
 * (:372-383) -- HIPBackend's hipblasSgemm / hipblasSgemmStridedBatched (hip_backend.hip:122-139,
 * 170-190, 277-295) -- and, through the prologue/epilogue modes, the op sequences of
 * lrp_rules::linear (lrp_rules.cpp:197-220), DeviceBackend::lrp_linear (:627), lrp_bilinear_matmul
 * (:643) and the tied head's epsilon rule (tied_lm_head_module.cpp:76-111).
 */
typedef struct pxk_operand {
    const float* ptr;
    int64_t ld;           /* row stride (elements) of the stored matrix */
    int64_t batch_stride; /* per outer batch index */
    int64_t inner_stride; /* per (inner index / inner_div) */
    int64_t inner_div;    /* <= 1: none */
    int64_t group_stride; /* per k-group sub-product */
} pxk_operand;

enum {
    PXK_CAUSAL_NONE = 0,
    PXK_CAUSAL_TRI = 1,    /* only output tiles touching n <= m are computed; the rest are not written */
    PXK_CAUSAL_K_LE_M = 2, /* the sum runs over k <= m (P @ V, S @ K) */
    PXK_CAUSAL_K_GE_M = 3  /* the sum runs over k >= m (P^T @ S, S^T @ Q) */
};

enum {
    PXK_PRO_NONE = 0,
    PXK_PRO_DIV_STAB = 1, /* A / (Z + bias[k] + eps * sign(Z + bias[k])), sign(0) = +1 (lrp_math.hpp:17) */
    PXK_PRO_RMS = 2       /* A is the input x of an RMSNorm over its K columns (rms_norm_module.cpp:51-68;
                             RMSNormForward, row_math.hpp) whose gamma the caller has folded into B
                             (B[k][n] = gamma[k] W[k][n], pxk_scale_rows): the product is taken over the
                             norm's output y[m][k] = gamma[k] x[m][k] / rms[m] with
                             rms[m] = sqrt(mean_k x[m][k]^2 + norm_eps), computed as
                             (sum_k x[m][k] B[k][n]) / rms[m]. A untransposed, no k-groups, causal range,
                             split-K, z or z_bias; row_rms (nullable) receives rms, batch b at b * m + row.
                             Replaces the norm's separate row kernel. */
};

enum {
    PXK_EPI_STORE = 0,       /* C = acc, or acc + beta * C when beta != 0 */
    PXK_EPI_STORE_BIAS = 1,  /* C = acc (pre-bias z); C2 = acc + bias[n] when bias given */
    PXK_EPI_ADD_RESID = 2,   /* C = acc; C2 = acc + bias[n] (bias optional, else C2 = C); C3 = X + C2 */
    PXK_EPI_MUL_X = 3,       /* C = X * acc, or Y + X * acc when Y is given */
    PXK_EPI_SPV = 4,         /* r = X * acc; C = r / (2 X + eps * sign X) */
    PXK_EPI_ROPE_REL = 5,    /* r = Y * acc; RoPE epsilon rule with x = X, y = Y over the head's pairs;
                                C = r_in (may be NULL); C2 = r_in / stab(Z + bias[n]) */
    PXK_EPI_VALUE_REL = 6,   /* r = Y * acc; C = r (may be NULL); C2 = r / stab(Z + bias[n]) */
    PXK_EPI_SWIGLU_REL = 7,  /* SwiGLU relevance: rh = X * acc (X = hidden); c = Y * W (gate_post * up);
                                rg = (c / (2c + eps sign c)) * rh; C = rg / stab(Z2 + bias[n]) (gate);
                                C2 = rg / stab(Z3 + bias2[n]) (up). Z stays the prologue's. Without
                                biases X, Y and W may all be NULL: gate_post = act(Z2) (gate_act),
                                up = Z3 and hidden = gate_post * up are recomputed as the forward
                                computed them, saving three reads per element. */
    PXK_EPI_MUL_X_SPLIT = 8, /* r = X * acc, or Y + X * acc; then the epsilon split of the residual sum
                                W = Z2 + Z3 whose relevance r is (lrp_residual_split, lrp_math.hpp:33-38):
                                C = (Z2 / stab(W)) * r, C2 = (Z3 / stab(W)) * r. W must hold Z2 + Z3 as the
                                forward computed it. Z stays the prologue's. With c2_den given, C2 is
                                that share divided by its consumer's stabilised denominator,
                                C2 = ((Z3 / stab(W)) * r) / stab(c2_den + c2_den_bias[n]): the next
                                relevance GEMM then reads it without the DIV_STAB prologue. */
    PXK_EPI_ROPE_FWD = 9,    /* C = acc; C2 = y = acc + bias[n] when a bias is given (else y = acc); and
                                for columns n < rope_cols, C3 = y rotated pairwise at position m
                                (rope_rotate, row_math.hpp:93-110; pairs inside each head_dim block) */
    PXK_EPI_SWIGLU_FWD = 10  /* SwiGLU gate (swiglu_module.cpp:80-88) on a gate/up GEMM whose B columns
                                alternate 32-wide gate and up blocks (block 2b: gate features 32b..32b+31,
                                block 2b+1: the same up features); N = 2F, F a multiple of 32, no bias.
                                C (ld >= 2F) = z as [gate | up] halves; C3 = gate_post = silu(z_gate)
                                (x / (1 + e^-x), cpu_backend.cpp:29; GeLU tanh with gate_act 1);
                                C2 = hidden = gate_post * z_up. */
};

enum {
    PXK_TILE_AUTO = 0,
    PXK_TILE_128x128 = 1, /* 4 waves of 64x64, K stage 32 */
    PXK_TILE_64x64 = 2,   /* 4 waves of 32x32, K stage 32 */
    PXK_TILE_32x64 = 3,   /* 4 waves each on a quarter of a 64-wide K stage, summed in LDS */
    PXK_TILE_32x32 = 4,   /* as 32x64 */
    PXK_TILE_32x64_DIRECT = 5, /* as 32x64, each wave streaming its operands from L2 into registers */
    PXK_TILE_32x32_DIRECT = 6,
    PXK_TILE_SKINNY = 7,  /* m <= 16, unbatched, A untransposed, no prologue or causal range: B streamed
                             with 128-bit vector loads, A in LDS, 64-column tiles; NN split over K
                             (STORE, STORE_BIAS, ADD_RESID, SWIGLU_FWD), NT in one pass (STORE, K up
                             to about 4000 rows at m <= 4). PXK_TILE_AUTO picks it whenever it applies */
    PXK_TILE_32x48_DIRECT = 8, /* as 32x64 direct, 48 columns: 192 workgroups over a 512 x 576 output */
    PXK_TILE_32x48 = 9        /* as 32x64, 48 columns */
};

typedef struct pxk_gemm_desc {
    int64_t m, n, k;
    int64_t batch;   /* >= 1 */
    int64_t inner;   /* >= 1 */
    int64_t kgroups; /* >= 1 */
    int32_t trans_a; /* A stored (K x M) instead of (M x K) */
    int32_t trans_b; /* B stored (N x K) instead of (K x N) */
    int32_t causal;
    int32_t prologue;
    int32_t epilogue;
    int32_t splits; /* split-K factor; 0 = chosen by the library */
    float beta;
    float eps;
    pxk_operand a, b, c;
    pxk_operand z;        /* prologue denominators, laid out like A */
    pxk_operand z_bias;   /* prologue bias over k (ld 0; batch strides as for A), ptr nullable */
    pxk_operand c2, c3;   /* extra outputs, laid out like C */
    pxk_operand x, y, w;  /* epilogue inputs, laid out like C */
    pxk_operand z2, z3;   /* SWIGLU_REL's gate / up denominators */
    pxk_operand e_bias;   /* epilogue bias over n (ld 0; batch strides as for C), ptr nullable */
    pxk_operand e_bias2;
    const float* cos_t;   /* RoPE tables (positions x head_dim/2), position = m */
    const float* sin_t;
    int64_t head_dim;     /* ROPE_REL: pairs live inside each head_dim-wide column block */
    int32_t rope_half;    /* 1: pair (i, i + D/2); 0: pair (2i, 2i+1) */
    int32_t tile;         /* 0 = chosen by the library; else PXK_TILE_* (a tuning override) */
    float* workspace;     /* split-K partials */
    size_t workspace_bytes;
    int64_t rope_cols;    /* ROPE_FWD: the leading columns (whole heads) that are rotated into C3 */
    int32_t gate_act;     /* SWIGLU_FWD's gate: 0 SiLU, 1 GeLU tanh (pointwise_math.hpp:32-36) */
    int32_t reserved;
    pxk_operand c2_den;      /* MUL_X_SPLIT, ptr nullable: C2 is divided by stab(c2_den + c2_den_bias[n]) */
    pxk_operand c2_den_bias; /* bias over n of that denominator (ld 0), ptr nullable */
    const float* x_rms;      /* MUL_X, MUL_X_SPLIT, nullable (with x_gamma): X holds an RMSNorm's input x and
                                the epilogue reads y = x_gamma[n] * X[m][n] / x_rms[m] (the norm's output,
                                as its row kernel computes it) in its place. Unbatched. */
    const float* x_gamma;
    float* row_rms;          /* PXK_PRO_RMS: receives rms[m] (nullable) */
    float norm_eps;          /* PXK_PRO_RMS */
    int32_t reserved2;
} pxk_gemm_desc;

/* Bytes of workspace pxk_gemm needs for this descriptor (0 when it runs without split-K). */
size_t pxk_gemm_workspace(const pxk_gemm_desc* d);
int pxk_gemm(const pxk_gemm_desc* d, void* stream);

/* pxk_gemm without a workspace argument and without any allocation: the split-K partials live in a
 * static device array of PXK_GEMM_SCRATCH_BYTES per GPU, held until the process ends (its device
 * address is looked up once per device, on the first split-K call there, which must be made outside
 * any stream capture: under capture that first call returns PXK_ERR_INVALID and launches nothing;
 * after it, captured calls are valid). d->workspace is ignored. The
 * plan, kernels and results are pxk_gemm's for the same descriptor; a plan whose partials exceed
 * the scratch returns PXK_ERR_WORKSPACE before any launch. The array is shared by every call on a
 * GPU and keeps the last call's partials: calls that overlap on one GPU (other streams, other
 * threads) race. It has no counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). */
#define PXK_GEMM_SCRATCH_BYTES ((size_t)64 << 20)
int pxk_gemm_noalloc(const pxk_gemm_desc* d, void* stream);

/* The tile shape (PXK_TILE_*) and split-K count pxk_gemm would launch for this descriptor, after
 * the same validation. Introspection for tuning and tests; no reference counterpart. */
int pxk_gemm_plan(const pxk_gemm_desc* d, int32_t* tile, int32_t* splits);

/* The (trans_a, trans_b, prologue, epilogue) combinations built into the library; pxk_gemm
 * rejects others with PXK_ERR_INVALID. */
int pxk_gemm_supported(int trans_a, int trans_b, int prologue, int epilogue);

/* Plain gemm_ex: out = op(a) op(b) + beta out, row-major, contiguous (device_backend.hpp:361). */
int pxk_gemm_ex(const float* a, int transpose_a, const float* b, int transpose_b, float* out, int64_t m, int64_t k,
                int64_t n, float beta, float* workspace, size_t workspace_bytes, void* stream);

/* ---- elementwise (memory-bound, 128-bit accesses where aligned) --------------------------------- */
/* DeviceBackend::fill (:291) */
int pxk_fill(float* ptr, float value, int64_t n, void* stream);
/* DeviceBackend::elementwise (:313); op = ElementwiseOp order: Relu, Neg, Tanh, Sigmoid, Silu, Exp,
 * GeluTanh, Gelu (device_backend.hpp:39-48). */
int pxk_elementwise(int op, const float* in, float* out, int64_t n, void* stream);
/* DeviceBackend::add (:328), mul (:344), axpby (:436) */
int pxk_add(const float* a, const float* b, float* out, int64_t n, void* stream);
int pxk_mul(const float* a, const float* b, float* out, int64_t n, void* stream);
int pxk_axpby(float alpha, const float* x, float beta, const float* y, float* out, int64_t n, void* stream);
/* DeviceBackend::add_row_vector (:405) */
int pxk_add_row_vector(const float* in, const float* row, float* out, int64_t rows, int64_t cols, void* stream);
/* out[i][j] = in[i][j] * scale[i]: an RMSNorm's gamma folded into the (in x out) weight of the
 * projection that reads the norm's output (PXK_PRO_RMS). No reference counterpart: the reference
 * applies gamma in the norm (rms_norm_module.cpp:51-68). */
int pxk_scale_rows(const float* in, const float* scale, float* out, int64_t rows, int64_t cols, void* stream);
/* DeviceBackend::lrp_residual_split (:631), lrp_bilinear_elementwise (:635), lrp_stabilized_divide (:712) */
int pxk_lrp_residual_split(const float* a, const float* b, const float* r, float* r_a, float* r_b, int64_t n,
                           float eps, void* stream);
int pxk_lrp_bilinear_elementwise(const float* a, const float* b, const float* r, float* r_out, int64_t n, float eps,
                                 void* stream);
int pxk_lrp_stabilized_divide(const float* r, const float* denom, const float* gate, float* out, int64_t n, float eps,
                              int gate_mode, void* stream);
/* The Eq. 15 scaled relevance of a product O = A B: s = r / (2 o + eps sign o) (lrp_math.hpp:57-61),
 * the shared factor of DeviceBackend::lrp_bilinear_matmul's two shares (:643). */
int pxk_lrp_bilinear_scale(const float* r, const float* o, float* s, int64_t n, float eps, void* stream);
/* SwiGLU gate (swiglu_module.cpp:80-88): gate_post = act(gate), hidden = gate_post * up, over an
 * (rows x 2F) [gate | up] buffer with row stride ld; act 0 SiLU, 1 GeLU tanh (Gemma's GeGLU). */
int pxk_swiglu_forward(const float* gu, int64_t ld, float* gate_post, float* hidden, int64_t rows, int64_t f, int act,
                       void* stream);
/* DeviceBackend::copy_2d (:783), accumulate_rows (:792), gather_rows (:596) */
/* buf[k * count + i] = buf[i] for k = 1 .. copies - 1 (buf holds copies * count floats): one forward
 * pass's activations repeated for several relevance seeds of the same sequences. No reference
 * counterpart; it replaces rerunning the forward per copy. */
int pxk_repeat_block(float* buf, int64_t count, int64_t copies, void* stream);
int pxk_copy_2d(float* dst, int64_t dst_stride, const float* src, int64_t src_stride, int64_t rows, int64_t cols,
                void* stream);
int pxk_accumulate_rows(const float* in, float* out, int64_t rows, int64_t cols, void* stream);
int pxk_gather_rows(const float* table, const float* indices, float* out, int64_t count, int64_t dim, void* stream);
/* DeviceBackend::column_sums (:399) */
int pxk_column_sums(const float* in, float* out, int64_t rows, int64_t cols, float beta, void* stream);

/* ---- row kernels (one wave64 per row, shuffle reductions) ------------------------------------- */
/* DeviceBackend::rms_norm_forward (:550); row_rms may be NULL. */
int pxk_rms_norm_forward(const float* in, const float* gamma, float* out, float* row_rms, int64_t rows, int64_t cols,
                         float eps, void* stream);
/* DeviceBackend::softmax_rows (:456) */
int pxk_softmax_rows(const float* in, float* out, int64_t rows, int64_t cols, void* stream);
/* DeviceBackend::lrp_softmax_rows (:648) */
int pxk_lrp_softmax_rows(const float* x, const float* y, const float* r, float* r_in, int64_t rows, int64_t cols,
                         void* stream);
/* Per-row sums (EmbeddingModule::propagate_relevance's ones-gemm, embedding_module.cpp:116-123). */
int pxk_row_sums(const float* in, float* out, int64_t rows, int64_t cols, void* stream);
/* DeviceBackend::sum (:504) / dot (:443): deterministic two-pass reduction into out[0]. */
int pxk_sum(const float* in, int64_t n, float* out, float* partials, void* stream);
int pxk_dot(const float* a, const float* b, int64_t n, float* out, float* partials, void* stream);
size_t pxk_reduce_partials(int64_t n);

/* ---- attention ------------------------------------------------------------------------------- */
/* Byte range of the attention forward's K or V tile buffer resource, counted from the tile's first
 * row key0 of one head's column segment in a row-major operand with row stride ld: it ends with the
 * head's head_dim values of the sequence's last row (l - 1), so rows past the sequence and columns
 * past head_dim on that row read 0. The kernel's own definition, on the host: introspection for
 * tests, no reference counterpart. -1 on bad arguments. */
int64_t pxk_attention_kv_tile_records(int64_t l, int64_t key0, int64_t ld, int64_t head_dim);
/* Fused causal (or full) GQA attention forward over (n, l) tokens: raw = Q K^T per query head,
 * P = softmax(scale * raw) over the visible keys, ctx = P V, in one launch. q, k, v are token-major
 * head-packed rows (row b*l + i, head h at column h*head_dim; query head h reads KV head
 * h / (heads / kv_heads)); raw and P are (n, heads, l, l), P with zeros past the visible keys and
 * raw defined on the visible keys only; ctx is written head-packed like q. Replaces the sequence of
 * MultiHeadAttentionModule::forward (multihead_attention_module.cpp:268-291): per-head gemm_ex,
 * axpby scale, attention_mask_fill, softmax_rows, gemm. pxk_attention_supported() tells whether
 * a shape is handled: head_dim a multiple of 4 up to 128, q/k row strides a multiple of 4, and a
 * workgroup's 16 score rows (16 x seq_len floats) within LDS, about 2000 tokens. */
int pxk_attention_supported(int64_t head_dim, int64_t seq_len, int64_t ldq, int64_t ldk, int64_t ldv);
int pxk_attention_forward(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v, int64_t ldv,
                          float* raw, float* p, float* ctx, int64_t ldctx, int64_t n, int64_t l, int64_t heads,
                          int64_t kv_heads, int64_t head_dim, float scale, int causal, void* stream);
/* The same forward with the softmax's row statistics: per query head and row, the max
 * m = max over the visible keys of scale * raw and 1 / sum of exp(scale * raw - m) into stats
 * (n, heads, l, 2), from which P = exp(scale * raw - m) * (1 / sum) is recomputed where the
 * relevance pass needs it (pxk_attention_relevance_q / _kv with their stats operand). raw and p
 * are optional here (NULL: not written); with neither there are no score rows in LDS and no
 * sequence-length limit beyond 65536. ctx as above; head_dim a multiple of 4 up to 128, q/k row
 * strides a multiple of 4. */
int pxk_attention_forward_stats(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                                int64_t ldv, float* raw, float* p, float* stats, float* ctx, int64_t ldctx,
                                int64_t n, int64_t l, int64_t heads, int64_t kv_heads, int64_t head_dim, float scale,
                                int causal, void* stream);
/* Whether pxk_attention_forward_stats, with neither raw nor p, runs a shape GQA-shared: one
 * workgroup per (sequence, KV head, 16-row block) whose waves are the KV head's query heads, each
 * K / V tile read into LDS once for the group (v 16-byte aligned with a row stride a multiple of 4
 * besides). 1 where each 16-row block has at least 16 (sequence, KV head) workgroups, 512 in all,
 * and 2, 3, 4 or 8 query heads per KV head; else 0 (the per-head kernel, whose waves split a
 * block's key tiles). No counterpart in the reference, whose forward is per head
 * (multihead_attention_module.cpp:268-291): it names the plan, as pxk_gemm_plan does. */
int pxk_attention_forward_gqa(int64_t n, int64_t l, int64_t heads, int64_t kv_heads);

/* The AttnLRP pass of one attention layer through the steps that need whole score rows, fused per
 * query head and 16-row block (MultiHeadAttentionModule::propagate_relevance,
 * multihead_attention_module.cpp:404-485, with lrp_bilinear_matmul lrp_math.hpp:57-86,
 * lrp_softmax_rows :89-98 and lrp_rope :104-123):
 *   r_attn = P * (s_pv V^T)                  P V bilinear share (s_pv = r_ctx / (2 ctx + eps sign ctx))
 *   s      = (scale raw)(r_attn - P sum_row r_attn) / (2 raw + eps sign raw), 0 where masked
 *   r_q    = Q * (s K)                        Q K^T bilinear share (Q, K after RoPE)
 *   g_q    = RoPE rule(x = Q before RoPE, y = Q, r_q) / stab(z_q + bias)   (no RoPE: r_q / stab(...))
 * s is written over whole rows (zeros past the visible keys) for the key share. Layouts as for
 * pxk_attention_forward; z, q_pre and g are head-packed rows with their own strides, bias (heads *
 * head_dim) is NULL under the pre-bias rule or without a q_proj bias. */
typedef struct pxk_attn_rel_desc {
    int64_t n, l, heads, kv_heads, head_dim;
    float scale, eps;
    int32_t causal, rope, rope_half;
    int32_t relevance_only; /* 1: g = the RoPE rule's r_q itself, no q_proj denominator (z may be NULL) */
    const float* spv;
    int64_t ld_spv;
    const float* v;
    int64_t ld_v;
    const float* k;
    int64_t ld_k;
    const float* p;
    const float* raw;
    float* s;
    const float* q;
    int64_t ld_q;
    const float* q_pre;
    int64_t ld_q_pre;
    const float* z;
    int64_t ld_z;
    const float* bias;
    const float* cos_t; /* (l x head_dim/2), position = row within the sequence */
    const float* sin_t;
    float* g;
    int64_t ld_g;
    /* The recomputing form, selected by a non-NULL stats: p and raw are not read (may be NULL).
     * Per 16-key tile the kernel recomputes raw = Q K^T (the forward's product, from q and k as
     * given here) and P = exp(scale raw - m) / sum from the forward's row statistics
     * (pxk_attention_forward_stats), and takes the softmax rule's row sum of r_attn as
     * s_pv . ctx, which equals the sum of P * (s_pv V^T) over the keys. s and p_out (both
     * nullable) receive s and P over each 16-row block's 16-key tiles up to its diagonal, zeros
     * at the masked keys within them (all that pxk_attention_relevance_kv reads under `causal`);
     * entries past those tiles are left as they were. No sequence-length limit beyond 65536; q, k
     * and ctx 16-byte aligned with row strides a multiple of 4. */
    const float* ctx;   /* the attention output P V, head-packed as the forward writes it */
    int64_t ld_ctx;
    const float* stats; /* (n, heads, l, 2): max of scale * raw and 1 / sum per row */
    float* row_sum;     /* nullable: receives s_pv . ctx per (n, heads, l) row */
    float* p_out;       /* nullable: receives P (n, heads, l, l) on the visible keys */
} pxk_attn_rel_desc;
int pxk_attention_relevance_q(const pxk_attn_rel_desc* d, void* stream);

/* The key and value shares of one attention layer's AttnLRP pass, fused per KV head, 16-key
 * block and 16-wide group of head dimensions (MultiHeadAttentionModule::propagate_relevance,
 * multihead_attention_module.cpp:446-475: the b-shares of lrp_bilinear_matmul, lrp_math.hpp:57-86,
 * summed over the query heads of each KV head as sum_kv_groups does, :173-188; lrp_rope
 * lrp_math.hpp:104-123 for the keys; then the k/v projections' stabilised denominators):
 *   r_k = K * sum_h s_h^T Q_h      -> key_rel = RoPE rule(x = k_pre, y = K, r_k),  g_k = key_rel / stab(z_k + bias_k)
 *   r_v = V * sum_h P_h^T s_pv_h   -> value_rel = r_v,                          g_v = r_v / stab(z_v + bias_v)
 * s and P are (n, heads, l, l) with zeros at masked entries (as pxk_attention_relevance_q and
 * pxk_attention_forward write them); under `causal` only queries at or after each key are read.
 * q (post-RoPE), s_pv, k (post-RoPE), k_pre, v, z_k, z_v, key_rel, value_rel, g_k and g_v are
 * token-major head-packed rows with the given strides (query head h at column h*head_dim, KV
 * head j at column j*head_dim). Without RoPE, key_rel = r_k and k_pre is unused. key_rel and
 * value_rel may be NULL; bias_k / bias_v are NULL under the pre-bias rule or without a bias.
 * Replaces the two transposed k/v-share GEMMs and their split-K reductions. */
typedef struct pxk_attn_rel_kv_desc {
    int64_t n, l, heads, kv_heads, head_dim;
    float eps;
    int32_t causal, rope, rope_half;
    const float* s;
    const float* p;
    const float* q;
    int64_t ld_q;
    const float* spv;
    int64_t ld_spv;
    const float* k;
    int64_t ld_k;
    const float* k_pre;
    int64_t ld_k_pre;
    const float* v;
    int64_t ld_v;
    const float* z_k;
    const float* z_v;
    int64_t ld_z;
    const float* bias_k;
    const float* bias_v;
    const float* cos_t; /* (l x head_dim/2), position = row within the sequence */
    const float* sin_t;
    float* key_rel;
    float* value_rel;
    int64_t ld_rel;
    float* g_k;
    float* g_v;
    int64_t ld_g;
    int32_t relevance_only; /* 1: g_k = key_rel and g_v = value_rel themselves (z_k, z_v may be NULL) */
} pxk_attn_rel_kv_desc;
int pxk_attention_relevance_kv(const pxk_attn_rel_kv_desc* d, void* stream);

/* Causal/plain softmax of scaled scores (the module's axpby + attention_mask_fill(lowest) +
 * softmax_rows, multihead_attention_module.cpp:280-285): P = softmax(scale * raw) over the keys
 * each query sees; masked entries of P are written 0. raw (slices, L, L); only its visible
 * entries are read. */
int pxk_attention_softmax(const float* raw, float* p, int64_t slices, int64_t l, float scale, int causal,
                          int64_t window, void* stream);
/* The AttnLRP score step, fused: r_sc = x * (r_attn - P * sum(r_attn)) with x = scale * raw
 * (SoftmaxModule rule, lrp_math.hpp:89-98), masked entries 0 (fill_masked(0), :441), then the
 * Q K^T bilinear denominator s = r_sc / (2 raw + eps sign raw) (lrp_math.hpp:57-61). Writes s
 * over whole rows (0 where masked). s may alias r_attn. */
int pxk_attention_lrp_scores(const float* r_attn, const float* p, const float* raw, float* s, int64_t slices,
                             int64_t l, float scale, float eps, int causal, int64_t window, void* stream);
/* QK-Norm (multihead_attention_module.cpp step 3): RMSNorm (row_math.hpp:59-71) over each head's
 * head_dim values of head-packed rows, in (rows x heads*head_dim, row stride ld_in) -> out (row
 * stride ld_out); gamma (head_dim) is the effective scale (weight offset already added). */
int pxk_rms_norm_heads(const float* in, int64_t ld_in, float* out, int64_t ld_out, const float* gamma, int64_t rows,
                       int64_t heads, int64_t head_dim, float eps, void* stream);
/* The query share's RoPE epsilon rule (lrp_math.hpp:104-123) on token-major head-packed rows, for
 * head_dims the ROPE_REL epilogue cannot take: r = y * acc (acc = s K, y the rotated queries),
 * r_in from x (the queries before rotation) per pair, then g = r_in / stab(z + bias), or g = r_in
 * when rel_only. Positions are row % seq_len. */
int pxk_lrp_rope_rows(const float* acc, int64_t ld_acc, const float* x, int64_t ldx, const float* y, int64_t ldy,
                      const float* z, int64_t ldz, const float* bias, const float* cos_t, const float* sin_t, float* g,
                      int64_t ldg, int64_t rows, int64_t seq_len, int64_t heads, int64_t head_dim, float eps,
                      int rotate_half, int rel_only, void* stream);
/* RoPE of the packed projections (rope_module.cpp:104-121 + permute-free layout): q_out (rows x H*D)
 * and k_out (rows x Hkv*D), both with row stride ld_out, from the q/k columns of `in` (row stride
 * ld_in), positions = row % seq_len. The attention forward's rotation where head_dim does not tile
 * the projection GEMM's epilogue. */
int pxk_rope_qk(const float* q_in, const float* k_in, int64_t ld_in, float* q_out, float* k_out, int64_t ld_out,
                const float* cos_t, const float* sin_t, int64_t rows, int64_t seq_len, int64_t heads, int64_t kv_heads,
                int64_t head_dim, int rotate_half, void* stream);
/* DeviceBackend::rope_rotate (:568) and lrp_rope (:652) over (slices, seq_len, head_dim). */
int pxk_rope_rotate(const float* in, const float* cos_t, const float* sin_t, float* out, int64_t slices,
                    int64_t seq_len, int64_t head_dim, int inverse, int rotate_half, void* stream);
int pxk_lrp_rope(const float* x, const float* y, const float* r, const float* cos_t, const float* sin_t, float* r_in,
                 int64_t slices, int64_t seq_len, int64_t head_dim, float eps, int rotate_half, void* stream);
/* DeviceBackend::permute_0213 (:576) */
int pxk_permute_0213(const float* in, float* out, int64_t d0, int64_t d1, int64_t d2, int64_t d3, void* stream);
/* DeviceBackend::attention_mask_fill (:592) */
int pxk_attention_mask_fill(float* scores, const float* key_keep, int64_t batch, int64_t heads, int64_t q_len,
                            int64_t k_len, int causal, int64_t q_offset, int64_t window, float value, void* stream);

/* ---- Zennit-compatible affine rules ------------------------------------------------------------
 * Gamma, AlphaBeta and ZBox for a dense layer y = x W + b with W (in x out), as lrp_rules::apply
 * defines them (lrp_rules.cpp:72-160; stab(z) = z + eps sign z, x+ = max(x, 0), x- = x - x+):
 *   Gamma:     Wa = W + g W+, Wb = W + g W-, ba = b + g b+, bb = b + g b-, z = x W + b;
 *              gp = [z > 0] R / stab(x+ Wa + x- Wb + ba), gn = [z < 0] R / stab(x+ Wb + x- Wa + bb);
 *              R_in = x+ (gp Wa^T + gn Wb^T) + x- (gp Wb^T + gn Wa^T)
 *   AlphaBeta: as Gamma with Wa = W+, Wb = W-, ba = b+, bb = b-, no gate, gp scaled by alpha and gn
 *              by -beta (R_in = alpha * positive - beta * negative)
 *   ZBox:      den = x W - low 1 W+ - high 1 W-; g = R / stab(den);
 *              R_in = x (g W^T) - g (low W+ + high W-)^T
 * Each becomes two MFMA GEMMs over weights stacked once per layer (pxk_lrp_rule_weights):
 *   Gamma / AlphaBeta: W2 (2in x 2out) = [[Wa, Wb], [Wb, Wa]], b2 = [ba | bb];
 *                      den = [x+ | x-] W2 (pxk_lrp_sign_split, then pxk_gemm), g from den
 *                      (pxk_lrp_rule_divide), C = g W2^T (2in wide), R_in from C (pxk_lrp_rule_combine)
 *   ZBox:              W2 (2in x out) = [W ; low W+ + high W-], b2 = [low 1 W+ | high 1 W-] (column
 *                      sums in the reference's order); den from the cached x W and b2, C = g W2^T
 * Every rule is independent per output column, so one call covers column-packed layers (q | k | v,
 * gate | up) and gives the sum of their input relevances. Replaces lrp_rules::apply's composition
 * of relu / axpby / gemm / add_row_vector / lrp_stabilized_divide / mul calls for LinearModule
 * (lrp_rules.cpp:197-215) and TiedLMHeadModule (tied_lm_head_module.cpp:76-111). */
enum { PXK_RULE_GAMMA = 1, PXK_RULE_ALPHA_BETA = 2, PXK_RULE_ZBOX = 3 }; /* LRPRule order */

typedef struct pxk_rule_params {
    int32_t rule;
    float eps, gamma, alpha, beta, low, high;
} pxk_rule_params;

/* One column block of a layer's W (in x cols): W[i][j] = w[i * ld + j], or w[j * ld + i] when
 * trans (the tied head reads the embedding table, vocab x hidden, in place). bias (cols) may be
 * NULL (a zero bias). */
typedef struct pxk_rule_block {
    const float* w;
    int64_t ld;
    int64_t cols;
    int32_t trans;
    const float* bias;
} pxk_rule_block;

/* W2 and b2 for the layer whose columns are the blocks in order (out = the sum of their cols):
 * W2 holds 2in x 2out floats (Gamma, AlphaBeta) or 2in x out (ZBox), b2 2 * out. */
int pxk_lrp_rule_weights(const pxk_rule_params* p, const pxk_rule_block* blocks, int nblocks, int64_t in,
                         float* w2, float* b2, void* stream);
/* out (rows x 2in, row stride 2in) = [x+ | x-] of x (rows x in, row stride ldx). */
int pxk_lrp_sign_split(const float* x, int64_t ldx, int64_t rows, int64_t in, float* out, void* stream);
/* The rule's gated quotients over rows x out outputs. r[m][j % r_cols] (row stride ldr) is the
 * output relevance, so r_cols < out repeats one relevance over several column blocks (the gate and
 * up projections of a SwiGLU both receive the product's share). Gamma / AlphaBeta: den (rows x 2out,
 * stride ld_den) from the den GEMM, g (rows x 2out, may alias den); z (pre-bias x W, stride ldz) and
 * bias (nullable) give Gamma's gate. ZBox: den is not read, g is rows x out from z and b2. */
int pxk_lrp_rule_divide(const pxk_rule_params* p, const float* r, int64_t ldr, int64_t r_cols, const float* den,
                        int64_t ld_den, const float* z, int64_t ldz, const float* bias, const float* b2, int64_t rows,
                        int64_t out, float* g, int64_t ldg, void* stream);
/* R_in from C (rows x 2in, stride ldc) and x: Gamma / AlphaBeta x+ C[:, :in] + x- C[:, in:],
 * ZBox x C[:, :in] - C[:, in:]; then + add (nullable). Without a split, r_in receives it. With
 * split_sum given, it is the relevance of the residual sum s = a + b (lrp_residual_split,
 * lrp_math.hpp:33-38): r_in = (a / stab(s)) R, r_b = (b / stab(s)) R. Every operand has row
 * stride ld. */
int pxk_lrp_rule_combine(int rule, const float* x, int64_t ldx, const float* c, int64_t ldc, const float* add,
                         int64_t rows, int64_t in, float* r_in, int64_t ld, const float* split_a,
                         const float* split_b, const float* split_sum, float* r_b, float eps, void* stream);

/* A sandwich block's sublayer output a, its post-norm and the residual add, then the norm that reads
 * the sum (Gemma 3; TransformerBlock::forward_cached, transformer_block.cpp:143-151: PostNorm, add,
 * then norm2 or the next block's norm1): y = x + gamma_a * a / rms(a), rms(a) = sqrt(mean(a^2) +
 * eps_a), and, when y_norm is given, y_norm = gamma_y * y / rms(y). Row-major rows x cols; replaces
 * rms_norm_forward + add + rms_norm_forward in one pass. */
int pxk_rms_norm_add(const float* x, const float* a, const float* gamma_a, float eps_a, float* y,
                     const float* gamma_y, float eps_y, float* y_norm, int64_t rows, int64_t cols, void* stream);

/* ---- KV-cached decode ----------------------------------------------------------------------------
 * The position-dependent steps of a batched greedy decode step. The position is an int32 in device
 * memory shared by the batch, so a step launches with the same arguments at every position (a HIP
 * graph of one step is replayed per token) and pxk_decode_advance() moves it after the step.
 * Replaces MakeCachedNextTokenLogits's per-step work (generation.cpp:189-258): KVCache::append
 * (kv_cache.cpp:18-39), MultiHeadAttentionModule::forward_cached (multihead_attention_module.cpp:
 * 501-587) and the host round trip of the last hidden row; batch 1 there, any batch here.
 * Cache layout: sequence b at cache + b * seq_stride, position p at + p * kv_heads * head_dim. */
/* q (rotated, at *pos) -> q_out (n x heads*head_dim); k (rotated) and v -> the caches at *pos, for
 * *pos < positions (the caches' length, also the RoPE tables' (positions x head_dim/2)). With q_gamma
 * and k_gamma (QK-Norm, Qwen3 / Gemma 3: both or neither), each q and k head is first normalised as
 * pxk_rms_norm_heads does (eps norm_eps), in the same launch. */
int pxk_decode_rope_append(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v, int64_t ldv,
                           float* q_out, float* k_cache, float* v_cache, int64_t seq_stride, int64_t positions,
                           const float* cos_t, const float* sin_t, const int32_t* pos, int64_t n, int64_t heads,
                           int64_t kv_heads, int64_t head_dim, int rope, int rotate_half, const float* q_gamma,
                           const float* k_gamma, float norm_eps, void* stream);
/* ctx (n x heads*head_dim) = softmax(scale q K^T) V over the cached keys 0..*pos (the last `window`
 * of them when window > 0); max_keys bounds *pos + 1. Two launches: every (sequence, query head,
 * 64-key chunk) scores its keys and keeps a max / exp-sum / exp-weighted context partial in the
 * workspace (pxk_decode_attention_workspace() bytes), then one workgroup per (sequence, head)
 * merges the partials. */
size_t pxk_decode_attention_workspace(int64_t n, int64_t heads, int64_t head_dim, int64_t max_keys);
/* The keys [j0, j1) that 64-key chunk `chunk` of pxk_decode_attention reads for a query at cache
 * position pos (clamped to [0, max_keys)) under a sliding window (0: none); j1 <= j0 when the chunk
 * holds none. The kernel's own definition, on the host: introspection for tests, no reference
 * counterpart. */
int pxk_decode_chunk_keys(int64_t pos, int64_t max_keys, int64_t window, int64_t chunk, int64_t* j0, int64_t* j1);
int pxk_decode_attention(const float* q, const float* k_cache, const float* v_cache, int64_t seq_stride, float* ctx,
                         const int32_t* pos, int64_t n, int64_t heads, int64_t kv_heads, int64_t head_dim,
                         int64_t window, int64_t max_keys, float scale, float* workspace, size_t workspace_bytes,
                         void* stream);
/* Greedy pick (the first maximum of each sequence's logits row, rows ld_logits apart): ids[b * ld_ids +
 * *pos + 1] and cur[b] get the id, picked_logit[b * ld_logit + *pos + 1] (nullable) its logit. Two
 * launches: 64 slices of each row reduced to their first maxima in a 16-byte aligned workspace of
 * pxk_decode_pick_workspace() bytes, then merged in index order. */
size_t pxk_decode_pick_workspace(int64_t n);
int pxk_decode_pick(const float* logits, int64_t ld_logits, int64_t n, int64_t vocab, float* ids, int64_t ld_ids,
                    float* cur, float* picked_logit, int64_t ld_logit, const int32_t* pos, void* workspace,
                    size_t workspace_bytes, void* stream);
/* *pos += 1 (one thread). */
int pxk_decode_advance(int32_t* pos, void* stream);
/* The LRP seed of one row per sequence (n x vocab, every other entry 0; the explained rows' logits
 * are rows ld_logits apart): one-hot at the id targets[b * stride] (a float, rounded; an id outside
 * the vocabulary seeds id 0) with that logit as its value (LRPSeed::OutputValue) or 1 (unit,
 * OneHot); targets_out (n int64, nullable) receives the ids. The device-resident-targets form of
 * pxk_lm_seed, for explaining tokens a decode generated. */
int pxk_seed_rows(const float* logits, int64_t ld_logits, const float* targets, int64_t stride, int64_t n,
                  int64_t vocab, float* seed, int64_t* targets_out, int unit, void* stream);

/* ---- checkpoint loading ----------------------------------------------------------------------
 * A checkpoint tensor's raw little-endian bytes (already copied to the device) widened to fp32 as
 * SafetensorsFile::tensor does on the host (src/safetensors.cpp:676-740): BF16 and F16 and both
 * F8 kinds exactly (subnormals, infinities, NaN), F64 rounded to nearest. With `transpose`, the
 * (rows x cols) source lands as (cols x rows): the (out, in) -> (in, out) Linear weight transform
 * of the Hugging Face mapping (src/causal_lm.cpp:257-291, WeightTransform::Transpose). */
enum {
    PXK_DTYPE_F32 = 0,
    PXK_DTYPE_F16 = 1,
    PXK_DTYPE_BF16 = 2,
    PXK_DTYPE_F64 = 3,
    PXK_DTYPE_F8_E4M3 = 4,
    PXK_DTYPE_F8_E5M2 = 5
};
int pxk_convert_weight(const void* src, int dtype, int64_t rows, int64_t cols, int transpose, float* dst,
                       void* stream);

/* Device-side token id validation for EmbeddingModule::forward (embedding_module.cpp:48-59, which
 * reads the ids back to the host): ids_out[i] = llround(ids[i]) (halves away from zero) when that
 * lies in [0, vocab); otherwise ids_out[i] = 0, so the gather that follows stays inside the table,
 * and the id is reported. *status (device memory) is set to 0 when every id is valid, else to 1;
 * it is written on every call (one workgroup, no atomics), so it needs no clearing. */
int pxk_embedding_ids(const float* ids, int64_t count, int64_t vocab, float* ids_out, int32_t* status, void* stream);

/* ---- seeding ------------------------------------------------------------------------------------
 * On-device LRP seed for a causal LM (src/attnlrp_parity.cpp:104-109 moved to the device): for
 * each sequence n, target[n] = argmax of logits[n, L-1, :] (lowest index on ties) unless targets
 * are given (targets_in != NULL), and seed = one-hot(target) * logit (OutputValue) or one-hot
 * (unit). seed (N, L, V) is fully written; targets_out (N) as int64. */
int pxk_lm_seed(const float* logits, int64_t n, int64_t l, int64_t vocab, const int64_t* targets_in,
                int64_t* targets_out, float* seed, int unit, void* stream);

/* The tied LM head's epsilon-rule relevance (bias in the denominator or not: the tied head's bias
 * is zero) for the seed pxk_lm_seed forms, without forming it: targets as pxk_lm_seed; for the
 * last row of each sequence r = x * (R / stab(z_t) * E[t, :]) with R the target's logit z_t
 * (OutputValue) or 1 (unit); every other row is exactly zero. That is the dense result of
 * TiedLMHeadModule::propagate_relevance (tied_lm_head_module.cpp:76-111) under
 * lrp_rules::epsilon_with_bias (lrp_rules.cpp:177-194) for such a seed: the dense product only adds
 * zeros to the target's term. With a split (r_a != NULL) the relevance of the residual sum
 * s = a + b is split as lrp_residual_split does (lrp_math.hpp:33-38) into r_a and r_b instead of
 * being written to r. */
typedef struct pxk_seed_head_desc {
    const float* logits;     /* (n * l, vocab) */
    const float* x;          /* (n * l, d): the head's input */
    const float* e;          /* (vocab, d): the tied embedding */
    int64_t n, l, vocab, d;
    float eps;
    int32_t unit;
    const int64_t* targets_in; /* host, n ids, or NULL: the first maximum of each last row */
    int64_t* targets_out;    /* device, n */
    float* r;                /* (n * l, d) when there is no split */
    const float* a;          /* split: (n * l, d) each */
    const float* b;
    const float* s;
    float* r_a;
    float* r_b;
    const float* b_den;      /* split, nullable: r_b is divided by stab(b_den + b_den_bias[j]), the */
    const float* b_den_bias; /* denominator of the relevance GEMM that reads it (as PXK_EPI_MUL_X_SPLIT's c2_den) */
} pxk_seed_head_desc;
int pxk_lm_seed_head_relevance(const pxk_seed_head_desc* d, void* stream);

/* ---- training and the non-LLM modules' row and element ops (training.hip) ---------------------
 * Simple kernels for the DeviceBackend virtuals outside the forward + AttnLRP path: one thread per
 * element, or one wave64 per row with fixed-order wave reductions. Each is the reference's
 * per-element expression; row sums differ from its sequential loops only by rounding. */
/* elementwise_backward (device_backend.hpp:428; cpu_backend.cpp:226-270); op as ElementwiseOp. */
int pxk_elementwise_backward(int op, const float* x, const float* grad_out, float* grad_in, int64_t n, void* stream);
/* softmax_rows_backward (device_backend.hpp:462; cpu_backend.cpp:312-323): dx = y (dy - sum y dy). */
int pxk_softmax_rows_backward(const float* y, const float* dy, float* dx, int64_t rows, int64_t cols, void* stream);
/* rms_norm_backward (device_backend.hpp:557; row_math.hpp:75-86). */
int pxk_rms_norm_backward(const float* grad_out, const float* gamma, const float* in, const float* row_rms,
                          float* grad_in, float* gamma_terms, int64_t rows, int64_t cols, void* stream);
/* layer_norm_forward / layer_norm_backward (device_backend.hpp; row_math.hpp:15-56). */
int pxk_layer_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                           float* row_std, int64_t rows, int64_t cols, float eps, void* stream);
int pxk_layer_norm_backward(const float* grad_out, const float* gamma, const float* xhat, const float* row_std,
                            float* grad_in, int64_t rows, int64_t cols, void* stream);
/* logsumexp_rows (cpu_backend.cpp:325-338). */
int pxk_logsumexp_rows(const float* in, float* out, int64_t rows, int64_t cols, void* stream);
/* scatter_add_rows (cpu_backend.cpp:468-475): table[indices[i]] += src[i], i ascending per column. */
int pxk_scatter_add_rows(const float* src, const float* indices, float* table, int64_t count, int64_t dim,
                         void* stream);
/* adam_step (cpu_backend.cpp:340-351). */
int pxk_adam_step(float* param, const float* grad, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                  float eps, float bias_correction1, float bias_correction2, void* stream);
/* dropout_forward (cpu_backend.cpp:362-369): the counter-based SplitMix64 uniform of (seed, offset + i). */
int pxk_dropout_forward(const float* in, float* out, float* mask, int64_t n, float p, float scale, uint64_t seed,
                        uint64_t offset, void* stream);
/* bce_with_logits (grad 0) and bce_with_logits_grad (grad 1, times scale) (cpu_backend.cpp:371-383). */
int pxk_bce_with_logits(const float* logits, const float* target, float* out, int64_t n, int grad, float scale,
                        void* stream);
/* tanh_gaussian_forward / tanh_gaussian_backward (row_math.hpp:131-160); the row log-probability in double. */
int pxk_tanh_gaussian_forward(const float* mean, const float* log_std, const float* eps, float* action,
                              float* std_cache, float* log_prob, int64_t rows, int64_t cols, float stabilizer,
                              double half_log_two_pi, void* stream);
int pxk_tanh_gaussian_backward(const float* action, const float* std_cache, const float* eps, const float* grad_action,
                               const float* grad_log_prob, float* grad_mean, float* grad_log_std, int64_t n,
                               float stabilizer, void* stream);
/* top_k_rows (top_k_math.hpp:20-48): NaN ranks highest, ties keep the lower column; indices as floats. */
int pxk_top_k_rows(const float* in, float* values, float* indices, int64_t rows, int64_t cols, int64_t k, int largest,
                   void* stream);

/* ---- the non-LLM modules' ops (module_ops.hip): simple, correct kernels, one thread per output,
 * lane or row, adding in the reference's loop order; no atomics. Op codes are the reference enums'
 * declaration order. -------------------------------------------------------------------------- */

/* logic_pointwise (device_backend.hpp:663, lrp_math.hpp:125-270): op 0-2 Conjunction forward /
 * backward / LRP, 3-5 Disjunction; norm 0 product, 1 Lukasiewicz, 2 Godel. g_or_r is read by the
 * backward and LRP passes, y by LRP only; out_b is written by the backward and LRP passes. */
int pxk_logic_pointwise(int op, int norm, const float* a, const float* b, const float* g_or_r, const float* y,
                        float* out_a, float* out_b, int64_t n, float eps, void* stream);
/* aggregator_forward / _backward / _lrp (device_backend.hpp:667-676, lrp_math.hpp:272-306): the power
 * mean over the leading axis of (n, cols), one thread per column. */
int pxk_aggregator_forward(const float* x, float* mean_pow, float* out, int64_t n, int64_t cols, float p,
                           void* stream);
int pxk_aggregator_backward(const float* x, const float* mean_pow, const float* grad_out, float* grad_in, int64_t n,
                            int64_t cols, float p, void* stream);
int pxk_aggregator_lrp(const float* x, const float* mean_pow, const float* r_out, float* r_in, int64_t n, int64_t cols,
                       float p, float eps, void* stream);

/* ConvGeometry (device_backend.hpp:173-180). */
typedef struct pxk_conv_geometry {
    int64_t kh, kw, stride_h, stride_w, pad_h, pad_w;
} pxk_conv_geometry;
/* im2col (device_backend.hpp:683): (n, c, h, w) -> (n, c kh kw, out_h out_w) patches, padding reads 0. */
int pxk_im2col(const float* in, float* col, int64_t n, int64_t c, int64_t h, int64_t w, const pxk_conv_geometry* g,
               void* stream);
/* col2im_add (device_backend.hpp:691): patches added back into out (n, c, h, w), one thread per pixel
 * gathering its taps in the CPU scatter's order. */
int pxk_col2im_add(const float* col, float* out, int64_t n, int64_t c, int64_t h, int64_t w,
                   const pxk_conv_geometry* g, void* stream);
/* add_channel_vector (device_backend.hpp:695): out[i][ch][k] = in[i][ch][k] + vec[ch]; out may alias in. */
int pxk_add_channel_vector(const float* in, const float* vec, float* out, int64_t n, int64_t c, int64_t inner,
                           void* stream);
/* lrp_conv (device_backend.hpp:702, cnn_math.hpp:84-93): the Conv2D epsilon rule in patch space. */
int pxk_lrp_conv(const float* col, const float* kernel, const float* pre_bias, const float* r, float* r_col, int64_t n,
                 int64_t out_channels, int64_t p, int64_t q, float eps, void* stream);
/* max_pool_forward / max_unpool (device_backend.hpp:720-729, cnn_math.hpp:106-160). */
int pxk_max_pool_forward(const float* in, float* out, float* argmax, int64_t planes, int64_t h, int64_t w, int64_t kh,
                         int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, void* stream);
int pxk_max_unpool(const float* src, const float* argmax, float* dst, int64_t planes, int64_t h, int64_t w, int64_t kh,
                   int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, void* stream);
/* avg_pool_forward / avg_pool_backward / lrp_avg_pool (device_backend.hpp:731-741, cnn_math.hpp:162-184):
 * non-overlapping windows; grad_in and r_in cover the windows only (the caller zeroes the rest). */
int pxk_avg_pool_forward(const float* in, float* out, int64_t planes, int64_t h, int64_t w, int64_t kh, int64_t kw,
                         void* stream);
int pxk_avg_pool_backward(const float* grad_out, float* grad_in, int64_t planes, int64_t h, int64_t w, int64_t kh,
                          int64_t kw, void* stream);
int pxk_lrp_avg_pool(const float* x, const float* r, float* r_in, int64_t planes, int64_t h, int64_t w, int64_t kh,
                     int64_t kw, float eps, void* stream);
/* batch_norm_forward / _backward / _update_running / _eval_forward / _eval_backward
 * (device_backend.hpp:743-766, cnn_math.hpp:186-330): one thread per channel of (n, c, spatial). */
int pxk_batch_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                           float* channel_std, int64_t n, int64_t c, int64_t spatial, float eps, void* stream);
int pxk_batch_norm_backward(const float* grad_out, const float* gamma, const float* xhat, const float* channel_std,
                            float* grad_in, float* gamma_grad, float* beta_grad, int64_t n, int64_t c, int64_t spatial,
                            void* stream);
int pxk_batch_norm_update_running(const float* in, float* running_mean, float* running_var, int64_t n, int64_t c,
                                  int64_t spatial, float momentum, void* stream);
int pxk_batch_norm_eval_forward(const float* in, const float* gamma, const float* beta, const float* running_mean,
                                const float* running_var, float* xhat, float* out, float* channel_std, int64_t n,
                                int64_t c, int64_t spatial, float eps, void* stream);
int pxk_batch_norm_eval_backward(const float* grad_out, const float* gamma, const float* xhat,
                                 const float* channel_std, float* grad_in, float* gamma_grad, float* beta_grad,
                                 int64_t n, int64_t c, int64_t spatial, void* stream);
/* group_norm_forward / _backward (device_backend.hpp:768-776, cnn_math.hpp:332-413): one thread per
 * (example, group); the parameter gradients one thread per channel. */
int pxk_group_norm_forward(const float* in, const float* gamma, const float* beta, float* xhat, float* out,
                           float* group_std, int64_t n, int64_t c, int64_t spatial, int64_t groups, float eps,
                           void* stream);
int pxk_group_norm_backward(const float* grad_out, const float* gamma, const float* xhat, const float* group_std,
                            float* grad_in, float* gamma_grad, float* beta_grad, int64_t n, int64_t c, int64_t spatial,
                            int64_t groups, void* stream);

/* RecurrentCellArgs (device_backend.hpp:91-95); recurrent_cell (:795, recurrent_math.hpp:18-106), op 0
 * RnnBackward, 1 LstmForward, 2 LstmBackward, 3 LstmLrp, 4 GruBackward, 5 GruLrp, slots as
 * device_backend.hpp:75-87 documents; n elements. */
typedef struct pxk_recurrent_args {
    const float* in[10];
    float* out[6];
    float eps;
} pxk_recurrent_args;
int pxk_recurrent_cell(int op, const pxk_recurrent_args* args, int64_t n, void* stream);
/* gru_lrp_hprev (device_backend.hpp:801, recurrent_math.hpp:108-124). */
int pxk_gru_lrp_hprev(const float* h_prev, const float* w_hn, const float* hn, const float* r_term_b,
                      const float* direct, float* r_hprev, int64_t rows, int64_t hidden, float eps, void* stream);
/* SsmPassArgs (device_backend.hpp:158-167); ssm_pass (:813, ssm_math.hpp), op = SsmPassOp's order
 * (0 MambaForward .. 18 ReverseTimeSum), slots and lanes as device_backend.hpp:97-134 documents.
 * Carry and state buffers the reference's callers zero are zeroed by them here too. */
typedef struct pxk_ssm_args {
    const float* in[12];
    float* out[10];
    int64_t n, l, d, s;
    float eps, gamma;
} pxk_ssm_args;
int pxk_ssm_pass(int op, const pxk_ssm_args* args, void* stream);
/* RlRowArgs (device_backend.hpp:208-219); rl_rows (:824, rl_math.hpp), op = RlRowOp's order (0 DqnLoss
 * .. 8 TokenCeLoss); one thread per row (per element for PolyakBlend). */
typedef struct pxk_rl_args {
    const float* in[5];
    float* out[4];
    int64_t rows, cols;
    float scale, lower, upper, gamma, tau;
    int64_t ignore_index;
} pxk_rl_args;
int pxk_rl_rows(int op, const pxk_rl_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PXK_H */
