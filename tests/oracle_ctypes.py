"""ctypes bindings for the CPU oracle (oracle/liboracle.so) and, where it was built, the compiled
reference (oracle/_ref/libpxref.so).

Test infrastructure: the oracle is the checker for the MI355X path, never part of it.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libpxref.so")
REF_MI355X_SO = os.path.join(ROOT, "oracle", "_ref", "libpxref_mi355x.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i64p = ctypes.POINTER(ctypes.c_int64)


class ModelConfig(ctypes.Structure):
    """px_model_config (oracle/pxo.h, include/pulsatrix_amd.h)."""

    _fields_ = [
        ("vocab_size", ctypes.c_int64),
        ("hidden_size", ctypes.c_int64),
        ("num_layers", ctypes.c_int64),
        ("num_heads", ctypes.c_int64),
        ("num_kv_heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("intermediate_size", ctypes.c_int64),
        ("rms_norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("use_rope", ctypes.c_int32),
        ("rope_rotate_half", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("qkv_bias", ctypes.c_int32),
        ("out_bias", ctypes.c_int32),
        ("mlp_bias", ctypes.c_int32),
        ("tie_word_embeddings", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("hidden_act", ctypes.c_int32),
        ("qk_norm", ctypes.c_int32),
        ("post_norms", ctypes.c_int32),
        ("rope_scaling", ctypes.c_int32),
        ("norm_weight_offset", ctypes.c_float),
        ("embed_scale", ctypes.c_float),
        ("query_pre_attn_scalar", ctypes.c_float),
        ("rope_local_base", ctypes.c_float),
        ("rope_factor", ctypes.c_float),
        ("rope_low_freq_factor", ctypes.c_float),
        ("rope_high_freq_factor", ctypes.c_float),
        ("reserved2", ctypes.c_int32),
        ("rope_original_max_position", ctypes.c_int64),
        ("sliding_window", ctypes.c_int64),
        ("sliding_layers", ctypes.c_uint64),
    ]

    def kv_heads(self):
        return self.num_kv_heads if self.num_kv_heads > 0 else self.num_heads

    def hd(self):
        return self.head_dim if self.head_dim > 0 else self.hidden_size // self.num_heads


EPSILON, GAMMA, ALPHA_BETA, ZBOX = 0, 1, 2, 3  # LRPRule order (include/pulsatrix/lrp_rule_config.hpp)


class LrpRule(ctypes.Structure):
    """px_lrp_rule (oracle/pxo.h, include/pulsatrix_amd.h): LRPRuleConfig's fields."""

    _fields_ = [
        ("epsilon", ctypes.c_float),
        ("rule", ctypes.c_int32),
        ("gamma", ctypes.c_float),
        ("alpha", ctypes.c_float),
        ("beta", ctypes.c_float),
        ("low", ctypes.c_float),
        ("high", ctypes.c_float),
        ("bias_in_denominator", ctypes.c_int32),
    ]


def lrp_rule(rule=EPSILON, epsilon=1e-6, gamma=0.25, alpha=1.0, beta=0.0, low=0.0, high=1.0,
             bias_in_denominator=False):
    return LrpRule(epsilon, rule, gamma, alpha, beta, low, high, int(bias_in_denominator))


def model_config(**kw):
    base = dict(vocab_size=0, hidden_size=0, num_layers=1, num_heads=1, num_kv_heads=0, head_dim=0,
                intermediate_size=0, rms_norm_eps=1e-5, rope_theta=10000.0, use_rope=1, rope_rotate_half=1,
                causal=1, qkv_bias=0, out_bias=0, mlp_bias=0, tie_word_embeddings=1, reserved=0)
    base.update(kw)
    return ModelConfig(**base)


def fptr(a):
    return a.ctypes.data_as(_f32p) if a is not None else None


def block_layout(cfg):
    """(name, shape) of one block's parameters in the flat blob order."""
    d, q, kv, f = cfg.hidden_size, cfg.num_heads * cfg.hd(), cfg.kv_heads() * cfg.hd(), cfg.intermediate_size
    out = [("norm1.weight", (d,))]

    def lin(name, i, o, bias):
        out.append((name + ".weight", (i, o)))
        if bias:
            out.append((name + ".bias", (o,)))

    lin("mha.q_proj", d, q, cfg.qkv_bias)
    lin("mha.k_proj", d, kv, cfg.qkv_bias)
    lin("mha.v_proj", d, kv, cfg.qkv_bias)
    lin("mha.out_proj", q, d, cfg.out_bias)
    if cfg.qk_norm:
        out += [("mha.q_norm.weight", (cfg.hd(),)), ("mha.k_norm.weight", (cfg.hd(),))]
    out.append(("norm2.weight", (d,)))
    lin("swiglu.gate_proj", d, f, cfg.mlp_bias)
    lin("swiglu.up_proj", d, f, cfg.mlp_bias)
    lin("swiglu.down_proj", f, d, cfg.mlp_bias)
    if cfg.post_norms:
        out += [("post_attn_norm.weight", (d,)), ("post_mlp_norm.weight", (d,))]
    return out


def lm_layout(cfg):
    out = [("embed_tokens.weight", (cfg.vocab_size, cfg.hidden_size))]
    for i in range(cfg.num_layers):
        out += [("layers.%d.%s" % (i, n), s) for n, s in block_layout(cfg)]
    out.append(("norm.weight", (cfg.hidden_size,)))
    if not cfg.tie_word_embeddings:
        out.append(("lm_head.weight", (cfg.hidden_size, cfg.vocab_size)))
    return out


def pack(layout, tensors):
    parts = [np.ascontiguousarray(tensors[name], dtype=np.float32).reshape(shape) for name, shape in layout]
    return np.concatenate([p.ravel() for p in parts]).astype(np.float32)


class _Lib:
    def __init__(self, path, prefix):
        self.lib = ctypes.CDLL(path)
        self.p = prefix
        L = self.lib
        cfgp = ctypes.POINTER(ModelConfig)
        for name, res, args in [
            ("block_create", ctypes.c_void_p, [cfgp, _f32p]),
            ("block_forward", ctypes.c_int, [ctypes.c_void_p, _f32p, ctypes.c_int64, ctypes.c_int64, _f32p]),
            ("block_relevance", ctypes.c_int, [ctypes.c_void_p, _f32p, ctypes.c_float, ctypes.c_int, _f32p]),
            ("block_destroy", None, [ctypes.c_void_p]),
            ("lm_create", ctypes.c_void_p, [cfgp, _f32p]),
            ("lm_forward", ctypes.c_int, [ctypes.c_void_p, _i64p, ctypes.c_int64, ctypes.c_int64, _f32p]),
            ("lm_relevance", ctypes.c_int, [ctypes.c_void_p, _f32p, ctypes.c_float, ctypes.c_int, _f32p, _f32p, _f32p,
                                            _f32p]),
            ("lm_destroy", None, [ctypes.c_void_p]),
            ("block_relevance_rule", ctypes.c_int, [ctypes.c_void_p, _f32p, ctypes.POINTER(LrpRule), _f32p]),
            ("lm_relevance_rule", ctypes.c_int, [ctypes.c_void_p, _f32p, ctypes.POINTER(LrpRule), _f32p, _f32p,
                                                 _f32p, _f32p]),
            ("last_error", ctypes.c_char_p, []),
        ]:
            fn = getattr(L, prefix + name)
            fn.restype = res
            fn.argtypes = args

    def fn(self, name):
        return getattr(self.lib, self.p + name)

    def check(self, rc):
        if rc != 0:
            raise RuntimeError(self.fn("last_error")().decode())

    # ---- block ----
    def block(self, cfg, params):
        return _Block(self, cfg, params)

    def lm(self, cfg, params):
        return _LM(self, cfg, params)


class _Block:
    def __init__(self, lib, cfg, params):
        self.lib, self.cfg = lib, cfg
        self.params = np.ascontiguousarray(params, dtype=np.float32)
        self.h = lib.fn("block_create")(ctypes.byref(cfg), fptr(self.params))
        if not self.h:
            raise RuntimeError(lib.fn("last_error")().decode())

    def forward(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        n, l, _ = x.shape
        y = np.empty_like(x)
        self.lib.check(self.lib.fn("block_forward")(self.h, fptr(x), n, l, fptr(y)))
        return y

    def relevance(self, r, eps, bias_in_denominator):
        r = np.ascontiguousarray(r, dtype=np.float32)
        out = np.empty_like(r)
        self.lib.check(self.lib.fn("block_relevance")(self.h, fptr(r), eps, int(bias_in_denominator), fptr(out)))
        return out

    def relevance_rule(self, r, rule):
        r = np.ascontiguousarray(r, dtype=np.float32)
        out = np.empty_like(r)
        self.lib.check(self.lib.fn("block_relevance_rule")(self.h, fptr(r), ctypes.byref(rule), fptr(out)))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.fn("block_destroy")(self.h)
            self.h = None


class _LM:
    def __init__(self, lib, cfg, params):
        self.lib, self.cfg = lib, cfg
        self.params = np.ascontiguousarray(params, dtype=np.float32)
        self.h = lib.fn("lm_create")(ctypes.byref(cfg), fptr(self.params))
        if not self.h:
            raise RuntimeError(lib.fn("last_error")().decode())
        self.shape = None

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        n, l = ids.shape
        logits = np.empty((n, l, self.cfg.vocab_size), dtype=np.float32)
        self.lib.check(self.lib.fn("lm_forward")(self.h, ids.ctypes.data_as(_i64p), n, l, fptr(logits)))
        self.shape = (n, l)
        return logits

    def relevance(self, seed, eps, bias_in_denominator, want_kv=False):
        n, l = self.shape
        c = self.cfg
        seed = np.ascontiguousarray(seed, dtype=np.float32)
        r_embed = np.empty((n, l, c.hidden_size), dtype=np.float32)
        r_tok = np.empty((n, l), dtype=np.float32)
        kv = (c.num_layers, n * l, c.kv_heads() * c.hd())
        k = np.empty(kv, dtype=np.float32) if want_kv else None
        v = np.empty(kv, dtype=np.float32) if want_kv else None
        self.lib.check(self.lib.fn("lm_relevance")(self.h, fptr(seed), eps, int(bias_in_denominator), fptr(r_embed),
                                                    fptr(r_tok), fptr(k), fptr(v)))
        return (r_embed, r_tok, k, v) if want_kv else (r_embed, r_tok)

    def relevance_rule(self, seed, rule, want_kv=False):
        n, l = self.shape
        c = self.cfg
        seed = np.ascontiguousarray(seed, dtype=np.float32)
        r_embed = np.empty((n, l, c.hidden_size), dtype=np.float32)
        r_tok = np.empty((n, l), dtype=np.float32)
        kv = (c.num_layers, n * l, c.kv_heads() * c.hd())
        k = np.empty(kv, dtype=np.float32) if want_kv else None
        v = np.empty(kv, dtype=np.float32) if want_kv else None
        self.lib.check(self.lib.fn("lm_relevance_rule")(self.h, fptr(seed), ctypes.byref(rule), fptr(r_embed),
                                                         fptr(r_tok), fptr(k), fptr(v)))
        return (r_embed, r_tok, k, v) if want_kv else (r_embed, r_tok)

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.fn("lm_destroy")(self.h)
            self.h = None


_oracle = None
_ref = None


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle/liboracle.so is not built (run __graft_entry__.build())")
        _oracle = _Lib(ORACLE_SO, "pxo_")
        L = _oracle.lib
        L.pxo_fill_normal.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_double]
        L.pxo_fill_normal.restype = None
        L.pxo_param_count.argtypes = [ctypes.POINTER(ModelConfig)]
        L.pxo_param_count.restype = ctypes.c_int64
        L.pxo_block_param_count.argtypes = [ctypes.POINTER(ModelConfig)]
        L.pxo_block_param_count.restype = ctypes.c_int64
        L.pxo_set_threads.argtypes = [ctypes.c_int]
        L.pxo_get_threads.restype = ctypes.c_int
        L.pxo_set_split_threads.argtypes = [ctypes.c_int]
        # As a checker the oracle may spread lrp_linear / lrp_bilinear_matmul over threads (the same
        # numbers for any count); the CPU baseline sets 1 again, CPUBackend's schedule.
        L.pxo_set_split_threads(min(16, os.cpu_count() or 1))
        L.pxo_rope_tables.argtypes = [ctypes.c_int64, ctypes.c_float, ctypes.c_int64, ctypes.c_int64, _f32p, _f32p]
    return _oracle


def ref():
    """The compiled reference, or None where oracle/_ref was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        _ref = _Lib(REF_SO, "pxr_")
        _bind_backend_shim(_ref.lib)
        _bind_generate(_ref.lib)
    return _ref


def _bind_generate(L):
    """pxr_generate (the reference's Generate over a C next-token callback) and the reference
    CausalLM's own next_token_logits behind that callback (oracle/ref_driver.cpp)."""
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    L.pxr_generate.restype = ctypes.c_int
    L.pxr_generate.argtypes = [vp, vp, i64, _i64p, i64, i64, i64, _i64p, i64, ctypes.c_int, ctypes.c_float, i64,
                               ctypes.c_float, ctypes.c_float, ctypes.c_float, i64, _i64p, _f32p, i64, _i64p,
                               ctypes.POINTER(ctypes.c_int)]
    L.pxr_lm_next_token_logits_create.restype = vp
    L.pxr_lm_next_token_logits_create.argtypes = [vp, i64]
    L.pxr_lm_next_token_logits.restype = ctypes.c_int
    L.pxr_lm_next_token_logits.argtypes = [vp, _i64p, i64, _f32p, i64]
    L.pxr_lm_next_token_logits_destroy.restype = None
    L.pxr_lm_next_token_logits_destroy.argtypes = [vp]


def ref_generate(model, vocab, prompt, max_new_tokens, min_new_tokens=0, eos=(), do_sample=False, temperature=1.0,
                 top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0, seed=-1):
    """The reference's Generate (generation.hpp:95-135) over `model`, a next-token function object
    whose `callback` is its (C function pointer, context); the object stays referenced for the call.
    Returns (new tokens, their log-probabilities, finish reason 'eos' or 'length')."""
    lib = ref()
    fn, ctx = model.callback
    p = np.ascontiguousarray(prompt, dtype=np.int64)
    e = np.ascontiguousarray(list(eos) or [0], dtype=np.int64)
    cap = max(1, int(max_new_tokens))
    toks = np.zeros(cap, np.int64)
    logp = np.zeros(cap, np.float32)
    n_new, fin = ctypes.c_int64(), ctypes.c_int()
    lib.check(lib.lib.pxr_generate(fn, ctx, vocab, p.ctypes.data_as(_i64p), p.size, max_new_tokens, min_new_tokens,
                                   e.ctypes.data_as(_i64p), len(eos), int(do_sample), temperature, top_k, top_p, min_p,
                                   repetition_penalty, seed, toks.ctypes.data_as(_i64p), fptr(logp), cap,
                                   ctypes.byref(n_new), ctypes.byref(fin)))
    k = n_new.value
    return toks[:k], logp[:k], ("eos" if fin.value == 0 else "length")


class RefNextToken:
    """The compiled reference CausalLM's next_token_logits(max_length) (causal_lm.hpp:116)."""

    def __init__(self, lm, max_length):
        self.lm = lm
        L = lm.lib.lib
        self.h = L.pxr_lm_next_token_logits_create(lm.h, max_length)
        if not self.h:
            raise RuntimeError(lm.lib.fn("last_error")().decode())

    def __call__(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.int64)
        out = np.empty(self.lm.cfg.vocab_size, np.float32)
        self.lm.lib.check(self.lm.lib.lib.pxr_lm_next_token_logits(self.h, t.ctypes.data_as(_i64p), t.size, fptr(out),
                                                                   out.size))
        return out

    @property
    def callback(self):
        return ctypes.cast(self.lm.lib.lib.pxr_lm_next_token_logits, ctypes.c_void_p).value, self.h

    def __del__(self):
        if getattr(self, "h", None):
            self.lm.lib.lib.pxr_lm_next_token_logits_destroy(self.h)
            self.h = None


_ref_mi355x = None


def ref_mi355x():
    """The reference's modules on MI355XBackend (oracle/_ref/libpxref_mi355x.so: the drop-in, run),
    or None where it was not built. The same pxr_ entry points as ref(), on host arrays, plus
    pxr_be_* (each DeviceBackend virtual on device pointers) and pxr_mlp_explain."""
    global _ref_mi355x
    if _ref_mi355x is None and os.path.exists(REF_MI355X_SO):
        from pulsatrix_amd import native

        native.pxk()  # the HIP runtime torch loaded, and the kernel library, first
        lib = _Lib(REF_MI355X_SO, "pxr_")
        _bind_backend_shim(lib.lib)
        _ref_mi355x = lib
    return _ref_mi355x


def _bind_backend_shim(L):
    """Signatures of pxr_be_* (oracle/ref_driver.cpp): each DeviceBackend virtual of the library's
    backend, host pointers on the reference's CPUBackend, device pointers on MI355XBackend."""
    if True:
        vp, sz, i, f = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
        sig = {
            "copy": [vp, vp, sz, i], "fill": [vp, f, sz], "gemm": [vp, vp, vp, sz, sz, sz],
            "gemm_ex": [vp, i, vp, i, vp, sz, sz, sz, f],
            "gemm_strided_batched": [vp, i, sz, vp, i, sz, vp, sz, sz, sz, sz, sz, f],
            "elementwise": [i, vp, vp, sz], "add": [vp, vp, vp, sz], "mul": [vp, vp, vp, sz],
            "axpby": [f, vp, f, vp, vp, sz], "column_sums": [vp, vp, sz, sz, f], "add_row_vector": [vp, vp, vp, sz, sz],
            "dot_into": [vp, vp, sz, vp], "softmax_rows": [vp, vp, sz, sz],
            "rms_norm_forward": [vp, vp, vp, vp, sz, sz, f], "rope_rotate": [vp, vp, vp, vp, sz, sz, sz, i, i],
            "permute_0213": [vp, vp, sz, sz, sz, sz], "attention_mask_fill": [vp, vp, sz, sz, sz, sz, i, sz, sz, f],
            "gather_rows": [vp, vp, vp, sz, sz], "lrp_linear": [vp, vp, vp, vp, vp, sz, sz, sz, f],
            "lrp_residual_split": [vp, vp, vp, vp, vp, sz, f], "lrp_bilinear_elementwise": [vp, vp, vp, vp, sz, f],
            "lrp_bilinear_matmul": [vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, f, i],
            "lrp_softmax_rows": [vp, vp, vp, vp, sz, sz], "lrp_rope": [vp, vp, vp, vp, vp, vp, sz, sz, sz, f, i],
            "lrp_stabilized_divide": [vp, vp, vp, vp, sz, f, i], "copy_2d": [vp, sz, vp, sz, sz, sz],
            "accumulate_rows": [vp, vp, sz, sz], "synchronize": [], "sum": [vp, sz, vp], "dot": [vp, vp, sz, vp],
            "allocate": [sz, ctypes.POINTER(vp)],
            "elementwise_backward": [i, vp, vp, vp, sz], "softmax_rows_backward": [vp, vp, vp, sz, sz],
            "rms_norm_backward": [vp, vp, vp, vp, vp, vp, sz, sz],
            "layer_norm_forward": [vp, vp, vp, vp, vp, vp, sz, sz, f], "layer_norm_backward": [vp, vp, vp, vp, vp, sz, sz],
            "logsumexp_rows": [vp, vp, sz, sz], "scatter_add_rows": [vp, vp, vp, sz, sz],
            "adam_step": [vp, vp, vp, vp, sz, f, f, f, f, f, f],
            "dropout_forward": [vp, vp, vp, sz, f, f, ctypes.c_uint64, ctypes.c_uint64],
            "bce_with_logits": [vp, vp, vp, sz], "bce_with_logits_grad": [vp, vp, vp, sz, f],
            "tanh_gaussian_forward": [vp, vp, vp, vp, vp, vp, sz, sz, f, ctypes.c_double],
            "tanh_gaussian_backward": [vp, vp, vp, vp, vp, vp, vp, sz, f],
            "top_k_rows": [vp, vp, vp, sz, sz, sz, i],
            "logic_pointwise": [i, i, vp, vp, vp, vp, vp, vp, sz, f],
            "aggregator_forward": [vp, vp, vp, sz, sz, f], "aggregator_backward": [vp, vp, vp, vp, sz, sz, f],
            "aggregator_lrp": [vp, vp, vp, vp, sz, sz, f, f],
            "im2col": [vp, vp] + [sz] * 10, "col2im_add": [vp, vp] + [sz] * 10,
            "add_channel_vector": [vp, vp, vp, sz, sz, sz], "lrp_conv": [vp, vp, vp, vp, vp, sz, sz, sz, sz, f],
            "max_pool_forward": [vp, vp, vp] + [sz] * 9, "max_unpool": [vp, vp, vp] + [sz] * 9,
            "avg_pool_forward": [vp, vp, sz, sz, sz, sz, sz], "avg_pool_backward": [vp, vp, sz, sz, sz, sz, sz],
            "lrp_avg_pool": [vp, vp, vp, sz, sz, sz, sz, sz, f],
            "batch_norm_forward": [vp, vp, vp, vp, vp, vp, sz, sz, sz, f],
            "batch_norm_backward": [vp, vp, vp, vp, vp, vp, vp, sz, sz, sz],
            "batch_norm_update_running": [vp, vp, vp, sz, sz, sz, f],
            "batch_norm_eval_forward": [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, f],
            "batch_norm_eval_backward": [vp, vp, vp, vp, vp, vp, vp, sz, sz, sz],
            "group_norm_forward": [vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, f],
            "group_norm_backward": [vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz],
            "gru_lrp_hprev": [vp, vp, vp, vp, vp, vp, sz, sz, f],
            "recurrent_cell": [i, ctypes.POINTER(vp), ctypes.POINTER(vp), f, sz],
            "ssm_pass": [i, ctypes.POINTER(vp), ctypes.POINTER(vp)] + [ctypes.c_int64] * 4 + [f, f],
            "rl_rows": [i, ctypes.POINTER(vp), ctypes.POINTER(vp), ctypes.c_int64, ctypes.c_int64, f, f, f, f, f,
                        ctypes.c_int64],
        }
        for name, args in sig.items():
            fn = getattr(L, "pxr_be_" + name)
            fn.argtypes, fn.restype = args, ctypes.c_int
        L.pxr_be_free.argtypes, L.pxr_be_free.restype = [vp], None
        L.pxr_be_device.restype = ctypes.c_int
        L.pxr_linear_relevance_rule.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                                                ctypes.c_int64, ctypes.POINTER(LrpRule), _f32p]


def mlp_explain(lib, layers, x, targets, rule, preset=0):
    """LRP::explain over Linear -> ReLU -> ... -> Linear (pxr_mlp_explain) on `lib`'s backend.
    layers: [(w (in, out), b (out,) or None)]; preset 0 applies `rule` everywhere, 1-3 are the
    reference's epsilon_plus, epsilon_alpha2_beta1 and epsilon_gamma_box(-3, 3) composites.
    Returns (relevance (n, in), relevance_in_sum)."""
    fn = lib.lib.pxr_mlp_explain
    fn.argtypes = [ctypes.c_int, _i64p, _i64p, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p), _f32p,
                   ctypes.c_int64, _i64p, ctypes.POINTER(LrpRule), ctypes.c_int, _f32p, _f32p]
    fn.restype = ctypes.c_int
    ins = np.array([w.shape[0] for w, _ in layers], np.int64)
    outs = np.array([w.shape[1] for w, _ in layers], np.int64)
    keep = [np.ascontiguousarray(w, np.float32) for w, _ in layers] + \
           [None if b is None else np.ascontiguousarray(b, np.float32) for _, b in layers]
    nl = len(layers)
    wp = (ctypes.c_void_p * nl)(*[k.ctypes.data for k in keep[:nl]])
    bp = (ctypes.c_void_p * nl)(*[None if k is None else k.ctypes.data for k in keep[nl:]])
    x = np.ascontiguousarray(x, np.float32)
    t = np.ascontiguousarray(targets, np.int64)
    out = np.empty((x.shape[0], ins[0]), np.float32)
    total = ctypes.c_float(0)
    lib.check(lib.lib.pxr_mlp_explain(nl, ins.ctypes.data_as(_i64p), outs.ctypes.data_as(_i64p), wp, bp, fptr(x),
                                      x.shape[0], t.ctypes.data_as(_i64p), ctypes.byref(rule), preset, fptr(out),
                                      ctypes.byref(total)))
    return out, total.value


def fill_normal(n, seed, std):
    out = np.empty(n, dtype=np.float32)
    oracle().lib.pxo_fill_normal(fptr(out), n, seed, std)
    return out


def is_norm_weight(name):
    return name.endswith("norm.weight") or name.endswith("norm1.weight") or name.endswith("norm2.weight")


def synthetic_params(cfg, seed, std=0.02, block=False):
    """The flat blob of a random-init model: N(0, std) from seed, every RMSNorm's effective scale
    (norm_weight_offset + gamma) 1."""
    layout = block_layout(cfg) if block else lm_layout(cfg)
    total = sum(int(np.prod(s)) for _, s in layout)
    blob = fill_normal(total, seed, std)
    off = 0
    for name, shape in layout:
        size = int(np.prod(shape))
        if is_norm_weight(name):
            blob[off:off + size] = np.float32(1.0) - np.float32(cfg.norm_weight_offset)
        off += size
    return blob


def linear_forward(x, w, b):
    """Oracle LinearModule::forward: returns (pre_bias, y)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, i = x.shape
    o = w.shape[1]
    pre, y = np.empty((n, o), np.float32), np.empty((n, o), np.float32)
    bb = None if b is None else np.ascontiguousarray(b, dtype=np.float32)
    L = oracle()
    L.lib.pxo_linear_forward.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _f32p,
                                         _f32p]
    L.check(L.lib.pxo_linear_forward(fptr(x), fptr(w), fptr(bb), n, i, o, fptr(pre), fptr(y)))
    return pre, y


def linear_relevance(x, w, b, pre, r, eps, bias_in_denominator):
    x, w, pre, r = (np.ascontiguousarray(a, dtype=np.float32) for a in (x, w, pre, r))
    n, i = x.shape
    o = w.shape[1]
    out = np.empty((n, i), np.float32)
    bb = None if b is None else np.ascontiguousarray(b, dtype=np.float32)
    L = oracle()
    L.lib.pxo_linear_relevance.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_int64, ctypes.c_float, ctypes.c_int, _f32p]
    L.check(L.lib.pxo_linear_relevance(fptr(x), fptr(w), fptr(bb), fptr(pre), fptr(r), n, i, o, eps,
                                       int(bias_in_denominator), fptr(out)))
    return out


def linear_relevance_rule(x, w, b, pre, r, rule):
    """Oracle LinearModule::propagate_relevance under `rule` (an LrpRule)."""
    x, w, pre, r = (np.ascontiguousarray(a, dtype=np.float32) for a in (x, w, pre, r))
    n, i = x.shape
    o = w.shape[1]
    out = np.empty((n, i), np.float32)
    bb = None if b is None else np.ascontiguousarray(b, dtype=np.float32)
    L = oracle()
    L.lib.pxo_linear_relevance_rule.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                                                ctypes.c_int64, ctypes.POINTER(LrpRule), _f32p]
    L.check(L.lib.pxo_linear_relevance_rule(fptr(x), fptr(w), fptr(bb), fptr(pre), fptr(r), n, i, o,
                                            ctypes.byref(rule), fptr(out)))
    return out


def ref_linear_relevance_rule(x, w, b, r, rule):
    """The compiled reference's LinearModule (forward, then propagate_relevance under `rule`)."""
    R = ref()
    x, w, r = (np.ascontiguousarray(a, dtype=np.float32) for a in (x, w, r))
    n, i = x.shape
    o = w.shape[1]
    out = np.empty((n, i), np.float32)
    bb = None if b is None else np.ascontiguousarray(b, dtype=np.float32)
    R.lib.pxr_linear_relevance_rule.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int64, ctypes.c_int64,
                                                ctypes.c_int64, ctypes.POINTER(LrpRule), _f32p]
    R.check(R.lib.pxr_linear_relevance_rule(fptr(x), fptr(w), fptr(bb), fptr(r), n, i, o, ctypes.byref(rule),
                                            fptr(out)))
    return out
