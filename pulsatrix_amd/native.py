"""ctypes bindings of the MI355X libraries' C ABI (include/pxk.h, include/pulsatrix_amd.h).

This is the binding a Python caller of the library uses. It loads the in-tree libraries built by
pulsatrix_amd/build.py and raises if they are missing: there is no fallback path.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
PXK_SO = os.path.join(LIB_DIR, "libpxk_gfx950.so")
HOST_SO = os.path.join(LIB_DIR, "libpulsatrix_amd.so")

c_f32p = ctypes.POINTER(ctypes.c_float)
c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p


class PxkError(RuntimeError):
    pass


class Operand(ctypes.Structure):
    _fields_ = [("ptr", c_vp), ("ld", c_i64), ("batch_stride", c_i64), ("inner_stride", c_i64),
                ("inner_div", c_i64), ("group_stride", c_i64)]


class GemmDesc(ctypes.Structure):
    _fields_ = [("m", c_i64), ("n", c_i64), ("k", c_i64), ("batch", c_i64), ("inner", c_i64), ("kgroups", c_i64),
                ("trans_a", ctypes.c_int32), ("trans_b", ctypes.c_int32), ("causal", ctypes.c_int32),
                ("prologue", ctypes.c_int32), ("epilogue", ctypes.c_int32), ("splits", ctypes.c_int32),
                ("beta", ctypes.c_float), ("eps", ctypes.c_float),
                ("a", Operand), ("b", Operand), ("c", Operand), ("z", Operand), ("z_bias", Operand),
                ("c2", Operand), ("c3", Operand), ("x", Operand), ("y", Operand), ("w", Operand), ("z2", Operand), ("z3", Operand),
                ("e_bias", Operand), ("e_bias2", Operand),
                ("cos_t", c_vp), ("sin_t", c_vp), ("head_dim", c_i64), ("rope_half", ctypes.c_int32),
                ("tile", ctypes.c_int32), ("workspace", c_vp), ("workspace_bytes", ctypes.c_size_t),
                ("rope_cols", c_i64), ("gate_act", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("c2_den", Operand), ("c2_den_bias", Operand), ("x_rms", c_vp), ("x_gamma", c_vp), ("row_rms", c_vp),
                ("norm_eps", ctypes.c_float), ("reserved2", ctypes.c_int32)]


CAUSAL_NONE, CAUSAL_TRI, CAUSAL_K_LE_M, CAUSAL_K_GE_M = 0, 1, 2, 3
PRO_NONE, PRO_DIV_STAB, PRO_RMS = 0, 1, 2
(EPI_STORE, EPI_STORE_BIAS, EPI_ADD_RESID, EPI_MUL_X, EPI_SPV, EPI_ROPE_REL, EPI_VALUE_REL,
 EPI_SWIGLU_REL, EPI_MUL_X_SPLIT, EPI_ROPE_FWD, EPI_SWIGLU_FWD) = range(11)
TILE_AUTO, TILE_128x128, TILE_64x64, TILE_32x64, TILE_32x32, TILE_32x64_DIRECT, TILE_32x32_DIRECT, TILE_SKINNY = range(8)
TILE_32x48_DIRECT = 8
TILE_32x48 = 9

# (name, restype, argtypes) of every pxk entry point; `p` = device pointer (void*), `i` = int64,
# `f` = float, `n` = int, `s` = size_t.
_T = {"p": c_vp, "i": c_i64, "f": ctypes.c_float, "n": ctypes.c_int, "s": ctypes.c_size_t}
PXK_SIGNATURES = {
    "pxk_gemm_ex": "pnpnpiiifps" + "p",
    "pxk_fill": "pfip",
    "pxk_elementwise": "nppip",
    "pxk_add": "pppip",
    "pxk_mul": "pppip",
    "pxk_axpby": "fpfppip",
    "pxk_add_row_vector": "pppiip",
    "pxk_scale_rows": "pppiip",
    "pxk_lrp_residual_split": "pppppifp",
    "pxk_lrp_bilinear_elementwise": "ppppifp",
    "pxk_lrp_stabilized_divide": "ppppifnp",
    "pxk_lrp_bilinear_scale": "pppifp",
    "pxk_swiglu_forward": "pippiinp",
    "pxk_copy_2d": "pipiiip",
    "pxk_repeat_block": "piip",
    "pxk_accumulate_rows": "ppiip",
    "pxk_gather_rows": "pppiip",
    "pxk_embedding_ids": "piippp",
    "pxk_convert_weight": "pniinpp",
    "pxk_column_sums": "ppiifp",
    "pxk_rms_norm_forward": "ppppiifp",
    "pxk_softmax_rows": "ppiip",
    "pxk_lrp_softmax_rows": "ppppiip",
    "pxk_row_sums": "ppiip",
    "pxk_sum": "pippp",
    "pxk_dot": "ppippp",
    "pxk_attention_supported": "iiiii",
    "pxk_attention_forward": "pipipipppiiiiiifnp",
    "pxk_attention_forward_stats": "pipipippppiiiiiifnp",
    "pxk_attention_softmax": "ppiifnip",
    "pxk_attention_lrp_scores": "ppppiiffnip",
    "pxk_rms_norm_heads": "pipipiiifp",
    "pxk_rms_norm_add": "pppfppfpiip",
    "pxk_lrp_rope_rows": "pipipipippppiiiiifnnp",
    "pxk_rope_qk": "ppippipppiiiiinp",
    "pxk_rope_rotate": "ppppiiinnp",
    "pxk_lrp_rope": "ppppppiiifnp",
    "pxk_permute_0213": "ppiiiip",
    "pxk_attention_mask_fill": "ppiiiiniifp",
    "pxk_lm_seed": "piiipppnp",
    "pxk_decode_advance": "pp",
    "pxk_seed_rows": "pipiiippnp",
    "pxk_decode_pick": "piiipippippsp",
    "pxk_decode_attention": "pppippiiiiiifpsp",
    "pxk_decode_rope_append": "pipipipppiipppiiiinnppfp",
}


def _bind(lib, sigs):
    for name, sig in sigs.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [_T[c] for c in sig]


_pxk = None


def _share_hip_runtime():
    """Load PyTorch's HIP runtime first when PyTorch is installed, so the native libraries bind to
    that same libamdhip64.so.7 (by soname) and the process holds one HIP runtime. Loaded the other
    way round, PyTorch brings a second copy of the runtime that cannot see the device."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def pxk():
    """The kernel library, loaded once; raises PxkError if it was not built."""
    global _pxk
    if _pxk is None:
        _share_hip_runtime()
        if not os.path.exists(PXK_SO):
            raise PxkError("%s is missing: build it with __graft_entry__.build()" % PXK_SO)
        lib = ctypes.CDLL(PXK_SO)
        _bind(lib, PXK_SIGNATURES)
        lib.pxk_last_error.restype = ctypes.c_char_p
        lib.pxk_version.restype = ctypes.c_char_p
        lib.pxk_gemm.restype = ctypes.c_int
        lib.pxk_gemm.argtypes = [ctypes.POINTER(GemmDesc), c_vp]
        lib.pxk_gemm_noalloc.restype = ctypes.c_int
        lib.pxk_gemm_noalloc.argtypes = [ctypes.POINTER(GemmDesc), c_vp]
        lib.pxk_gemm_workspace.restype = ctypes.c_size_t
        lib.pxk_gemm_workspace.argtypes = [ctypes.POINTER(GemmDesc)]
        lib.pxk_gemm_plan.restype = ctypes.c_int
        lib.pxk_gemm_plan.argtypes = [ctypes.POINTER(GemmDesc), ctypes.POINTER(ctypes.c_int32),
                                      ctypes.POINTER(ctypes.c_int32)]
        lib.pxk_attention_relevance_q.restype = ctypes.c_int
        lib.pxk_attention_relevance_q.argtypes = [ctypes.POINTER(AttnRelDesc), c_vp]
        lib.pxk_attention_relevance_kv.restype = ctypes.c_int
        lib.pxk_attention_relevance_kv.argtypes = [ctypes.POINTER(AttnRelKvDesc), c_vp]
        lib.pxk_gemm_supported.restype = ctypes.c_int
        lib.pxk_gemm_supported.argtypes = [ctypes.c_int] * 4
        lib.pxk_lrp_rule_weights.restype = ctypes.c_int
        lib.pxk_lrp_rule_weights.argtypes = [ctypes.POINTER(RuleParams), ctypes.POINTER(RuleBlock), ctypes.c_int,
                                             c_i64, c_vp, c_vp, c_vp]
        lib.pxk_lrp_sign_split.restype = ctypes.c_int
        lib.pxk_lrp_sign_split.argtypes = [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp]
        lib.pxk_lrp_rule_divide.restype = ctypes.c_int
        lib.pxk_lrp_rule_divide.argtypes = [ctypes.POINTER(RuleParams), c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64,
                                            c_vp, c_vp, c_i64, c_i64, c_vp, c_i64, c_vp]
        lib.pxk_lrp_rule_combine.restype = ctypes.c_int
        lib.pxk_lrp_rule_combine.argtypes = [ctypes.c_int, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64,
                                             c_vp, c_vp, c_vp, c_vp, ctypes.c_float, c_vp]
        lib.pxk_reduce_partials.restype = ctypes.c_size_t
        lib.pxk_reduce_partials.argtypes = [c_i64]
        _pxk = lib
    return _pxk


def check(rc):
    if rc != 0:
        raise PxkError(pxk().pxk_last_error().decode())


def call(name, *args):
    check(getattr(pxk(), name)(*args))


def operand(ptr, ld, batch_stride=0, inner_stride=0, inner_div=0, group_stride=0):
    return Operand(ptr, ld, batch_stride, inner_stride, inner_div, group_stride)


class AttnRelDesc(ctypes.Structure):
    """pxk_attn_rel_desc."""

    _fields_ = [("n", c_i64), ("l", c_i64), ("heads", c_i64), ("kv_heads", c_i64), ("head_dim", c_i64),
                ("scale", ctypes.c_float), ("eps", ctypes.c_float), ("causal", ctypes.c_int32),
                ("rope", ctypes.c_int32), ("rope_half", ctypes.c_int32), ("relevance_only", ctypes.c_int32),
                ("spv", c_vp), ("ld_spv", c_i64), ("v", c_vp), ("ld_v", c_i64), ("k", c_vp), ("ld_k", c_i64),
                ("p", c_vp), ("raw", c_vp), ("s", c_vp), ("q", c_vp), ("ld_q", c_i64), ("q_pre", c_vp),
                ("ld_q_pre", c_i64), ("z", c_vp), ("ld_z", c_i64), ("bias", c_vp), ("cos_t", c_vp), ("sin_t", c_vp),
                ("g", c_vp), ("ld_g", c_i64), ("ctx", c_vp), ("ld_ctx", c_i64),
                ("stats", c_vp), ("row_sum", c_vp), ("p_out", c_vp)]


class AttnRelKvDesc(ctypes.Structure):
    """pxk_attn_rel_kv_desc."""

    _fields_ = [("n", c_i64), ("l", c_i64), ("heads", c_i64), ("kv_heads", c_i64), ("head_dim", c_i64),
                ("eps", ctypes.c_float), ("causal", ctypes.c_int32), ("rope", ctypes.c_int32),
                ("rope_half", ctypes.c_int32), ("s", c_vp), ("p", c_vp), ("q", c_vp), ("ld_q", c_i64),
                ("spv", c_vp), ("ld_spv", c_i64), ("k", c_vp), ("ld_k", c_i64), ("k_pre", c_vp),
                ("ld_k_pre", c_i64), ("v", c_vp), ("ld_v", c_i64), ("z_k", c_vp), ("z_v", c_vp), ("ld_z", c_i64),
                ("bias_k", c_vp), ("bias_v", c_vp), ("cos_t", c_vp), ("sin_t", c_vp), ("key_rel", c_vp),
                ("value_rel", c_vp), ("ld_rel", c_i64), ("g_k", c_vp), ("g_v", c_vp), ("ld_g", c_i64),
                ("relevance_only", ctypes.c_int32)]


class RuleParams(ctypes.Structure):
    """pxk_rule_params."""

    _fields_ = [("rule", ctypes.c_int32), ("eps", ctypes.c_float), ("gamma", ctypes.c_float),
                ("alpha", ctypes.c_float), ("beta", ctypes.c_float), ("low", ctypes.c_float),
                ("high", ctypes.c_float)]


class RuleBlock(ctypes.Structure):
    """pxk_rule_block."""

    _fields_ = [("w", c_vp), ("ld", c_i64), ("cols", c_i64), ("trans", ctypes.c_int32), ("bias", c_vp)]


def gemm(desc, stream=None):
    check(pxk().pxk_gemm(ctypes.byref(desc), stream))


def gemm_workspace(desc):
    return pxk().pxk_gemm_workspace(ctypes.byref(desc))


def gemm_plan(desc):
    """(tile, splits) pxk_gemm would launch for `desc`."""
    tile, splits = ctypes.c_int32(), ctypes.c_int32()
    check(pxk().pxk_gemm_plan(ctypes.byref(desc), ctypes.byref(tile), ctypes.byref(splits)))
    return tile.value, splits.value


# ---- the host framework (include/pulsatrix_amd.h) ----------------------------------------------

class ModelConfig(ctypes.Structure):
    """px_model_config."""

    _fields_ = [("vocab_size", c_i64), ("hidden_size", c_i64), ("num_layers", c_i64), ("num_heads", c_i64),
                ("num_kv_heads", c_i64), ("head_dim", c_i64), ("intermediate_size", c_i64),
                ("rms_norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("use_rope", ctypes.c_int32),
                ("rope_rotate_half", ctypes.c_int32), ("causal", ctypes.c_int32), ("qkv_bias", ctypes.c_int32),
                ("out_bias", ctypes.c_int32), ("mlp_bias", ctypes.c_int32), ("tie_word_embeddings", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("hidden_act", ctypes.c_int32), ("qk_norm", ctypes.c_int32),
                ("post_norms", ctypes.c_int32), ("rope_scaling", ctypes.c_int32),
                ("norm_weight_offset", ctypes.c_float), ("embed_scale", ctypes.c_float),
                ("query_pre_attn_scalar", ctypes.c_float), ("rope_local_base", ctypes.c_float),
                ("rope_factor", ctypes.c_float), ("rope_low_freq_factor", ctypes.c_float),
                ("rope_high_freq_factor", ctypes.c_float), ("reserved2", ctypes.c_int32),
                ("rope_original_max_position", c_i64), ("sliding_window", c_i64),
                ("sliding_layers", ctypes.c_uint64)]


EPSILON, GAMMA, ALPHA_BETA, ZBOX = 0, 1, 2, 3  # LRPRule order


class LrpRule(ctypes.Structure):
    """px_lrp_rule: LRPRuleConfig's fields (rule in LRPRule order)."""

    _fields_ = [("epsilon", ctypes.c_float), ("rule", ctypes.c_int32), ("gamma", ctypes.c_float),
                ("alpha", ctypes.c_float), ("beta", ctypes.c_float), ("low", ctypes.c_float),
                ("high", ctypes.c_float), ("bias_in_denominator", ctypes.c_int32)]


def lrp_rule(rule=EPSILON, epsilon=1e-6, gamma=0.25, alpha=1.0, beta=0.0, low=0.0, high=1.0,
             bias_in_denominator=False):
    return LrpRule(epsilon, rule, gamma, alpha, beta, low, high, int(bias_in_denominator))


def as_rule(r):
    """An LrpRule from any object with LRPRuleConfig's field names (the oracle's struct included)."""
    return LrpRule(*[getattr(r, f) for f, _ in LrpRule._fields_])


_host = None


def host():
    """libpulsatrix_amd.so, loaded once; raises PxkError if it was not built."""
    global _host
    if _host is None:
        if not os.path.exists(HOST_SO):
            raise PxkError("%s is missing: build it with __graft_entry__.build()" % HOST_SO)
        pxk()  # its dependency, from the same directory
        lib = ctypes.CDLL(HOST_SO)
        cfgp = ctypes.POINTER(ModelConfig)
        i64p = ctypes.POINTER(ctypes.c_int64)
        rulep = ctypes.POINTER(LrpRule)
        sigs = {
            "pxa_last_error": (ctypes.c_char_p, []),
            "pxa_device_count": (ctypes.c_int, []),
            "pxa_backend": (c_vp, []),
            "pxa_backend_stream": (c_vp, []),
            "pxa_backend_synchronize": (ctypes.c_int, []),
            "pxa_backend_memory": (ctypes.c_int, [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
            "pxa_launch_log_start": (ctypes.c_int, []),
            "pxa_launch_log_stop": (ctypes.c_int, [ctypes.POINTER(c_i64)]),
            "pxa_launch_log_entry": (ctypes.c_int, [c_i64, ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p,
                                                    ctypes.c_size_t, ctypes.POINTER(ctypes.c_double),
                                                    ctypes.POINTER(ctypes.c_double)]),
            "pxa_launch_log_time": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
            "pxa_launch_log_dispatches": (ctypes.c_int, [c_i64, ctypes.POINTER(ctypes.c_int32)]),
            "pxa_fill_normal": (None, [c_vp, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_double]),
            "pxa_param_count": (c_i64, [cfgp]),
            "pxa_block_param_count": (c_i64, [cfgp]),
            "pxa_synthetic_params": (ctypes.c_int, [cfgp, ctypes.c_int, ctypes.c_uint64, ctypes.c_double, c_vp]),
            "pxa_block_create": (c_vp, [cfgp, c_vp]),
            "pxa_block_forward": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_vp]),
            "pxa_block_relevance": (ctypes.c_int, [c_vp, c_vp, ctypes.c_float, ctypes.c_int, c_vp]),
            "pxa_block_destroy": (None, [c_vp]),
            "pxa_lm_create": (c_vp, [cfgp, c_vp]),
            "pxa_lm_create_random": (c_vp, [cfgp, ctypes.c_uint64, ctypes.c_double]),
            "pxa_lm_load": (c_vp, [ctypes.c_char_p, cfgp]),
            "pxa_lm_forward": (ctypes.c_int, [c_vp, i64p, c_i64, c_i64, c_vp]),
            "pxa_lm_relevance": (ctypes.c_int, [c_vp, c_vp, ctypes.c_float, ctypes.c_int, c_vp, c_vp, c_vp, c_vp]),
            "pxa_lm_explain_device": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, ctypes.c_float, ctypes.c_int, c_vp,
                                                     c_vp, i64p, ctypes.c_int]),
            "pxa_lm_capture_explain": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, ctypes.c_float, ctypes.c_int, c_vp,
                                                      c_vp]),
            "pxa_lm_replay": (ctypes.c_int, [c_vp]),
            "pxa_block_relevance_rule": (ctypes.c_int, [c_vp, c_vp, rulep, c_vp]),
            "pxa_linear_relevance_rule": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, rulep, c_vp,
                                                         c_vp]),
            "pxa_lm_relevance_rule": (ctypes.c_int, [c_vp, c_vp, rulep, c_vp, c_vp, c_vp, c_vp]),
            "pxa_lm_explain_device_rule": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, rulep, c_vp, c_vp, i64p,
                                                          ctypes.c_int]),
            "pxa_lm_capture_explain_rule": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, rulep, c_vp, c_vp]),
            "pxa_lm_explain_rows_device": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_vp, c_i64, rulep, c_vp, c_vp,
                                                          ctypes.c_int]),
            "pxa_lm_generate_device": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp]),
            "pxa_lm_explain_generated_device": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, rulep, c_vp,
                                                               ctypes.c_int]),
            "pxa_lm_next_token_logits_create": (c_vp, [c_vp, c_i64]),
            "pxa_lm_next_token_logits": (ctypes.c_int, [c_vp, i64p, c_i64, c_vp, c_i64]),
            "pxa_lm_next_token_logits_destroy": (None, [c_vp]),
            "pxa_lm_check_device_ids": (ctypes.c_int, [c_vp]),
            "pxa_lm_last_logits": (c_vp, [c_vp]),
            "pxa_lm_last_embedding_relevance": (c_vp, [c_vp]),
            "pxa_lm_destroy": (None, [c_vp]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _host = lib
    return _host


def host_check(rc):
    if rc != 0:
        raise PxkError(host().pxa_last_error().decode())


def model_config(**kw):
    base = dict(vocab_size=0, hidden_size=0, num_layers=1, num_heads=1, num_kv_heads=0, head_dim=0,
                intermediate_size=0, rms_norm_eps=1e-5, rope_theta=10000.0, use_rope=1, rope_rotate_half=1,
                causal=1, qkv_bias=0, out_bias=0, mlp_bias=0, tie_word_embeddings=1, reserved=0)
    base.update(kw)
    return ModelConfig(**base)
