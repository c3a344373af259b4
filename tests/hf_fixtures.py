"""Loaders for the committed golden fixtures (tests/golden/), shared by the oracle and GPU tests."""
import json
import os

import numpy as np

from oracle_ctypes import lm_layout, model_config, pack

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load_st(path):
    from safetensors.torch import load_file  # bf16-capable loader; no code runs from the file

    return {k: v.float().numpy() if v.is_floating_point() else v.numpy() for k, v in load_file(path).items()}


def hf_tiny(name):
    """(cfg, flat params, golden, attnlrp) for tests/golden/hf_tiny/<name>.

    The checkpoint's (out, in) Linear weights are transposed to the (in, out) layout the
    reference's LinearModule keeps (HuggingFaceMapping, src/causal_lm.cpp:257-291).
    """
    d = os.path.join(GOLDEN, "hf_tiny", name)
    hc = json.load(open(os.path.join(d, "config.json")))
    tensors = {}
    for f in sorted(os.listdir(d)):
        if f.startswith("model") and f.endswith(".safetensors"):
            tensors.update(_load_st(os.path.join(d, f)))
    cfg = config_of(hc)
    gemma = hc["model_type"] in ("gemma3", "gemma3_text")
    named = {"embed_tokens.weight": tensors["model.embed_tokens.weight"], "norm.weight": tensors["model.norm.weight"]}
    for i in range(cfg.num_layers):
        hf, px = "model.layers.%d." % i, "layers.%d." % i
        named[px + "norm1.weight"] = tensors[hf + "input_layernorm.weight"]
        if gemma:  # sandwich norms (HuggingFaceMapping, src/causal_lm.cpp:257-291)
            named[px + "norm2.weight"] = tensors[hf + "pre_feedforward_layernorm.weight"]
            named[px + "post_attn_norm.weight"] = tensors[hf + "post_attention_layernorm.weight"]
            named[px + "post_mlp_norm.weight"] = tensors[hf + "post_feedforward_layernorm.weight"]
        else:
            named[px + "norm2.weight"] = tensors[hf + "post_attention_layernorm.weight"]
        for p in ("q_proj", "k_proj", "v_proj"):
            named[px + "mha.%s.weight" % p] = tensors[hf + "self_attn.%s.weight" % p].T
            if cfg.qkv_bias:
                named[px + "mha.%s.bias" % p] = tensors[hf + "self_attn.%s.bias" % p]
        named[px + "mha.out_proj.weight"] = tensors[hf + "self_attn.o_proj.weight"].T
        if cfg.qk_norm:
            named[px + "mha.q_norm.weight"] = tensors[hf + "self_attn.q_norm.weight"]
            named[px + "mha.k_norm.weight"] = tensors[hf + "self_attn.k_norm.weight"]
        for p in ("gate_proj", "up_proj", "down_proj"):
            named[px + "swiglu.%s.weight" % p] = tensors[hf + "mlp.%s.weight" % p].T
    if not cfg.tie_word_embeddings:
        named["lm_head.weight"] = tensors["lm_head.weight"].T
    params = pack(lm_layout(cfg), named)
    golden = _load_st(os.path.join(d, "golden.safetensors"))
    attnlrp = _load_st(os.path.join(d, "attnlrp.safetensors"))
    return cfg, params, golden, attnlrp


def gradient_x_input(name):
    """The negative control of tests/fixtures/hf_tiny/<name>/gradient_x_input.safetensors: LXT with
    its AttnLRP patches off (plain gradient x input) for the same ids and targets as attnlrp."""
    return _load_st(os.path.join(GOLDEN, "hf_tiny", name, "gradient_x_input.safetensors"))


def config_of(hc):
    """px_model_config of a Hugging Face config.json, as ParseHfConfig + ToAttentionConfig read it
    (src/hf_model.cpp:99-313) for the Llama, Qwen2, Qwen3 and Gemma 3 fields."""
    heads = hc["num_attention_heads"]
    mt = hc["model_type"]
    gemma = mt in ("gemma3", "gemma3_text")
    rp = hc.get("rope_parameters") or {}
    full, sliding = rp.get("full_attention"), rp.get("sliding_attention")
    if "rope_theta" in hc:
        rope = hc["rope_theta"]
    elif isinstance(full, dict):
        rope = full.get("rope_theta", 10000.0)
    else:
        rope = rp.get("rope_theta", 10000.0)
    scaling = full if isinstance(full, dict) else (rp or hc.get("rope_scaling") or {})
    stype = scaling.get("rope_type", scaling.get("type", "default"))
    local = hc.get("rope_local_base_freq", sliding.get("rope_theta") if isinstance(sliding, dict) else None)
    window = hc.get("sliding_window") if hc.get("use_sliding_window", True) else None
    if window is not None and 0 < hc.get("max_position_embeddings", 0) <= window:
        window = None
    types = hc.get("layer_types") or []
    mask = sum(1 << i for i, t in enumerate(types) if t == "sliding_attention") if window else 0
    act = hc.get("hidden_act", hc.get("hidden_activation", "silu"))
    qkv_bias = bool(hc.get("attention_bias", mt == "qwen2"))
    return model_config(
        vocab_size=hc["vocab_size"], hidden_size=hc["hidden_size"], num_layers=hc["num_hidden_layers"],
        num_heads=heads, num_kv_heads=hc.get("num_key_value_heads", heads),
        head_dim=hc.get("head_dim", hc["hidden_size"] // heads), intermediate_size=hc["intermediate_size"],
        rms_norm_eps=hc.get("rms_norm_eps", 1e-6), rope_theta=float(rope), use_rope=1, rope_rotate_half=1, causal=1,
        qkv_bias=int(qkv_bias), out_bias=0, mlp_bias=int(hc.get("mlp_bias", False)),
        tie_word_embeddings=int(hc.get("tie_word_embeddings", True)),
        hidden_act=0 if act == "silu" else 1, qk_norm=int(mt in ("qwen3", "qwen3_moe", "gemma3", "gemma3_text")),
        post_norms=int(gemma), norm_weight_offset=1.0 if gemma else 0.0,
        embed_scale=float(np.float32(np.sqrt(np.float64(hc["hidden_size"])))) if gemma else 0.0,
        query_pre_attn_scalar=float(hc.get("query_pre_attn_scalar") or 0.0),
        rope_local_base=float(local or 0.0), rope_scaling={"default": 0, "linear": 1, "llama3": 2}[stype],
        rope_factor=float(scaling.get("factor", 1.0)), rope_low_freq_factor=float(scaling.get("low_freq_factor", 1.0)),
        rope_high_freq_factor=float(scaling.get("high_freq_factor", 1.0)),
        rope_original_max_position=int(scaling.get("original_max_position_embeddings", 0)),
        sliding_window=int(window or 0), sliding_layers=mask)


def sequences(fixture, prefix="ids"):
    k = 0
    while "%s.%d" % (prefix, k) in fixture:
        yield k
        k += 1


def lxt_values():
    return json.load(open(os.path.join(GOLDEN, "lxt_values.json")))


def det(n, mul, add, div):
    """The LXT generator's det(): float(((i * mul + add) % 17) - 8) / float(div) (tests/lrp_reference_test.cpp:63-69)."""
    i = np.arange(n, dtype=np.int64)
    return (((i * mul + add) % 17) - 8).astype(np.float32) / np.float32(div)


def pearson(x, y):
    x = np.asarray(x, dtype=np.float64).ravel()
    y = np.asarray(y, dtype=np.float64).ravel()
    x = x - x.mean()
    y = y - y.mean()
    sxx, syy = (x * x).sum(), (y * y).sum()
    return 0.0 if sxx == 0 or syy == 0 else float((x * y).sum() / np.sqrt(sxx * syy))


def per_head(rel, L, kv_heads):
    """(Hkv, L) per-(head, token) totals of an (L, Hkv*D) projection relevance (src/attnlrp_parity.cpp:33-45)."""
    r = np.asarray(rel, dtype=np.float64).reshape(L, kv_heads, -1).sum(axis=2)
    return r.T.astype(np.float32)
