"""The reference's Hugging Face attention cases and its independent NumPy AttnLRP block, run through
the reference's own modules (oracle/ref_driver.cpp: pxr_mha_case, pxr_legacy_block_case) on either
of its backends: the reference's CPUBackend (oracle/_ref/libpxref.so) or MI355XBackend
(oracle/_ref/libpxref_mi355x.so, the drop-in).

The attention cases restate tests/attention_reference_test.cpp:139-200: LlamaAttention (GQA 4/2,
head_dim 4, RoPE base 100, causal, the second sequence's last two positions padded), Qwen2Attention
(MQA 3/1, Q/K/V biases, base 1000, left padding, position offset 3) and Qwen3Attention (2/1,
head_dim 6 with d_model 8, QK-Norm with gains 1 + Det, base 10000), weights and inputs from the
test's Det() formula (:25-31), two sequences of 5 tokens. Each runs forward, then the backward of
sum(out * G) with G zero on padding queries (:115-131). The expected forward outputs and input
gradients are the values the reference pasted from transformers 5.18.0
(tests/golden/hf_attention_values.json). Tolerance 1e-4 * max(1, |expected|) per element (:35-42).

The block case is tests/transformer_block_test.cpp:262-318 (tests/golden/legacy_block_values.json):
forward within 1e-4 and LRPRuleConfig{} input relevance within 1e-4 of the NumPy values."""
import ctypes
import json
import os

import numpy as np

from hf_fixtures import det

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


class MhaSpec(ctypes.Structure):
    """pxr_mha_spec (oracle/ref_driver.cpp)."""
    _fields_ = [("d_model", ctypes.c_int64), ("heads", ctypes.c_int64), ("kv_heads", ctypes.c_int64),
                ("head_dim", ctypes.c_int64), ("rope_base", ctypes.c_float), ("qkv_bias", ctypes.c_int32),
                ("qk_norm", ctypes.c_int32), ("causal", ctypes.c_int32), ("position_offset", ctypes.c_int64),
                ("n", ctypes.c_int64), ("l", ctypes.c_int64)] + \
               [(f, ctypes.c_void_p) for f in ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "q_gamma", "k_gamma", "keep")]


# name: (config, Det() arguments of each tensor, keep flags, x Det(), G Det(), expected keys)
CASES = {
    "llama": dict(d_model=8, heads=4, kv_heads=2, head_dim=4, rope_base=100.0, qkv_bias=0, qk_norm=0, offset=0,
                  wq=(5, 1, 7), wk=(3, 2, 9), wv=(7, 3, 8), wo=(11, 4, 10),
                  keep=[1, 1, 1, 1, 1, 1, 1, 1, 0, 0], x=(5, 3, 4), g=(7, 2, 5),
                  expected=("kLlamaOutput", "kLlamaInputGrad")),
    "qwen2": dict(d_model=6, heads=3, kv_heads=1, head_dim=4, rope_base=1000.0, qkv_bias=1, qk_norm=0, offset=3,
                  wq=(5, 2, 6), bq=(3, 1, 5), wk=(3, 1, 7), bk=(3, 4, 6), wv=(7, 5, 9), bv=(3, 2, 7), wo=(13, 3, 11),
                  keep=[0, 1, 1, 1, 1, 1, 1, 1, 1, 1], x=(3, 1, 4), g=(5, 4, 6),
                  expected=("kQwen2Output", "kQwen2InputGrad")),
    "qwen3": dict(d_model=8, heads=2, kv_heads=1, head_dim=6, rope_base=10000.0, qkv_bias=0, qk_norm=1, offset=0,
                  wq=(5, 1, 6), wk=(3, 4, 7), wv=(7, 2, 8), wo=(11, 5, 9), q_gamma=(5, 1, 20), k_gamma=(7, 3, 20),
                  keep=[1] * 10, x=(7, 1, 4), g=(3, 5, 5),
                  expected=("kQwen3Output", "kQwen3InputGrad")),
}
N, L = 2, 5


def expected(name):
    values = json.load(open(os.path.join(GOLDEN, "hf_attention_values.json")))
    out_key, grad_key = CASES[name]["expected"]
    return np.array(values[out_key], np.float32), np.array(values[grad_key], np.float32)


def run_mha_case(lib, name):
    """(forward output, input gradient) of one case through the reference's module on lib's backend."""
    c = CASES[name]
    d, qd, kvd = c["d_model"], c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]
    keep = np.array(c["keep"], np.float32)
    arrays = {"wq": det(d * qd, *c["wq"]), "wk": det(d * kvd, *c["wk"]), "wv": det(d * kvd, *c["wv"]),
              "wo": det(qd * d, *c["wo"]), "keep": keep}
    if c["qkv_bias"]:
        arrays.update(bq=det(qd, *c["bq"]), bk=det(kvd, *c["bk"]), bv=det(kvd, *c["bv"]))
    if c["qk_norm"]:
        arrays.update(q_gamma=det(c["head_dim"], *c["q_gamma"]) + np.float32(1.0),
                      k_gamma=det(c["head_dim"], *c["k_gamma"]) + np.float32(1.0))
    arrays = {k: np.ascontiguousarray(v, np.float32) for k, v in arrays.items()}
    spec = MhaSpec(d_model=d, heads=c["heads"], kv_heads=c["kv_heads"], head_dim=c["head_dim"],
                   rope_base=c["rope_base"], qkv_bias=c["qkv_bias"], qk_norm=c["qk_norm"], causal=1,
                   position_offset=c["offset"], n=N, l=L,
                   **{k: v.ctypes.data for k, v in arrays.items()})
    x = np.ascontiguousarray(det(N * L * d, *c["x"]), np.float32)
    g = det(N * L * d, *c["g"]).reshape(N * L, d) * keep[:, None]  # G zero on padding queries
    g = np.ascontiguousarray(g.ravel(), np.float32)
    out, grad = np.empty_like(x), np.empty_like(x)
    fn = lib.fn("mha_case")
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(MhaSpec)] + [ctypes.c_void_p] * 4
    lib.check(fn(ctypes.byref(spec), x.ctypes.data, g.ctypes.data, out.ctypes.data, grad.ctypes.data))
    return out, grad


def assert_matches_reference(got, want, what):
    tol = 1e-4 * np.maximum(1.0, np.abs(want))
    bad = np.abs(got - want) > tol
    assert not bad.any(), "%s: %d elements outside 1e-4 * max(1, |x|); first at %d: %r vs %r" % (
        what, bad.sum(), int(np.argmax(bad)), float(got[np.argmax(bad)]), float(want[np.argmax(bad)]))


def legacy_block_values():
    return json.load(open(os.path.join(GOLDEN, "legacy_block_values.json")))


def run_legacy_block_case(lib):
    """(y, r_in) of the NumPy AttnLRP block through the reference's TransformerBlock on lib's backend."""
    v = legacy_block_values()
    params = np.ascontiguousarray(np.concatenate([v[k] for k in ("norm1", "q", "k", "v", "out", "norm2", "gate",
                                                                 "up", "down")]), np.float32)
    x = np.ascontiguousarray(v["x"], np.float32)
    r_out = np.ascontiguousarray(v["relevance_out"], np.float32)
    y, r_in = np.empty_like(x), np.empty_like(x)
    fn = lib.fn("legacy_block_case")
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_void_p] * 5
    lib.check(fn(v["d_model"], v["heads"], v["d_ff"], x.size // v["d_model"], params.ctypes.data, x.ctypes.data,
                 r_out.ctypes.data, y.ctypes.data, r_in.ctypes.data))
    return y, r_in
