"""Pins the CPU oracle (oracle/pxo.cpp) before anything is checked against it.

* Against the reference's own fixtures (committed under tests/golden/): transformers logits and
  LXT 2.1 AttnLRP relevance of the hf_tiny checkpoints, and the LXT TransformerBlock values of
  tests/lrp_reference_test.cpp.
* Against the compiled reference (oracle/_ref, where this container built it): bit for bit, on
  the B block shape, a GQA causal LM, biases, both LRP rules.
* Against closed forms the mathematics fixes: the Eq. 15 shares of a bilinear product each sum
  to half the output relevance; a zero-weight block is the identity.
"""
import numpy as np
import pytest

import oracle_ctypes as oc
from hf_fixtures import det, gradient_x_input, hf_tiny, lxt_values, pearson, per_head, sequences

LXT_EPS = 1e-9  # LxtAttnLrpConfig(), src/attnlrp_parity.cpp:67-72


def close(actual, expected, rel=1e-4):
    expected = np.asarray(expected, dtype=np.float32)
    tol = rel * np.maximum(1.0, np.abs(expected))
    return np.all(np.abs(np.asarray(actual) - expected) <= tol)


@pytest.mark.parametrize("name", ["llama", "qwen2", "qwen3", "gemma3"])
def test_oracle_logits_match_transformers(name):
    cfg, params, golden, _ = hf_tiny(name)
    lm = oc.oracle().lm(cfg, params)
    for k in sequences(golden):
        ids = golden["ids.%d" % k].reshape(1, -1)
        logits = lm.forward(ids)[0]
        assert close(logits, golden["logits.%d" % k]), (name, k, np.abs(logits - golden["logits.%d" % k]).max())


@pytest.mark.parametrize("name", ["llama", "qwen2", "qwen3", "gemma3"])
def test_oracle_attnlrp_matches_lxt(name):
    """The checks of tests/attnlrp_parity_test.cpp:28-51 (via CompareToAttnLrp)."""
    cfg, params, _, ref = hf_tiny(name)
    lm = oc.oracle().lm(cfg, params)
    for k in sequences(ref):
        ids = ref["ids.%d" % k].reshape(1, -1)
        L = ids.shape[1]
        target = int(ref["target.%d" % k][0])
        logits = lm.forward(ids)
        seed = np.zeros_like(logits)
        seed[0, L - 1, target] = logits[0, L - 1, target]
        r_embed, r_tok, key, value = lm.relevance(seed, LXT_EPS, True, want_kv=True)
        expected = ref["relevance.%d" % k]
        assert pearson(r_tok[0], expected) > 0.99999
        assert np.abs(r_tok[0] - expected).max() / np.abs(expected).max() < 1e-4
        assert abs(r_tok.sum() - expected.sum()) <= 1e-4 * abs(expected.sum())
        hkv = cfg.kv_heads()
        ek, ev = ref["key_relevance.%d" % k], ref["value_relevance.%d" % k]
        for i in range(cfg.num_layers):
            assert pearson(per_head(key[i], L, hkv), ek[i]) > 0.99999
            assert pearson(per_head(value[i], L, hkv), ev[i]) > 0.99999


def test_oracle_attnlrp_negative_control():
    """Seeding the wrong target must fail the correlation gate (tests/attnlrp_parity_test.cpp:42-49 spirit)."""
    cfg, params, _, ref = hf_tiny("llama")
    lm = oc.oracle().lm(cfg, params)
    ids = ref["ids.2"].reshape(1, -1)
    L = ids.shape[1]
    logits = lm.forward(ids)
    target = (int(ref["target.2"][0]) + 1) % cfg.vocab_size
    seed = np.zeros_like(logits)
    seed[0, L - 1, target] = logits[0, L - 1, target]
    _, r_tok = lm.relevance(seed, LXT_EPS, True)
    assert pearson(r_tok[0], ref["relevance.2"]) < 0.99999


@pytest.mark.parametrize("name", ["llama", "qwen2", "qwen3", "gemma3"])
def test_oracle_attnlrp_does_not_match_gradient_x_input(name):
    """The reference's negative control (tests/attnlrp_parity_test.cpp:42-49): against LXT's plain
    gradient x input for the same ids and targets, the AttnLRP relevance fails the gate, with a
    token correlation below 0.9 on some sequence."""
    cfg, params, _, ref = hf_tiny(name)
    neg = gradient_x_input(name)
    lm = oc.oracle().lm(cfg, params)
    worst = 1.0
    for k in sequences(neg):
        ids = neg["ids.%d" % k].reshape(1, -1)
        L = ids.shape[1]
        target = int(neg["target.%d" % k][0])
        logits = lm.forward(ids)
        seed = np.zeros_like(logits)
        seed[0, L - 1, target] = logits[0, L - 1, target]
        _, r_tok = lm.relevance(seed, LXT_EPS, True)
        worst = min(worst, pearson(r_tok[0], neg["relevance.%d" % k]))
    assert worst < 0.9, worst


def lxt_block_params():
    """The LXT TransformerBlock of tests/lrp_reference_test.cpp:360-375 (d 4, 2 heads, d_ff 6, biases)."""
    cfg = oc.model_config(hidden_size=4, num_heads=2, num_kv_heads=2, head_dim=2, intermediate_size=6,
                          rms_norm_eps=1e-6, use_rope=0, causal=0, qkv_bias=1, out_bias=1, mlp_bias=1)
    t = {"norm1.weight": det(4, 3, 14, 8) + 1.0, "norm2.weight": det(4, 5, 11, 8) + 1.0}

    def lin(name, i, o, mul, add, div, badd, bdiv):
        t[name + ".weight"] = det(i * o, mul, add, div).reshape(i, o)
        t[name + ".bias"] = det(o, 3, badd, bdiv)

    lin("mha.q_proj", 4, 4, 5, 1, 6, 2, 11)
    lin("mha.k_proj", 4, 4, 7, 3, 5, 5, 13)
    lin("mha.v_proj", 4, 4, 11, 6, 7, 8, 9)
    lin("mha.out_proj", 4, 4, 13, 2, 8, 1, 10)
    lin("swiglu.gate_proj", 4, 6, 5, 9, 6, 4, 12)
    lin("swiglu.up_proj", 4, 6, 7, 2, 7, 7, 10)
    lin("swiglu.down_proj", 6, 4, 3, 8, 6, 9, 11)
    return cfg, oc.pack(oc.block_layout(cfg), t)


def test_oracle_block_matches_lxt():
    """Block -> Flatten -> Linear(12, 3), ZennitEpsilon(1e-6), one-hot targets {0, 2}."""
    cfg, params = lxt_block_params()
    vals = lxt_values()
    blk = oc.oracle().block(cfg, params)
    x = det(24, 5, 7, 4).reshape(2, 3, 4)
    y = blk.forward(x)
    w, b = det(36, 11, 5, 9).reshape(12, 3), det(3, 3, 3, 7)
    pre, logits = oc.linear_forward(y.reshape(2, 12), w, b)
    assert close(logits.ravel(), vals["kBlockLogits"])
    seed = np.zeros((2, 3), np.float32)
    seed[0, 0] = 1.0
    seed[1, 2] = 1.0
    r_flat = oc.linear_relevance(y.reshape(2, 12), w, b, pre, seed, 1e-6, True)
    r_in = blk.relevance(r_flat.reshape(2, 3, 4), 1e-6, True)
    assert close(r_in.ravel(), vals["kBlockRelevance"])


def b_config(**kw):
    base = dict(hidden_size=576, num_heads=9, num_kv_heads=3, head_dim=64, intermediate_size=1536,
                rms_norm_eps=1e-5, rope_theta=10000.0)
    base.update(kw)
    return oc.model_config(**base)


needs_ref = pytest.mark.skipif(oc.ref() is None, reason="oracle/_ref (compiled reference) not built here")


@needs_ref
@pytest.mark.parametrize("bias_in_denominator,eps", [(False, 1e-6), (True, 1e-9)])
def test_oracle_block_bit_identical_to_reference(bias_in_denominator, eps):
    cfg = b_config()
    params = oc.synthetic_params(cfg, 11, block=True)
    x = oc.fill_normal(48 * 576, 5, 1.0).reshape(1, 48, 576)
    o, r = oc.oracle().block(cfg, params), oc.ref().block(cfg, params)
    yo, yr = o.forward(x), r.forward(x)
    assert np.array_equal(yo, yr)
    seed = np.zeros_like(yo)
    seed[..., 0] = yo[..., 0]  # OutputValue seed at channel 0
    assert np.array_equal(o.relevance(seed, eps, bias_in_denominator), r.relevance(seed, eps, bias_in_denominator))


@needs_ref
def test_oracle_block_with_biases_bit_identical_to_reference():
    cfg = b_config(hidden_size=48, num_heads=4, num_kv_heads=2, head_dim=12, intermediate_size=40, qkv_bias=1,
                   out_bias=1, mlp_bias=1, causal=0, rope_rotate_half=0)
    params = oc.synthetic_params(cfg, 3, std=0.2, block=True)
    x = oc.fill_normal(2 * 7 * 48, 6, 1.0).reshape(2, 7, 48)
    o, r = oc.oracle().block(cfg, params), oc.ref().block(cfg, params)
    yo = o.forward(x)
    assert np.array_equal(yo, r.forward(x))
    seed = oc.fill_normal(yo.size, 8, 1.0).reshape(yo.shape)
    for bid in (False, True):
        assert np.array_equal(o.relevance(seed, 1e-6, bid), r.relevance(seed, 1e-6, bid))


@needs_ref
@pytest.mark.parametrize("tied", [1, 0])
def test_oracle_lm_bit_identical_to_reference(tied):
    cfg = oc.model_config(vocab_size=300, hidden_size=64, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=16,
                          intermediate_size=80, rope_theta=100000.0, tie_word_embeddings=tied)
    params = oc.synthetic_params(cfg, 21)
    ids = np.random.RandomState(1).randint(0, 300, size=(2, 19))
    o, r = oc.oracle().lm(cfg, params), oc.ref().lm(cfg, params)
    lo, lr = o.forward(ids), r.forward(ids)
    assert np.array_equal(lo, lr)
    seed = np.zeros_like(lo)
    for n in range(2):
        t = int(np.argmax(lo[n, -1]))
        seed[n, -1, t] = lo[n, -1, t]
    for a, b in zip(o.relevance(seed, LXT_EPS, True, want_kv=True), r.relevance(seed, LXT_EPS, True, want_kv=True)):
        assert np.array_equal(a, b)


def test_oracle_bilinear_shares_sum_to_half():
    """Eq. 15: with eps -> 0, r_a and r_b each sum to half of sum(R_O) (lrp_math.hpp:47-56)."""
    import ctypes

    rng = np.random.RandomState(0)
    m, p, q = 5, 7, 3
    a = rng.uniform(0.5, 1.5, (m, p)).astype(np.float32)
    b = rng.uniform(0.5, 1.5, (p, q)).astype(np.float32)
    o = (a.astype(np.float64) @ b).astype(np.float32)
    r = rng.uniform(-1, 1, (m, q)).astype(np.float32)
    ra, rb = np.empty_like(a), np.empty_like(b)
    L = oc.oracle().lib
    L.pxo_lrp_bilinear_matmul.argtypes = [oc._f32p] * 6 + [ctypes.c_size_t] * 4 + [ctypes.c_float, ctypes.c_int]
    L.pxo_lrp_bilinear_matmul(oc.fptr(a), oc.fptr(b), oc.fptr(o), oc.fptr(r), oc.fptr(ra), oc.fptr(rb), 1, m, p, q,
                              1e-12, 0)
    assert abs(ra.sum() - 0.5 * r.sum()) < 1e-5 and abs(rb.sum() - 0.5 * r.sum()) < 1e-5


def test_oracle_zero_weight_block_is_identity():
    """All-zero projections: attention and MLP outputs vanish, y = x (transformer_block_test.cpp:46)."""
    cfg = b_config(hidden_size=32, num_heads=4, num_kv_heads=2, head_dim=8, intermediate_size=48)
    params = np.zeros(oc.oracle().lib.pxo_block_param_count(oc.ModelConfig(**{f: getattr(cfg, f) for f, _ in
                                                                                cfg._fields_})), np.float32)
    x = oc.fill_normal(3 * 32, 2, 1.0).reshape(1, 3, 32)
    assert np.array_equal(oc.oracle().block(cfg, params).forward(x), x)


def test_fill_normal_moments():
    v = oc.fill_normal(200000, 42, 0.02).astype(np.float64)
    assert abs(v.mean()) < 3e-4 and abs(v.std() - 0.02) < 3e-4


def gemma_config(**kw):
    """A Gemma-3-style config: GeLU-tanh gates, QK-norm, sandwich norms, (1 + w) norms, scaled
    embeddings, query_pre_attn_scalar, sliding layers with their own RoPE base, linear RoPE scaling
    on the full layers (the hf_tiny gemma3 fixture's settings at other sizes)."""
    base = dict(vocab_size=211, hidden_size=48, num_layers=3, num_heads=4, num_kv_heads=1, head_dim=24,
                intermediate_size=56, rms_norm_eps=1e-6, rope_theta=10000.0, hidden_act=1, qk_norm=1, post_norms=1,
                norm_weight_offset=1.0, embed_scale=float(np.float32(np.sqrt(48.0))), query_pre_attn_scalar=20.0,
                rope_local_base=100.0, rope_scaling=1, rope_factor=2.0, sliding_window=5, sliding_layers=0b101)
    base.update(kw)
    return oc.model_config(**base)


@needs_ref
@pytest.mark.parametrize("tied", [1, 0])
def test_oracle_gemma_lm_bit_identical_to_reference(tied):
    """Every Gemma 3 variant at once, LXT and pre-bias epsilon rules and Gamma, against the compiled
    reference built through its own ToAttentionConfig(config, layer)."""
    cfg = gemma_config(tie_word_embeddings=tied)
    params = oc.synthetic_params(cfg, 23, std=0.1)
    ids = np.random.RandomState(2).randint(0, 211, size=(2, 13))
    o, r = oc.oracle().lm(cfg, params), oc.ref().lm(cfg, params)
    lo = o.forward(ids)
    assert np.array_equal(lo, r.forward(ids))
    seed = np.zeros_like(lo)
    for n in range(2):
        t = int(np.argmax(lo[n, -1]))
        seed[n, -1, t] = lo[n, -1, t]
    for a, b in zip(o.relevance(seed, LXT_EPS, True, want_kv=True), r.relevance(seed, LXT_EPS, True, want_kv=True)):
        assert np.array_equal(a, b)
    for a, b in zip(o.relevance(seed, 1e-6, False), r.relevance(seed, 1e-6, False)):
        assert np.array_equal(a, b)
    g = oc.lrp_rule(oc.GAMMA, gamma=0.25)
    for a, b in zip(o.relevance_rule(seed, g), r.relevance_rule(seed, g)):
        assert np.array_equal(a, b)


@needs_ref
@pytest.mark.parametrize("kw", [dict(sliding_layers=0), dict(rope_scaling=2, rope_factor=8.0, rope_low_freq_factor=1.0,
                                                              rope_high_freq_factor=4.0,
                                                              rope_original_max_position=8, sliding_window=0)])
def test_oracle_variant_lm_bit_identical_to_reference(kw):
    """A window on every layer (Mistral's form), and llama3 RoPE scaling without windows."""
    cfg = gemma_config(**kw)
    params = oc.synthetic_params(cfg, 29, std=0.1)
    ids = np.random.RandomState(3).randint(0, 211, size=(1, 17))
    o, r = oc.oracle().lm(cfg, params), oc.ref().lm(cfg, params)
    lo = o.forward(ids)
    assert np.array_equal(lo, r.forward(ids))
    seed = np.zeros_like(lo)
    t = int(np.argmax(lo[0, -1]))
    seed[0, -1, t] = lo[0, -1, t]
    for a, b in zip(o.relevance(seed, LXT_EPS, True), r.relevance(seed, LXT_EPS, True)):
        assert np.array_equal(a, b)


@needs_ref
def test_oracle_gemma_block_bit_identical_to_reference():
    cfg = gemma_config(num_layers=1, sliding_layers=1)
    params = oc.synthetic_params(cfg, 5, std=0.2, block=True)
    x = oc.fill_normal(2 * 9 * 48, 6, 1.0).reshape(2, 9, 48)
    o, r = oc.oracle().block(cfg, params), oc.ref().block(cfg, params)
    yo = o.forward(x)
    assert np.array_equal(yo, r.forward(x))
    seed = oc.fill_normal(yo.size, 8, 1.0).reshape(yo.shape)
    assert np.array_equal(o.relevance(seed, 0.1, True), r.relevance(seed, 0.1, True))


@pytest.mark.skipif(oc.ref() is None, reason="oracle/_ref was not built (no reference sources)")
def test_oracle_backward_rows_bit_identical_to_reference():
    """The oracle's elementwise_backward (every op), softmax_rows_backward and rms_norm_backward
    against the compiled reference CPUBackend on the same data: bit for bit."""
    import gpu_util as G
    R = oc.ref().lib
    n, rows, cols = 4099, 37, 129
    x, g = G.uniform((n,), 1) * 3, G.uniform((n,), 2)
    for op in range(8):
        a, b = np.empty_like(x), np.empty_like(x)
        G.oracle_call("pxo_elementwise_backward", op, x, g, a, n)
        R.pxr_be_elementwise_backward(op, x.ctypes.data, g.ctypes.data, b.ctypes.data, n)
        assert np.array_equal(a, b, equal_nan=True), op
    # ReLU is a select: a non-finite gradient where x <= 0 still gives 0
    gi = g.copy()
    gi[x <= 0] = np.inf
    a = np.empty_like(x)
    G.oracle_call("pxo_elementwise_backward", 0, x, gi, a, n)
    assert np.all(a[x <= 0] == 0)
    y = np.exp(G.uniform((rows, cols), 3))
    y /= y.sum(axis=1, keepdims=True)
    dy = G.uniform((rows, cols), 4)
    a, b = np.empty_like(y), np.empty_like(y)
    G.oracle_call("pxo_softmax_rows_backward", y, dy, a, rows, cols)
    R.pxr_be_softmax_rows_backward(y.ctypes.data, dy.ctypes.data, b.ctypes.data, rows, cols)
    assert np.array_equal(a, b)
    # closed form: each row of dx sums to sum(y dy) (1 - sum y) = 0 for a softmax row
    assert np.abs(a.astype(np.float64).sum(axis=1)).max() < 1e-5
    xin, gamma = G.uniform((rows, cols), 5), G.uniform((cols,), 6)
    rms = np.sqrt((xin.astype(np.float64) ** 2).mean(axis=1) + 1e-5).astype(np.float32)
    ga, gb, ta, tb = (np.empty_like(xin) for _ in range(4))
    G.oracle_call("pxo_rms_norm_backward", dy, gamma, xin, rms, ga, ta, rows, cols)
    R.pxr_be_rms_norm_backward(dy.ctypes.data, gamma.ctypes.data, xin.ctypes.data, rms.ctypes.data, gb.ctypes.data,
                               tb.ctypes.data, rows, cols)
    assert np.array_equal(ga, gb) and np.array_equal(ta, tb)
    # against the derivative itself, by central differences of RMSNorm in float64
    x64, g64, gam = xin.astype(np.float64), dy.astype(np.float64), gamma.astype(np.float64)

    def f(x):
        return ((gam * x / np.sqrt((x ** 2).mean(axis=1, keepdims=True) + 1e-5)) * g64).sum()

    h = 1e-6
    for (r, c) in ((0, 0), (5, 17), (36, 128)):
        e = np.zeros_like(x64)
        e[r, c] = h
        num = (f(x64 + e) - f(x64 - e)) / (2 * h)
        assert abs(num - ga[r, c]) <= 1e-4 * max(1.0, abs(num)), (r, c, num, ga[r, c])
