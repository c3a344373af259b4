"""The Gemma 3 architecture on the MI355X path (GeLU-tanh gates, QK-Norm, sandwich norms, (1 + w)
norms, scaled embeddings, query_pre_attn_scalar, sliding-window layers with their own RoPE base,
linear RoPE scaling, head_dim 256), called through the C ABI:

* the hf_tiny gemma3 checkpoint (tests/fixtures/hf_tiny/gemma3, committed under tests/golden/):
  transformers logits at 1e-4 and LXT 2.1 relevance at the reference's own thresholds
  (tests/attnlrp_parity_test.cpp:28-51), from host parameters and through the device loader;
* Gemma-style configs and the Gemma-3-270m widths against the oracle (itself pinned to the same
  fixture and bit-identical to the compiled reference, tests/test_oracle.py), with the gates of
  test_model_gpu.py.
"""
import os

import numpy as np
import pytest

import gpu_util as G
import oracle_ctypes as oc
from hf_fixtures import GOLDEN, hf_tiny, pearson, per_head, sequences
from pulsatrix_amd import models
from pulsatrix_amd import native as N
from test_model_gpu import LXT_EPS, argmax_seed, expect_logits_agree, expect_relevance_agrees, to_px
from test_oracle import gemma_config

pytestmark = pytest.mark.gpu


def check_hf_tiny(lm, cfg, golden, ref):
    for k in sequences(golden):
        ids = golden["ids.%d" % k].reshape(1, -1)
        logits = lm.forward(ids)[0]
        exp = golden["logits.%d" % k]
        assert np.all(np.abs(logits - exp) <= 1e-4 * np.maximum(1.0, np.abs(exp))), k
    for k in sequences(ref):
        ids = ref["ids.%d" % k].reshape(1, -1)
        L = ids.shape[1]
        target = int(ref["target.%d" % k][0])
        logits = lm.forward(ids)
        seed = np.zeros_like(logits)
        seed[0, L - 1, target] = logits[0, L - 1, target]
        _, r_tok, key, value = lm.relevance(seed, LXT_EPS, True, want_kv=True)
        expected = ref["relevance.%d" % k]
        assert pearson(r_tok[0], expected) > 0.99999
        assert np.abs(r_tok[0] - expected).max() / np.abs(expected).max() < 1e-4
        assert abs(r_tok.sum() - expected.sum()) <= 1e-4 * abs(expected.sum())
        for i in range(cfg.num_layers):
            assert pearson(per_head(key[i], L, cfg.kv_heads()), ref["key_relevance.%d" % k][i]) > 0.99999
            assert pearson(per_head(value[i], L, cfg.kv_heads()), ref["value_relevance.%d" % k][i]) > 0.99999


def test_gemma3_hf_tiny_matches_transformers_and_lxt():
    """Sliding window 3 on three of four layers (local RoPE base 100), linear RoPE scaling x2 on the
    full layer, QK-Norm, sandwich norms, GeLU-tanh, scaled embeddings, query_pre_attn_scalar 12."""
    cfg, params, golden, ref = hf_tiny("gemma3")
    check_hf_tiny(models.CausalLM(to_px(cfg), params), cfg, golden, ref)


def test_gemma3_hf_tiny_loads_to_the_device():
    """The BF16 checkpoint through LoadCausalLM: config.json parsed for every Gemma 3 field, the
    sandwich and QK norms mapped, weights widened and transposed on the GPU."""
    cfg, params, golden, ref = hf_tiny("gemma3")
    lm = models.CausalLM.load(os.path.join(GOLDEN, "hf_tiny", "gemma3"))
    for f, _ in cfg._fields_:
        if f not in ("reserved", "reserved2"):
            assert getattr(lm.cfg, f) == pytest.approx(getattr(cfg, f)), f
    check_hf_tiny(lm, cfg, golden, ref)


def compare_lm(cfg, params, ids, rules):
    ref, gpu = oc.oracle().lm(cfg, params), models.CausalLM(to_px(cfg), params)
    lr, lg = ref.forward(ids), gpu.forward(ids)
    expect_logits_agree(lg, lr, "logits")
    seed = argmax_seed(lr)
    for name, rule in rules:
        a = gpu.relevance_rule(seed, rule, want_kv=True)
        b = ref.relevance_rule(seed, rule, want_kv=True)
        for what, u, v in zip(("embedding", "tokens", "keys", "values"), a, b):
            expect_relevance_agrees(u, v, "%s %s" % (what, name))


LXT = ("lxt", oc.lrp_rule(oc.EPSILON, epsilon=LXT_EPS, bias_in_denominator=True))
DEFAULT = ("pre-bias eps 1e-6", oc.lrp_rule(oc.EPSILON, epsilon=1e-6))
GAMMA = ("gamma 0.25", oc.lrp_rule(oc.GAMMA, gamma=0.25))


@pytest.mark.parametrize("tied", [1, 0])
def test_gemma_style_lm_matches_oracle(tied):
    """Every Gemma 3 variant at small widths (head_dim 24, a window of 5 on layers 0 and 2) at a length
    where the window masks, under LXT, the default epsilon rule and Gamma."""
    cfg = gemma_config(tie_word_embeddings=tied)
    params = oc.synthetic_params(cfg, 23, std=0.1)
    ids = np.random.RandomState(2).randint(0, cfg.vocab_size, size=(2, 29))
    compare_lm(cfg, params, ids, [LXT, DEFAULT, GAMMA])


@pytest.mark.parametrize("kw", [dict(sliding_layers=0, head_dim=16, num_heads=6, num_kv_heads=2),
                                dict(rope_scaling=2, rope_factor=8.0, rope_low_freq_factor=1.0,
                                     rope_high_freq_factor=4.0, rope_original_max_position=8, sliding_window=0),
                                dict(hidden_act=0, qk_norm=1, post_norms=0, norm_weight_offset=0.0, embed_scale=0.0,
                                     sliding_window=0, rope_scaling=0)])
def test_variant_lms_match_oracle(kw):
    """A window on every layer on the fused-size head_dim (Mistral's form), llama3 RoPE scaling, and
    a Qwen3-style model (QK-Norm alone)."""
    cfg = gemma_config(**kw)
    params = oc.synthetic_params(cfg, 31, std=0.1)
    ids = np.random.RandomState(5).randint(0, cfg.vocab_size, size=(2, 23))
    compare_lm(cfg, params, ids, [LXT])


def gemma_270m(**kw):
    """Gemma-3-270m's widths: hidden 640, 4 query / 1 KV heads of 256, FFN 2048 GeGLU, vocab 262144,
    RMSNorm eps 1e-6, query_pre_attn_scalar 256, RoPE 1e6 globally and 1e4 on the sliding layers
    (window 512), sandwich norms, (1 + w) norms, embeddings scaled by sqrt(640)."""
    base = dict(vocab_size=262144, hidden_size=640, num_layers=2, num_heads=4, num_kv_heads=1, head_dim=256,
                intermediate_size=2048, rms_norm_eps=1e-6, rope_theta=1e6, hidden_act=1, qk_norm=1, post_norms=1,
                norm_weight_offset=1.0, embed_scale=float(np.float32(np.sqrt(640.0))), query_pre_attn_scalar=256.0,
                rope_local_base=10000.0, sliding_window=512, sliding_layers=0b01)
    base.update(kw)
    return oc.model_config(**base)


def test_gemma3_270m_widths_match_oracle():
    """head_dim 256 (the unfused attention and the row-wise RoPE rule), the 262144-entry tied head,
    one sliding and one full layer, 2 x 80 tokens, under LXT."""
    cfg = gemma_270m()
    params = oc.synthetic_params(cfg, 270)
    ids = np.random.RandomState(6).randint(0, cfg.vocab_size, size=(2, 80))
    compare_lm(cfg, params, ids, [LXT])


def test_gemma3_270m_block_rules_match_oracle():
    """One Gemma-3-270m block (head_dim 256) under Gamma and ZBox, whose attention relevance runs in
    the relevance-only mode through the row-wise RoPE rule; eps 0.1 keeps the oracle stable under
    N(0, 1) relevance seeds."""
    cfg = gemma_270m(num_layers=1, vocab_size=0)
    params = oc.synthetic_params(cfg, 7, std=0.05, block=True)
    x = oc.fill_normal(2 * 40 * 640, 9, 1.0).reshape(2, 40, 640)
    ref, gpu = oc.oracle().block(cfg, params), models.Block(to_px(cfg), params)
    G.assert_close(gpu.forward(x), ref.forward(x), 1e-4, "forward")
    seed = oc.fill_normal(x.size, 12, 1.0).reshape(x.shape)
    for name, c in (("gamma", oc.lrp_rule(oc.GAMMA, epsilon=0.1, gamma=0.25)),
                    ("zbox", oc.lrp_rule(oc.ZBOX, epsilon=0.1, low=-4.0, high=4.0)),
                    ("lxt-style eps 0.1", oc.lrp_rule(oc.EPSILON, epsilon=0.1, bias_in_denominator=True))):
        expect_relevance_agrees(gpu.relevance_rule(seed, c), ref.relevance_rule(seed, c), "block " + name)


def test_rms_norm_heads_matches_oracle_rows():
    """QK-Norm's kernel: each head's D values of head-packed rows, strided in and out."""
    rows, heads, D, ld_in, ld_out = 37, 3, 40, 130, 125
    x = G.uniform((rows, ld_in), 1, -2, 2)
    gamma = G.uniform((D,), 2, 0.5, 1.5)
    out = G.empty((rows, ld_out), 0.0)
    N.call("pxk_rms_norm_heads", G.ptr(G.dev(x)), ld_in, G.ptr(out), ld_out, G.ptr(G.dev(gamma)), rows, heads, D,
           1e-6, G.stream())
    got = G.host(out)
    want = np.zeros_like(got)
    for h in range(heads):
        seg = np.ascontiguousarray(x[:, h * D:(h + 1) * D])
        o = np.empty_like(seg)
        rms = np.empty(rows, np.float32)
        G.oracle_call("pxo_rms_norm_forward", seg, gamma, o, rms, rows, D, 1e-6)
        want[:, h * D:(h + 1) * D] = o
    G.assert_close(got, want, 1e-5, "rms_norm_heads")
