"""Pins the oracle's Zennit-compatible affine rules (Gamma, AlphaBeta, ZBox and the
bias-in-denominator epsilon rule; src/lrp_rules.cpp:13-215) before the MI355X path is checked
against them:

* known answers worked out by hand for a one-output layer (both output signs for Gamma);
* the Zennit 1.0.0 values of the reference's MLP (tests/lrp_reference_test.cpp:285-303, committed
  as tests/golden/zennit_values.json) at the reference's tolerance;
* each rule's definition term by term in float64 (rules_cases.rule_by_definition) on the
  reference's batch layer and on random layers;
* invariants: AlphaBeta conserves without a bias, Gamma(0) is the bias-in-denominator epsilon
  rule, ZBox with a zero box is the pre-bias epsilon rule;
* bit-identical results to the compiled reference (oracle/_ref) for Linear layers, a tied-head
  causal LM and a block, under every rule.
"""
import numpy as np
import pytest

import oracle_ctypes as oc
import rules_cases as rc

needs_ref = pytest.mark.skipif(oc.ref() is None, reason="oracle/_ref (compiled reference) not built here")


def oracle_rule(x, w, b, r, c):
    pre, _ = oc.linear_forward(x, w, b)
    return oc.linear_relevance_rule(x, w, b, pre, r, c)


@pytest.mark.parametrize("case", range(len(rc.SINGLE_CASES)))
def test_oracle_rules_known_answers(case):
    _, c, want = rc.SINGLE_CASES[case]
    got = oracle_rule(rc.SINGLE_X, rc.SINGLE_W, rc.SINGLE_B, np.ones((1, 1), np.float32), c)
    np.testing.assert_allclose(got[0], want, rtol=1e-5, atol=1e-6)


def test_oracle_gamma_uses_the_negative_pair_for_negative_outputs():
    got = oracle_rule(rc.SINGLE_X, rc.NEG_W, rc.NEG_B, rc.NEG_R, rc.rule(rc.G, gamma=0.5))
    np.testing.assert_allclose(got[0], rc.NEG_EXPECTED, rtol=1e-5, atol=1e-6)


def mlp_relevance(c, relevance_fn):
    """The reference MLP explained under `c`: forward through the oracle's Linear layers with ReLU
    between them, then each layer's rule from the one-hot seed; ReLU passes relevance unchanged."""
    x = rc.mlp_input()
    cache = []
    for i, (w, b) in enumerate(rc.mlp_params()):
        pre, y = oc.linear_forward(x, w, b)
        cache.append((x, w, b, pre))
        x = np.maximum(y, 0.0) if i < 2 else y
    r = rc.mlp_seed()
    for x, w, b, pre in reversed(cache):
        r = relevance_fn(x, w, b, pre, r, c)
    return r


@pytest.mark.parametrize("case", range(8))
def test_oracle_rules_match_zennit_mlp(case):
    name, c, key = rc.mlp_cases()[case]
    rc.expect_reference_close(mlp_relevance(c, oc.linear_relevance_rule), rc.zennit_values()[key])


def test_zennit_values_reject_a_wrong_rule():
    """The goldens tell the rules apart: Gamma's values are not ZPlus's, and a sign slip in
    AlphaBeta's negative branch (alpha + beta instead of alpha - beta) fails them."""
    vals = rc.zennit_values()
    gamma = mlp_relevance(rc.rule(rc.G, gamma=0.25), oc.linear_relevance_rule)
    assert np.abs(gamma - np.reshape(vals["kMlpZPlus"], gamma.shape)).max() > 1e-2
    with pytest.raises(AssertionError):  # AlphaBeta(2, -1) stands in for the slipped sign
        bad = oc.lrp_rule(rc.AB, alpha=2.0, beta=-1.0)
        rc.expect_reference_close(mlp_relevance(bad, lambda x, w, b, pre, r, c: rc.rule_by_definition(
            x, w, b, r, c).astype(np.float32)), vals["kMlpAlphaBeta21"])


@pytest.mark.parametrize("case", range(5))
def test_oracle_rules_match_definition_on_the_batch_layer(case):
    _, c = rc.all_rules()[case]
    got = oracle_rule(rc.BATCH_X, rc.BATCH_W, rc.BATCH_B, rc.BATCH_R, c)
    want = rc.rule_by_definition(rc.BATCH_X, rc.BATCH_W, rc.BATCH_B, rc.BATCH_R, c)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("case", range(5))
@pytest.mark.parametrize("bias", [True, False])
def test_oracle_rules_match_definition_on_random_layers(case, bias):
    _, c = rc.all_rules()[case]
    rng = np.random.RandomState(case + 10 * bias)
    n, i, o = 5, 23, 17
    x = rng.uniform(-1, 1, (n, i)).astype(np.float32)
    w = rng.uniform(-1, 1, (i, o)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, o).astype(np.float32) if bias else None
    r = rng.uniform(-1, 1, (n, o)).astype(np.float32)
    got = oracle_rule(x, w, b, r, c)
    want = rc.rule_by_definition(x, w, b, r, c)
    # well-conditioned rows only: a denominator near 0 amplifies float32 rounding
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 1e-3 * scale


def test_oracle_alpha_beta_conserves_without_bias():
    x = np.array([1.0, 2.0, 0.5, 3.0, 1.5, 0.25, 2.0, 0.75], np.float32).reshape(2, 4)
    zero = np.zeros(3, np.float32)
    for a, bt in ((1.0, 0.0), (2.0, 1.0), (3.0, 2.0)):
        got = oracle_rule(x, rc.BATCH_W, zero, rc.BATCH_R, rc.rule(rc.AB, alpha=a, beta=bt))
        np.testing.assert_allclose(got.sum(1), rc.BATCH_R.sum(1), atol=1e-4)


def test_oracle_gamma_zero_is_epsilon_with_bias():
    g0 = oracle_rule(rc.BATCH_X, rc.BATCH_W, rc.BATCH_B, rc.BATCH_R, rc.rule(rc.G, gamma=0.0))
    ep = oracle_rule(rc.BATCH_X, rc.BATCH_W, rc.BATCH_B, rc.BATCH_R, rc.eps_bias())
    np.testing.assert_allclose(g0, ep, atol=1e-5)


def test_oracle_zbox_zero_box_is_pre_bias_epsilon():
    zb = oracle_rule(rc.BATCH_X, rc.BATCH_W, rc.BATCH_B, rc.BATCH_R, rc.rule(rc.ZB, low=0.0, high=0.0))
    ep = oracle_rule(rc.BATCH_X, rc.BATCH_W, rc.BATCH_B, rc.BATCH_R, oc.lrp_rule(rc.E))
    np.testing.assert_allclose(zb, ep, atol=1e-5)


@pytest.mark.parametrize("alpha,beta,msg", [(2.0, 0.0, "alpha - beta == 1"), (-1.0, -2.0, "alpha >= 0 and beta >= 0")])
def test_oracle_invalid_alpha_beta_throws(alpha, beta, msg):
    with pytest.raises(RuntimeError, match=msg):
        oracle_rule(rc.SINGLE_X, rc.SINGLE_W, rc.SINGLE_B, np.ones((1, 1), np.float32),
                    rc.rule(rc.AB, alpha=alpha, beta=beta))


@needs_ref
@pytest.mark.parametrize("case", range(5))
@pytest.mark.parametrize("bias", [True, False])
def test_oracle_rules_bit_identical_to_reference(case, bias):
    _, c = rc.all_rules()[case]
    rng = np.random.RandomState(100 + case)
    n, i, o = 7, 40, 33
    x = rng.uniform(-1, 1, (n, i)).astype(np.float32)
    w = rng.uniform(-1, 1, (i, o)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, o).astype(np.float32) if bias else None
    r = rng.uniform(-1, 1, (n, o)).astype(np.float32)
    assert np.array_equal(oracle_rule(x, w, b, r, c), oc.ref_linear_relevance_rule(x, w, b, r, c))


@needs_ref
@pytest.mark.parametrize("tied,case", [(1, 3), (1, 2), (0, 1), (1, 4)])
def test_oracle_lm_rules_bit_identical_to_reference(tied, case):
    """A causal LM under a rule: the reference hands the config to every Linear and the head."""
    cfg = oc.model_config(vocab_size=97, hidden_size=32, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=8,
                          intermediate_size=40, rope_theta=100000.0, tie_word_embeddings=tied)
    params = oc.synthetic_params(cfg, 5, std=0.1)
    ids = np.random.RandomState(2).randint(0, 97, size=(2, 9))
    o, r = oc.oracle().lm(cfg, params), oc.ref().lm(cfg, params)
    lo = o.forward(ids)
    assert np.array_equal(lo, r.forward(ids))
    seed = np.zeros_like(lo)
    for s in range(2):
        t = int(np.argmax(lo[s, -1]))
        seed[s, -1, t] = lo[s, -1, t]
    _, c = rc.all_rules()[case]
    for a, b in zip(o.relevance_rule(seed, c, want_kv=True), r.relevance_rule(seed, c, want_kv=True)):
        assert np.array_equal(a, b)


@needs_ref
def test_oracle_block_rule_bit_identical_to_reference():
    cfg = oc.model_config(hidden_size=24, num_heads=2, num_kv_heads=1, head_dim=12, intermediate_size=20,
                          qkv_bias=1, out_bias=1, mlp_bias=1)
    params = oc.synthetic_params(cfg, 4, std=0.2, block=True)
    x = oc.fill_normal(2 * 5 * 24, 6, 1.0).reshape(2, 5, 24)
    o, r = oc.oracle().block(cfg, params), oc.ref().block(cfg, params)
    y = o.forward(x)
    assert np.array_equal(y, r.forward(x))
    seed = oc.fill_normal(y.size, 8, 1.0).reshape(y.shape)
    for _, c in rc.all_rules():
        assert np.array_equal(o.relevance_rule(seed, c), r.relevance_rule(seed, c))


@pytest.mark.skipif(oc.ref() is None, reason="oracle/_ref was not built (no reference sources)")
@pytest.mark.parametrize("case", __import__("dropin_cases").explain_cases(), ids=lambda c: c[0])
def test_reference_lrp_explain_reproduces_zennit_mlp(case):
    """The harness the drop-in tests run on MI355XBackend, on the reference's own CPUBackend:
    LRP::explain over the Zennit MLP (ExplainerContext, OneHot seeds at targets {2, 1}) matches
    the Zennit 1.0.0 values; relevance_in_sum is the attribution's sum."""
    name, rule, preset, key = case
    rel, total = oc.mlp_explain(oc.ref(), rc.mlp_params(), rc.mlp_input(), rc.MLP_TARGETS, rule, preset)
    rc.expect_reference_close(rel, rc.zennit_values()[key])
    assert abs(total - float(rel.astype(np.float64).sum())) <= 1e-5 * max(1.0, abs(total))
