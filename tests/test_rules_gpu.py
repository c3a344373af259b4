"""The Zennit-compatible affine rules (Gamma, AlphaBeta, ZBox; src/lrp_rules.cpp:72-160) on the
MI355X path, called through the C ABI, against the oracle (itself pinned in test_oracle_rules.py to
hand-computed answers, the Zennit 1.0.0 values and the compiled reference) and against those same
hand-computed and Zennit answers directly.

Gates: the hand-computed single-output answers at 1e-5; the Zennit MLP values at the reference's
tolerance (lrp_reference_test.cpp:85-91); everything else per ExpectRelevanceAgrees
(tests/gpu_training_equivalence_cases.hpp:528-549): every element within 1e-3 * max|R_cpu|, sums
within 1e-3 * sum|R_cpu|, no sign flip where |R_cpu| > 1% of max|R_cpu|.
"""
import numpy as np
import pytest

import gpu_util as G
import oracle_ctypes as oc
import rules_cases as rc
from pulsatrix_amd import models
from pulsatrix_amd import native as N
from test_model_gpu import argmax_seed, expect_logits_agree, expect_relevance_agrees, small_lm_config, to_px

pytestmark = pytest.mark.gpu

RULES = rc.all_rules()[1:]  # the epsilon rule has its own tests; these are the three others, four settings


@pytest.fixture(autouse=True)
def _fresh_rules():
    """Tests may change a rule's epsilon; every test starts from the shared settings."""
    global RULES
    RULES = rc.all_rules()[1:]
    yield


def gpu_rule(x, w, b, r, c):
    return models.linear_relevance_rule(x, w, b, r, c)[1]


@pytest.mark.parametrize("case", range(len(rc.SINGLE_CASES)))
def test_linear_rules_known_answers(case):
    _, c, want = rc.SINGLE_CASES[case]
    got = gpu_rule(rc.SINGLE_X, rc.SINGLE_W, rc.SINGLE_B, np.ones((1, 1), np.float32), c)
    np.testing.assert_allclose(got[0], want, rtol=1e-5, atol=1e-6)


def test_gamma_uses_the_negative_pair_for_negative_outputs():
    got = gpu_rule(rc.SINGLE_X, rc.NEG_W, rc.NEG_B, rc.NEG_R, rc.rule(rc.G, gamma=0.5))
    np.testing.assert_allclose(got[0], rc.NEG_EXPECTED, rtol=1e-5, atol=1e-6)


def gpu_mlp_relevance(c):
    """The reference's three-layer MLP explained under `c` on the device, ReLU (identity rule) on the host."""
    x = rc.mlp_input()
    cache = []
    for i, (w, b) in enumerate(rc.mlp_params()):
        y, _ = models.linear_relevance_rule(x, w, b, np.zeros((x.shape[0], w.shape[1]), np.float32), c)
        cache.append((x, w, b))
        x = np.maximum(y, 0.0) if i < 2 else y
    r = rc.mlp_seed()
    for x, w, b in reversed(cache):
        r = gpu_rule(x, w, b, r, c)
    return r


@pytest.mark.parametrize("case", range(8))
def test_linear_rules_match_zennit_mlp(case):
    _, c, key = rc.mlp_cases()[case]
    rc.expect_reference_close(gpu_mlp_relevance(c), rc.zennit_values()[key])


@pytest.mark.parametrize("case", range(len(RULES)))
@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("shape", [(5, 23, 17), (64, 96, 80), (512, 576, 1536), (300, 1536, 577)])
def test_linear_rules_match_oracle(case, bias, shape):
    """Ragged and full-width layers (512 x 576 -> 1536 is the S MLP's gate) against the oracle; the
    inputs sit inside ZBox's box, so every rule's denominators keep one sign per term."""
    _, c = RULES[case]
    n, i, o = shape
    rng = np.random.RandomState(7 * case + bias + i)
    x = rng.uniform(-1, 1, (n, i)).astype(np.float32)
    w = rng.uniform(-1, 1, (i, o)).astype(np.float32) / np.sqrt(i)
    b = rng.uniform(-0.5, 0.5, o).astype(np.float32) if bias else None
    r = rng.uniform(-1, 1, (n, o)).astype(np.float32)
    y, got = models.linear_relevance_rule(x, w, b, r, c)
    pre, y_ref = oc.linear_forward(x, w, b)
    G.assert_close(y, y_ref, 1e-4, "forward")
    expect_relevance_agrees(got, oc.linear_relevance_rule(x, w, b, pre, r, c), "%s %s" % (RULES[case][0], shape))


def test_alpha_beta_conserves_without_bias():
    """AlphaBeta with alpha - beta = 1 and no bias conserves each row's relevance exactly (up to
    rounding): a property the reference's rule has whatever the sizes."""
    rng = np.random.RandomState(11)
    x = rng.uniform(-1, 1, (64, 576)).astype(np.float32)
    w = rng.uniform(-1, 1, (576, 1536)).astype(np.float32) / 24
    r = rng.uniform(0, 1, (64, 1536)).astype(np.float32)
    for a, b in ((1.0, 0.0), (2.0, 1.0)):
        got = gpu_rule(x, w, None, r, rc.rule(rc.AB, alpha=a, beta=b))
        np.testing.assert_allclose(got.sum(1), r.sum(1), rtol=2e-4)


def test_gamma_zero_is_epsilon_with_bias_and_zero_box_is_pre_bias_epsilon():
    x, w, b, r = rc.BATCH_X, rc.BATCH_W, rc.BATCH_B, rc.BATCH_R
    np.testing.assert_allclose(gpu_rule(x, w, b, r, rc.rule(rc.G, gamma=0.0)), gpu_rule(x, w, b, r, rc.eps_bias()),
                               atol=1e-5)
    np.testing.assert_allclose(gpu_rule(x, w, b, r, rc.rule(rc.ZB, low=0.0, high=0.0)),
                               gpu_rule(x, w, b, r, oc.lrp_rule(rc.E)), atol=1e-5)


@pytest.mark.parametrize("alpha,beta,msg", [(2.0, 0.0, "alpha - beta == 1"), (-1.0, -2.0, "alpha >= 0 and beta >= 0")])
def test_invalid_alpha_beta_throws_the_reference_message(alpha, beta, msg):
    with pytest.raises(N.PxkError, match="LinearModule::propagate_relevance: AlphaBeta rule needs " + msg):
        gpu_rule(rc.SINGLE_X, rc.SINGLE_W, rc.SINGLE_B, np.ones((1, 1), np.float32),
                 rc.rule(rc.AB, alpha=alpha, beta=beta))


def oracle_rule_sensitivity(cfg, params, x, seed, c, trials=3):
    """Largest relative change of the oracle's block relevance under `c` when params and x move by
    ~2e-7 relative (float32 rounding): the attention, SwiGLU and residual rules divide by
    activations with only the rule's epsilon as a stabilizer, so a parity case must first show
    that the oracle itself is stable there."""
    ref = oc.oracle().block(cfg, params)
    ref.forward(x)
    r0 = ref.relevance_rule(seed, c)
    worst = 0.0
    for t in range(trials):
        rs = np.random.RandomState(200 + t)
        p2 = (params * (1 + 2e-7 * rs.standard_normal(params.shape))).astype(np.float32)
        x2 = (x * (1 + 2e-7 * rs.standard_normal(x.shape))).astype(np.float32)
        other = oc.oracle().block(cfg, p2)
        other.forward(x2)
        worst = max(worst, float(np.abs(other.relevance_rule(seed, c) - r0).max() / np.abs(r0).max()))
    return worst


@pytest.mark.parametrize("biased", [True, False])
def test_block_rules_match_oracle(biased):
    """A block under every rule: the projections take the rule, the attention and SwiGLU products
    and the residual splits take epsilon. With biases the MLP runs its unfused gate; head_dim 24
    rotates outside the projection GEMM. Under seeded N(0, 1) relevance the epsilon-only rules are
    ill-conditioned at eps 1e-6 (the oracle moves by more than the gate under rounding-level input
    changes); eps 0.1 keeps the oracle stable, which each case checks first."""
    kw = dict(qkv_bias=1, out_bias=1, mlp_bias=1) if biased else {}
    cfg = oc.model_config(hidden_size=96, num_heads=4, num_kv_heads=2, head_dim=24, intermediate_size=64,
                          rope_theta=10000.0, **kw)
    params = oc.synthetic_params(cfg, 31, std=0.1, block=True)
    x = oc.fill_normal(2 * 19 * 96, 9, 1.0).reshape(2, 19, 96)
    ref, gpu = oc.oracle().block(cfg, params), models.Block(to_px(cfg), params)
    G.assert_close(gpu.forward(x), ref.forward(x), 1e-4, "forward")
    seed = oc.fill_normal(x.size, 12, 1.0).reshape(x.shape)
    for name, c in RULES:
        c.epsilon = 0.1
        assert oracle_rule_sensitivity(cfg, params, x, seed, c) < 1e-4, name
        expect_relevance_agrees(gpu.relevance_rule(seed, c), ref.relevance_rule(seed, c), "block " + name)


def oracle_lm_sensitivity(cfg, params, ids, seed, c, trials=2):
    """As oracle_rule_sensitivity, for a causal LM's embedding-level relevance (weights moved by
    ~2e-7 relative)."""
    ref = oc.oracle().lm(cfg, params)
    ref.forward(ids)
    r0 = ref.relevance_rule(seed, c)[0]
    worst = 0.0
    for t in range(trials):
        rs = np.random.RandomState(300 + t)
        other = oc.oracle().lm(cfg, (params * (1 + 2e-7 * rs.standard_normal(params.shape))).astype(np.float32))
        other.forward(ids)
        worst = max(worst, float(np.abs(other.relevance_rule(seed, c)[0] - r0).max() / np.abs(r0).max()))
    return worst


@pytest.mark.parametrize("tied", [1, 0])
@pytest.mark.parametrize("case", range(len(RULES)))
def test_causal_lm_rules_match_oracle(tied, case):
    """The whole LM: the head (tied: on E^T in place) and every projection under the rule, key and
    value relevance included. ZBox's box does not hold the normalised activations, so some of its
    denominators cross zero: at eps 1e-6 the oracle itself moves by ~1e-3 under rounding-level
    weight changes, at eps 1e-2 by ~1e-7. Each case checks the oracle's stability first."""
    name, c = RULES[case]
    if c.rule == rc.ZB:
        c.epsilon = 1e-2
    cfg = small_lm_config(tie_word_embeddings=tied)
    params = oc.synthetic_params(cfg, 99 + case)
    ids = np.random.RandomState(3).randint(0, cfg.vocab_size, size=(2, 37))
    ref, gpu = oc.oracle().lm(cfg, params), models.CausalLM(to_px(cfg), params)
    lr, lg = ref.forward(ids), gpu.forward(ids)
    expect_logits_agree(lg, lr, "logits")
    seed = argmax_seed(lr)
    assert oracle_lm_sensitivity(cfg, params, ids, seed, c) < 1e-4, name
    a = gpu.relevance_rule(seed, c, want_kv=True)
    b = ref.relevance_rule(seed, c, want_kv=True)
    for what, u, v in zip(("embedding", "tokens", "keys", "values"), a, b):
        expect_relevance_agrees(u, v, "%s %s tied=%d" % (what, name, tied))


def test_causal_lm_rule_errors_name_the_head():
    cfg = small_lm_config()
    gpu = models.CausalLM(to_px(cfg), oc.synthetic_params(cfg, 1))
    logits = gpu.forward(np.arange(8).reshape(1, 8))
    with pytest.raises(N.PxkError, match="TiedLMHeadModule::propagate_relevance: AlphaBeta rule needs alpha - beta"):
        gpu.relevance_rule(argmax_seed(logits), rc.rule(rc.AB, alpha=3.0, beta=1.0))


def test_rule_weights_follow_weight_and_rule_changes():
    """The stacked weights are cached per layer: a second rule, a new gamma and new weights must each
    be seen (the cache key), matching the oracle every time."""
    cfg = small_lm_config(num_layers=1, vocab_size=300)
    ids = np.random.RandomState(5).randint(0, 300, size=(1, 21))
    p1, p2 = oc.synthetic_params(cfg, 1), oc.synthetic_params(cfg, 2)
    gpu = models.CausalLM(to_px(cfg), p1)
    logits = gpu.forward(ids)
    seed = argmax_seed(logits)
    ref = oc.oracle().lm(cfg, p1)
    ref.forward(ids)
    for c in (rc.rule(rc.G, gamma=0.25), rc.rule(rc.G, gamma=1.0), rc.rule(rc.ZB, low=-2.0, high=2.0),
              rc.rule(rc.G, gamma=0.25)):
        expect_relevance_agrees(gpu.relevance_rule(seed, c)[0], ref.relevance_rule(seed, c)[0], "rule change")
    gpu2 = models.CausalLM(to_px(cfg), p2)
    ref2 = oc.oracle().lm(cfg, p2)
    seed2 = argmax_seed(ref2.forward(ids))
    gpu2.forward(ids)
    c = rc.rule(rc.G, gamma=0.25)
    expect_relevance_agrees(gpu2.relevance_rule(seed2, c)[0], ref2.relevance_rule(seed2, c)[0], "second model")


@pytest.mark.parametrize("case", [0, 2, 3])
def test_explain_device_rule_and_graph_replay_match_host_path(case):
    """The device hot path under a rule, eagerly and replayed from a HIP graph several times with
    other eager work in between, against the host-tensor path."""
    torch = G.torch_cuda()
    _, c = RULES[case]
    cfg = small_lm_config()
    params = oc.synthetic_params(cfg, 5)
    lm = models.CausalLM(to_px(cfg), params)
    ids = np.random.RandomState(4).randint(0, cfg.vocab_size, size=(3, 29))
    logits = lm.forward(ids)
    _, r_tok = lm.relevance_rule(argmax_seed(logits), c)
    ids_d = G.dev(ids.astype(np.float32))
    tok = G.empty((3, 29))
    tgt = G.keep(torch.zeros(3, dtype=torch.int64, device="cuda"))
    lm.explain_device_rule(G.ptr(ids_d), 3, 29, c, G.ptr(tok), G.ptr(tgt))
    models.synchronize()
    eager = G.host(tok)
    np.testing.assert_array_equal(G.host(tgt), logits[:, -1].argmax(-1))
    expect_relevance_agrees(eager, r_tok, "explain_device")
    lm.capture_explain_rule(G.ptr(ids_d), 3, 29, c, G.ptr(tok), G.ptr(tgt))
    for _ in range(3):
        tok.fill_(float("nan"))
        models.synchronize()
        lm.replay()
        models.synchronize()
        np.testing.assert_array_equal(G.host(tok), eager)
        lm.forward(ids)  # eager work between the replays


def test_smollm2_widths_gamma_matches_oracle():
    """SmolLM2-135M widths and vocab (576 hidden, 9/3 heads, FFN 1536, 49152 tokens, tied), two
    layers, 64 tokens: the Gamma rule through the full-size head and projections."""
    cfg = oc.model_config(vocab_size=49152, hidden_size=576, num_layers=2, num_heads=9, num_kv_heads=3,
                          head_dim=64, intermediate_size=1536, rms_norm_eps=1e-5, rope_theta=100000.0)
    params = oc.synthetic_params(cfg, 77)
    ids = np.random.RandomState(8).randint(0, 49152, size=(1, 64))
    ref, gpu = oc.oracle().lm(cfg, params), models.CausalLM(to_px(cfg), params)
    lr, lg = ref.forward(ids), gpu.forward(ids)
    expect_logits_agree(lg, lr, "logits")
    seed = argmax_seed(lr)
    c = rc.rule(rc.G, gamma=0.25)
    for what, u, v in zip(("embedding", "tokens"), gpu.relevance_rule(seed, c), ref.relevance_rule(seed, c)):
        expect_relevance_agrees(u, v, what)
