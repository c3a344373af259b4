"""Batched KV-cached greedy decode and the AttnLRP explanation of every generated token on the
MI355X path (CausalLM::generate_greedy_device / explain_generated_device through the C ABI), against
the oracle's greedy decode (a full forward over the whole sequence each step, MakeNextTokenLogits,
generation.cpp:160-187) and the oracle's relevance of each prefix seeded at its last row.

Gates: generated ids bit-exact where the oracle's top-2 margin is at least 1e-3 of max(1, max|logit|)
(the cases are chosen so); picked logits within 1e-4 * max(1, |logit|); relevance per
ExpectRelevanceAgrees (tests/gpu_training_equivalence_cases.hpp:528-549).
"""
import numpy as np
import pytest

import decode_cases as dc
import gpu_util as G
import oracle_ctypes as oc
from pulsatrix_amd import models
from pulsatrix_amd import native as N
from test_model_gpu import LXT_EPS, expect_relevance_agrees, to_px
from test_oracle import gemma_config

pytestmark = pytest.mark.gpu
LXT = oc.lrp_rule(oc.EPSILON, epsilon=LXT_EPS, bias_in_denominator=True)


def generate(lm, prompts, new_tokens, extra=0):
    n, p = prompts.shape
    ld = p + new_tokens + extra
    ids = np.full((n, ld), -1.0, np.float32)
    ids[:, :p] = prompts
    ids_d = G.dev(ids)
    picked = G.empty((n, ld), 0.0)
    lm.generate_device(G.ptr(ids_d), n, p, new_tokens, ld, G.ptr(picked))
    models.synchronize()
    return ids_d, G.host(ids_d), G.host(picked)


@pytest.mark.parametrize("name", sorted(dc.CASES))
def test_generate_matches_oracle_greedy(name):
    cfg, params, prompts, new = dc.case(name)
    want, want_logit, margin = dc.oracle_greedy(cfg, params, prompts, new)
    assert margin > 1e-3, "the case needs a clear greedy path"
    lm = models.CausalLM(to_px(cfg), params)
    _, ids, picked = generate(lm, prompts, new, extra=3)
    p = prompts.shape[1]
    np.testing.assert_array_equal(ids[:, :p + new].astype(np.int64), want)
    assert np.all(ids[:, p + new:] == -1.0), "nothing is written past the new tokens"
    got = picked[:, p:p + new]
    assert np.all(np.abs(got - want_logit) <= 1e-4 * np.maximum(1.0, np.abs(want_logit)))


def test_sliding_window_spanning_several_key_chunks():
    """A window of 100 keys over up to 239 positions (150-token prompts, 90 new tokens) on a Gemma 3
    variant whose layers 0 and 2 slide: at the last steps the query sees keys 140-239, so the
    64-key chunks 0 and 1 hold nothing visible (empty partials the merge skips), chunk 2 is cut by
    the window and chunk 3 by the position. Greedy ids against the oracle's uncached decode, the
    picked logits within 1e-4."""
    cfg = gemma_config(vocab_size=300, sliding_window=100)
    params = oc.synthetic_params(cfg, 64, std=0.05)
    prompts = np.random.RandomState(9).randint(0, 300, size=(2, 150))
    new = 90
    want, want_logit, margin = dc.oracle_greedy(cfg, params, prompts, new)
    assert margin > 1e-3, "the case needs a clear greedy path"
    lm = models.CausalLM(to_px(cfg), params)
    _, ids, picked = generate(lm, prompts, new)
    p = prompts.shape[1]
    np.testing.assert_array_equal(ids[:, :p + new].astype(np.int64), want)
    got = picked[:, p:p + new]
    assert np.all(np.abs(got - want_logit) <= 1e-4 * np.maximum(1.0, np.abs(want_logit)))


def test_generate_is_deterministic_and_handles_short_runs():
    """Replays of one captured step reproduce an eager run; 1 and 2 new tokens take the paths
    without a graph."""
    cfg, params, prompts, new = dc.case("llama")
    lm = models.CausalLM(to_px(cfg), params)
    a = generate(lm, prompts, new)[1]
    b = generate(lm, prompts, new)[1]
    np.testing.assert_array_equal(a, b)
    p = prompts.shape[1]
    for t in (1, 2):
        np.testing.assert_array_equal(generate(lm, prompts, t)[1][:, :p + t], a[:, :p + t])


def oracle_prefix_relevance(cfg, params, ids, l, rule):
    """The oracle's token relevance of the prefix ids[:, :l], seeded at its last row with the next id
    and its logit (LRPSeed::OutputValue)."""
    ref = oc.oracle().lm(cfg, params)
    logits = ref.forward(ids[:, :l].astype(np.int64))
    seed = np.zeros_like(logits)
    for b in range(ids.shape[0]):
        t = int(ids[b, l])
        seed[b, -1, t] = logits[b, -1, t]
    return ref.relevance_rule(seed, rule)[1]


@pytest.mark.parametrize("name", sorted(dc.CASES))
def test_explain_generated_matches_oracle(name):
    cfg, params, prompts, new = dc.case(name)
    lm = models.CausalLM(to_px(cfg), params)
    ids_d, ids, _ = generate(lm, prompts, new)
    n, p = prompts.shape
    W = p + new - 1
    out = G.empty((new, n, W))
    lm.explain_generated_device(G.ptr(ids_d), n, p, new, ids.shape[1], LXT, G.ptr(out))
    rel = G.host(out)
    for t in (0, new // 2, new - 1):
        l = p + t
        expect_relevance_agrees(rel[t][:, :l], oracle_prefix_relevance(cfg, params, ids, l, LXT), "token %d" % t)
        assert np.all(rel[t][:, l:] == 0.0)


@pytest.mark.parametrize("name", sorted(dc.CASES))
def test_grouped_explanation_matches_single_prefix_passes(name):
    """explain_generated_device runs consecutive tokens as seeded copies of their longest prefix; each
    token's relevance against explain_rows_device over its own prefix alone, for every token."""
    cfg, params, prompts, new = dc.case(name)
    lm = models.CausalLM(to_px(cfg), params)
    ids_d, ids, _ = generate(lm, prompts, new)
    n, p = prompts.shape
    ld, W = ids.shape[1], p + new - 1
    out = G.empty((new, n, W))
    lm.explain_generated_device(G.ptr(ids_d), n, p, new, ld, LXT, G.ptr(out))
    grouped = G.host(out)
    for t in range(new):
        l = p + t
        pid = G.dev(np.ascontiguousarray(ids[:, :l]))
        tg = G.dev(np.ascontiguousarray(ids[:, l]))
        rows = G.empty((n * l,))
        lm.explain_rows_device(G.ptr(pid), n, l, G.ptr(tg), 1, LXT, G.ptr(rows))
        expect_relevance_agrees(grouped[t][:, :l], G.host(rows).reshape(n, l), "token %d" % t)
        assert np.all(grouped[t][:, l:] == 0.0)


@pytest.mark.parametrize("name", ["llama", "gemma"])
def test_grouped_explanation_under_gamma_matches_single_prefix_passes(name):
    """The shared-forward groups under Zennit's Gamma (whose rule reads the MLP's hidden and gate
    activations and the stacked weights) against single-prefix passes, every third token."""
    cfg, params, prompts, new = dc.case(name)
    lm = models.CausalLM(to_px(cfg), params)
    ids_d, ids, _ = generate(lm, prompts, new)
    n, p = prompts.shape
    ld, W = ids.shape[1], p + new - 1
    gamma = oc.lrp_rule(oc.GAMMA, epsilon=0.1, gamma=0.25)
    out = G.empty((new, n, W))
    lm.explain_generated_device(G.ptr(ids_d), n, p, new, ld, gamma, G.ptr(out))
    grouped = G.host(out)
    for t in range(0, new, 3):
        l = p + t
        pid = G.dev(np.ascontiguousarray(ids[:, :l]))
        tg = G.dev(np.ascontiguousarray(ids[:, l]))
        rows = G.empty((n * l,))
        lm.explain_rows_device(G.ptr(pid), n, l, G.ptr(tg), 1, gamma, G.ptr(rows))
        expect_relevance_agrees(grouped[t][:, :l], G.host(rows).reshape(n, l), "token %d" % t)
        assert np.all(grouped[t][:, l:] == 0.0)


def test_explain_rows_matches_the_dense_explain():
    """Seeding the last rows only (the head on n rows) against the dense explain_device (the head on
    every row) for the same targets, under LXT and Gamma."""
    torch = G.torch_cuda()
    cfg, params, prompts, _ = dc.case("llama")
    lm = models.CausalLM(to_px(cfg), params)
    n, l = prompts.shape
    ids_d = G.dev(prompts.astype(np.float32))
    targets = np.array([3, 77, 499])
    tg = G.dev(targets.astype(np.float32))
    for rule in (LXT, oc.lrp_rule(oc.GAMMA, gamma=0.25)):
        dense = G.empty((n * l,))
        tgt = G.keep(torch.zeros(n, dtype=torch.int64, device="cuda"))
        lm.explain_device_rule(G.ptr(ids_d), n, l, rule, G.ptr(dense), G.ptr(tgt), targets=targets)
        rows = G.empty((n * l,))
        tgt2 = G.keep(torch.zeros(n, dtype=torch.int64, device="cuda"))
        lm.explain_rows_device(G.ptr(ids_d), n, l, G.ptr(tg), 1, rule, G.ptr(rows), G.ptr(tgt2))
        models.synchronize()
        np.testing.assert_array_equal(G.host(tgt2), targets)
        expect_relevance_agrees(G.host(rows), G.host(dense), "rows vs dense")


def test_gemma3_270m_widths_generate_and_explain():
    """Gemma-3-270m's widths (head_dim 256, vocab 262144, a sliding and a full layer), 2 sequences:
    greedy ids against the oracle and the last token's explanation."""
    from test_gemma_gpu import gemma_270m

    cfg = gemma_270m()
    params = oc.synthetic_params(cfg, 270, std=0.05)
    prompts = np.random.RandomState(9).randint(0, cfg.vocab_size, size=(2, 10))
    new = 5
    want, _, margin = dc.oracle_greedy(cfg, params, prompts, new)
    assert margin > 1e-3
    lm = models.CausalLM(to_px(cfg), params)
    ids_d, ids, _ = generate(lm, prompts, new)
    np.testing.assert_array_equal(ids.astype(np.int64), want)
    out = G.empty((new, 2, 10 + new - 1))
    lm.explain_generated_device(G.ptr(ids_d), 2, 10, new, ids.shape[1], LXT, G.ptr(out))
    l = 10 + new - 1
    expect_relevance_agrees(G.host(out)[new - 1][:, :l], oracle_prefix_relevance(cfg, params, ids, l, LXT), "last")


def test_full_gemma3_270m_decode_job_properties():
    """The whole decode workload at its full size (Gemma-3-270m shape: 18 layers, 5 sliding : 1 full,
    vocab 262144; batch 4, 64-token prompts, 256 new tokens), checked by properties that hold at any
    size: every cached greedy pick is the first maximum of the uncached forward's logits over the
    same ids (MakeNextTokenLogits), wherever that row's top-2 margin leaves the order decided, with
    the picked logit within 1e-4; and three generated tokens' grouped explanations equal
    explain_rows_device over their prefixes alone."""
    n, p, T = 4, 64, 256
    cfg = N.model_config(vocab_size=262144, hidden_size=640, num_layers=18, num_heads=4, num_kv_heads=1,
                         head_dim=256, intermediate_size=2048, rms_norm_eps=1e-6, rope_theta=1e6, hidden_act=1,
                         qk_norm=1, post_norms=1, norm_weight_offset=1.0,
                         embed_scale=float(np.float32(np.sqrt(640.0))), query_pre_attn_scalar=256.0,
                         rope_local_base=10000.0, sliding_window=512,
                         sliding_layers=sum(1 << i for i in range(18) if i % 6 != 5))
    lm = models.CausalLM(cfg, seed=1234, std=0.02)
    prompts = np.random.RandomState(1234).randint(0, cfg.vocab_size, size=(n, p))
    ids_d, ids, picked = generate(lm, prompts, T)
    seq = ids.astype(np.int64)
    logits = lm.forward(seq[:, :p + T - 1])[:, p - 1:]  # rows predicting columns p .. p + T - 1
    want = logits.argmax(-1)
    two = np.partition(logits, cfg.vocab_size - 2, axis=-1)[..., -2:]
    first, second = two.max(-1), two.min(-1)
    scale = np.maximum(1.0, np.abs(logits).max(-1))
    decided = (first - second) > 1e-4 * scale
    got = seq[:, p:]
    assert decided.mean() > 0.9
    np.testing.assert_array_equal(got[decided], want[decided])
    chosen = np.take_along_axis(logits, got[..., None], -1)[..., 0]
    assert np.all(np.abs(chosen - first) <= 1e-4 * scale)  # an undecided pick is still a maximum
    assert np.all(np.abs(picked[:, p:] - chosen) <= 1e-4 * scale)
    W = p + T - 1
    out = G.empty((T, n, W))
    lm.explain_generated_device(G.ptr(ids_d), n, p, T, ids.shape[1], LXT, G.ptr(out))
    rel = G.host(out)
    for t in (0, 137, T - 1):
        l = p + t
        pid = G.dev(np.ascontiguousarray(ids[:, :l]))
        tg = G.dev(np.ascontiguousarray(ids[:, l]))
        rows = G.empty((n * l,))
        lm.explain_rows_device(G.ptr(pid), n, l, G.ptr(tg), 1, LXT, G.ptr(rows))
        expect_relevance_agrees(rel[t][:, :l], G.host(rows).reshape(n, l), "token %d" % t)
        assert np.all(rel[t][:, l:] == 0.0)


def test_generate_errors_follow_the_reference():
    cfg, params, prompts, _ = dc.case("llama")
    lm = models.CausalLM(to_px(cfg), params)
    ids = G.dev(np.zeros((3, 8), np.float32))
    with pytest.raises(N.PxkError, match="must hold the prompt and every new token"):
        lm.generate_device(G.ptr(ids), 3, 7, 4, 8)
    bidir = models.CausalLM(to_px(oc.model_config(**{**{f: getattr(cfg, f) for f, _ in cfg._fields_},
                                                      "causal": 0})), params)
    with pytest.raises(N.PxkError, match="attends bidirectionally"):
        bidir.generate_device(G.ptr(ids), 3, 2, 2, 8)
