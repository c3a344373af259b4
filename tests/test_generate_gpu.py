"""The reference's Generate() on the MI355X decode path: CausalLM::next_token_logits(max_length)
(include/pulsatrix/causal_lm.hpp:116) through the C ABI (pxa_lm_next_token_logits), driven by the
compiled reference's own Generate (generation.hpp:95-135, oracle/_ref) as a C callback.

Gates: greedy ids bit-exact against the oracle's uncached greedy decode (MakeNextTokenLogits,
generation.cpp:160-187; the cases have a top-2 margin of at least 1e-3 of max(1, max|logit|)); the
same ids and log-probabilities within 1e-4 * max(1, |x|) as the reference's Generate over the
reference CausalLM's own next_token_logits on CPUBackend; next-token logits within
1e-4 * max(1, max|logit|) of the oracle's full forward after every kind of history change.
"""
import numpy as np
import pytest

import decode_cases as dc
import gpu_util as G
import oracle_ctypes as oc
from pulsatrix_amd import models
from pulsatrix_amd import native as N
from test_model_gpu import LXT_EPS, to_px

pytestmark = pytest.mark.gpu


def need_ref():
    if oc.ref() is None:
        pytest.fail("oracle/_ref is not built: the boundary evidence needs it "
                    "(__graft_entry__.build() builds it where the reference sources are)")


def oracle_last_logits(cfg, params, tokens):
    return oc.oracle().lm(cfg, params).forward(np.asarray(tokens, np.int64)[None])[0, -1]


def close(got, want, what):
    scale = max(1.0, float(np.abs(want).max()))
    err = float(np.abs(np.asarray(got, np.float64) - want).max())
    assert err <= 1e-4 * scale, "%s: max |diff| %.3e > 1e-4 * %.3e" % (what, err, scale)


@pytest.mark.parametrize("name", sorted(dc.CASES))
def test_reference_generate_greedy_on_mi355x_next_token_logits(name):
    need_ref()
    cfg, params, prompts, new = dc.case(name)
    want, _, margin = dc.oracle_greedy(cfg, params, prompts, new)
    assert margin > 1e-3, "the case needs a clear greedy path"
    lm = models.CausalLM(to_px(cfg), params)
    ref_lm = oc.ref().lm(cfg, params)
    p = prompts.shape[1]
    for b in range(prompts.shape[0]):
        f = lm.next_token_logits(p + new)
        toks, logp, fin = oc.ref_generate(f, cfg.vocab_size, prompts[b], new)
        assert fin == "length"
        np.testing.assert_array_equal(toks, want[b, p:], err_msg="sequence %d" % b)
        cpu = oc.RefNextToken(ref_lm, p + new)
        rtoks, rlogp, _ = oc.ref_generate(cpu, cfg.vocab_size, prompts[b], new)
        np.testing.assert_array_equal(toks, rtoks)
        close(logp, rlogp.astype(np.float64), "log-probabilities, sequence %d" % b)


def test_reference_sampling_on_mi355x_matches_its_cpu_run():
    """Seeded sampling (temperature, top-k, top-p, min-p, repetition penalty, min_new_tokens and an
    EOS id) draws the same tokens from the MI355X logits as from CPUBackend's."""
    need_ref()
    cfg, params, prompts, _ = dc.case("llama")
    lm = models.CausalLM(to_px(cfg), params)
    ref_lm = oc.ref().lm(cfg, params)
    kw = dict(min_new_tokens=3, eos=(7, 11), do_sample=True, temperature=0.8, top_k=40, top_p=0.9, min_p=0.02,
              repetition_penalty=1.3)
    for seed in (3, 1234):
        ours = oc.ref_generate(lm.next_token_logits(40), cfg.vocab_size, prompts[0], 16, seed=seed, **kw)
        cpu = oc.ref_generate(oc.RefNextToken(ref_lm, 40), cfg.vocab_size, prompts[0], 16, seed=seed, **kw)
        np.testing.assert_array_equal(ours[0], cpu[0], err_msg="seed %d" % seed)
        assert ours[2] == cpu[2]
        close(ours[1], cpu[1].astype(np.float64), "log-probabilities, seed %d" % seed)


def test_next_token_logits_follows_the_history_like_the_reference():
    """Extensions (decode steps, the second one a graph replay), the same sequence again, a prefix of
    the history, a new prompt, a long extension (one forward), and steps after unrelated work that
    reallocated the backend's buffers (the step's graph is captured again): each call's logits against
    the oracle's forward over that sequence."""
    cfg, params, prompts, _ = dc.case("llama")
    lm = models.CausalLM(to_px(cfg), params)
    f = lm.next_token_logits(40)
    rng = np.random.RandomState(5)
    s = [int(t) for t in prompts[0]]
    seqs = [s, s + [3, 9], s + [3, 9, 4], s + [3, 9, 4], s[:5], s[:5] + [8], [int(t) for t in prompts[1]]]
    seqs.append(seqs[-1] + [int(t) for t in rng.randint(0, cfg.vocab_size, 10)])
    for i, seq in enumerate(seqs):
        close(f(seq), oracle_last_logits(cfg, params, seq), "call %d (%d tokens)" % (i, len(seq)))
    # unrelated work on the same backend grows buffers the captured step uses
    big = rng.randint(0, cfg.vocab_size, size=(4, 33)).astype(np.float32)
    ids = G.dev(big)
    rel = G.empty((4, 33), 0.0)
    tg = G.torch_cuda().empty(4, dtype=G.torch_cuda().int64, device="cuda")
    lm.explain_device_rule(G.ptr(ids), 4, 33, oc.lrp_rule(oc.EPSILON, epsilon=LXT_EPS, bias_in_denominator=True),
                           G.ptr(rel), G.ptr(G.keep(tg)))
    models.synchronize()
    seq = seqs[-1]
    for t in (2, 6, 1):
        seq = seq + [t]
        close(f(seq), oracle_last_logits(cfg, params, seq), "after other work (%d tokens)" % len(seq))


def test_next_token_logits_errors_follow_the_reference():
    cfg, params, _, _ = dc.case("llama")
    lm = models.CausalLM(to_px(cfg), params)
    f = lm.next_token_logits(6)
    with pytest.raises(N.PxkError, match="MakeCachedNextTokenLogits: the sequence is empty"):
        f([])
    with pytest.raises(N.PxkError, match="7 tokens don't fit in caches of 6"):
        f([1] * 7)
    with pytest.raises(N.PxkError, match="index out of range"):
        f([1, cfg.vocab_size])
    with pytest.raises(N.PxkError, match="max_length must be positive"):
        lm.next_token_logits(0)
    close(f([1, 2, 3]), oracle_last_logits(cfg, params, [1, 2, 3]), "after the errors")
    bidir = dc.llama_decode_config()
    bidir.causal = 0
    with pytest.raises(N.PxkError, match="attends bidirectionally"):
        models.CausalLM(to_px(bidir), params).next_token_logits(8)
