"""The Generate() harness on the CPU: the compiled reference's Generate (generation.hpp:95-135) over
its own CausalLM::next_token_logits (MakeCachedNextTokenLogits, generation.cpp:189-258) through the
C callback that the MI355X tests hand the product's pxa_lm_next_token_logits to. Its greedy ids
equal the oracle's uncached greedy decode (a full forward per step, MakeNextTokenLogits), so the
callback plumbing, the config fields and the result layout are pinned before any GPU runs them.
"""
import numpy as np
import pytest

import decode_cases as dc
import oracle_ctypes as oc

pytestmark = pytest.mark.skipif(oc.ref() is None, reason="oracle/_ref (compiled reference) not built here")


@pytest.mark.parametrize("name", sorted(dc.CASES))
def test_reference_cached_generate_matches_oracle_greedy(name):
    cfg, params, prompts, new = dc.case(name)
    want, _, margin = dc.oracle_greedy(cfg, params, prompts, new)
    assert margin > 1e-3
    lm = oc.ref().lm(cfg, params)
    p = prompts.shape[1]
    for b in range(prompts.shape[0]):
        toks, logp, fin = oc.ref_generate(oc.RefNextToken(lm, p + new), cfg.vocab_size, prompts[b], new)
        assert fin == "length" and len(toks) == new
        np.testing.assert_array_equal(toks, want[b, p:])
        assert np.all(logp <= 0.0) and np.all(np.isfinite(logp))


def test_reference_generate_stops_at_eos_and_reports_it():
    cfg, params, prompts, new = dc.case("llama")
    want, _, _ = dc.oracle_greedy(cfg, params, prompts[:1], new)
    p = prompts.shape[1]
    eos = int(want[0, p + 4])  # the fifth greedy token
    first = int(np.argmax(want[0, p:] == eos))
    lm = oc.ref().lm(cfg, params)
    toks, _, fin = oc.ref_generate(oc.RefNextToken(lm, p + new), cfg.vocab_size, prompts[0], new, eos=(eos,))
    assert fin == "eos"
    np.testing.assert_array_equal(toks, want[0, p:p + first + 1])


def test_reference_next_token_logits_follow_the_history():
    """The reference's cached function against the oracle's forward over each sequence: an
    extension, the same sequence, a prefix, a new prompt."""
    cfg, params, prompts, _ = dc.case("llama")
    f = oc.RefNextToken(oc.ref().lm(cfg, params), 32)
    o = oc.oracle().lm(cfg, params)
    s = [int(t) for t in prompts[0]]
    for seq in (s, s + [3, 9], s + [3, 9], s[:4], [int(t) for t in prompts[1]]):
        want = o.forward(np.asarray(seq, np.int64)[None])[0, -1]
        got = f(seq)
        assert np.abs(got - want).max() <= 1e-4 * max(1.0, float(np.abs(want).max()))
