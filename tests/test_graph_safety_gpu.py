"""Captured explain graphs and launch logs refuse to run on device memory that has moved.

A captured graph addresses the model's buffers and the backend's shared split-K pool as they were
at capture time. Each model handle owns its graph; pxa_lm_replay checks on the host, before any
launch, that no block the graph may address has been freed since the capture (a longer pass
regrows the model's buffers, the pool grows, the model is destroyed). The same holds for the
launch log bench.py times. Every refusal here is a host-side check: nothing stale is launched.
"""
import ctypes

import numpy as np
import pytest

import gpu_util as G
import oracle_ctypes as oc
from pulsatrix_amd import models
from pulsatrix_amd import native as N

pytestmark = pytest.mark.gpu
LXT_EPS = 1e-9


def small_model():
    cfg = oc.model_config(vocab_size=1000, hidden_size=64, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=16,
                          intermediate_size=96, rms_norm_eps=1e-5, rope_theta=100000.0)
    px = N.ModelConfig(**{f: getattr(cfg, f) for f, _ in cfg._fields_})
    return cfg, models.CausalLM(px, oc.synthetic_params(cfg, 5))


def device_inputs(cfg, n, l, seed):
    torch = G.torch_cuda()
    ids = np.random.RandomState(seed).randint(0, cfg.vocab_size, size=(n, l)).astype(np.float32)
    return G.dev(ids), G.empty((n, l)), G.keep(torch.zeros(n, dtype=torch.int64, device="cuda"))


def eager(lm, ids, tok, tgt):
    n, l = tok.shape
    lm.explain_device(ids.data_ptr(), n, l, LXT_EPS, 1, tok.data_ptr(), tgt.data_ptr())
    models.synchronize()
    return G.host(tok).copy()


def replay_equals(lm, tok, expected):
    tok.fill_(float("nan"))
    models.synchronize()
    lm.replay()
    models.synchronize()
    return np.array_equal(G.host(tok), expected)


def test_replay_refused_after_longer_pass_then_recaptured():
    cfg, lm = small_model()
    ids16, tok16, tgt16 = device_inputs(cfg, 1, 16, 1)
    ref16 = eager(lm, ids16, tok16, tgt16)
    lm.capture_explain(ids16.data_ptr(), 1, 16, LXT_EPS, 1, tok16.data_ptr(), tgt16.data_ptr())
    assert replay_equals(lm, tok16, ref16)
    # A pass at a longer length regrows the model's buffers: the graph now addresses freed blocks.
    ids40, tok40, tgt40 = device_inputs(cfg, 2, 40, 2)
    eager(lm, ids40, tok40, tgt40)
    tok16.fill_(7.0)
    models.synchronize()
    with pytest.raises(N.PxkError, match="freed or reallocated since the capture"):
        lm.replay()
    models.synchronize()
    assert np.all(G.host(tok16) == 7.0)  # nothing ran
    # The shorter pass fits the regrown buffers: captured again, it replays to the eager result.
    ref16b = eager(lm, ids16, tok16, tgt16)
    np.testing.assert_array_equal(ref16b, ref16)
    lm.capture_explain(ids16.data_ptr(), 1, 16, LXT_EPS, 1, tok16.data_ptr(), tgt16.data_ptr())
    for _ in range(2):
        assert replay_equals(lm, tok16, ref16)
        eager(lm, ids16, tok16, tgt16)  # eager work at the captured shape between replays moves nothing


def test_replay_after_destroy_and_without_capture_refused():
    cfg, lm = small_model()
    with pytest.raises(N.PxkError, match="nothing was captured"):
        lm.replay()
    ids, tok, tgt = device_inputs(cfg, 1, 12, 3)
    ref = eager(lm, ids, tok, tgt)
    lm.capture_explain(ids.data_ptr(), 1, 12, LXT_EPS, 1, tok.data_ptr(), tgt.data_ptr())
    assert replay_equals(lm, tok, ref)
    handle = lm.h
    N.host().pxa_lm_destroy(handle)
    lm.h = None
    assert N.host().pxa_lm_replay(handle) != 0
    assert "unknown or destroyed model handle" in N.host().pxa_last_error().decode()
    N.host().pxa_lm_destroy(handle)  # a second destroy is a no-op


def test_other_models_do_not_invalidate_a_graph():
    """Blocks of another model, freed after this model's capture, are not this graph's."""
    cfg, lm = small_model()
    ids, tok, tgt = device_inputs(cfg, 1, 12, 4)
    ref = eager(lm, ids, tok, tgt)
    _, other = small_model()
    ids2, tok2, tgt2 = device_inputs(cfg, 1, 20, 5)
    eager(other, ids2, tok2, tgt2)
    lm.capture_explain(ids.data_ptr(), 1, 12, LXT_EPS, 1, tok.data_ptr(), tgt.data_ptr())
    del other  # destroys the other model, freeing blocks allocated before this capture
    assert replay_equals(lm, tok, ref)


def test_capture_at_a_new_length_runs_it_eagerly_first():
    """A capture at a length longer than any earlier pass runs the pass once eagerly (growing the
    buffers) before capturing it, so the graph never addresses a block the growth freed."""
    cfg, lm = small_model()
    ids, tok, tgt = device_inputs(cfg, 1, 8, 6)
    eager(lm, ids, tok, tgt)
    ids2, tok2, tgt2 = device_inputs(cfg, 1, 48, 7)
    lm.capture_explain(ids2.data_ptr(), 1, 48, LXT_EPS, 1, tok2.data_ptr(), tgt2.data_ptr())
    models.synchronize()
    captured_pass = G.host(tok2).copy()  # written by the capture's eager run
    ref = eager(lm, ids2, tok2, tgt2)
    np.testing.assert_array_equal(captured_pass, ref)
    for _ in range(2):
        assert replay_equals(lm, tok2, ref)


def test_launch_log_refused_after_model_destroyed():
    cfg, lm = small_model()
    ids, tok, tgt = device_inputs(cfg, 1, 12, 8)
    eager(lm, ids, tok, tgt)
    h = N.host()
    N.host_check(h.pxa_launch_log_start())
    lm.explain_device(ids.data_ptr(), 1, 12, LXT_EPS, 1, tok.data_ptr(), tgt.data_ptr())
    count = ctypes.c_int64(0)
    N.host_check(h.pxa_launch_log_stop(ctypes.byref(count)))
    assert count.value > 0
    secs = (ctypes.c_double * count.value)()
    N.host_check(h.pxa_launch_log_time(1, secs))  # the model is alive: the log replays
    del lm
    assert h.pxa_launch_log_time(1, secs) != 0
    assert "freed since the log closed" in h.pxa_last_error().decode()
