"""The Llama-3.2-1B-shaped configuration: hidden 2048, 32 query / 8 KV heads of 64, SwiGLU FFN
8192, vocab 128256, RoPE theta 500000, fp32, random init N(0, 0.02).

* At its widths, with 2 layers and batch 2 x 64 tokens, the MI355X path is held to the oracle at
  the module gates (logits 1e-4 scaled, argmax exact, ExpectRelevanceAgrees for token, embedding,
  key and value relevance).
* At its full shape (16 layers, batch 8 x 1024) the oracle would take hours, so the path is held to
  properties that do not depend on size: the explain step is deterministic (bit-identical on a
  second run), the on-device targets are the argmax of the on-device logits, and a sequence's
  relevance does not depend on the batch it runs in (sequence 3 of the batch against the same
  sequence run alone, at the relevance gate)."""
import ctypes
import time

import numpy as np
import pytest

import gpu_util as G
import oracle_ctypes as oc
from pulsatrix_amd import models
from pulsatrix_amd import native as N
from test_model_gpu import argmax_seed, expect_logits_agree, expect_relevance_agrees, to_px

pytestmark = pytest.mark.gpu
LXT_EPS = 1e-9


def l1b_config(**kw):
    base = dict(vocab_size=128256, hidden_size=2048, num_layers=16, num_heads=32, num_kv_heads=8, head_dim=64,
                intermediate_size=8192, rms_norm_eps=1e-5, rope_theta=500000.0)
    base.update(kw)
    return oc.model_config(**base)


class _DeviceArray:
    """A float32 view of backend-owned device memory for torch.as_tensor (only read here)."""

    def __init__(self, ptr, count):
        self.__cuda_array_interface__ = {"shape": (count,), "typestr": "<f4", "data": (ptr, False), "version": 2,
                                         "strides": None}


def device_view(torch, ptr, count):
    return torch.as_tensor(_DeviceArray(ptr, count), device="cuda")


def test_l1b_widths_match_oracle():
    cfg = l1b_config(num_layers=2)
    print("L1B widths, 2 layers, batch 2 x 64", flush=True)
    params = oc.synthetic_params(cfg, 41)
    ids = np.random.RandomState(42).randint(0, cfg.vocab_size, size=(2, 64))
    gpu = models.CausalLM(to_px(cfg), params)
    lg = gpu.forward(ids)
    ref = oc.oracle().lm(cfg, params)
    lr = ref.forward(ids)
    expect_logits_agree(lg, lr, "logits")
    seed = argmax_seed(lr)
    a = gpu.relevance(seed, LXT_EPS, True, want_kv=True)
    b = ref.relevance(seed, LXT_EPS, True, want_kv=True)
    for what, x, y in zip(("embedding", "tokens", "keys", "values"), a, b):
        expect_relevance_agrees(x, y, what)


def test_wide_grid_attention_matches_oracle():
    """A batch wide enough for the attention kernels' wide-grid forms (8 sequences x 4 KV heads: the
    GQA-shared forward and q side, the key side with two key blocks per workgroup), at reduced
    widths so the oracle runs it: 2 layers, hidden 256, 16 / 4 heads of 64, batch 8 x 256."""
    cfg = oc.model_config(vocab_size=1000, hidden_size=256, num_layers=2, num_heads=16, num_kv_heads=4, head_dim=64,
                          intermediate_size=512, rms_norm_eps=1e-5, rope_theta=10000.0)
    print("wide-grid attention, 2 layers, batch 8 x 256", flush=True)
    fn = N.pxk().pxk_attention_forward_gqa
    fn.argtypes = [ctypes.c_int64] * 4
    fn.restype = ctypes.c_int
    assert fn(8, 256, 16, 4) == 1
    params = oc.synthetic_params(cfg, 43)
    ids = np.random.RandomState(44).randint(0, cfg.vocab_size, size=(8, 256))
    gpu = models.CausalLM(to_px(cfg), params)
    lg = gpu.forward(ids)
    ref = oc.oracle().lm(cfg, params)
    lr = ref.forward(ids)
    expect_logits_agree(lg, lr, "logits")
    seed = argmax_seed(lr)
    a = gpu.relevance(seed, LXT_EPS, True, want_kv=True)
    b = ref.relevance(seed, LXT_EPS, True, want_kv=True)
    for what, x, y in zip(("embedding", "tokens", "keys", "values"), a, b):
        expect_relevance_agrees(x, y, what)


def test_l1b_full_shape_properties():
    torch = G.torch_cuda()
    cfg = l1b_config()
    n, L = 8, 1024
    print("L1B full shape: 16 layers, batch %d x %d" % (n, L), flush=True)
    lm = models.CausalLM(to_px(cfg), seed=7, std=0.02)
    ids = np.random.RandomState(8).randint(0, cfg.vocab_size, size=(n, L)).astype(np.float32)
    ids_d = G.dev(ids)
    tok, tok2 = G.empty((n, L)), G.empty((n, L))
    tgt, tgt2 = (G.keep(torch.empty(n, dtype=torch.int64, device="cuda")) for _ in range(2))
    models.synchronize()
    t0 = time.perf_counter()
    lm.explain_device(ids_d.data_ptr(), n, L, LXT_EPS, 1, tok.data_ptr(), tgt.data_ptr())
    models.synchronize()
    t1 = time.perf_counter()
    print("explain step (first call, includes buffer set-up): %.3f s" % (t1 - t0), flush=True)
    # the on-device targets are the argmax of the last position's logits, read from HBM
    base, V = lm.last_logits_ptr(), cfg.vocab_size
    logits_last = np.stack([device_view(torch, base + 4 * (s * L + L - 1) * V, V).cpu().numpy() for s in range(n)])
    assert list(G.host(tgt)) == list(np.argmax(logits_last, axis=1))
    r1 = G.host(tok)
    assert np.all(np.isfinite(r1))
    lm.explain_device(ids_d.data_ptr(), n, L, LXT_EPS, 1, tok2.data_ptr(), tgt2.data_ptr())
    models.synchronize()
    t2 = time.perf_counter()
    print("explain step (second call): %.3f s = %.0f tokens/s" % (t2 - t1, n * L / (t2 - t1)), flush=True)
    assert np.array_equal(G.host(tok2), r1), "explain step not deterministic"
    assert np.array_equal(G.host(tgt2), G.host(tgt))
    # batch invariance: sequence 3 alone
    one, tgt1 = G.empty((1, L)), G.keep(torch.empty(1, dtype=torch.int64, device="cuda"))
    lm.explain_device(ids_d.data_ptr() + 3 * L * 4, 1, L, LXT_EPS, 1, one.data_ptr(), tgt1.data_ptr())
    models.synchronize()
    assert int(G.host(tgt1)[0]) == int(G.host(tgt)[3])
    expect_relevance_agrees(G.host(one)[0], r1[3], "sequence 3 alone vs in the batch")

