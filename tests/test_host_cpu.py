"""CPU-side checks of the host framework library (no GPU calls): it loads, exports every entry
point include/pulsatrix_amd.h declares, and its synthetic initialisation and parameter layout
agree with the oracle's bit for bit (so GPU and oracle runs see the same weights)."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle_ctypes as oc
from pulsatrix_amd import models
from pulsatrix_amd import native as N


def test_host_library_exports_every_declared_symbol():
    header = open(os.path.join(oc.ROOT, "include", "pulsatrix_amd.h")).read()
    names = sorted(set(re.findall(r"\b(pxa_[a-z0-9_]+)\s*\(", header)))
    lib = N.host()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert len(names) >= 20


def as_oracle_cfg(cfg):
    return oc.ModelConfig(**{f: getattr(cfg, f) for f, _ in cfg._fields_})


@pytest.mark.parametrize("tied,bias", [(1, 0), (0, 1)])
def test_synthetic_params_match_oracle(tied, bias):
    cfg = N.model_config(vocab_size=97, hidden_size=24, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=6,
                         intermediate_size=40, tie_word_embeddings=tied, qkv_bias=bias, mlp_bias=bias, out_bias=bias)
    ocfg = as_oracle_cfg(cfg)
    assert models.param_count(cfg) == oc.oracle().lib.pxo_param_count(ctypes.byref(ocfg))
    assert models.param_count(cfg, block=True) == oc.oracle().lib.pxo_block_param_count(ctypes.byref(ocfg))
    for block in (False, True):
        mine = models.synthetic_params(cfg, 1234, 0.02, block=block)
        ref = oc.synthetic_params(ocfg, 1234, 0.02, block=block)
        assert np.array_equal(mine, ref)


def test_fill_normal_matches_oracle():
    a = np.empty(10001, np.float32)
    N.host().pxa_fill_normal(a.ctypes.data_as(ctypes.c_void_p), a.size, 77, 1.5)
    assert np.array_equal(a, oc.fill_normal(a.size, 77, 1.5))


def test_backend_reports_missing_device_without_crashing():
    if N.host().pxa_device_count() > 0:
        pytest.skip("a GPU is present")
    assert N.host().pxa_backend() is None
    assert N.host().pxa_last_error()
