"""The fused attention kernels (pxk_attention_*) against float64 numpy restatements of the module
sequences they replace (multihead_attention_module.cpp:268-291 forward; :404-485 relevance).

Inputs are seeded uniform(-1, 1) (the reference's equivalence-test convention). Tolerances are
the primitive contract's 1e-4 scaled by max(1, |ref|), applied to every output the relevance
pass later reads: raw scores on the visible keys, P on every key (zeros past the visible ones),
and the head-packed context.
"""
import numpy as np
import pytest

import gpu_util as G
from pulsatrix_amd import native as N

gpu = pytest.mark.gpu

CASES = [  # n, L, H, Hkv, D
    (1, 37, 4, 2, 16),
    (2, 64, 3, 1, 12),
    (1, 128, 9, 3, 64),
    (1, 50, 2, 2, 128),
    (1, 512, 9, 3, 64),
    (1, 1030, 2, 1, 64),
]


def attention_reference(q, k, v, n, L, H, Hkv, D, scale, causal):
    """raw, P (n, H, L, L) and ctx (n*L, H*D) in float64."""
    grp = H // Hkv
    qh = q.reshape(n, L, H, D).transpose(0, 2, 1, 3).astype(np.float64)
    kh = np.repeat(k.reshape(n, L, Hkv, D).transpose(0, 2, 1, 3), grp, axis=1).astype(np.float64)
    vh = np.repeat(v.reshape(n, L, Hkv, D).transpose(0, 2, 1, 3), grp, axis=1).astype(np.float64)
    raw = qh @ kh.transpose(0, 1, 3, 2)
    x = scale * raw
    vis = np.tril(np.ones((L, L), bool)) if causal else np.ones((L, L), bool)
    x = np.where(vis, x, -np.inf)
    x = x - x.max(axis=-1, keepdims=True)
    e = np.where(vis, np.exp(x), 0.0)
    p = e / e.sum(axis=-1, keepdims=True)
    ctx = (p @ vh).transpose(0, 2, 1, 3).reshape(n * L, H * D)
    return raw, p, ctx, vis


@gpu
@pytest.mark.parametrize("causal", [1, 0])
@pytest.mark.parametrize("n,L,H,Hkv,D", CASES)
def test_fused_attention_forward_matches_numpy(n, L, H, Hkv, D, causal):
    qd, kvd = H * D, Hkv * D
    w3 = qd + 2 * kvd
    qkv = G.uniform((n * L, w3), 11 + L + D)  # the module's packed [q | k | v] rows
    scale = 1.0 / np.sqrt(D)
    qkv_d = G.dev(qkv)
    raw, p, ctx = G.empty((n, H, L, L)), G.empty((n, H, L, L)), G.empty((n * L, qd))
    base = qkv_d.data_ptr()
    N.call("pxk_attention_forward", base, w3, base + 4 * qd, w3, base + 4 * (qd + kvd), w3, G.ptr(raw), G.ptr(p),
           G.ptr(ctx), qd, n, L, H, Hkv, D, scale, causal, G.stream())
    r_raw, r_p, r_ctx, vis = attention_reference(qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:], n, L, H, Hkv, D,
                                                 scale, causal)
    got_raw, got_p = G.host(raw), G.host(p)
    G.assert_close(got_raw[..., vis], r_raw[..., vis], 1e-4, "raw")
    G.assert_close(got_p, r_p, 1e-5, "P")
    assert np.all(got_p[..., ~vis] == 0.0), "P must be 0 on masked keys"
    G.assert_close(G.host(ctx), r_ctx, 1e-4, "ctx")
    np.testing.assert_allclose(got_p.sum(axis=-1), 1.0, rtol=1e-5)  # rows of P sum to 1


@gpu
def test_fused_attention_is_deterministic():
    n, L, H, Hkv, D = 1, 200, 4, 2, 64
    q, k, v = G.uniform((n * L, H * D), 1), G.uniform((n * L, Hkv * D), 2), G.uniform((n * L, Hkv * D), 3)
    qd_, kd_, vd_ = G.dev(q), G.dev(k), G.dev(v)
    outs = []
    for _ in range(2):
        raw, p, ctx = G.empty((n, H, L, L)), G.empty((n, H, L, L)), G.empty((n * L, H * D))
        N.call("pxk_attention_forward", G.ptr(qd_), H * D, G.ptr(kd_), Hkv * D, G.ptr(vd_), Hkv * D, G.ptr(raw),
               G.ptr(p), G.ptr(ctx), H * D, n, L, H, Hkv, D, 0.125, 1, G.stream())
        outs.append((G.host(p), G.host(ctx)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def test_fused_attention_support_and_rejection():
    """CPU-side: supported layouts, and a bad one rejected before any launch."""
    lib = N.pxk()
    assert lib.pxk_attention_supported(64, 512, 960, 960, 960) == 1
    assert lib.pxk_attention_supported(64, 1024, 960, 960, 960) == 1
    assert lib.pxk_attention_supported(6, 512, 960, 960, 960) == 0  # head_dim not a multiple of 4
    assert lib.pxk_attention_supported(256, 512, 4096, 4096, 4096) == 0
    assert lib.pxk_attention_supported(64, 4096, 960, 960, 960) == 0  # score rows beyond LDS
    rc = lib.pxk_attention_forward(16, 64, 16, 64, 16, 64, 16, 16, 16, 64, 1, 8, 3, 2, 16, 0.25, 1, None)
    assert rc == 1  # 3 query heads over 2 KV heads
