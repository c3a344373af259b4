"""The fused attention kernels (pxk_attention_*) against float64 numpy restatements of the module
sequences they replace (multihead_attention_module.cpp:268-291 forward; :404-485 relevance).

Inputs are seeded uniform(-1, 1) (the reference's equivalence-test convention). Tolerances are
the primitive contract's 1e-4 scaled by max(1, |ref|), applied to every output the relevance
pass later reads: raw scores on the visible keys, P on every key (zeros past the visible ones),
and the head-packed context.
"""
import ctypes

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
@pytest.mark.parametrize("with_p", [0, 1])
@pytest.mark.parametrize("n,L,H,Hkv,D", [(1, 37, 4, 2, 16), (2, 64, 3, 1, 12), (1, 512, 9, 3, 64), (1, 50, 2, 2, 128),
                                         (1, 2600, 2, 1, 64)])
def test_fused_attention_forward_stats_matches_numpy(n, L, H, Hkv, D, with_p):
    """The statistics form: ctx and, per row, the softmax max of scale * raw and 1 / sum. Without P
    or raw it needs no LDS for score rows, so 2600 tokens (past the score-row form's limit) run."""
    print("forward stats n=%d L=%d H=%d Hkv=%d D=%d with_p=%d" % (n, L, H, Hkv, D, with_p), flush=True)
    if with_p and L > 2000:
        pytest.skip("P is kept only within the score-row form's LDS limit")
    qd, kvd = H * D, Hkv * D
    w3 = qd + 2 * kvd
    qkv = G.uniform((n * L, w3), 21 + L + D)
    scale = 1.0 / np.sqrt(D)
    qkv_d = G.dev(qkv)
    stats, ctx = G.empty((n, H, L, 2)), G.empty((n * L, qd))
    p = G.empty((n, H, L, L)) if with_p else None
    base = qkv_d.data_ptr()
    N.call("pxk_attention_forward_stats", base, w3, base + 4 * qd, w3, base + 4 * (qd + kvd), w3, None,
           G.ptr(p) if with_p else None, G.ptr(stats), G.ptr(ctx), qd, n, L, H, Hkv, D, scale, 1, G.stream())
    q, k, v = qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:]
    grp = H // Hkv
    qh = q.reshape(n, L, H, D).transpose(0, 2, 1, 3).astype(np.float64)
    kh = np.repeat(k.reshape(n, L, Hkv, D).transpose(0, 2, 1, 3), grp, axis=1).astype(np.float64)
    vh = np.repeat(v.reshape(n, L, Hkv, D).transpose(0, 2, 1, 3), grp, axis=1).astype(np.float64)
    want_st = np.empty((n, H, L, 2))
    want_ctx = np.empty((n, H, L, D))
    for b in range(n):  # per head, so the 2600-token case stays small
        for h in range(H):
            x = scale * (qh[b, h] @ kh[b, h].T)
            x = np.where(np.tril(np.ones((L, L), bool)), x, -np.inf)
            m = x.max(-1)
            e = np.exp(x - m[:, None])
            ssum = e.sum(-1)
            want_st[b, h, :, 0], want_st[b, h, :, 1] = m, 1.0 / ssum
            want_ctx[b, h] = (e / ssum[:, None]) @ vh[b, h]
            if with_p:
                G.assert_close(G.host(p)[b, h], e / ssum[:, None], 1e-4, "P")
    got = G.host(stats)
    G.assert_close(got[..., 0], want_st[..., 0], 1e-4, "row max")
    G.assert_close(got[..., 1], want_st[..., 1], 1e-4, "1 / row sum")
    G.assert_close(G.host(ctx), want_ctx.transpose(0, 2, 1, 3).reshape(n * L, qd), 1e-4, "ctx")


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


def stab(z, eps):
    return z + eps * np.where(z >= 0, 1.0, -1.0)


def relevance_q_reference(spv, q, q_pre, k, v, z, bias, p, raw, cos, sin, n, L, H, Hkv, D, scale, eps, causal, rope,
                          half):
    """s (n, H, L, L) and g_q (n*L, H*D) in float64: the module's steps 2-4 (multihead_attention_module.cpp
    :435-447 with lrp_bilinear_matmul, lrp_softmax_rows and lrp_rope)."""
    grp = H // Hkv
    f = lambda a, heads: a.reshape(n, L, heads, D).transpose(0, 2, 1, 3).astype(np.float64)
    spv_h, q_h, qx_h, z_h = f(spv, H), f(q, H), f(q_pre, H), f(z, H)
    k_h = np.repeat(f(k, Hkv), grp, axis=1)
    v_h = np.repeat(f(v, Hkv), grp, axis=1)
    vis = np.tril(np.ones((L, L), bool)) if causal else np.ones((L, L), bool)
    r_attn = np.where(vis, p * (spv_h @ v_h.transpose(0, 1, 3, 2)), 0.0)
    tot = r_attn.sum(axis=-1, keepdims=True)
    s = np.where(vis, (scale * raw) * (r_attn - p * tot) / (2.0 * raw + eps * np.where(raw >= 0, 1.0, -1.0)), 0.0)
    sk = s @ k_h
    r = q_h * sk
    if rope:
        d = np.arange(D)
        hf = D // 2
        i = np.where(d < hf, d, d - hf) if half else d // 2
        lo = i if half else 2 * i
        hi = i + hf if half else 2 * i + 1
        c, sn = cos[:, i][None, None], sin[:, i][None, None]
        y_lo, y_hi = q_h[..., lo], q_h[..., hi]
        d0, d1 = stab(y_lo, eps), stab(y_hi, eps)
        r_lo, r_hi = r[..., lo], r[..., hi]
        is_lo = (d == lo)
        r_in = np.where(is_lo, qx_h * c / d0 * r_lo + qx_h * sn / d1 * r_hi, qx_h * -sn / d0 * r_lo + qx_h * c / d1 * r_hi)
    else:
        r_in = r
    zz = z_h + (bias.reshape(1, H, 1, D) if bias is not None else 0.0)
    g = (r_in / stab(zz, eps)).transpose(0, 2, 1, 3).reshape(n * L, H * D)
    return s, g


@gpu
@pytest.mark.parametrize("recompute", [0, 1])
@pytest.mark.parametrize("rope,half,bias", [(1, 1, 0), (1, 0, 1), (0, 0, 1)])
@pytest.mark.parametrize("causal", [1, 0])
@pytest.mark.parametrize("n,L,H,Hkv,D", [(1, 37, 4, 2, 16), (2, 64, 3, 1, 12), (1, 128, 9, 3, 64), (1, 40, 2, 2, 128),
                                         (1, 512, 9, 3, 64)])
def test_fused_attention_relevance_matches_numpy(n, L, H, Hkv, D, causal, rope, half, bias, recompute):
    """recompute: the kernel gets no raw scores or P, only the forward's row statistics and the
    attention output ctx = P V; it recomputes raw = Q K^T and P and takes the softmax rule's row
    sums as s_pv . ctx, while the reference sums r_attn over the keys. Its q and k hold multiples
    of 0.5 up to 1 in magnitude, so raw = Q K^T is exact in float32 and float64 alike."""
    print("q relevance n=%d L=%d H=%d Hkv=%d D=%d causal=%d rope=%d half=%d recompute=%d"
          % (n, L, H, Hkv, D, causal, rope, half, recompute), flush=True)
    qd, kvd = H * D, Hkv * D
    grp = H // Hkv
    scale, eps = 1.0 / np.sqrt(D), 1e-6
    rs = np.random.RandomState(L + D)
    away = lambda *shape: (rs.uniform(0.5, 1.5, shape) * rs.choice([-1.0, 1.0], shape)).astype(np.float32)
    halves = lambda *shape: rs.choice([-1.0, -0.5, 0.5, 1.0], shape).astype(np.float32)
    spv, q, q_pre, z = G.uniform((n * L, qd), 1), away(n * L, qd), G.uniform((n * L, qd), 3), away(n * L, qd)
    k, v = G.uniform((n * L, kvd), 4), G.uniform((n * L, kvd), 5)
    b = (G.uniform((qd,), 6) * 0.1) if bias else None
    if recompute:
        q, k = halves(n * L, qd), halves(n * L, kvd)
        qh = q.reshape(n, L, H, D).transpose(0, 2, 1, 3).astype(np.float64)
        kh = np.repeat(k.reshape(n, L, Hkv, D).transpose(0, 2, 1, 3), grp, axis=1).astype(np.float64)
        raw = (qh @ kh.transpose(0, 1, 3, 2)).astype(np.float32)
    else:
        raw = away(n, H, L, L)  # denominators 2 raw + eps sign raw stay clear of 0
    vis = np.tril(np.ones((L, L), bool)) if causal else np.ones((L, L), bool)
    x = np.where(vis, scale * raw.astype(np.float64), -np.inf)
    mx = x.max(-1, keepdims=True)
    e = np.exp(x - mx)
    p = (e / e.sum(-1, keepdims=True)).astype(np.float32)
    stats = np.stack([mx[..., 0], 1.0 / e.sum(-1)], axis=-1).astype(np.float32)
    ang = np.arange(L)[:, None] * (10000.0 ** (-np.arange(D // 2) * 2.0 / D))[None, :]
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    want_s, want_g = relevance_q_reference(spv, q, q_pre, k, v, z, b, p.astype(np.float64), raw.astype(np.float64),
                                           cos.astype(np.float64), sin.astype(np.float64), n, L, H, Hkv, D, scale,
                                           eps, causal, rope, half)
    dv = {key: G.dev(a) for key, a in dict(spv=spv, q=q, q_pre=q_pre, z=z, k=k, v=v, p=p, raw=raw, cos=cos,
                                            sin=sin).items()}
    s_out, g_out = G.empty((n, H, L, L)), G.empty((n * L, qd))
    d = N.AttnRelDesc()
    d.n, d.l, d.heads, d.kv_heads, d.head_dim = n, L, H, Hkv, D
    d.scale, d.eps, d.causal, d.rope, d.rope_half = scale, eps, causal, rope, half
    d.spv, d.ld_spv = G.ptr(dv["spv"]).value, qd
    d.v, d.ld_v, d.k, d.ld_k = G.ptr(dv["v"]).value, kvd, G.ptr(dv["k"]).value, kvd
    d.p, d.raw, d.s = G.ptr(dv["p"]).value, G.ptr(dv["raw"]).value, G.ptr(s_out).value
    d.q, d.ld_q, d.q_pre, d.ld_q_pre = G.ptr(dv["q"]).value, qd, G.ptr(dv["q_pre"]).value, qd
    d.z, d.ld_z = G.ptr(dv["z"]).value, qd
    d.bias = G.ptr(G.dev(b)).value if bias else None
    d.cos_t, d.sin_t = G.ptr(dv["cos"]).value, G.ptr(dv["sin"]).value
    d.g, d.ld_g = G.ptr(g_out).value, qd
    if recompute:
        v_h = np.repeat(v.reshape(n, L, Hkv, D).transpose(0, 2, 1, 3), grp, axis=1).astype(np.float64)
        ctx = (p.astype(np.float64) @ v_h).transpose(0, 2, 1, 3).reshape(n * L, qd).astype(np.float32)
        ctx_d, stats_d, rsum, p_out = G.dev(ctx), G.dev(stats), G.empty((n, H, L)), G.empty((n, H, L, L))
        d.ctx, d.ld_ctx, d.stats, d.row_sum = G.ptr(ctx_d).value, qd, G.ptr(stats_d).value, G.ptr(rsum).value
        d.p_out = G.ptr(p_out).value
        d.p = d.raw = None  # not read
    assert N.pxk().pxk_attention_relevance_q(ctypes.byref(d), G.stream()) == 0, N.pxk().pxk_last_error()
    if recompute:  # s_pv . ctx per row
        spv_h = spv.reshape(n, L, H, D).transpose(0, 2, 1, 3).astype(np.float64)
        ctx_h = ctx.reshape(n, L, H, D).transpose(0, 2, 1, 3).astype(np.float64)
        G.assert_close(G.host(rsum), (spv_h * ctx_h).sum(-1), 1e-4, "row_sum")
    got_s = G.host(s_out)
    if recompute:  # s and P on the visible keys, zeros at the masked keys of the diagonal tiles
        got_p = G.host(p_out)
        G.assert_close(got_s[..., vis], want_s[..., vis], 1e-4, "s")
        G.assert_close(got_p[..., vis], p.astype(np.float64)[..., vis], 1e-4, "P")
        if causal:
            i, j = np.meshgrid(np.arange(L), np.arange(L), indexing="ij")
            diag = (j > i) & (j < np.minimum(16 * (i // 16 + 1), L))
            assert np.all(got_s[..., diag] == 0.0) and np.all(got_p[..., diag] == 0.0)
    else:
        G.assert_close(got_s, want_s, 1e-4, "s")
        assert np.all(got_s[..., ~vis] == 0.0)
    G.assert_close(G.host(g_out), want_g, 1e-4, "g_q")


def relevance_kv_reference(s, p, q, spv, k, k_pre, v, z_k, z_v, bk, bv, cos, sin, n, L, H, Hkv, D, eps, causal, rope,
                           half):
    """key_rel, value_rel, g_k, g_v (n*L, Hkv*D) in float64: the module's b-shares of the two
    bilinear products (multihead_attention_module.cpp:446-447 and :435-436), sum_kv_groups
    (:173-188), lrp_rope on the keys and the k/v projections' denominators."""
    grp = H // Hkv
    f = lambda a, heads: a.reshape(n, L, heads, D).transpose(0, 2, 1, 3).astype(np.float64)
    q_h, spv_h = f(q, H), f(spv, H)
    k_h, kp_h, v_h, zk_h, zv_h = f(k, Hkv), f(k_pre, Hkv), f(v, Hkv), f(z_k, Hkv), f(z_v, Hkv)
    vis = np.tril(np.ones((L, L), bool)) if causal else np.ones((L, L), bool)
    sm, pm = np.where(vis, s, 0.0), np.where(vis, p, 0.0)
    sk = np.einsum("nhij,nhid->nhjd", sm, q_h).reshape(n, Hkv, grp, L, D).sum(axis=2)
    pv = np.einsum("nhij,nhid->nhjd", pm, spv_h).reshape(n, Hkv, grp, L, D).sum(axis=2)
    r = k_h * sk
    if rope:
        d = np.arange(D)
        hf = D // 2
        i = np.where(d < hf, d, d - hf) if half else d // 2
        lo = i if half else 2 * i
        hi = i + hf if half else 2 * i + 1
        c, sn = cos[:, i][None, None], sin[:, i][None, None]
        d0, d1 = stab(k_h[..., lo], eps), stab(k_h[..., hi], eps)
        r_lo, r_hi = r[..., lo], r[..., hi]
        r = np.where(d == lo, kp_h * c / d0 * r_lo + kp_h * sn / d1 * r_hi,
                     kp_h * -sn / d0 * r_lo + kp_h * c / d1 * r_hi)
    rv = v_h * pv
    gk = r / stab(zk_h + (bk.reshape(1, Hkv, 1, D) if bk is not None else 0.0), eps)
    gv = rv / stab(zv_h + (bv.reshape(1, Hkv, 1, D) if bv is not None else 0.0), eps)
    t = lambda a: a.transpose(0, 2, 1, 3).reshape(n * L, Hkv * D)
    return t(r), t(rv), t(gk), t(gv)


@gpu
@pytest.mark.parametrize("rope,half,bias", [(1, 1, 0), (1, 0, 1), (0, 0, 1)])
@pytest.mark.parametrize("causal", [1, 0])
@pytest.mark.parametrize("n,L,H,Hkv,D", [(1, 37, 4, 2, 16), (2, 64, 3, 1, 12), (1, 128, 9, 3, 64), (1, 40, 2, 2, 128),
                                         (1, 512, 9, 3, 64), (2, 70, 4, 4, 20), (1, 23, 6, 2, 8)])
def test_fused_attention_kv_relevance_matches_numpy(n, L, H, Hkv, D, causal, rope, half, bias):
    print("kv relevance n=%d L=%d H=%d Hkv=%d D=%d causal=%d rope=%d half=%d" % (n, L, H, Hkv, D, causal, rope, half),
          flush=True)
    qd, kvd = H * D, Hkv * D
    eps = 1e-6
    rs = np.random.RandomState(3 * L + D)
    away = lambda *shape: (rs.uniform(0.5, 1.5, shape) * rs.choice([-1.0, 1.0], shape)).astype(np.float32)
    vis = np.tril(np.ones((L, L), bool)) if causal else np.ones((L, L), bool)
    s = np.where(vis, G.uniform((n, H, L, L), 1), 0.0).astype(np.float32)  # zeros where masked, as written upstream
    p = np.where(vis, G.uniform((n, H, L, L), 2, 0.0, 1.0), 0.0).astype(np.float32)
    q, spv = G.uniform((n * L, qd), 3), G.uniform((n * L, qd), 4)
    k, k_pre, v = away(n * L, kvd), G.uniform((n * L, kvd), 6), G.uniform((n * L, kvd), 7)
    z_k, z_v = away(n * L, kvd), away(n * L, kvd)
    bk, bv = ((G.uniform((kvd,), 8) * 0.1, G.uniform((kvd,), 9) * 0.1) if bias else (None, None))
    ang = np.arange(L)[:, None] * (10000.0 ** (-np.arange(D // 2) * 2.0 / D))[None, :]
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    want = relevance_kv_reference(s.astype(np.float64), p.astype(np.float64), q, spv, k, k_pre, v, z_k, z_v,
                                  bk, bv, cos.astype(np.float64), sin.astype(np.float64), n, L, H, Hkv, D, eps,
                                  causal, rope, half)
    dv = {key: G.dev(a) for key, a in dict(s=s, p=p, q=q, spv=spv, k=k, k_pre=k_pre, v=v, z_k=z_k, z_v=z_v, cos=cos,
                                            sin=sin).items()}
    outs = [G.empty((n * L, kvd)) for _ in range(4)]
    d = N.AttnRelKvDesc()
    d.n, d.l, d.heads, d.kv_heads, d.head_dim = n, L, H, Hkv, D
    d.eps, d.causal, d.rope, d.rope_half = eps, causal, rope, half
    d.s, d.p = G.ptr(dv["s"]).value, G.ptr(dv["p"]).value
    d.q, d.ld_q, d.spv, d.ld_spv = G.ptr(dv["q"]).value, qd, G.ptr(dv["spv"]).value, qd
    d.k, d.ld_k, d.k_pre, d.ld_k_pre = G.ptr(dv["k"]).value, kvd, G.ptr(dv["k_pre"]).value, kvd
    d.v, d.ld_v = G.ptr(dv["v"]).value, kvd
    d.z_k, d.z_v, d.ld_z = G.ptr(dv["z_k"]).value, G.ptr(dv["z_v"]).value, kvd
    d.bias_k = G.ptr(G.dev(bk)).value if bias else None
    d.bias_v = G.ptr(G.dev(bv)).value if bias else None
    d.cos_t, d.sin_t = G.ptr(dv["cos"]).value, G.ptr(dv["sin"]).value
    d.key_rel, d.value_rel, d.ld_rel = G.ptr(outs[0]).value, G.ptr(outs[1]).value, kvd
    d.g_k, d.g_v, d.ld_g = G.ptr(outs[2]).value, G.ptr(outs[3]).value, kvd
    assert N.pxk().pxk_attention_relevance_kv(ctypes.byref(d), G.stream()) == 0, N.pxk().pxk_last_error()
    for got, ref, name in zip(outs, want, ("key_rel", "value_rel", "g_k", "g_v")):
        G.assert_close(G.host(got), ref, 1e-4, name)


@gpu
@pytest.mark.parametrize("n,L,H,Hkv,D", [(4, 256, 32, 32, 64), (4, 232, 32, 32, 64), (4, 200, 16, 8, 128),
                                         (4, 230, 32, 32, 64), (2, 500, 8, 4, 64), (1, 1030, 6, 3, 64)])
@pytest.mark.parametrize("causal,rope,half,bias", [(1, 1, 1, 0), (0, 0, 0, 1), (1, 1, 0, 1)])
def test_fused_attention_kv_relevance_large_grid(n, L, H, Hkv, D, causal, rope, half, bias):
    """The wide-grid launch, four head-dim groups and two 16-key blocks per workgroup, taken from 512
    (KV head, key block, four groups) units: 4 x 32 x 16 (x 4 / 4) = 2048 at 4 x 256 tokens; an odd
    count of key blocks at 232 tokens (15: the last workgroup's second block lies past the
    sequence); head_dim 128 (8 groups) with 13 key blocks; 230 tokens, whose last 4-row chunk holds
    two rows. Then the four-group, one-block launch for 128 to 511 (KV head, key block) pairs: 256
    at 2 x 500 tokens with 4 KV heads, 195 at 1030 tokens with 3 (its last chunk two rows long)."""
    test_fused_attention_kv_relevance_matches_numpy(n, L, H, Hkv, D, causal, rope, half, bias)


@gpu
@pytest.mark.parametrize("n,L,H,Hkv,D", [(1, 200, 4, 2, 64), (2, 37, 3, 1, 16), (1, 512, 9, 3, 64), (4, 512, 8, 4, 64)])
def test_recomputing_chain_matches_score_row_chain(n, L, H, Hkv, D):
    """The step's attention relevance chain in its recomputing form (forward with row statistics,
    q side recomputing raw and P and writing s and P into NaN-filled buffers, key side reading
    them) against the score-row form (forward keeping raw and P, two-pass q side): the same
    [g_q | g_k | g_v]. q and k hold multiples of 0.5, so raw = Q K^T is exact. At 4 x 512 with
    8 / 4 heads the recomputing forward and q side run GQA-shared."""
    print("recomputing chain n=%d L=%d H=%d Hkv=%d D=%d" % (n, L, H, Hkv, D), flush=True)
    qd, kvd = H * D, Hkv * D
    w3 = qd + 2 * kvd
    scale, eps = 1.0 / np.sqrt(D), 1e-9
    rs = np.random.RandomState(7 * L + D)
    qkv = rs.choice([-1.0, -0.5, 0.5, 1.0], (n * L, w3)).astype(np.float32)
    qkv[:, qd + kvd:] = G.uniform((n * L, kvd), 1)  # v
    spv = G.uniform((n * L, qd), 2)
    pre = G.uniform((n * L, qd + kvd), 3)  # q | k before the rotation
    z = (rs.uniform(0.5, 1.5, (n * L, w3)) * rs.choice([-1.0, 1.0], (n * L, w3))).astype(np.float32)
    ang = np.arange(L)[:, None] * (10000.0 ** (-np.arange(D // 2) * 2.0 / D))[None, :]
    cos, sin = G.dev(np.cos(ang).astype(np.float32)), G.dev(np.sin(ang).astype(np.float32))
    qkv_d, spv_d, pre_d, z_d = G.dev(qkv), G.dev(spv), G.dev(pre), G.dev(z)
    base = qkv_d.data_ptr()

    def chain(recompute):
        ctx, g = G.empty((n * L, qd)), G.empty((n * L, w3))
        s_buf, p_buf = G.empty((n, H, L, L)), G.empty((n, H, L, L))  # NaN: unwritten entries show
        stats = G.empty((n, H, L, 2))
        if recompute:
            N.call("pxk_attention_forward_stats", base, w3, base + 4 * qd, w3, base + 4 * (qd + kvd), w3, None, None,
                   G.ptr(stats), G.ptr(ctx), qd, n, L, H, Hkv, D, scale, 1, G.stream())
        else:
            raw = G.empty((n, H, L, L))
            N.call("pxk_attention_forward", base, w3, base + 4 * qd, w3, base + 4 * (qd + kvd), w3, G.ptr(raw),
                   G.ptr(p_buf), G.ptr(ctx), qd, n, L, H, Hkv, D, scale, 1, G.stream())
        d = N.AttnRelDesc()
        d.n, d.l, d.heads, d.kv_heads, d.head_dim = n, L, H, Hkv, D
        d.scale, d.eps, d.causal, d.rope, d.rope_half = scale, eps, 1, 1, 1
        d.spv, d.ld_spv = spv_d.data_ptr(), qd
        d.v, d.ld_v, d.k, d.ld_k = base + 4 * (qd + kvd), w3, base + 4 * qd, w3
        d.s = G.ptr(s_buf).value
        d.q, d.ld_q, d.q_pre, d.ld_q_pre = base, w3, pre_d.data_ptr(), qd + kvd
        d.z, d.ld_z = z_d.data_ptr(), w3
        d.cos_t, d.sin_t = cos.data_ptr(), sin.data_ptr()
        d.g, d.ld_g = G.ptr(g).value, w3
        if recompute:
            d.ctx, d.ld_ctx, d.stats, d.p_out = G.ptr(ctx).value, qd, G.ptr(stats).value, G.ptr(p_buf).value
        else:
            d.p, d.raw = G.ptr(p_buf).value, G.ptr(raw).value
        assert N.pxk().pxk_attention_relevance_q(ctypes.byref(d), G.stream()) == 0, N.pxk().pxk_last_error()
        kd = N.AttnRelKvDesc()
        kd.n, kd.l, kd.heads, kd.kv_heads, kd.head_dim = n, L, H, Hkv, D
        kd.eps, kd.causal, kd.rope, kd.rope_half = eps, 1, 1, 1
        kd.s, kd.p, kd.q, kd.ld_q = G.ptr(s_buf).value, G.ptr(p_buf).value, base, w3
        kd.spv, kd.ld_spv = spv_d.data_ptr(), qd
        kd.k, kd.ld_k, kd.k_pre, kd.ld_k_pre = base + 4 * qd, w3, pre_d.data_ptr() + 4 * qd, qd + kvd
        kd.v, kd.ld_v = base + 4 * (qd + kvd), w3
        kd.z_k, kd.z_v, kd.ld_z = z_d.data_ptr() + 4 * qd, z_d.data_ptr() + 4 * (qd + kvd), w3
        kd.cos_t, kd.sin_t = cos.data_ptr(), sin.data_ptr()
        kd.g_k, kd.g_v, kd.ld_g = G.ptr(g).value + 4 * qd, G.ptr(g).value + 4 * (qd + kvd), w3
        assert N.pxk().pxk_attention_relevance_kv(ctypes.byref(kd), G.stream()) == 0, N.pxk().pxk_last_error()
        return G.host(g)

    want, got = chain(False), chain(True)
    assert np.all(np.isfinite(got))
    G.assert_close(got, want, 1e-4, "[g_q | g_k | g_v]")


def test_fused_attention_kv_relevance_rejects_bad_descs():
    """CPU-side validation: nothing is launched for a bad descriptor."""
    d = N.AttnRelKvDesc()
    d.n, d.l, d.heads, d.kv_heads, d.head_dim = 1, 8, 3, 2, 16
    assert N.pxk().pxk_attention_relevance_kv(ctypes.byref(d), None) == 1  # heads not a multiple of kv_heads
    d.heads = 4
    assert N.pxk().pxk_attention_relevance_kv(ctypes.byref(d), None) == 1  # NULL operands
    assert b"NULL" in N.pxk().pxk_last_error()


@gpu
def test_recomputed_scores_match_the_forwards_raw_with_random_inputs():
    """Uniform-random q and k (products not exact in float32) at the SmolLM2 shapes, causal GQA with
    RoPE. The q side recomputes raw = Q K^T and P from the forward's row statistics; s = r_sc /
    (2 raw + eps sign raw) is most sensitive where raw is near 0. The reference is float64
    arithmetic on the score-row forward's own float32 raw scores. Some query rows and key rows are
    planted so that their scores are a single product (the key's head zero apart from its first
    coordinate kappa, the query's first half zero apart from delta): raw = delta * kappa exactly, whatever the
    summation order, at 0, +-1e-7 .. 5e-6 (both sides of eps = 1e-6, both signs), so the sign rule
    and the small-denominator range are checked at known scores. The key side then reads the s and P
    the q side wrote: g_k and g_v against the float64 key-side sequence on the same s and P."""
    n, L, H, Hkv, D = 1, 512, 9, 3, 64
    print("recomputed scores vs forward raw, random inputs", flush=True)
    qd, kvd = H * D, Hkv * D
    w3 = qd + 2 * kvd
    scale, eps = 1.0 / np.sqrt(D), 1e-6
    qkv = G.uniform((n * L, w3), 11)
    q_rows, deltas = [64, 200, 333, 400, 511], [0.0, 1e-7, -2.5e-7, 1e-6, -5e-6]
    k_rows, kappas = [0, 17, 63, 64, 150, 333], [1.0, 0.5, -3.0, 0.25, -1.0, 2.0]
    for i, delta in zip(q_rows, deltas):
        for h in range(H):
            qkv[i, h * D:h * D + D // 2] = 0.0
            qkv[i, h * D] = delta
    for j, kappa in zip(k_rows, kappas):
        for hk in range(Hkv):
            col = qd + hk * D
            qkv[j, col:col + D] = 0.0
            qkv[j, col] = kappa
    spv, q_pre = G.uniform((n * L, qd), 12), G.uniform((n * L, qd + kvd), 13)
    rs = np.random.RandomState(14)
    z = (rs.uniform(0.5, 1.5, (n * L, w3)) * rs.choice([-1.0, 1.0], (n * L, w3))).astype(np.float32)
    ang = np.arange(L)[:, None] * (10000.0 ** (-np.arange(D // 2) * 2.0 / D))[None, :]
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    qkv_d, spv_d, pre_d, z_d, cos_d, sin_d = (G.dev(a) for a in (qkv, spv, q_pre, z, cos, sin))
    base = qkv_d.data_ptr()
    raw, p_fwd, ctx = G.empty((n, H, L, L)), G.empty((n, H, L, L)), G.empty((n * L, qd))
    N.call("pxk_attention_forward", base, w3, base + 4 * qd, w3, base + 4 * (qd + kvd), w3, G.ptr(raw), G.ptr(p_fwd),
           G.ptr(ctx), qd, n, L, H, Hkv, D, scale, 1, G.stream())
    stats, ctx2 = G.empty((n, H, L, 2)), G.empty((n * L, qd))
    N.call("pxk_attention_forward_stats", base, w3, base + 4 * qd, w3, base + 4 * (qd + kvd), w3, None, None,
           G.ptr(stats), G.ptr(ctx2), qd, n, L, H, Hkv, D, scale, 1, G.stream())
    raw_h = G.host(raw).astype(np.float64)
    vis = np.tril(np.ones((L, L), bool))
    planted = np.zeros((L, L), bool)
    for i, delta in zip(q_rows, deltas):
        for j, kappa in zip(k_rows, kappas):
            if j <= i:
                planted[i, j] = True
                assert np.all(raw_h[0, :, i, j] == np.float64(np.float32(delta) * np.float32(kappa)))
    q_h, k_h, v_h = qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:]
    x = np.where(vis, scale * raw_h, -np.inf)
    mx = x.max(-1, keepdims=True)
    e = np.exp(x - mx)
    p = e / e.sum(-1, keepdims=True)
    want_s, want_g = relevance_q_reference(spv, q_h, q_pre[:, :qd], k_h, v_h, z[:, :qd], None, p, raw_h,
                                           cos.astype(np.float64), sin.astype(np.float64), n, L, H, Hkv, D, scale,
                                           eps, 1, 1, 1)
    s_buf, p_buf, g = G.empty((n, H, L, L)), G.empty((n, H, L, L)), G.empty((n * L, qd))
    d = N.AttnRelDesc()
    d.n, d.l, d.heads, d.kv_heads, d.head_dim = n, L, H, Hkv, D
    d.scale, d.eps, d.causal, d.rope, d.rope_half = scale, eps, 1, 1, 1
    d.spv, d.ld_spv = spv_d.data_ptr(), qd
    d.v, d.ld_v, d.k, d.ld_k = base + 4 * (qd + kvd), w3, base + 4 * qd, w3
    d.s, d.p_out = G.ptr(s_buf).value, G.ptr(p_buf).value
    d.q, d.ld_q, d.q_pre, d.ld_q_pre = base, w3, pre_d.data_ptr(), qd + kvd
    d.z, d.ld_z = z_d.data_ptr(), w3
    d.cos_t, d.sin_t = cos_d.data_ptr(), sin_d.data_ptr()
    d.g, d.ld_g = G.ptr(g).value, qd
    d.ctx, d.ld_ctx, d.stats = G.ptr(ctx2).value, qd, G.ptr(stats).value
    assert N.pxk().pxk_attention_relevance_q(ctypes.byref(d), G.stream()) == 0, N.pxk().pxk_last_error()
    got_s, got_p = G.host(s_buf), G.host(p_buf)
    G.assert_close(got_p[..., vis], p[..., vis], 1e-5, "P")
    G.assert_close(got_s[..., vis], want_s[..., vis], 1e-4, "s")
    G.assert_close(got_s[..., planted], want_s[..., planted], 1e-4, "s at the planted scores near 0")
    G.assert_close(G.host(g), want_g, 1e-4, "g_q")
    # The key side over the s and P the q side wrote.
    k_pre, z_k, z_v = q_pre[:, qd:], z[:, qd:qd + kvd], z[:, qd + kvd:]
    want_kv = relevance_kv_reference(want_s, p, q_h, spv, k_h, k_pre, v_h, z_k, z_v, None, None,
                                     cos.astype(np.float64), sin.astype(np.float64), n, L, H, Hkv, D, eps, 1, 1, 1)
    gk, gv = G.empty((n * L, kvd)), G.empty((n * L, kvd))
    kd = N.AttnRelKvDesc()
    kd.n, kd.l, kd.heads, kd.kv_heads, kd.head_dim = n, L, H, Hkv, D
    kd.eps, kd.causal, kd.rope, kd.rope_half = eps, 1, 1, 1
    kd.q, kd.ld_q, kd.spv, kd.ld_spv = base, w3, spv_d.data_ptr(), qd
    kd.k, kd.ld_k, kd.k_pre, kd.ld_k_pre = base + 4 * qd, w3, pre_d.data_ptr() + 4 * qd, qd + kvd
    kd.v, kd.ld_v = base + 4 * (qd + kvd), w3
    kd.z_k, kd.z_v, kd.ld_z = z_d.data_ptr() + 4 * qd, z_d.data_ptr() + 4 * (qd + kvd), w3
    kd.cos_t, kd.sin_t = cos_d.data_ptr(), sin_d.data_ptr()
    kd.g_k, kd.g_v, kd.ld_g = G.ptr(gk).value, G.ptr(gv).value, kvd
    kd.s, kd.p = G.ptr(s_buf).value, G.ptr(p_buf).value
    assert N.pxk().pxk_attention_relevance_kv(ctypes.byref(kd), G.stream()) == 0, N.pxk().pxk_last_error()
    G.assert_close(G.host(gk), want_kv[2], 1e-4, "g_k")
    G.assert_close(G.host(gv), want_kv[3], 1e-4, "g_v")


def gqa_plan():
    fn = N.pxk().pxk_attention_forward_gqa
    fn.argtypes = [ctypes.c_int64] * 4
    fn.restype = ctypes.c_int
    return fn


def test_gqa_shared_forward_plan():
    """CPU-side: which statistics-form shapes run GQA-shared (the shapes the rule was measured on)."""
    plan = gqa_plan()
    assert plan(8, 1024, 32, 8) == 1 and plan(4, 1024, 32, 8) == 1 and plan(2, 1024, 32, 8) == 1
    assert plan(1, 1024, 32, 8) == 0 and plan(1, 2048, 32, 8) == 0 and plan(1, 4096, 16, 8) == 0
    assert plan(1, 512, 9, 3) == 0 and plan(4, 512, 9, 3) == 0  # the 135M shape: the per-head kernel
    assert plan(2, 1024, 16, 2) == 0  # four (sequence, KV head) workgroups per row block
    assert plan(16, 512, 40, 8) == 0  # five query heads per KV head: no GQA-shared build
    assert plan(16, 16, 32, 8) == 0  # 128 workgroups in all
    assert plan(0, 512, 32, 8) == 0 and plan(8, 1024, 30, 8) == 0 and plan(8, 0, 32, 8) == 0


@gpu
@pytest.mark.parametrize("causal", [1, 0])
@pytest.mark.parametrize("n,L,H,Hkv,D", [(4, 512, 8, 4, 64), (2, 500, 24, 8, 40), (4, 520, 16, 4, 32),
                                         (16, 512, 8, 1, 12), (4, 512, 8, 4, 128)])
def test_gqa_shared_forward_matches_numpy(n, L, H, Hkv, D, causal):
    """The statistics form on shapes that run GQA-shared (one workgroup per KV head and 16-row block,
    a wave per query head over all of the block's key tiles, K / V tiles through LDS): ctx and the
    rows' max and 1 / sum against float64 numpy, ragged lengths and head_dims below a 16 multiple
    included; and two launches bitwise equal."""
    print("gqa forward n=%d L=%d H=%d Hkv=%d D=%d causal=%d" % (n, L, H, Hkv, D, causal), flush=True)
    assert gqa_plan()(n, L, H, Hkv) == 1
    qd, kvd = H * D, Hkv * D
    w3 = qd + 2 * kvd
    qkv = G.uniform((n * L, w3), 31 + L + D)
    scale = 1.0 / np.sqrt(D)
    qkv_d = G.dev(qkv)
    base = qkv_d.data_ptr()
    outs = []
    for _ in range(2):
        stats, ctx = G.empty((n, H, L, 2)), G.empty((n * L, qd))
        N.call("pxk_attention_forward_stats", base, w3, base + 4 * qd, w3, base + 4 * (qd + kvd), w3, None, None,
               G.ptr(stats), G.ptr(ctx), qd, n, L, H, Hkv, D, scale, causal, G.stream())
        outs.append((G.host(stats), G.host(ctx)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    raw, p, want_ctx, vis = attention_reference(qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:], n, L, H, Hkv, D,
                                                scale, causal)
    x = np.where(vis, scale * raw, -np.inf)
    m = x.max(-1)
    ssum = np.exp(x - m[..., None]).sum(-1)
    got_st, got_ctx = outs[0]
    G.assert_close(got_st[..., 0], m, 1e-4, "row max")
    G.assert_close(got_st[..., 1], 1.0 / ssum, 1e-4, "1 / row sum")
    G.assert_close(got_ctx, want_ctx, 1e-4, "ctx")


@gpu
@pytest.mark.parametrize("causal", [1, 0])
@pytest.mark.parametrize("n,L,H,Hkv,D,rope,half,bias", [(4, 512, 8, 4, 64, 1, 1, 0), (2, 500, 24, 8, 40, 1, 0, 1),
                                                       (16, 512, 8, 1, 12, 0, 0, 1), (4, 520, 16, 4, 32, 1, 1, 1)])
def test_gqa_shared_q_relevance_matches_numpy(n, L, H, Hkv, D, rope, half, bias, causal):
    """The recomputing q side on shapes that run GQA-shared (one workgroup per KV head and 16-row
    block, a wave per query head over all of the block's key tiles, K / V tiles through LDS), with
    the checks of test_fused_attention_relevance_matches_numpy: s and P on the visible keys, zeros
    at the masked keys of the diagonal tiles, the row sums s_pv . ctx and g_q, against float64."""
    assert gqa_plan()(n, L, H, Hkv) == 1
    test_fused_attention_relevance_matches_numpy(n, L, H, Hkv, D, causal, rope, half, bias, 1)
