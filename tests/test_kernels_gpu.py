"""Kernel-level parity of libpxk_gfx950.so (called through its C ABI) against the CPU oracle.

The reference's primitive contract (tests/backend_primitive_equivalence_cases.hpp:22-31, 66-75):
seeded uniform(-1, 1) inputs, non-square shapes, |gpu - cpu| <= 1e-4. GEMM tolerances scale with
K, since fp32 MFMA accumulation order differs from the CPU's sequential sum.
"""
import ctypes
import re

import numpy as np
import pytest

import gpu_util as G
import oracle_ctypes as oc
from pulsatrix_amd import native as N

gpu = pytest.mark.gpu


def skip_if_device_present():
    """The argument-rejection tests hand the launchers placeholder pointers and rely on host-side
    validation refusing them. Where a GPU is visible they are skipped, so a regression in that
    validation can never launch a kernel on a placeholder address."""
    if N.host().pxa_device_count() > 0:
        pytest.skip("a GPU is present: placeholder-pointer rejection tests run only without one")


def test_library_exports_every_declared_symbol():
    """CPU-side: the kernel library loads and exports each entry point include/pxk.h declares."""
    header = open(oc.ROOT + "/include/pxk.h").read()
    names = sorted(set(re.findall(r"\b(pxk_[a-z0-9_]+)\s*\(", header)))
    lib = N.pxk()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert len(names) > 30
    assert lib.pxk_gemm_supported(0, 1, N.PRO_DIV_STAB, N.EPI_MUL_X) == 1
    assert lib.pxk_gemm_supported(1, 1, N.PRO_DIV_STAB, N.EPI_SWIGLU_REL) == 0


def test_gemm_rejects_bad_descriptors_without_launching():
    """CPU-side: validation happens on the host, before any launch."""
    skip_if_device_present()
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = 4, 4, 4, 1, 1, 1
    d.epilogue = 99
    assert N.pxk().pxk_gemm(ctypes.byref(d), None) == 1
    d.epilogue = N.EPI_STORE
    d.batch, d.inner = 3, 2  # batch must be a multiple of inner
    assert N.pxk().pxk_gemm(ctypes.byref(d), None) == 1


def test_decode_and_row_entry_points_reject_bad_arguments_without_launching():
    """CPU-side: the decode, fused-norm and repeat launchers validate on the host (the reference
    throws on the same misuse; here the C ABI returns PXK_ERR_INVALID with a message)."""
    skip_if_device_present()
    lib = N.pxk()
    p = ctypes.c_void_p(4096)
    f = ctypes.c_float
    # QK-Norm needs both scales
    assert lib.pxk_decode_rope_append(p, 64, p, 64, p, 64, p, p, p, 64, 1, p, p, p, 1, 1, 1, 64, 1, 1, p, None,
                                      f(1e-6), None) == 1
    assert b"both" in lib.pxk_last_error()
    # the cache must hold `positions`
    assert lib.pxk_decode_rope_append(p, 64, p, 64, p, 64, p, p, p, 63, 1, p, p, p, 1, 1, 1, 64, 1, 1, None, None,
                                      f(0.0), None) == 1
    # the next norm needs its scale; NULL operands
    assert lib.pxk_rms_norm_add(p, p, p, f(1e-6), p, None, f(1e-6), p, 4, 64, None) == 1
    assert lib.pxk_rms_norm_add(None, p, p, f(1e-6), p, None, f(1e-6), None, 4, 64, None) == 1
    assert lib.pxk_repeat_block(p, -1, 2, None) == 1 and lib.pxk_repeat_block(p, 8, 0, None) == 1
    assert lib.pxk_repeat_block(p, 8, 1, None) == 0  # one copy: nothing to write
    # the pick needs its workspace
    assert lib.pxk_decode_pick(p, 10, 2, 10, p, 4, p, None, 0, p, None, 0, None) == 3
    assert lib.pxk_decode_attention(p, p, p, 64, p, p, 1, 1, 1, 64, 0, 1, f(1.0), None, 0, None) == 3


class SeedHeadDesc(ctypes.Structure):
    """pxk_seed_head_desc (include/pxk.h)."""
    _fields_ = [("logits", ctypes.c_void_p), ("x", ctypes.c_void_p), ("e", ctypes.c_void_p),
                ("n", ctypes.c_int64), ("l", ctypes.c_int64), ("vocab", ctypes.c_int64), ("d", ctypes.c_int64),
                ("eps", ctypes.c_float), ("unit", ctypes.c_int32), ("targets_in", ctypes.c_void_p),
                ("targets_out", ctypes.c_void_p), ("r", ctypes.c_void_p), ("a", ctypes.c_void_p),
                ("b", ctypes.c_void_p), ("s", ctypes.c_void_p), ("r_a", ctypes.c_void_p), ("r_b", ctypes.c_void_p),
                ("b_den", ctypes.c_void_p), ("b_den_bias", ctypes.c_void_p)]


def test_seed_head_relevance_rejects_bad_descriptors_without_launching():
    """CPU-side: a b_den without the split (or a bias without b_den) is refused before the targets
    kernel launches, so nothing is written (a launch here would fail with PXK_ERR_LAUNCH instead)."""
    skip_if_device_present()
    lib = N.pxk()
    p = 4096
    d = SeedHeadDesc(logits=p, x=p, e=p, n=1, l=4, vocab=16, d=8, eps=1e-9, unit=0, targets_out=p, r=p, b_den=p)
    assert lib.pxk_lm_seed_head_relevance(ctypes.byref(d), None) == 1
    assert b"b_den belongs to the split" in lib.pxk_last_error()
    d = SeedHeadDesc(logits=p, x=p, e=p, n=1, l=4, vocab=16, d=8, eps=1e-9, unit=0, targets_out=p, a=p, b=p, s=p,
                     r_a=p, r_b=p, b_den_bias=p)
    assert lib.pxk_lm_seed_head_relevance(ctypes.byref(d), None) == 1
    assert b"b_den belongs to the split" in lib.pxk_last_error()


def gemm_tol(k):
    return 1e-4 * max(1.0, k / 1024.0)


@gpu
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 7, 3), (64, 64, 64), (130, 70, 33), (257, 129, 131),
                                   (512, 576, 192)])
def test_gemm_ex_matches_oracle(ta, tb, m, k, n):
    a = G.uniform((k, m) if ta else (m, k), 1)
    b = G.uniform((n, k) if tb else (k, n), 2)
    ref = np.empty((m, n), np.float32)
    G.oracle_call("pxo_gemm_ex", a, ta, b, tb, ref, m, k, n, 0.0)
    out = G.empty((m, n))
    N.call("pxk_gemm_ex", G.ptr(G.dev(a)), ta, G.ptr(G.dev(b)), tb, G.ptr(out), m, k, n, 0.0, None, 0, G.stream())
    G.assert_close(G.host(out), ref, gemm_tol(k), "gemm_ex")


@gpu
def test_gemm_ex_beta_accumulates():
    m, k, n = 96, 80, 72
    a, b, c0 = G.uniform((m, k), 3), G.uniform((k, n), 4), G.uniform((m, n), 5)
    ref = c0.copy()
    G.oracle_call("pxo_gemm_ex", a, 0, b, 0, ref, m, k, n, 1.0)
    out = G.dev(c0)
    N.call("pxk_gemm_ex", G.ptr(G.dev(a)), 0, G.ptr(G.dev(b)), 0, G.ptr(out), m, k, n, 1.0, None, 0, G.stream())
    G.assert_close(G.host(out), ref, 1e-4, "beta")


def plain_desc(m, n, k, a, b, c, ta=0, tb=0):
    d = N.GemmDesc()
    d.m, d.n, d.k = m, n, k
    d.batch = d.inner = d.kgroups = 1
    d.trans_a, d.trans_b = ta, tb
    d.a = N.operand(G.ptr(a).value, m if ta else k)
    d.b = N.operand(G.ptr(b).value, k if tb else n)
    d.c = N.operand(G.ptr(c).value, n)
    return d


@gpu
@pytest.mark.parametrize("splits", [2, 8])
@pytest.mark.parametrize("m,k,n", [(512, 4096, 576), (100, 1000, 60)])
def test_split_k_matches_single_pass(splits, m, k, n):
    a, b = G.dev(G.uniform((m, k), 6)), G.dev(G.uniform((k, n), 7))
    one, many = G.empty((m, n)), G.empty((m, n))
    d1 = plain_desc(m, n, k, a, b, one)
    d1.splits = 1
    N.gemm(d1, G.stream())
    d2 = plain_desc(m, n, k, a, b, many)
    d2.splits = splits
    ws = G.empty((splits * m * n,), 0.0)
    d2.workspace, d2.workspace_bytes = G.ptr(ws).value, splits * m * n * 4
    N.gemm(d2, G.stream())
    ref = G.host(a).astype(np.float64) @ G.host(b).astype(np.float64)
    G.assert_close(G.host(one), ref, gemm_tol(k), "single")
    G.assert_close(G.host(many), ref, gemm_tol(k), "split")


@gpu
def test_split_k_requires_workspace():
    m, k, n = 64, 1024, 64
    a, b, c = G.dev(G.uniform((m, k), 1)), G.dev(G.uniform((k, n), 2)), G.empty((m, n))
    d = plain_desc(m, n, k, a, b, c)
    d.splits = 4
    assert N.pxk().pxk_gemm(ctypes.byref(d), None) == 3


def launch(d, tile, splits):
    """pxk_gemm with a pinned tile shape / split count (0 = the library's choice)."""
    d.tile, d.splits = tile, splits
    nbytes = N.gemm_workspace(d)
    if nbytes:
        ws = G.empty((nbytes // 4,), 0.0)
        d.workspace, d.workspace_bytes = G.ptr(ws).value, nbytes
    N.gemm(d, G.stream())


@gpu
@pytest.mark.parametrize("tile,splits", [(0, 0), (N.TILE_128x128, 1), (N.TILE_64x64, 2), (N.TILE_32x64, 1),
                                         (N.TILE_32x32, 3)])
@pytest.mark.parametrize("L,H,Hkv,D", [(37, 4, 2, 16), (128, 9, 3, 64)])
def test_gqa_attention_gemms_match_numpy(L, H, Hkv, D, tile, splits):
    """Scores (TRI), P @ V (K <= M) and the GQA key sum (kgroups, K >= M) with head-packed layouts."""
    torch = G.torch_cuda()
    grp = H // Hkv
    q = G.uniform((L, H * D), 1)
    kk = G.uniform((L, Hkv * D), 2)
    p = np.tril(G.uniform((H, L, L), 3, 0.0, 1.0))
    qd, kd, pd = G.dev(q), G.dev(kk), G.dev(p)
    raw = G.empty((H, L, L), 0.0)
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = L, L, D, H, H, 1
    d.trans_b, d.causal = 1, N.CAUSAL_TRI
    d.a = N.operand(G.ptr(qd).value, H * D, 0, D)
    d.b = N.operand(G.ptr(kd).value, Hkv * D, 0, D, grp)
    d.c = N.operand(G.ptr(raw).value, L, 0, L * L)
    launch(d, tile, splits)
    qh = q.reshape(L, H, D).transpose(1, 0, 2).astype(np.float64)
    kh = kk.reshape(L, Hkv, D).transpose(1, 0, 2).astype(np.float64)
    ref = np.einsum("hid,hjd->hij", qh, np.repeat(kh, grp, axis=0))
    got = G.host(raw)
    lower = np.tril(np.ones((L, L), bool))
    G.assert_close(got[:, lower], ref[:, lower], 1e-4, "scores")
    # context = P @ V into the head-packed (L, H*D) layout, sum over k <= m only
    ctx = G.empty((L, H * D))
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = L, D, L, H, H, 1
    d.causal = N.CAUSAL_K_LE_M
    d.a = N.operand(G.ptr(pd).value, L, 0, L * L)
    d.b = N.operand(G.ptr(kd).value, Hkv * D, 0, D, grp)
    d.c = N.operand(G.ptr(ctx).value, H * D, 0, D)
    launch(d, tile, splits)
    ref = np.einsum("hij,hjd->ihd", p.astype(np.float64), np.repeat(kh, grp, axis=0)).reshape(L, H * D)
    G.assert_close(G.host(ctx), ref, 1e-4, "context")
    # per KV head: sum over its query heads of P_h^T @ Q_h, i >= j
    out = G.empty((L, Hkv * D))
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = L, D, L, Hkv, Hkv, grp
    d.trans_a, d.causal = 1, N.CAUSAL_K_GE_M
    d.a = N.operand(G.ptr(pd).value, L, 0, grp * L * L, 0, L * L)
    d.b = N.operand(G.ptr(qd).value, H * D, 0, grp * D, 0, D)
    d.c = N.operand(G.ptr(out).value, Hkv * D, 0, D)
    launch(d, tile, splits)
    per_head = np.einsum("hij,hid->hjd", p.astype(np.float64), qh)
    ref = per_head.reshape(Hkv, grp, L, D).sum(axis=1).transpose(1, 0, 2).reshape(L, Hkv * D)
    G.assert_close(G.host(out), ref, 1e-4, "kv sum")
    del torch


@gpu
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("n,i,o", [(7, 12, 5), (128, 576, 1536)])
def test_linear_relevance_fused_matches_oracle(bias, n, i, o):
    """DIV_STAB prologue + MUL_X epilogue = lrp_rules::linear (both rules)."""
    x, w = G.uniform((n, i), 1), G.uniform((i, o), 2) * 0.1
    b = G.uniform((o,), 3) if bias else None
    pre, _ = oc.linear_forward(x, w, b)
    r = G.uniform((n, o), 4)
    for bid, eps in ((True, 1e-9), (False, 1e-6)):
        ref = oc.linear_relevance(x, w, b, pre, r, eps, bid)
        xd, wd, zd, rd = G.dev(x), G.dev(w), G.dev(pre), G.dev(r)
        bd = G.dev(b) if (bias and bid) else None
        out = G.empty((n, i))
        d = N.GemmDesc()
        d.m, d.n, d.k, d.batch, d.inner, d.kgroups = n, i, o, 1, 1, 1
        d.trans_b, d.prologue, d.epilogue, d.eps = 1, N.PRO_DIV_STAB, N.EPI_MUL_X, eps
        d.a = N.operand(G.ptr(rd).value, o)
        d.z = N.operand(G.ptr(zd).value, o)
        if bd is not None:
            d.z_bias = N.operand(G.ptr(bd).value, 0)
        d.b = N.operand(G.ptr(wd).value, o)
        d.c = N.operand(G.ptr(out).value, i)
        d.x = N.operand(G.ptr(xd).value, i)
        N.gemm(d, G.stream())
        G.assert_close(G.host(out), ref, 1e-4, "linear relevance bid=%s" % bid)


@gpu
def test_elementwise_ops_match_oracle():
    n = 100003  # odd: exercises the scalar tail
    a, b, r = G.uniform((n,), 1), G.uniform((n,), 2), G.uniform((n,), 3)
    ad, bd, rd = G.dev(a), G.dev(b), G.dev(r)
    s = G.stream()
    for op in range(8):
        ref = np.empty_like(a)
        G.oracle_call("pxo_elementwise", op, a, ref, n)
        out = G.empty((n,))
        N.call("pxk_elementwise", op, G.ptr(ad), G.ptr(out), n, s)
        G.assert_close(G.host(out), ref, 1e-6, "op %d" % op)
    for name in ("add", "mul"):
        ref = np.empty_like(a)
        G.oracle_call("pxo_" + name, a, b, ref, n)
        out = G.empty((n,))
        N.call("pxk_" + name, G.ptr(ad), G.ptr(bd), G.ptr(out), n, s)
        assert np.array_equal(G.host(out), ref), name  # one fp32 op: bit-exact
    for beta in (0.0, -0.5):
        ref = np.empty_like(a)
        G.oracle_call("pxo_axpby", 1.5, a, beta, b, ref, n)
        out = G.empty((n,))
        N.call("pxk_axpby", 1.5, G.ptr(ad), beta, G.ptr(bd), G.ptr(out), n, s)
        G.assert_close(G.host(out), ref, 1e-6, "axpby")
    ra, rb = np.empty_like(a), np.empty_like(a)
    G.oracle_call("pxo_lrp_residual_split", a, b, r, ra, rb, n, 1e-6)
    oa, ob = G.empty((n,)), G.empty((n,))
    N.call("pxk_lrp_residual_split", G.ptr(ad), G.ptr(bd), G.ptr(rd), G.ptr(oa), G.ptr(ob), n, 1e-6, s)
    assert np.array_equal(G.host(oa), ra) and np.array_equal(G.host(ob), rb)
    ref = np.empty_like(a)
    G.oracle_call("pxo_lrp_bilinear_elementwise", a, b, r, ref, n, 1e-9)
    out = G.empty((n,))
    N.call("pxk_lrp_bilinear_elementwise", G.ptr(ad), G.ptr(bd), G.ptr(rd), G.ptr(out), n, 1e-9, s)
    assert np.array_equal(G.host(out), ref)
    for mode in (0, 1, 2):
        ref = np.empty_like(a)
        G.oracle_call("pxo_lrp_stabilized_divide", r, a, b, ref, n, 1e-6, mode)
        out = G.empty((n,))
        N.call("pxk_lrp_stabilized_divide", G.ptr(rd), G.ptr(ad), G.ptr(bd), G.ptr(out), n, 1e-6, mode, s)
        assert np.array_equal(G.host(out), ref), mode


@gpu
@pytest.mark.parametrize("rows,cols,offset", [(7, 100, 0), (513, 576, 0), (64, 1024, 0), (130, 2048, 0),
                                              (33, 4096, 0), (9, 4100, 0), (17, 6, 0), (40, 576, 1)])
def test_rms_norm_widths_match_oracle(rows, cols, offset):
    """Every register-resident width class (2, 3, 4, 8, 16 float4 per lane), the scalar fallback for
    wide, odd and misaligned rows, and rows_rms, against the oracle (row_math.hpp:59-71)."""
    x, g = G.uniform((rows, cols), 4 + cols), G.uniform((cols,), 5)
    ref, rms = np.empty_like(x), np.empty((rows,), np.float32)
    G.oracle_call("pxo_rms_norm_forward", x, g, ref, rms, rows, cols, 1e-5)
    xd = G.dev(np.concatenate([np.zeros(offset, np.float32), x.ravel()]))
    out, orms = G.empty((rows * cols + offset,)), G.empty((rows,))
    N.call("pxk_rms_norm_forward", xd.data_ptr() + 4 * offset, G.ptr(G.dev(g)), out.data_ptr() + 4 * offset,
           G.ptr(orms), rows, cols, 1e-5, G.stream())
    G.assert_close(G.host(out)[offset:].reshape(rows, cols), ref, 1e-5, "rmsnorm")
    G.assert_close(G.host(orms), rms, 1e-5, "rms")


@gpu
@pytest.mark.parametrize("rows,cols,offset,with_next", [(4, 640, 0, 1), (37, 576, 0, 1), (5, 2048, 0, 1),
                                                       (9, 100, 0, 0), (6, 4100, 0, 1), (8, 640, 1, 1)])
def test_rms_norm_add_matches_oracle_composition(rows, cols, offset, with_next):
    """A sandwich block's post-norm + residual add + next norm in one kernel, against the oracle's
    rms_norm_forward, the add and rms_norm_forward again; register-resident widths (2, 3, 8 float4 per
    lane), the scalar fallback for wide and misaligned rows, and without the next norm."""
    x, a = G.uniform((rows, cols), 11), G.uniform((rows, cols), 12, -3, 3)
    ga, gy = G.uniform((cols,), 13, 0.5, 1.5), G.uniform((cols,), 14, 0.5, 1.5)
    an, rms = np.empty_like(a), np.empty((rows,), np.float32)
    G.oracle_call("pxo_rms_norm_forward", a, ga, an, rms, rows, cols, 1e-6)
    y_ref = (x + an).astype(np.float32)
    yn_ref = np.empty_like(y_ref)
    G.oracle_call("pxo_rms_norm_forward", y_ref, gy, yn_ref, rms, rows, cols, 1e-5)
    pad = np.zeros(offset, np.float32)
    xd, ad = G.dev(np.concatenate([pad, x.ravel()])), G.dev(np.concatenate([pad, a.ravel()]))
    y, yn = G.empty((rows * cols + offset,)), G.empty((rows * cols + offset,))
    o = 4 * offset
    N.call("pxk_rms_norm_add", xd.data_ptr() + o, ad.data_ptr() + o, G.ptr(G.dev(ga)), 1e-6, y.data_ptr() + o,
           G.ptr(G.dev(gy)) if with_next else None, 1e-5, yn.data_ptr() + o if with_next else None, rows, cols,
           G.stream())
    G.assert_close(G.host(y)[offset:].reshape(rows, cols), y_ref, 1e-5, "norm + add")
    if with_next:
        G.assert_close(G.host(yn)[offset:].reshape(rows, cols), yn_ref, 1e-5, "next norm")
    else:
        assert np.all(np.isnan(G.host(yn)))  # untouched


@gpu
def test_row_kernels_match_oracle():
    rows, cols = 333, 2048
    x, g = G.uniform((rows, cols), 1), G.uniform((cols,), 2)
    s = G.stream()
    ref, rms = np.empty_like(x), np.empty((rows,), np.float32)
    G.oracle_call("pxo_rms_norm_forward", x, g, ref, rms, rows, cols, 1e-5)
    out, orms = G.empty((rows, cols)), G.empty((rows,))
    N.call("pxk_rms_norm_forward", G.ptr(G.dev(x)), G.ptr(G.dev(g)), G.ptr(out), G.ptr(orms), rows, cols, 1e-5, s)
    G.assert_close(G.host(out), ref, 1e-5, "rmsnorm")
    G.assert_close(G.host(orms), rms, 1e-5, "rms")
    ref = np.empty_like(x)
    G.oracle_call("pxo_softmax_rows", x, ref, rows, cols)
    out = G.empty((rows, cols))
    N.call("pxk_softmax_rows", G.ptr(G.dev(x)), G.ptr(out), rows, cols, s)
    G.assert_close(G.host(out), ref, 1e-6, "softmax")
    y, r = ref, G.uniform((rows, cols), 3)
    ref2 = np.empty_like(x)
    G.oracle_call("pxo_lrp_softmax_rows", x, y, r, ref2, rows, cols)
    out = G.empty((rows, cols))
    N.call("pxk_lrp_softmax_rows", G.ptr(G.dev(x)), G.ptr(G.dev(y)), G.ptr(G.dev(r)), G.ptr(out), rows, cols, s)
    G.assert_close(G.host(out), ref2, 1e-5, "lrp softmax")
    out = G.empty((rows,))
    N.call("pxk_row_sums", G.ptr(G.dev(x)), G.ptr(out), rows, cols, s)
    G.assert_close(G.host(out), x.astype(np.float64).sum(axis=1), 1e-5, "row sums")
    # deterministic two-pass sum / dot
    part = G.empty((N.pxk().pxk_reduce_partials(x.size) // 4,), 0.0)
    o1, o2 = G.empty((1,)), G.empty((1,))
    xd = G.dev(x)
    N.call("pxk_sum", G.ptr(xd), x.size, G.ptr(o1), G.ptr(part), s)
    N.call("pxk_sum", G.ptr(xd), x.size, G.ptr(o2), G.ptr(part), s)
    assert G.host(o1)[0] == G.host(o2)[0]
    assert abs(G.host(o1)[0] - x.astype(np.float64).sum()) < 1e-2
    N.call("pxk_dot", G.ptr(xd), G.ptr(xd), x.size, G.ptr(o1), G.ptr(part), s)
    assert abs(G.host(o1)[0] / (x.astype(np.float64) ** 2).sum() - 1) < 1e-5


@gpu
@pytest.mark.parametrize("half", [0, 1])
def test_rope_kernels_match_oracle(half):
    slices, L, D = 6, 37, 64
    cs, sn = np.empty((L, D // 2), np.float32), np.empty((L, D // 2), np.float32)
    oc.oracle().lib.pxo_rope_tables(D, 10000.0, L, 0, oc.fptr(cs), oc.fptr(sn))
    x = G.uniform((slices, L, D), 1)
    s = G.stream()
    for inverse in (0, 1):
        ref = np.empty_like(x)
        G.oracle_call("pxo_rope_rotate", x, cs, sn, ref, slices, L, D, inverse, half)
        out = G.empty(x.shape)
        N.call("pxk_rope_rotate", G.ptr(G.dev(x)), G.ptr(G.dev(cs)), G.ptr(G.dev(sn)), G.ptr(out), slices, L, D,
               inverse, half, s)
        G.assert_close(G.host(out), ref, 1e-6, "rope")  # the device contracts a*b - c*d into an FMA
    y = np.empty_like(x)
    G.oracle_call("pxo_rope_rotate", x, cs, sn, y, slices, L, D, 0, half)
    r = G.uniform(x.shape, 2)
    ref = np.empty_like(x)
    G.oracle_call("pxo_lrp_rope", x, y, r, cs, sn, ref, slices, L, D, 1e-9, half)
    out = G.empty(x.shape)
    N.call("pxk_lrp_rope", G.ptr(G.dev(x)), G.ptr(G.dev(y)), G.ptr(G.dev(r)), G.ptr(G.dev(cs)), G.ptr(G.dev(sn)),
           G.ptr(out), slices, L, D, 1e-9, half, s)
    G.assert_close(G.host(out), ref, 1e-5, "lrp rope")


@gpu
def test_data_movement_kernels_match_oracle():
    s = G.stream()
    x = G.uniform((2, 5, 3, 7), 1)
    ref = np.empty((2, 3, 5, 7), np.float32)
    G.oracle_call("pxo_permute_0213", x, ref, 2, 5, 3, 7)
    out = G.empty(ref.shape)
    N.call("pxk_permute_0213", G.ptr(G.dev(x)), G.ptr(out), 2, 5, 3, 7, s)
    assert np.array_equal(G.host(out), ref)
    sc = G.uniform((2, 3, 9, 9), 2)
    keep = (G.uniform((2, 9), 3) > -0.5).astype(np.float32)
    for causal, window, kp in ((1, 0, None), (1, 3, None), (0, 0, keep), (1, 0, keep)):
        ref = sc.copy()
        G.oracle_call("pxo_attention_mask_fill", ref, kp, 2, 3, 9, 9, causal, 0, window, -7.0)
        out = G.dev(sc)
        N.call("pxk_attention_mask_fill", G.ptr(out), G.ptr(G.dev(kp)) if kp is not None else None, 2, 3, 9, 9, causal,
               0, window, -7.0, s)
        assert np.array_equal(G.host(out), ref)
    table, idx = G.uniform((50, 24), 4), np.array([3, 0, 49, 7, 7], np.float32)
    ref = np.empty((5, 24), np.float32)
    G.oracle_call("pxo_gather_rows", table, idx, ref, 5, 24)
    out = G.empty((5, 24))
    N.call("pxk_gather_rows", G.ptr(G.dev(table)), G.ptr(G.dev(idx)), G.ptr(out), 5, 24, s)
    assert np.array_equal(G.host(out), ref)
    src = G.uniform((6, 10), 5)
    dst = G.uniform((6, 16), 6)
    ref = dst.copy()
    G.oracle_call("pxo_copy_2d", ref, 16, src, 10, 6, 10)
    out = G.dev(dst)
    N.call("pxk_copy_2d", G.ptr(out), 16, G.ptr(G.dev(src)), 10, 6, 10, s)
    assert np.array_equal(G.host(out), ref)
    acc = G.uniform((10,), 7)
    ref = acc.copy()
    G.oracle_call("pxo_accumulate_rows", src, ref, 6, 10)
    out = G.dev(acc)
    N.call("pxk_accumulate_rows", G.ptr(G.dev(src)), G.ptr(out), 6, 10, s)
    assert np.array_equal(G.host(out), ref)  # same order, one thread per column
    ref = acc.copy()
    G.oracle_call("pxo_column_sums", src, ref, 6, 10, 0.5)
    out = G.dev(acc)
    N.call("pxk_column_sums", G.ptr(G.dev(src)), G.ptr(out), 6, 10, 0.5, s)
    assert np.array_equal(G.host(out), ref)


@gpu
@pytest.mark.parametrize("causal,window", [(1, 0), (0, 0), (1, 7), (1, 1)])
def test_attention_row_kernels_match_oracle(causal, window):
    """pxk_attention_softmax / pxk_attention_lrp_scores = the module's op sequences on the oracle,
    causal, full, and causal with a sliding window (attention_mask_fill's window, row_math.hpp:117-126)."""
    H, L, scale, eps = 3, 45, 0.125, 1e-9
    raw = G.uniform((H, L, L), 1, -4, 4)
    scaled = np.empty_like(raw)
    G.oracle_call("pxo_axpby", scale, raw, 0.0, raw, scaled, raw.size)
    if causal:
        G.oracle_call("pxo_attention_mask_fill", scaled, None, 1, H, L, L, 1, 0, window,
                      float(np.finfo(np.float32).min))
    p_ref = np.empty_like(raw)
    G.oracle_call("pxo_softmax_rows", scaled, p_ref, H * L, L)
    s = G.stream()
    p = G.empty(raw.shape)
    rawd = G.dev(raw)
    N.call("pxk_attention_softmax", G.ptr(rawd), G.ptr(p), H, L, scale, causal, window, s)
    G.assert_close(G.host(p), p_ref, 1e-6, "softmax")
    r_attn = G.uniform((H, L, L), 2) * (p_ref > 0)
    r_sc = np.empty_like(raw)
    G.oracle_call("pxo_lrp_softmax_rows", scaled, p_ref, r_attn, r_sc, H * L, L)
    if causal:
        G.oracle_call("pxo_attention_mask_fill", r_sc, None, 1, H, L, L, 1, 0, window, 0.0)
    ref = r_sc / (2 * raw + eps * np.where(raw >= 0, 1, -1).astype(np.float32))
    out = G.empty(raw.shape)
    N.call("pxk_attention_lrp_scores", G.ptr(G.dev(r_attn)), G.ptr(G.dev(p_ref)), G.ptr(rawd), G.ptr(out), H, L,
           scale, eps, causal, window, s)
    G.assert_close(G.host(out), ref.astype(np.float32), 1e-5, "lrp scores")


@gpu
def test_lm_seed_picks_argmax_and_writes_one_hot():
    n, l, v = 3, 4, 1000
    logits = G.uniform((n, l, v), 1)
    logits[1, -1, 17] = 5.0
    logits[1, -1, 900] = 5.0  # tie: the lower index wins
    seed, tgt = G.empty((n, l, v)), G.keep(G.torch_cuda().empty(n, dtype=G.torch_cuda().int64, device="cuda"))
    N.call("pxk_lm_seed", G.ptr(G.dev(logits)), n, l, v, None, G.ptr(tgt), G.ptr(seed), 0, G.stream())
    got, t = G.host(seed), tgt.cpu().numpy()
    expect = np.argmax(logits[:, -1], axis=1)
    assert list(t) == list(expect) and t[1] == 17
    ref = np.zeros_like(logits)
    for i in range(n):
        ref[i, -1, expect[i]] = logits[i, -1, expect[i]]
    assert np.array_equal(got, ref)


@gpu
def test_embedding_ids_validated_on_device():
    """pxk_embedding_ids: llround (halves away from zero) and the [0, vocab) range check of
    embedding_module.cpp:48-59; out-of-range ids become 0 and set the status."""
    torch = G.torch_cuda()
    vocab = 50
    good = np.array([0, 49, 2.5, -0.4, 48.6, 7], np.float32)
    out, status = G.empty((good.size,)), G.keep(torch.full((1,), 7, dtype=torch.int32, device="cuda"))
    N.call("pxk_embedding_ids", G.ptr(G.dev(good)), good.size, vocab, G.ptr(out), G.ptr(status), G.stream())
    assert list(G.host(out)) == [0, 49, 3, 0, 49, 7] and int(status.cpu()[0]) == 0
    bad = np.array([3, -1, 50, np.nan, np.inf, 49.5, 1e9], np.float32)
    out = G.empty((bad.size,))
    N.call("pxk_embedding_ids", G.ptr(G.dev(bad)), bad.size, vocab, G.ptr(out), G.ptr(status), G.stream())
    assert list(G.host(out)) == [3, 0, 0, 0, 0, 0, 0] and int(status.cpu()[0]) == 1
    many = np.random.RandomState(3).randint(0, vocab, size=5000).astype(np.float32)
    out = G.empty((many.size,))
    N.call("pxk_embedding_ids", G.ptr(G.dev(many)), many.size, vocab, G.ptr(out), G.ptr(status), G.stream())
    assert np.array_equal(G.host(out), many) and int(status.cpu()[0]) == 0
