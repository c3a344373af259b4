"""Every (transpose, prologue, epilogue) combination of pxk_gemm on every tile shape and with
split-K, against float64 numpy.

The library picks a tile shape and split count per descriptor; the tuning override
(pxk_gemm_desc.tile, .splits) pins each one here so that every kernel instance the library can
launch is exercised, including ragged M/N/K edges and an odd split count that leaves uneven K
ranges. The fused prologue/epilogue semantics are the ones include/pxk.h states; the model
tests pin them end to end against the oracle (lrp_rules.cpp, multihead_attention_module.cpp).
"""
import ctypes

import numpy as np
import pytest

import gpu_util as G
from pulsatrix_amd import native as N

gpu = pytest.mark.gpu

COMBOS = [
    (0, 0, N.PRO_NONE, N.EPI_STORE), (0, 1, N.PRO_NONE, N.EPI_STORE), (1, 0, N.PRO_NONE, N.EPI_STORE),
    (1, 1, N.PRO_NONE, N.EPI_STORE), (0, 0, N.PRO_NONE, N.EPI_STORE_BIAS), (0, 0, N.PRO_NONE, N.EPI_ADD_RESID),
    (0, 0, N.PRO_NONE, N.EPI_MUL_X), (0, 1, N.PRO_NONE, N.EPI_MUL_X), (1, 0, N.PRO_NONE, N.EPI_MUL_X),
    (0, 0, N.PRO_DIV_STAB, N.EPI_MUL_X), (0, 1, N.PRO_DIV_STAB, N.EPI_MUL_X), (0, 1, N.PRO_DIV_STAB, N.EPI_SPV),
    (0, 0, N.PRO_NONE, N.EPI_ROPE_REL), (1, 0, N.PRO_NONE, N.EPI_ROPE_REL), (0, 0, N.PRO_NONE, N.EPI_VALUE_REL),
    (1, 0, N.PRO_NONE, N.EPI_VALUE_REL), (0, 1, N.PRO_DIV_STAB, N.EPI_SWIGLU_REL),
    (0, 1, N.PRO_NONE, N.EPI_MUL_X_SPLIT), (0, 0, N.PRO_DIV_STAB, N.EPI_MUL_X_SPLIT),
    (0, 1, N.PRO_DIV_STAB, N.EPI_MUL_X_SPLIT), (0, 0, N.PRO_NONE, N.EPI_ROPE_FWD),
    (0, 1, N.PRO_NONE, N.EPI_SPV), (0, 1, N.PRO_NONE, N.EPI_SWIGLU_REL),
]
TILES = [N.TILE_128x128, N.TILE_64x64, N.TILE_32x64, N.TILE_32x32, N.TILE_32x64_DIRECT, N.TILE_32x32_DIRECT,
         N.TILE_32x48_DIRECT, N.TILE_32x48]
TILE_BN = {N.TILE_128x128: 128, N.TILE_64x64: 64, N.TILE_32x64: 64, N.TILE_32x32: 32, N.TILE_32x64_DIRECT: 64,
           N.TILE_32x32_DIRECT: 32, N.TILE_32x48_DIRECT: 48, N.TILE_32x48: 48}
EPS = 1e-6


def away(shape, seed):
    """Uniform magnitudes in [0.5, 1.5) with random signs: denominators stay clear of zero."""
    r = np.random.RandomState(seed)
    return (r.uniform(0.5, 1.5, size=shape) * r.choice([-1.0, 1.0], size=shape)).astype(np.float32)


def stab(z):
    return z + EPS * np.where(z >= 0, 1.0, -1.0)


def rope_tables(m, d, theta=10000.0):
    half = d // 2
    inv = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / d)
    ang = np.arange(m, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rotate(y, cos, sin, D, half_layout):
    """rope_rotate (row_math.hpp:93-110) of every head_dim block of y's columns, position = row."""
    m, n = y.shape
    half = D // 2
    col = np.arange(n)
    d = col % D
    hb = col - d
    if half_layout:
        i = np.where(d < half, d, d - half)
        lo, hi = hb + i, hb + i + half
    else:
        i = d // 2
        lo, hi = hb + 2 * i, hb + 2 * i + 1
    c, s = cos[:, i], sin[:, i]
    x0, x1 = y[:, lo], y[:, hi]
    return np.where((col == lo)[None, :], x0 * c - x1 * s, x0 * s + x1 * c)


def expected(epi, acc, t, D, half_layout):
    """The epilogue of include/pxk.h on a float64 accumulator tile."""
    X, Y, W, Z, Z2, Z3, C0 = (t.get(k) for k in ("x", "y", "w", "z", "z2", "z3", "c0"))
    eb, eb2 = t.get("eb"), t.get("eb2")
    if epi == N.EPI_STORE:
        return {"c": acc + 0.5 * C0}
    if epi == N.EPI_STORE_BIAS:
        return {"c": acc, "c2": acc + eb}
    if epi == N.EPI_ADD_RESID:
        return {"c": acc, "c2": acc + eb, "c3": X + acc + eb}
    if epi == N.EPI_MUL_X:
        return {"c": Y + X * acc}
    if epi == N.EPI_SPV:
        return {"c": X * acc / (2 * X + EPS * np.where(X >= 0, 1.0, -1.0))}
    if epi == N.EPI_VALUE_REL:
        r = Y * acc
        return {"c": r, "c2": r / stab(Z + eb)}
    if epi == N.EPI_ROPE_FWD:
        y = acc + eb
        return {"c": acc, "c2": y, "c3": rotate(y, t["cos"], t["sin"], D, half_layout)}
    if epi == N.EPI_MUL_X_SPLIT:
        r = Y + X * acc
        den = stab(W)
        return {"c": (Z2 / den) * r, "c2": (Z3 / den) * r}
    if epi == N.EPI_SWIGLU_REL:
        c = Y * W
        rg = (c / (2 * c + EPS * np.where(c >= 0, 1.0, -1.0))) * (X * acc)
        return {"c": rg / stab(Z2 + eb), "c2": rg / stab(Z3 + eb2)}
    assert epi == N.EPI_ROPE_REL
    m, n = acc.shape
    cos, sin = t["cos"].astype(np.float64), t["sin"].astype(np.float64)
    half = D // 2
    col = np.arange(n)
    d = col % D
    hb = col - d
    if half_layout:
        i = np.where(d < half, d, d - half)
        lo, hi = hb + i, hb + i + half
    else:
        i = d // 2
        lo, hi = hb + 2 * i, hb + 2 * i + 1
    r_lo, r_hi = Y[:, lo] * acc[:, lo], Y[:, hi] * acc[:, hi]
    c, s = cos[:, i], sin[:, i]
    d0, d1 = stab(Y[:, lo]), stab(Y[:, hi])
    is_lo = (col == lo)[None, :]
    r_in = np.where(is_lo, X * c / d0 * r_lo + X * s / d1 * r_hi, X * -s / d0 * r_lo + X * c / d1 * r_hi)
    return {"c": r_in, "c2": r_in / stab(Z + eb)}


def run(d, splits):
    d.splits = splits
    if splits > 1:
        nbytes = N.gemm_workspace(d)
        assert nbytes >= splits * d.m * d.n * 4
        ws = G.empty((nbytes // 4,), 0.0)
        d.workspace, d.workspace_bytes = G.ptr(ws).value, nbytes
    return N.pxk().pxk_gemm(ctypes.byref(d), G.stream())


@gpu
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("combo", COMBOS, ids=lambda c: "ta%d_tb%d_pro%d_epi%d" % c)
def test_fused_gemm_on_every_tile(combo, tile, splits):
    ta, tb, pro, epi = combo
    rope = epi in (N.EPI_ROPE_REL, N.EPI_ROPE_FWD)
    D = 64 if rope and TILE_BN[tile] >= 64 else 16
    m, n, k = 77, 128, 150  # ragged M and K; N = whole heads for the RoPE rule
    a, b = G.uniform((k, m) if ta else (m, k), 1), G.uniform((n, k) if tb else (k, n), 2)
    t = {"x": G.uniform((m, n), 3), "y": away((m, n), 4), "w": away((m, n), 5), "z": away((m, n), 6),
         "z2": away((m, n), 7), "z3": away((m, n), 8), "c0": G.uniform((m, n), 9),
         "eb": G.uniform((n,), 10), "eb2": G.uniform((n,), 11)}
    t["cos"], t["sin"] = rope_tables(m, D)
    zp, zb = away((m, k), 12), G.uniform((k,), 13)  # prologue denominators over A's layout, bias over k
    a64 = (a.T if ta else a).astype(np.float64)
    b64 = (b.T if tb else b).astype(np.float64)
    if pro == N.PRO_DIV_STAB:
        a64 = a64 / stab(zp.astype(np.float64) + zb)
    acc = a64 @ b64
    t64 = {key: v.astype(np.float64) for key, v in t.items()}
    want = expected(epi, acc, t64, D, True)

    dv = {key: G.dev(v) for key, v in t.items()}
    outs = {key: G.empty((m, n)) for key in ("c", "c2", "c3")}
    if epi == N.EPI_STORE:
        outs["c"] = G.dev(t["c0"])
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = m, n, k, 1, 1, 1
    d.trans_a, d.trans_b, d.prologue, d.epilogue, d.eps, d.tile = ta, tb, pro, epi, EPS, tile
    d.beta = 0.5 if epi == N.EPI_STORE else 0.0
    d.a = N.operand(G.ptr(G.dev(a)).value, m if ta else k)
    d.b = N.operand(G.ptr(G.dev(b)).value, k if tb else n)
    for key in ("c", "c2", "c3"):
        setattr(d, key, N.operand(G.ptr(outs[key]).value, n))
    for key in ("x", "y", "w", "z2", "z3"):
        setattr(d, key, N.operand(G.ptr(dv[key]).value, n))
    if pro == N.PRO_DIV_STAB:
        d.z = N.operand(G.ptr(G.dev(zp)).value, k)
        d.z_bias = N.operand(G.ptr(G.dev(zb)).value, 0)
    else:
        d.z = N.operand(G.ptr(dv["z"]).value, n)
    d.e_bias = N.operand(G.ptr(dv["eb"]).value, 0)
    d.e_bias2 = N.operand(G.ptr(dv["eb2"]).value, 0)
    d.cos_t, d.sin_t = G.ptr(dv["cos"]).value, G.ptr(dv["sin"]).value
    d.head_dim, d.rope_half = D, 1
    d.rope_cols = n - D  # every head but the last is rotated
    if epi == N.EPI_MUL_X and pro == N.PRO_NONE and ta == 0 and tb == 0:
        d.y = N.operand(None, 0)  # the Y-less form: C = X * acc
        want = {"c": t64["x"] * acc}
    rc = run(d, splits)
    assert rc == 0, N.pxk().pxk_last_error()
    for key, ref in want.items():
        got = G.host(outs[key])
        if epi == N.EPI_ROPE_FWD and key == "c3":
            got, ref = got[:, :n - D], ref[:, :n - D]
        G.assert_close(got, ref, 2e-5, "tile %d splits %d output %s" % (tile, splits, key))


@gpu
@pytest.mark.parametrize("tile", [N.TILE_32x48_DIRECT, N.TILE_32x48])
@pytest.mark.parametrize("D", [2, 6])
def test_rope_forward_with_head_dim_not_a_multiple_of_4(D, tile):
    """ROPE_FWD where a thread's four columns cross a head boundary (head_dim 2 and 6 on 48-wide
    tiles, 96 columns, whole heads per tile), against float64 numpy."""
    m, n, k = 70, 96, 40
    a, b = G.uniform((m, k), 1), G.uniform((k, n), 2)
    eb = G.uniform((n,), 10)
    cos, sin = rope_tables(m, D)
    acc = a.astype(np.float64) @ b.astype(np.float64)
    t64 = {"eb": eb.astype(np.float64), "cos": cos.astype(np.float64), "sin": sin.astype(np.float64)}
    want = expected(N.EPI_ROPE_FWD, acc, t64, D, True)
    outs = {key: G.empty((m, n)) for key in ("c", "c2", "c3")}
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = m, n, k, 1, 1, 1
    d.epilogue, d.eps, d.tile = N.EPI_ROPE_FWD, EPS, tile
    d.a, d.b = N.operand(G.ptr(G.dev(a)).value, k), N.operand(G.ptr(G.dev(b)).value, n)
    for key in ("c", "c2", "c3"):
        setattr(d, key, N.operand(G.ptr(outs[key]).value, n))
    d.e_bias = N.operand(G.ptr(G.dev(eb)).value, 0)
    dc, ds = G.dev(cos), G.dev(sin)
    d.cos_t, d.sin_t = G.ptr(dc).value, G.ptr(ds).value
    d.head_dim, d.rope_half = D, 1
    d.rope_cols = n - 2 * D
    assert run(d, 1) == 0, N.pxk().pxk_last_error()
    for key, ref in want.items():
        got = G.host(outs[key])
        if key == "c3":
            got, ref = got[:, :n - 2 * D], ref[:, :n - 2 * D]
        G.assert_close(got, ref, 2e-5, "head_dim %d tile %d output %s" % (D, tile, key))


@gpu
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("tb,pro,bias", [(1, N.PRO_NONE, True), (0, N.PRO_DIV_STAB, False), (1, N.PRO_DIV_STAB, True)])
def test_split_share_divided_by_the_next_denominator(tb, pro, bias, tile, splits):
    """MUL_X_SPLIT with c2_den: C2 = ((Z3 / stab(W)) r) / stab(c2_den + c2_den_bias[n]), the share the next
    relevance GEMM then reads without its DIV_STAB prologue; C is the plain first share."""
    m, n, k = 77, 128, 150
    a, b = G.uniform((m, k), 1), G.uniform((n, k) if tb else (k, n), 2)
    x, y, w = G.uniform((m, n), 3), G.uniform((m, n), 4), away((m, n), 5)
    z2, z3, den, db = G.uniform((m, n), 7), G.uniform((m, n), 8), away((m, n), 9), G.uniform((n,), 10, -0.2, 0.2)
    zp, zb = away((m, k), 12), G.uniform((k,), 13)
    a64 = a.astype(np.float64)
    if pro == N.PRO_DIV_STAB:
        a64 = a64 / stab(zp.astype(np.float64) + zb)
    acc = a64 @ (b.T if tb else b).astype(np.float64)
    r = y + x * acc
    want_c = (z2 / stab(w)) * r
    want_c2 = (z3 / stab(w)) * r / stab(den + (db if bias else 0.0))
    c, c2 = G.empty((m, n)), G.empty((m, n))
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = m, n, k, 1, 1, 1
    d.trans_b, d.prologue, d.epilogue, d.eps, d.tile = tb, pro, N.EPI_MUL_X_SPLIT, EPS, tile
    d.a = N.operand(G.ptr(G.dev(a)).value, k)
    d.b = N.operand(G.ptr(G.dev(b)).value, k if tb else n)
    d.c, d.c2 = N.operand(G.ptr(c).value, n), N.operand(G.ptr(c2).value, n)
    for key, v in (("x", x), ("y", y), ("w", w), ("z2", z2), ("z3", z3), ("c2_den", den)):
        setattr(d, key, N.operand(G.ptr(G.dev(v)).value, n))
    if bias:
        d.c2_den_bias = N.operand(G.ptr(G.dev(db)).value, 0)
    if pro == N.PRO_DIV_STAB:
        d.z = N.operand(G.ptr(G.dev(zp)).value, k)
        d.z_bias = N.operand(G.ptr(G.dev(zb)).value, 0)
    rc = run(d, splits)
    assert rc == 0, N.pxk().pxk_last_error()
    G.assert_close(G.host(c), want_c, 2e-5, "tile %d splits %d first share" % (tile, splits))
    G.assert_close(G.host(c2), want_c2, 2e-5, "tile %d splits %d divided second share" % (tile, splits))


def skip_if_device_present():
    """Placeholder-pointer rejection tests rely on host validation refusing the descriptor; where a
    GPU is visible they are skipped, so a regression there can never launch on a placeholder."""
    if N.host().pxa_device_count() > 0:
        pytest.skip("a GPU is present: placeholder-pointer rejection tests run only without one")


def test_split_denominator_only_with_the_split_epilogue():
    """CPU-side: c2_den is refused on any other epilogue, and its bias without it; nothing is launched."""
    skip_if_device_present()
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = 8, 8, 8, 1, 1, 1
    for key in ("a", "b", "c", "c2", "x", "w", "z2", "z3"):
        setattr(d, key, N.operand(16, 8))  # never dereferenced: validation fails first
    d.epilogue = N.EPI_MUL_X
    d.c2_den = N.operand(16, 8)
    assert N.pxk().pxk_gemm(ctypes.byref(d), None) == 1
    assert b"c2_den" in N.pxk().pxk_last_error()
    d.epilogue = N.EPI_MUL_X_SPLIT
    d.c2_den = N.operand(None, 0)
    d.c2_den_bias = N.operand(16, 0)
    assert N.pxk().pxk_gemm(ctypes.byref(d), None) == 1


@gpu
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("tile", [t for t in TILES if TILE_BN[t] % 64 == 0])
def test_swiglu_gate_epilogue(tile, splits):
    """SWIGLU_FWD: B's columns alternate 32-wide gate and up blocks; C gets z as [gate | up] halves,
    C3 = silu(gate), C2 = silu(gate) * up (swiglu_module.cpp:80-88)."""
    m, k, F = 77, 150, 96
    a, wg, wu = G.uniform((m, k), 31), G.uniform((k, F), 32), G.uniform((k, F), 33)
    b = np.empty((k, 2 * F), np.float32)
    for blk in range(F // 32):
        b[:, 64 * blk:64 * blk + 32] = wg[:, 32 * blk:32 * blk + 32]
        b[:, 64 * blk + 32:64 * blk + 64] = wu[:, 32 * blk:32 * blk + 32]
    zg = a.astype(np.float64) @ wg.astype(np.float64)
    zu = a.astype(np.float64) @ wu.astype(np.float64)
    gp = zg / (1.0 + np.exp(-zg))
    c, hid, gpo = G.empty((m, 2 * F)), G.empty((m, F)), G.empty((m, F))
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = m, 2 * F, k, 1, 1, 1
    d.epilogue, d.tile = N.EPI_SWIGLU_FWD, tile
    d.a, d.b = N.operand(G.ptr(G.dev(a)).value, k), N.operand(G.ptr(G.dev(b)).value, 2 * F)
    d.c, d.c2, d.c3 = N.operand(G.ptr(c).value, 2 * F), N.operand(G.ptr(hid).value, F), N.operand(G.ptr(gpo).value, F)
    assert run(d, splits) == 0, N.pxk().pxk_last_error()
    G.assert_close(G.host(c), np.concatenate([zg, zu], axis=1), 2e-5, "z")
    G.assert_close(G.host(gpo), gp, 2e-5, "gate_post")
    G.assert_close(G.host(hid), gp * zu, 2e-5, "hidden")


@gpu
@pytest.mark.parametrize("half", [0, 1])
@pytest.mark.parametrize("tile", [N.TILE_64x64, N.TILE_32x64])
def test_rope_rule_epilogue_interleaved_and_half_pairs(half, tile):
    """ROPE_REL for both pair layouts (rotate-half and interleaved)."""
    m, n, k, D = 45, 128, 40, 64
    a, b = G.uniform((m, k), 21), G.uniform((k, n), 22)
    t = {"x": G.uniform((m, n), 23), "y": away((m, n), 24), "z": away((m, n), 25), "eb": G.uniform((n,), 26)}
    t["cos"], t["sin"] = rope_tables(m, D)
    acc = a.astype(np.float64) @ b.astype(np.float64)
    want = expected(N.EPI_ROPE_REL, acc, {key: v.astype(np.float64) for key, v in t.items()}, D, half == 1)
    dv = {key: G.dev(v) for key, v in t.items()}
    c, c2 = G.empty((m, n)), G.empty((m, n))
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = m, n, k, 1, 1, 1
    d.epilogue, d.eps, d.tile = N.EPI_ROPE_REL, EPS, tile
    d.a, d.b = N.operand(G.ptr(G.dev(a)).value, k), N.operand(G.ptr(G.dev(b)).value, n)
    d.c, d.c2 = N.operand(G.ptr(c).value, n), N.operand(G.ptr(c2).value, n)
    d.x, d.y, d.z = (N.operand(G.ptr(dv[key]).value, n) for key in ("x", "y", "z"))
    d.e_bias = N.operand(G.ptr(dv["eb"]).value, 0)
    d.cos_t, d.sin_t = G.ptr(dv["cos"]).value, G.ptr(dv["sin"]).value
    d.head_dim, d.rope_half = D, half
    assert run(d, 1) == 0, N.pxk().pxk_last_error()
    G.assert_close(G.host(c), want["c"], 2e-5, "r_in")
    G.assert_close(G.host(c2), want["c2"], 2e-5, "r_in / z")


def test_rope_rule_rejects_heads_wider_than_the_tile():
    """CPU-side: a 64-wide head cannot be split across 32-wide tiles; nothing is launched."""
    skip_if_device_present()
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = 8, 128, 8, 1, 1, 1
    d.epilogue, d.tile, d.head_dim = N.EPI_ROPE_REL, N.TILE_32x32, 64
    for key in ("a", "b", "c2", "x", "y", "z"):
        setattr(d, key, N.operand(16, 8))  # never dereferenced: validation fails first
    d.cos_t = d.sin_t = 16
    assert N.pxk().pxk_gemm(ctypes.byref(d), None) == 1
    assert b"do not fit" in N.pxk().pxk_last_error()


def gate_np(x, act):
    x = x.astype(np.float64)
    if act == 1:
        return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))
    return x / (1.0 + np.exp(-x))


@gpu
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("pro", [N.PRO_DIV_STAB, N.PRO_NONE])
@pytest.mark.parametrize("tile,splits", [(0, 0), (N.TILE_128x128, 1), (N.TILE_64x64, 3), (N.TILE_32x32_DIRECT, 1),
                                         (N.TILE_32x48_DIRECT, 1), (N.TILE_32x32, 1)])
def test_swiglu_rel_recomputes_its_factors_without_biases(act, pro, tile, splits):
    """SWIGLU_REL with X, Y and W omitted (no biases): gate_post = act(z_gate), up = z_up and hidden =
    gate_post * up recomputed in the epilogue, against float64 numpy of the stored-operand form; with
    the DIV_STAB prologue, or on an A already divided (the fused path's pre-divided relevance)."""
    m, k, F = 77, 150, 96
    a, b = G.uniform((m, k), 1), G.uniform((F, k), 2)
    zd, zg, zu = away((m, k), 6), G.uniform((m, F), 7, -3, 3), G.uniform((m, F), 8, -3, 3)
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = m, F, k, 1, 1, 1
    d.trans_b, d.prologue, d.epilogue, d.eps, d.gate_act = 1, pro, N.EPI_SWIGLU_REL, EPS, act
    c, c2 = G.empty((m, F)), G.empty((m, F))
    if pro == N.PRO_NONE:
        a = (a.astype(np.float64) / stab(zd)).astype(np.float32)
        zd = np.ones_like(zd)
    d.a = N.operand(G.ptr(G.dev(a)).value, k)
    if pro == N.PRO_DIV_STAB:
        d.z = N.operand(G.ptr(G.dev(zd)).value, k)
    d.b = N.operand(G.ptr(G.dev(b)).value, k)
    d.c, d.c2 = N.operand(G.ptr(c).value, F), N.operand(G.ptr(c2).value, F)
    d.z2, d.z3 = N.operand(G.ptr(G.dev(zg)).value, F), N.operand(G.ptr(G.dev(zu)).value, F)
    d.tile = tile
    assert run(d, splits) == 0, N.pxk().pxk_last_error()
    acc = (a.astype(np.float64) / (stab(zd) if pro == N.PRO_DIV_STAB else 1.0)) @ b.astype(np.float64).T
    gp, up = gate_np(zg, act), zu.astype(np.float64)
    cc = gp * up
    rg = (cc / (2 * cc + EPS * np.where(cc >= 0, 1.0, -1.0))) * (gp * up * acc)
    G.assert_close(G.host(c), rg / stab(zg), 1e-4, "gate share")
    G.assert_close(G.host(c2), rg / stab(zu), 1e-4, "up share")
    d.e_bias = N.operand(G.ptr(G.dev(zg[0])).value, 0)
    assert N.pxk().pxk_gemm(ctypes.byref(d), G.stream()) == 1  # recomputing is only for bias-free layers


def rms_norm_np(x, gamma, eps):
    """RMSNormForward (row_math.hpp; rms_norm_module.cpp:51-68) in float64: gamma * x / rms."""
    x = x.astype(np.float64)
    rms = np.sqrt((x * x).mean(axis=1) + eps)
    return gamma.astype(np.float64)[None, :] * x / rms[:, None], rms


@gpu
@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("epi", [N.EPI_STORE, N.EPI_STORE_BIAS, N.EPI_ROPE_FWD, N.EPI_SWIGLU_FWD])
def test_rms_prologue_on_every_tile(tile, epi):
    """PXK_PRO_RMS: A is an RMSNorm's input x and B the weight scaled by gamma; the product runs over
    y = gamma x / rms (the norm's row kernel folded into the GEMM) and row_rms receives rms, against
    float64 numpy of the unfolded y W."""
    if epi == N.EPI_SWIGLU_FWD and TILE_BN[tile] % 64:
        pytest.skip("SWIGLU_FWD needs 64-wide tile multiples")
    D = 64 if TILE_BN[tile] >= 64 else 16
    if epi == N.EPI_ROPE_FWD and TILE_BN[tile] < D:
        pytest.skip("heads wider than the tile")
    m, k, n, eps = 77, 148, 128, 1e-5
    x, gamma = G.uniform((m, k), 41), G.uniform((k,), 42, 0.5, 1.5)
    w = G.uniform((k, n), 43)
    b = (gamma[:, None] * w).astype(np.float32)  # gamma folded into the weight, as pxk_scale_rows does
    y, rms = rms_norm_np(x, gamma, eps)
    acc = y @ w.astype(np.float64)
    eb = G.uniform((n,), 44)
    c, c2, c3 = G.empty((m, n)), G.empty((m, n)), G.empty((m, n))
    rms_out = G.empty((m,))
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = m, n, k, 1, 1, 1
    d.prologue, d.epilogue, d.tile, d.norm_eps = N.PRO_RMS, epi, tile, eps
    d.a, d.b = N.operand(G.ptr(G.dev(x)).value, k), N.operand(G.ptr(G.dev(b)).value, n)
    d.row_rms = G.ptr(rms_out).value
    d.c, d.c2, d.c3 = (N.operand(G.ptr(t).value, n) for t in (c, c2, c3))
    want = {"c": acc}
    if epi == N.EPI_STORE_BIAS:
        d.e_bias = N.operand(G.ptr(G.dev(eb)).value, 0)
        want["c2"] = acc + eb
    if epi == N.EPI_ROPE_FWD:
        cos, sin = rope_tables(m, D)
        d.cos_t, d.sin_t = G.ptr(G.dev(cos)).value, G.ptr(G.dev(sin)).value
        d.head_dim, d.rope_half, d.rope_cols = D, 1, n - D
        want["c3"] = rotate(acc, cos, sin, D, True)
    if epi == N.EPI_SWIGLU_FWD:
        F = n // 2
        hid, gp = G.empty((m, F)), G.empty((m, F))
        d.c2, d.c3 = N.operand(G.ptr(hid).value, F), N.operand(G.ptr(gp).value, F)
        blocks = np.arange(n).reshape(-1, 64)
        zg, zu = acc[:, blocks[:, :32].ravel()], acc[:, blocks[:, 32:].ravel()]
        want = {"c": np.concatenate([zg, zu], axis=1)}
        gate = zg / (1.0 + np.exp(-zg))
    assert N.pxk().pxk_gemm(ctypes.byref(d), G.stream()) == 0, N.pxk().pxk_last_error()
    got = {"c": c, "c2": c2, "c3": c3}
    for key, ref in want.items():
        out = G.host(got[key])
        if epi == N.EPI_ROPE_FWD and key == "c3":
            out, ref = out[:, :n - D], ref[:, :n - D]
        G.assert_close(out, ref, 2e-5, "tile %d output %s" % (tile, key))
    if epi == N.EPI_SWIGLU_FWD:
        G.assert_close(G.host(gp), gate, 2e-5, "gate_post")
        G.assert_close(G.host(hid), gate * zu, 2e-5, "hidden")
    G.assert_close(G.host(rms_out), rms, 1e-6, "rms")


@gpu
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("tile", [0, N.TILE_32x48_DIRECT, N.TILE_32x32, N.TILE_64x64])
@pytest.mark.parametrize("epi", [N.EPI_MUL_X, N.EPI_MUL_X_SPLIT])
def test_relevance_epilogue_reads_a_norm_input(epi, tile, splits):
    """MUL_X / MUL_X_SPLIT with x_rms and x_gamma: X holds the norm's input x, and the epilogue uses
    y = gamma x / rms in its place (the value the norm's row kernel would have stored)."""
    m, k, n, eps = 77, 150, 128, 1e-5
    a, b = G.uniform((m, k), 51), G.uniform((n, k), 52)
    x, gamma = G.uniform((m, n), 53), G.uniform((n,), 54, 0.5, 1.5)
    y, rms = rms_norm_np(x, gamma, eps)
    acc = a.astype(np.float64) @ b.astype(np.float64).T
    r = y * acc
    out, out2 = G.empty((m, n)), G.empty((m, n))
    d = N.GemmDesc()
    d.m, d.n, d.k, d.batch, d.inner, d.kgroups = m, n, k, 1, 1, 1
    d.trans_b, d.epilogue, d.eps, d.tile = 1, epi, EPS, tile
    d.a, d.b = N.operand(G.ptr(G.dev(a)).value, k), N.operand(G.ptr(G.dev(b)).value, k)
    d.c, d.c2 = N.operand(G.ptr(out).value, n), N.operand(G.ptr(out2).value, n)
    d.x = N.operand(G.ptr(G.dev(x)).value, n)
    d.x_rms = G.ptr(G.dev(rms.astype(np.float32))).value
    d.x_gamma = G.ptr(G.dev(gamma)).value
    want = {"c": r}
    if epi == N.EPI_MUL_X_SPLIT:
        z2, z3, w = G.uniform((m, n), 55), G.uniform((m, n), 56), away((m, n), 57)
        for key, v in (("z2", z2), ("z3", z3), ("w", w)):
            setattr(d, key, N.operand(G.ptr(G.dev(v)).value, n))
        want = {"c": (z2 / stab(w)) * r, "c2": (z3 / stab(w)) * r}
    assert run(d, splits) == 0, N.pxk().pxk_last_error()
    got = {"c": out, "c2": out2}
    for key, ref in want.items():
        G.assert_close(G.host(got[key]), ref, 2e-5, "tile %d splits %d %s" % (tile, splits, key))


def test_rms_prologue_and_normed_input_reject_misuse():
    """CPU-side: the RMS prologue takes gamma in B, an untransposed A, no k-groups and no split-K; x_rms and
    x_gamma go together on MUL_X / MUL_X_SPLIT. Nothing is launched."""
    skip_if_device_present()
    lib = N.pxk()

    def base():
        d = N.GemmDesc()
        d.m, d.n, d.k, d.batch, d.inner, d.kgroups = 8, 8, 8, 1, 1, 1
        for key in ("a", "b", "c", "c2", "x", "w", "z2", "z3"):
            setattr(d, key, N.operand(16, 8))  # never dereferenced: validation fails first
        d.prologue, d.norm_eps = N.PRO_RMS, 1e-5
        return d

    d = base()
    d.z_bias = N.operand(16, 0)  # gamma belongs in B
    assert lib.pxk_gemm(ctypes.byref(d), None) == 1 and b"RMS prologue" in lib.pxk_last_error()
    d = base()
    d.norm_eps = -1.0
    assert lib.pxk_gemm(ctypes.byref(d), None) == 1
    d = base()
    d.trans_a = 1
    assert lib.pxk_gemm(ctypes.byref(d), None) == 1
    d = base()
    d.kgroups = 2
    assert lib.pxk_gemm(ctypes.byref(d), None) == 1
    d = base()
    d.splits = 2
    assert lib.pxk_gemm(ctypes.byref(d), None) == 1
    d = base()
    d.prologue, d.epilogue, d.x_rms = N.PRO_NONE, N.EPI_MUL_X, 16
    assert lib.pxk_gemm(ctypes.byref(d), None) == 1 and b"x_gamma" in lib.pxk_last_error()
    d.x_gamma, d.epilogue = 16, N.EPI_SPV
    assert lib.pxk_gemm(ctypes.byref(d), None) == 1
