"""The skinny-M GEMM path of pxk_gemm (PXK_TILE_SKINNY: up to 16 rows, the decode steps' and the
last-row heads' shape), called through the C ABI against float64 numpy products of the same
operands, for every epilogue it is built with, ragged N and K, forced and chosen K splits, and the
tied head's transposed table.
"""
import ctypes

import numpy as np
import pytest

import gpu_util as G
from pulsatrix_amd import native as N
from test_kernels_gpu import gemm_tol, launch, plain_desc


def fake_desc(m, n, k, tb=0, epi=None):
    d = N.GemmDesc()
    d.m, d.n, d.k = m, n, k
    d.batch = d.inner = d.kgroups = 1
    d.trans_b = tb
    d.a = N.operand(4096, k)
    d.b = N.operand(8192, k if tb else n)
    d.c = N.operand(16384, n)
    if epi is not None:
        d.epilogue = epi
    return d


def test_planner_picks_the_skinny_path_for_few_rows():
    """CPU-side: plans only, nothing launches."""
    assert N.gemm_plan(fake_desc(4, 1536, 640))[0] == N.TILE_SKINNY
    assert N.gemm_plan(fake_desc(4, 640, 2048)) == (N.TILE_SKINNY, 1)
    tile, splits = N.gemm_plan(fake_desc(4, 640, 65536))
    assert tile == N.TILE_SKINNY and splits > 1  # a workgroup would stream 1 MiB of B: split over K
    assert N.gemm_plan(fake_desc(4, 262144, 640, tb=1)) == (N.TILE_SKINNY, 1)
    assert N.gemm_plan(fake_desc(16, 4096, 640))[0] == N.TILE_SKINNY
    assert N.gemm_plan(fake_desc(17, 4096, 640))[0] != N.TILE_SKINNY  # more than 16 rows
    d = fake_desc(4, 4096, 640, epi=N.EPI_MUL_X)
    d.x = N.operand(32768, 4096)
    assert N.gemm_plan(d)[0] != N.TILE_SKINNY  # not built
    assert N.gemm_plan(fake_desc(4, 1024, 1 << 15, tb=1))[0] != N.TILE_SKINNY  # A does not fit LDS
    d = fake_desc(17, 64, 64)
    d.tile = N.TILE_SKINNY
    assert N.pxk().pxk_gemm_plan(ctypes.byref(d), None, None) == 1  # forced where it does not apply


def nn_operands(m, k, n, seed):
    return G.uniform((m, k), seed), G.uniform((k, n), seed + 1)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 4, 7, 16])
@pytest.mark.parametrize("k,n", [(640, 1536), (2048, 640), (37, 70), (1000, 4100), (5000, 200)])
@pytest.mark.parametrize("splits", [0, 1, 3])
def test_skinny_nn_store_matches_numpy(m, k, n, splits):
    a, b = nn_operands(m, k, n, 3)
    c = G.empty((m, n))
    d = plain_desc(m, n, k, G.dev(a), G.dev(b), c)
    d.tile = N.TILE_SKINNY
    assert N.gemm_plan(d)[0] == N.TILE_SKINNY
    launch(d, N.TILE_SKINNY, splits)
    G.assert_close(G.host(c), a.astype(np.float64) @ b, gemm_tol(k), "skinny nn")


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n", [(4, 640, 640), (9, 300, 130)])
def test_skinny_nn_beta_accumulates(m, k, n):
    a, b = nn_operands(m, k, n, 5)
    c0 = G.uniform((m, n), 7)
    c = G.dev(c0)
    d = plain_desc(m, n, k, G.dev(a), G.dev(b), c)
    d.beta = 0.5
    launch(d, 0, 0)
    G.assert_close(G.host(c), 0.5 * c0 + a.astype(np.float64) @ b, gemm_tol(k), "skinny beta")


@pytest.mark.gpu
@pytest.mark.parametrize("m", [2, 12])
def test_skinny_nn_bias_and_residual_epilogues(m):
    k, n = 1024, 644
    a, b = nn_operands(m, k, n, 11)
    bias, resid = G.uniform((n,), 13), G.uniform((m, n), 14)
    ref = a.astype(np.float64) @ b
    z, y = G.empty((m, n)), G.empty((m, n))
    d = plain_desc(m, n, k, G.dev(a), G.dev(b), z)
    d.epilogue = N.EPI_STORE_BIAS
    d.c2 = N.operand(G.ptr(y).value, n)
    d.e_bias = N.operand(G.ptr(G.dev(bias)).value, 0)
    launch(d, 0, 0)
    assert N.gemm_plan(d)[0] == N.TILE_SKINNY
    G.assert_close(G.host(z), ref, gemm_tol(k), "store_bias z")
    G.assert_close(G.host(y), ref + bias, gemm_tol(k), "store_bias y")
    z, y, out = G.empty((m, n)), G.empty((m, n)), G.empty((m, n))
    d = plain_desc(m, n, k, G.dev(a), G.dev(b), z)
    d.epilogue = N.EPI_ADD_RESID
    d.c2 = N.operand(G.ptr(y).value, n)
    d.c3 = N.operand(G.ptr(out).value, n)
    d.x = N.operand(G.ptr(G.dev(resid)).value, n)
    d.e_bias = N.operand(G.ptr(G.dev(bias)).value, 0)
    launch(d, 0, 0)
    G.assert_close(G.host(z), ref, gemm_tol(k), "add_resid z")
    G.assert_close(G.host(out), resid + ref + bias, gemm_tol(k), "add_resid out")


def gate(x, act):
    if act == 1:
        return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))
    return x / (1.0 + np.exp(-x))


@pytest.mark.gpu
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("m", [4, 16])
def test_skinny_nn_swiglu_epilogue(act, m):
    """Gate and up columns interleaved in 32-wide blocks (the packed gate|up weight)."""
    k, F = 640, 2048
    n = 2 * F
    a, b = nn_operands(m, k, n, 17)
    ref = a.astype(np.float64) @ b
    cols = np.arange(n).reshape(-1, 2, 32)
    zg, zu = ref[:, cols[:, 0].ravel()], ref[:, cols[:, 1].ravel()]
    z, hid, gp = G.empty((m, n)), G.empty((m, F)), G.empty((m, F))
    d = plain_desc(m, n, k, G.dev(a), G.dev(b), z)
    d.epilogue = N.EPI_SWIGLU_FWD
    d.gate_act = act
    d.c2 = N.operand(G.ptr(hid).value, F)
    d.c3 = N.operand(G.ptr(gp).value, F)
    launch(d, 0, 0)
    assert N.gemm_plan(d)[0] == N.TILE_SKINNY
    tol = gemm_tol(k)
    G.assert_close(G.host(z), np.concatenate([zg, zu], axis=1), tol, "swiglu z")
    G.assert_close(G.host(gp), gate(zg, act), tol, "swiglu gate")
    G.assert_close(G.host(hid), gate(zg, act) * zu, tol, "swiglu hidden")


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n", [(4, 640, 262144), (1, 576, 49152), (13, 576, 49152), (8, 70, 1001),
                                   (5, 1022, 4098), (16, 768, 640)])
def test_skinny_nt_matches_numpy(m, k, n):
    """C = A E^T with E stored (n, k), a tied head's table."""
    a, e = G.uniform((m, k), 19), G.uniform((n, k), 20)
    c = G.empty((m, n))
    d = plain_desc(m, n, k, G.dev(a), G.dev(e), c, tb=1)
    launch(d, 0, 0)
    assert N.gemm_plan(d) == (N.TILE_SKINNY, 1)
    G.assert_close(G.host(c), a.astype(np.float64) @ e.T.astype(np.float64), gemm_tol(k), "skinny nt")


@pytest.mark.gpu
def test_skinny_nt_strided_a_and_c():
    """Row strides wider than the extents (the last rows of a sequence batch)."""
    m, k, n, lda, ldc = 5, 256, 3000, 1000, 3008
    a = G.uniform((m, lda), 21)
    e = G.uniform((n, k), 22)
    c = G.empty((m, ldc), 0.0)
    d = plain_desc(m, n, k, G.dev(a), G.dev(e), c, tb=1)
    d.a = N.operand(d.a.ptr, lda)
    d.c = N.operand(d.c.ptr, ldc)
    launch(d, 0, 0)
    got = G.host(c)
    G.assert_close(got[:, :n], a[:, :k].astype(np.float64) @ e.T, gemm_tol(k), "strided nt")
    assert np.all(got[:, n:] == 0.0)
