"""The raw op sweep at its full sizes: GEMMs M x K x N in {512x576x1536, 512x1536x576,
4096x2048x8192, 512x576x49152}, each forward (NN), as the Linear relevance form against the stored
W (NT: x * ((R / stab(z)) W^T), lrp_rules.cpp:197-215) and weight-side (TN: A^T S); elementwise ops
over 2^26 elements; RMSNorm over 32768 rows of 2048.

The GEMMs are checked on 24 sampled output rows (first, last and 22 seeded ones) against float64
numpy at the primitive contract's 1e-4 (backend_primitive_equivalence_cases.hpp:66-75). The
elementwise ops and RMSNorm are compared against the oracle over every element: bit-exact where
the kernel evaluates the reference's per-element expression in the same order, 1e-5 for RMSNorm
(its row sum is a different, fixed order)."""
import numpy as np
import pytest

import gpu_util as G
from pulsatrix_amd import native as N

gpu = pytest.mark.gpu

SHAPES = [(512, 576, 1536), (512, 1536, 576), (4096, 2048, 8192), (512, 576, 49152)]


def stab(z, eps):
    return z + eps * np.where(z >= 0, 1.0, -1.0)


def away(shape, seed):
    """uniform magnitudes in [0.5, 1.5) with random signs: stabilised denominators clear of 0."""
    rs = np.random.RandomState(seed)
    return (rs.uniform(0.5, 1.5, shape) * rs.choice([-1.0, 1.0], shape)).astype(np.float32)


def sample_rows(count, seed):
    rs = np.random.RandomState(seed)
    return np.unique(np.concatenate([[0, count - 1], rs.randint(0, count, 22)]))


@gpu
@pytest.mark.parametrize("orient", ["NN", "NT", "TN"])
@pytest.mark.parametrize("M,K,Nn", SHAPES)
def test_sweep_gemm_full_size(M, K, Nn, orient):
    print("sweep gemm %s %dx%dx%d" % (orient, M, K, Nn), flush=True)
    d = N.GemmDesc()
    d.batch, d.inner, d.kgroups = 1, 1, 1
    eps = 1e-6
    if orient == "NN":
        A, B = G.uniform((M, K), 1), G.uniform((K, Nn), 2)
        C = G.empty((M, Nn))
        d.m, d.n, d.k = M, Nn, K
        d.a, d.b, d.c = N.operand(G.dev(A).data_ptr(), K), N.operand(G.dev(B).data_ptr(), Nn), N.operand(C.data_ptr(), Nn)
        rows = sample_rows(M, 3)
        want = A[rows].astype(np.float64) @ B.astype(np.float64)
    elif orient == "NT":
        R, Z, W, X = G.uniform((M, Nn), 4), away((M, Nn), 5), G.uniform((K, Nn), 6), G.uniform((M, K), 7)
        C = G.empty((M, K))
        d.m, d.n, d.k, d.trans_b = M, K, Nn, 1
        d.prologue, d.epilogue, d.eps = N.PRO_DIV_STAB, N.EPI_MUL_X, eps
        d.a, d.z = N.operand(G.dev(R).data_ptr(), Nn), N.operand(G.dev(Z).data_ptr(), Nn)
        d.b, d.c, d.x = N.operand(G.dev(W).data_ptr(), Nn), N.operand(C.data_ptr(), K), N.operand(G.dev(X).data_ptr(), K)
        rows = sample_rows(M, 8)
        g = R[rows].astype(np.float64) / stab(Z[rows].astype(np.float64), eps)
        want = X[rows].astype(np.float64) * (g @ W.astype(np.float64).T)
    else:
        A, S = G.uniform((M, K), 9), G.uniform((M, Nn), 10)
        C = G.empty((K, Nn))
        d.m, d.n, d.k, d.trans_a = K, Nn, M, 1
        d.a, d.b, d.c = N.operand(G.dev(A).data_ptr(), K), N.operand(G.dev(S).data_ptr(), Nn), N.operand(C.data_ptr(), Nn)
        rows = sample_rows(K, 11)
        want = A[:, rows].astype(np.float64).T @ S.astype(np.float64)
    ws_bytes = N.gemm_workspace(d)
    ws = G.empty((max(ws_bytes // 4, 1),), 0.0)
    d.workspace, d.workspace_bytes = ws.data_ptr(), ws_bytes
    N.gemm(d, G.stream())
    got = G.host(C)
    assert np.all(np.isfinite(got)), "every output written"
    G.assert_close(got[rows], want, 1e-4, "sampled rows")


@gpu
@pytest.mark.parametrize("n", [1 << 26, (1 << 22) + 5])
def test_sweep_elementwise_full_size(n):
    """2^26 as swept; 2^22 + 5 takes the streaming path with a scalar tail."""
    print("sweep elementwise n=%d" % n, flush=True)
    a, b, r = G.uniform((n,), 21), G.uniform((n,), 22), G.uniform((n,), 23)
    ad, bd, rd = G.dev(a), G.dev(b), G.dev(r)
    s = G.stream()
    out, out2 = G.empty((n,)), G.empty((n,))
    ref, ref2 = np.empty_like(a), np.empty_like(a)
    for name in ("add", "mul"):
        G.oracle_call("pxo_" + name, a, b, ref, n)
        N.call("pxk_" + name, G.ptr(ad), G.ptr(bd), G.ptr(out), n, s)
        assert np.array_equal(G.host(out), ref), name
    G.oracle_call("pxo_elementwise", 0, a, ref, n)
    N.call("pxk_elementwise", 0, G.ptr(ad), G.ptr(out), n, s)
    assert np.array_equal(G.host(out), ref), "relu"
    for mode in (0, 1):
        G.oracle_call("pxo_lrp_stabilized_divide", r, a, b if mode else None, ref, n, 1e-6, mode)
        N.call("pxk_lrp_stabilized_divide", G.ptr(rd), G.ptr(ad), G.ptr(bd) if mode else None, G.ptr(out), n, 1e-6,
               mode, s)
        assert np.array_equal(G.host(out), ref), ("epsilon-divide", mode)
    G.oracle_call("pxo_lrp_residual_split", a, b, r, ref, ref2, n, 1e-6)
    N.call("pxk_lrp_residual_split", G.ptr(ad), G.ptr(bd), G.ptr(rd), G.ptr(out), G.ptr(out2), n, 1e-6, s)
    assert np.array_equal(G.host(out), ref) and np.array_equal(G.host(out2), ref2), "residual split"
    G.oracle_call("pxo_lrp_bilinear_elementwise", a, b, r, ref, n, 1e-6)
    N.call("pxk_lrp_bilinear_elementwise", G.ptr(ad), G.ptr(bd), G.ptr(rd), G.ptr(out), n, 1e-6, s)
    assert np.array_equal(G.host(out), ref), "bilinear elementwise"


@gpu
def test_sweep_rms_norm_full_size():
    rows, cols = 32768, 2048
    print("sweep rms_norm %dx%d" % (rows, cols), flush=True)
    x, g = G.uniform((rows, cols), 31), G.uniform((cols,), 32)
    ref, rms = np.empty_like(x), np.empty((rows,), np.float32)
    G.oracle_call("pxo_rms_norm_forward", x, g, ref, rms, rows, cols, 1e-5)
    out, orms = G.empty((rows, cols)), G.empty((rows,))
    N.call("pxk_rms_norm_forward", G.ptr(G.dev(x)), G.ptr(G.dev(g)), G.ptr(out), G.ptr(orms), rows, cols, 1e-5,
           G.stream())
    G.assert_close(G.host(out), ref, 1e-5, "rmsnorm")
    G.assert_close(G.host(orms), rms, 1e-5, "rms")
