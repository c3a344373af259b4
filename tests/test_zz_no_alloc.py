"""pxk_gemm_noalloc, the allocation-free variant of pxk_gemm (split-K partials in a static device
array of PXK_GEMM_SCRATCH_BYTES per GPU, looked up with hipGetSymbolAddress), against pxk_gemm with
a caller's workspace on the same descriptors: two calls in a row, the second smaller, each
bit-identical to pxk_gemm (the same plan and kernels). Plans whose partials exceed the scratch are
refused before any launch (host-side check, also on the CPU)."""
import ctypes

import numpy as np
import pytest

import gpu_util as G
from pulsatrix_amd import native as N

SCRATCH_BYTES = 64 << 20


def head_relevance_desc(torch, m, d, v, seed):
    """r_in (m x d) = x * ((R / stab(z)) E): the tied head's relevance GEMM, K = v (split-K)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    R = torch.rand(m, v, device="cuda", generator=g) * 2 - 1
    Z = torch.rand(m, v, device="cuda", generator=g) * 2 - 1
    E = (torch.rand(v, d, device="cuda", generator=g) * 2 - 1) * 0.05
    X = torch.rand(m, d, device="cuda", generator=g) * 2 - 1
    outs = [torch.full((m, d), float("nan"), device="cuda") for _ in range(2)]
    desc = N.GemmDesc()
    desc.m, desc.n, desc.k, desc.batch, desc.inner, desc.kgroups = m, d, v, 1, 1, 1
    desc.prologue, desc.epilogue, desc.eps = N.PRO_DIV_STAB, N.EPI_MUL_X, 1e-6
    desc.a, desc.z = N.operand(R.data_ptr(), v), N.operand(Z.data_ptr(), v)
    desc.b, desc.x = N.operand(E.data_ptr(), d), N.operand(X.data_ptr(), d)
    for t in (R, Z, E, X, *outs):
        G.keep(t)
    return desc, outs


def run_pair(torch, desc, outs):
    """pxk_gemm with a torch-allocated workspace into outs[0], pxk_gemm_noalloc into outs[1]."""
    st = G.stream()
    desc.c = N.operand(outs[0].data_ptr(), desc.n)  # set before planning: the plan validates C
    ws_bytes = N.gemm_workspace(desc)
    ws = G.keep(torch.empty(max(ws_bytes // 4, 1), device="cuda"))
    desc.workspace, desc.workspace_bytes = ws.data_ptr(), ws_bytes
    N.check(N.pxk().pxk_gemm(ctypes.byref(desc), st))
    desc.c = N.operand(outs[1].data_ptr(), desc.n)
    desc.workspace, desc.workspace_bytes = None, 0
    N.check(N.pxk().pxk_gemm_noalloc(ctypes.byref(desc), st))
    torch.cuda.synchronize()
    return G.host(outs[0]), G.host(outs[1]), ws_bytes


@pytest.mark.gpu
def test_gemm_noalloc_matches_gemm_on_two_calls_the_second_smaller():
    torch = G.torch_cuda()
    # 1: the SmolLM2-shaped head relevance, 512 x 576 x 49152 (the planner splits K; about 38 MB of partials)
    desc, outs = head_relevance_desc(torch, 512, 576, 49152, 1)
    ref, got, ws = run_pair(torch, desc, outs)
    assert 0 < ws <= SCRATCH_BYTES, ws
    assert np.all(np.isfinite(ref)) and np.array_equal(got, ref)
    # 2: smaller, with a forced split count, right after (the scratch still holds call 1's partials)
    desc, outs = head_relevance_desc(torch, 96, 200, 3000, 2)
    desc.splits = 6
    ref2, got2, ws2 = run_pair(torch, desc, outs)
    assert N.gemm_plan(desc)[1] == 6 and 0 < ws2 < ws
    assert np.all(np.isfinite(ref2)) and np.array_equal(got2, ref2)
    # 3: a plan without split-K touches no scratch at all
    desc, outs = head_relevance_desc(torch, 64, 64, 256, 3)
    desc.splits = 1
    ref3, got3, ws3 = run_pair(torch, desc, outs)
    assert ws3 == 0 and np.array_equal(got3, ref3)


def test_gemm_noalloc_refuses_plans_beyond_the_scratch_before_launching():
    """Host-side: 64 splits of 512 x 576 partials need 75.5 MB > 64 MiB. Placeholder pointers: the
    check runs before anything touches the device, and the test is skipped where a GPU is present."""
    if N.host().pxa_device_count() > 0:
        pytest.skip("a GPU is present: placeholder-pointer rejection tests run only without one")
    desc = N.GemmDesc()
    desc.m, desc.n, desc.k, desc.batch, desc.inner, desc.kgroups = 512, 576, 49152, 1, 1, 1
    desc.splits = 64
    p = ctypes.c_void_p(4096).value
    desc.a, desc.b, desc.c = N.operand(p, 49152), N.operand(p, 576), N.operand(p, 576)
    assert N.pxk().pxk_gemm_noalloc(ctypes.byref(desc), None) == 3
    assert b"static scratch" in N.pxk().pxk_last_error()
    assert N.pxk().pxk_gemm_noalloc(None, None) == 1


_CAPTURE_CHILD = r'''
import ctypes, sys
import numpy as np
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/tests"]
import torch
import gpu_util as G
from pulsatrix_amd import native as N
import test_zz_no_alloc as T

desc, outs = T.head_relevance_desc(torch, 96, 200, 3000, 4)
desc.splits = 6
side = torch.cuda.Stream()
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
desc.c = N.operand(outs[1].data_ptr(), desc.n)
with torch.cuda.graph(g, stream=side):
    rc_first = N.pxk().pxk_gemm_noalloc(ctypes.byref(desc), ctypes.c_void_p(side.cuda_stream))
msg = N.pxk().pxk_last_error().decode()
print("first-call-under-capture rc", rc_first, flush=True)
assert rc_first == 1 and "inside a stream capture" in msg, (rc_first, msg)
ref, got, _ = T.run_pair(torch, desc, outs)  # one eager call on the device: the scratch address is known
assert np.array_equal(got, ref)
out = G.keep(torch.full((96, 200), float("nan"), device="cuda"))
desc.c = N.operand(out.data_ptr(), desc.n)
g2 = torch.cuda.CUDAGraph()
with torch.cuda.graph(g2, stream=side):
    rc = N.pxk().pxk_gemm_noalloc(ctypes.byref(desc), ctypes.c_void_p(side.cuda_stream))
assert rc == 0, N.pxk().pxk_last_error()
for i in range(3):  # replays, with eager work between them
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    g2.replay()
    torch.cuda.synchronize()
    assert np.array_equal(G.host(out), ref), "replay %d" % i
    T.run_pair(torch, desc, outs)
print("captured replays match pxk_gemm", flush=True)
'''


@pytest.mark.gpu
def test_gemm_noalloc_first_call_under_capture_refused_then_captured_calls_replay():
    """In a fresh process, so that the first split-K call on the device is the captured one: it is
    refused without launching; after one eager call, a captured call replays to pxk_gemm's bits."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
