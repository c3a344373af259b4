"""Helpers for the GPU parity tests: device buffers (torch, used only as HBM plumbing), the
current stream, and oracle primitive calls on numpy arrays."""
import ctypes

import numpy as np

import oracle_ctypes as oc


def torch_cuda():
    import torch

    return torch


# Device buffers handed out here stay alive until release_all() (called after every test): a
# pointer taken from a temporary tensor would otherwise be recycled by torch's caching allocator
# before the kernel that reads it runs.
_alive = []


def keep(t):
    _alive.append(t)
    return t


def release_all():
    _alive.clear()


def dev(a):
    """numpy -> device float32 tensor."""
    torch = torch_cuda()
    return keep(torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda"))


def empty(shape, fill=np.nan):
    torch = torch_cuda()
    t = torch.empty(shape, dtype=torch.float32, device="cuda")
    t.fill_(float(fill))
    return keep(t)


def host(t):
    torch = torch_cuda()
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream():
    torch = torch_cuda()
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


_sig = {
    "pxo_gemm_ex": "pnpnpsssf",
    "pxo_add": "ppps",
    "pxo_mul": "ppps",
    "pxo_axpby": "fpfpps",
    "pxo_elementwise": "npps",
    "pxo_add_row_vector": "pppss",
    "pxo_softmax_rows": "ppss",
    "pxo_rms_norm_forward": "ppppssf",
    "pxo_rope_rotate": "ppppsssnn",
    "pxo_permute_0213": "ppssss",
    "pxo_attention_mask_fill": "ppssssnssf",
    "pxo_gather_rows": "pppss",
    "pxo_lrp_linear": "pppppsssf",
    "pxo_lrp_residual_split": "pppppsf",
    "pxo_lrp_bilinear_elementwise": "ppppsf",
    "pxo_lrp_bilinear_matmul": "ppppppssssfn",
    "pxo_lrp_softmax_rows": "ppppss",
    "pxo_lrp_rope": "ppppppsssfn",
    "pxo_lrp_stabilized_divide": "ppppsfn",
    "pxo_copy_2d": "psps" + "ss",
    "pxo_accumulate_rows": "ppss",
    "pxo_column_sums": "ppssf",
    "pxo_elementwise_backward": "nppps",
    "pxo_softmax_rows_backward": "pppss",
    "pxo_rms_norm_backward": "ppppppss",
}
_T = {"p": ctypes.c_void_p, "s": ctypes.c_size_t, "n": ctypes.c_int, "f": ctypes.c_float}
_bound = False


def oracle_call(name, *args):
    """Calls an oracle primitive; numpy arrays are passed by pointer."""
    global _bound
    lib = oc.oracle().lib
    if not _bound:
        for k, s in _sig.items():
            getattr(lib, k).argtypes = [_T[c] for c in s]
            getattr(lib, k).restype = None
        lib.pxo_sum.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        lib.pxo_sum.restype = ctypes.c_float
        lib.pxo_dot.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        lib.pxo_dot.restype = ctypes.c_float
        _bound = True
    conv = [a.ctypes.data_as(ctypes.c_void_p) if isinstance(a, np.ndarray) else a for a in args]
    return getattr(lib, name)(*conv)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def uniform(shape, seed, lo=-1.0, hi=1.0):
    """Seeded uniform(-1, 1) data, as the reference's equivalence tests use (mt19937 there)."""
    return np.random.RandomState(seed).uniform(lo, hi, size=shape).astype(np.float32)


def assert_close(actual, expected, rel=1e-4, what=""):
    """|actual - expected| <= rel * max(1, max|expected|) elementwise."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    assert actual.shape == expected.shape, (what, actual.shape, expected.shape)
    assert np.all(np.isfinite(actual)), (what, "non-finite values")
    scale = max(1.0, float(np.abs(expected).max()) if expected.size else 1.0)
    err = float(np.abs(actual - expected).max()) if expected.size else 0.0
    assert err <= rel * scale, "%s: max |diff| %.3e > %.1e * %.3e" % (what, err, rel, scale)
