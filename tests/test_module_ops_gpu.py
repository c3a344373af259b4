"""The DeviceBackend virtuals of the reference's non-LLM modules on MI355XBackend (module_ops.hip):
fuzzy logic and the aggregator, conv patches, pooling, batch / group norm, the RNN / LSTM / GRU
cells, the Mamba / RWKV / RetNet passes and the RL rows. Each runs through the pxr_be_* shim on
MI355XBackend (oracle/_ref/libpxref_mi355x.so, device buffers) and on the compiled reference's
CPUBackend (oracle/_ref/libpxref.so, host copies of the same seeded inputs): every output within
1e-5 of max(1, max|cpu|) (the GPU's exp / log / pow / tanh and fused multiply-adds differ from
glibc's by rounding), index outputs (argmax, decoded targets, masks) exactly. The shapes follow
the reference's equivalence cases (tests/backend_primitive_equivalence_cases.hpp): small,
non-square, with padding, overlapping windows and ragged edges.
"""
import ctypes

import numpy as np
import pytest

import gpu_util as G
import oracle_ctypes as oc
from test_dropin_gpu import be, cpu_vs_gpu, lib  # noqa: F401  (lib is the module fixture)

pytestmark = pytest.mark.gpu


def unit(shape, seed):
    """Uniform (0.05, 0.95): fuzzy truth values, activated gates, probabilities."""
    return np.random.RandomState(seed).uniform(0.05, 0.95, size=shape).astype(np.float32)


def away(shape, seed, lo=0.5, hi=1.5):
    """Magnitudes in [lo, hi) with random signs: denominators clear of zero."""
    r = np.random.RandomState(seed)
    return (r.uniform(lo, hi, size=shape) * r.choice([-1.0, 1.0], size=shape)).astype(np.float32)


def slots_vs_cpu(lib, name, op, ins, outs, tail, nin, nout, rel=1e-5, exact=()):
    """pxr_be_<name>(op, in[nin], out[nout], *tail) on both backends: ins / outs are lists of arrays
    (None for unused slots; outs hold the initial contents, e.g. zeroed carries and states)."""
    cpu = oc.ref()
    if cpu is None:
        pytest.fail("oracle/_ref/libpxref.so was not built: the boundary evidence needs it "
                    "(__graft_entry__.build() builds it where the reference sources are)")
    vp = ctypes.c_void_p
    h_in = [None if a is None else np.ascontiguousarray(a, np.float32).copy() for a in ins]
    h_out = [None if a is None else np.ascontiguousarray(a, np.float32).copy() for a in outs]
    d_in = [None if a is None else G.dev(a) for a in ins]
    d_out = [None if a is None else G.dev(a) for a in outs]

    def arr(n, vals):
        return (vp * n)(*([vp(v) if v else None for v in vals] + [None] * (n - len(vals))))

    cpu.check(getattr(cpu.lib, "pxr_be_" + name)(
        op, arr(nin, [None if a is None else a.ctypes.data for a in h_in]),
        arr(nout, [None if a is None else a.ctypes.data for a in h_out]), *tail))
    G.torch_cuda().cuda.synchronize()
    lib.check(getattr(lib.lib, "pxr_be_" + name)(
        op, arr(nin, [None if t is None else t.data_ptr() for t in d_in]),
        arr(nout, [None if t is None else t.data_ptr() for t in d_out]), *tail))
    lib.check(lib.lib.pxr_be_synchronize())
    for k, (h, d) in enumerate(zip(h_out, d_out)):
        if h is None:
            continue
        got = G.host(d)
        if k in exact:
            assert np.array_equal(got, h, equal_nan=True), (name, op, k)
        else:
            G.assert_close(got, h, rel, "%s op %d out[%d]" % (name, op, k))


# ---- fuzzy logic and the aggregator ---------------------------------------------------------------

@pytest.mark.parametrize("norm", [0, 1, 2])
def test_logic_pointwise(lib, norm):
    n = 4099
    a, b, g = unit((n,), 1), unit((n,), 2), G.uniform((n,), 3)
    a[:7] = b[:7]  # ties go to a
    for conj in (0, 3):
        y = np.zeros(n, np.float32)
        cpu_vs_gpu(lib, "logic_pointwise", {"a": a, "b": b, "y": y}, ["y"],
                   [conj, norm, "a", "b", None, None, "y", None, n, 1e-6])
        oc.ref().check(oc.ref().lib.pxr_be_logic_pointwise(conj, norm, a.ctypes.data, b.ctypes.data, None, None,
                                                           y.ctypes.data, None, n, 1e-6))
        for op in (conj + 1, conj + 2):
            arrays = {"a": a, "b": b, "g": g, "y": y, "oa": np.zeros(n, np.float32), "ob": np.zeros(n, np.float32)}
            cpu_vs_gpu(lib, "logic_pointwise", arrays, ["oa", "ob"], [op, norm, "a", "b", "g", "y", "oa", "ob", n, 1e-6],
                       exact=("oa", "ob") if norm == 2 else ())


def test_aggregator_forward_backward_lrp(lib):
    n, cols, p = 37, 53, 2.5
    x = unit((n, cols), 4) + 0.1
    mp, out = np.zeros(cols, np.float32), np.zeros(cols, np.float32)
    cpu_vs_gpu(lib, "aggregator_forward", {"x": x, "mp": mp, "out": out}, ["mp", "out"], ["x", "mp", "out", n, cols, p])
    oc.ref().check(oc.ref().lib.pxr_be_aggregator_forward(x.ctypes.data, mp.ctypes.data, out.ctypes.data, n, cols, p))
    go = G.uniform((cols,), 5)
    cpu_vs_gpu(lib, "aggregator_backward", {"x": x, "mp": mp, "go": go, "gi": np.zeros_like(x)}, ["gi"],
               ["x", "mp", "go", "gi", n, cols, p])
    cpu_vs_gpu(lib, "aggregator_lrp", {"x": x, "mp": mp, "ro": go, "ri": np.zeros_like(x)}, ["ri"],
               ["x", "mp", "ro", "ri", n, cols, p, 1e-6])


# ---- convolution patches ---------------------------------------------------------------------------

GEOMETRIES = [(3, 3, 1, 1, 0, 0), (3, 2, 2, 1, 1, 0), (2, 3, 1, 2, 0, 1), (5, 5, 2, 3, 2, 2), (1, 1, 1, 1, 0, 0)]


def out_size(x, k, s, p):
    return (x + 2 * p - k) // s + 1


@pytest.mark.parametrize("geo", GEOMETRIES, ids=lambda g: "k%dx%d_s%d%d_p%d%d" % g)
def test_im2col_col2im_and_conv_rule(lib, geo):
    kh, kw, sh, sw, ph, pw = geo
    n, c, h, w, oc_ = 2, 3, 9, 7, 4
    oh, ow = out_size(h, kh, sh, ph), out_size(w, kw, sw, pw)
    P, Q = c * kh * kw, oh * ow
    x = G.uniform((n, c, h, w), 6)
    cpu_vs_gpu(lib, "im2col", {"x": x, "col": np.full((n, P, Q), np.nan, np.float32)}, ["col"],
               ["x", "col", n, c, h, w, kh, kw, sh, sw, ph, pw], exact=("col",))
    col = G.uniform((n, P, Q), 7)
    cpu_vs_gpu(lib, "col2im_add", {"col": col, "out": G.uniform((n, c, h, w), 8)}, ["out"],
               ["col", "out", n, c, h, w, kh, kw, sh, sw, ph, pw])
    kern, z, r = G.uniform((oc_, P), 9), away((n, oc_, Q), 10), G.uniform((n, oc_, Q), 11)
    cpu_vs_gpu(lib, "lrp_conv", {"col": col, "k": kern, "z": z, "r": r, "rc": np.zeros((n, P, Q), np.float32)}, ["rc"],
               ["col", "k", "z", "r", "rc", n, oc_, P, Q, 1e-6])


def test_add_channel_vector(lib):
    n, c, inner = 3, 5, 17
    x, v = G.uniform((n, c, inner), 12), G.uniform((c,), 13)
    cpu_vs_gpu(lib, "add_channel_vector", {"x": x, "v": v, "o": np.zeros_like(x)}, ["o"], ["x", "v", "o", n, c, inner],
               exact=("o",))


# ---- pooling -----------------------------------------------------------------------------------------

@pytest.mark.parametrize("geo", [(2, 2, 2, 2, 0, 0), (3, 3, 2, 2, 1, 1), (3, 2, 1, 2, 1, 0), (4, 4, 3, 3, 2, 1)],
                         ids=lambda g: "k%dx%d_s%d%d_p%d%d" % g)
def test_max_pool_and_unpool(lib, geo):
    kh, kw, sh, sw, ph, pw = geo
    planes, h, w = 5, 9, 8
    oh, ow = out_size(h, kh, sh, ph), out_size(w, kw, sw, pw)
    x = G.uniform((planes, h, w), 14)
    x[0, :3, :3] = 0.25  # ties: the first maximum in window order wins
    cpu_vs_gpu(lib, "max_pool_forward", {"x": x, "o": np.zeros((planes, oh, ow), np.float32),
                                         "am": np.zeros((planes, oh, ow), np.float32)}, ["o", "am"],
               ["x", "o", "am", planes, h, w, kh, kw, sh, sw, ph, pw], exact=("o", "am"))
    am = np.zeros((planes, oh, ow), np.float32)
    o = np.zeros_like(am)
    oc.ref().check(oc.ref().lib.pxr_be_max_pool_forward(x.ctypes.data, o.ctypes.data, am.ctypes.data, planes, h, w, kh,
                                                        kw, sh, sw, ph, pw))
    src = G.uniform((planes, oh, ow), 15)
    cpu_vs_gpu(lib, "max_unpool", {"src": src, "am": am, "dst": np.full((planes, h, w), np.nan, np.float32)}, ["dst"],
               ["src", "am", "dst", planes, h, w, kh, kw, sh, sw, ph, pw])


def test_avg_pool_forward_backward_rule(lib):
    planes, h, w, kh, kw = 4, 8, 9, 2, 3
    oh, ow = (h - kh) // kh + 1, (w - kw) // kw + 1
    x = away((planes, h, w), 16)
    cpu_vs_gpu(lib, "avg_pool_forward", {"x": x, "o": np.zeros((planes, oh, ow), np.float32)}, ["o"],
               ["x", "o", planes, h, w, kh, kw])
    go = G.uniform((planes, oh, ow), 17)
    cpu_vs_gpu(lib, "avg_pool_backward", {"go": go, "gi": np.zeros_like(x)}, ["gi"], ["go", "gi", planes, h, w, kh, kw])
    cpu_vs_gpu(lib, "lrp_avg_pool", {"x": x, "r": go, "ri": np.zeros_like(x)}, ["ri"],
               ["x", "r", "ri", planes, h, w, kh, kw, 1e-6])


# ---- batch and group norm -------------------------------------------------------------------------

def test_batch_norm_train_and_eval(lib):
    n, c, sp, eps = 3, 5, 7, 1e-5
    x, gm, bt = G.uniform((n, c, sp), 18) * 2 + 0.3, G.uniform((c,), 19), G.uniform((c,), 20)
    z = lambda *s: np.zeros(s, np.float32)  # noqa: E731
    cpu_vs_gpu(lib, "batch_norm_forward", {"x": x, "g": gm, "b": bt, "xh": z(n, c, sp), "o": z(n, c, sp), "sd": z(c)},
               ["xh", "o", "sd"], ["x", "g", "b", "xh", "o", "sd", n, c, sp, eps])
    xh, o, sd = z(n, c, sp), z(n, c, sp), z(c)
    oc.ref().check(oc.ref().lib.pxr_be_batch_norm_forward(x.ctypes.data, gm.ctypes.data, bt.ctypes.data, xh.ctypes.data,
                                                          o.ctypes.data, sd.ctypes.data, n, c, sp, eps))
    go = G.uniform((n, c, sp), 21)
    for name in ("batch_norm_backward", "batch_norm_eval_backward"):
        cpu_vs_gpu(lib, name, {"go": go, "g": gm, "xh": xh, "sd": sd, "gi": z(n, c, sp), "gg": z(c), "bg": z(c)},
                   ["gi", "gg", "bg"], ["go", "g", "xh", "sd", "gi", "gg", "bg", n, c, sp])
    rm, rv = G.uniform((c,), 22), unit((c,), 23) + 0.5
    cpu_vs_gpu(lib, "batch_norm_eval_forward", {"x": x, "g": gm, "b": bt, "rm": rm, "rv": rv, "xh": z(n, c, sp),
                                                "o": z(n, c, sp), "sd": z(c)},
               ["xh", "o", "sd"], ["x", "g", "b", "rm", "rv", "xh", "o", "sd", n, c, sp, eps])
    for nn, spp in ((n, sp), (1, 1)):  # one value per channel keeps the running variance
        xs = x[:nn, :, :spp].copy()
        cpu_vs_gpu(lib, "batch_norm_update_running", {"x": xs, "rm": rm, "rv": rv}, ["rm", "rv"],
                   ["x", "rm", "rv", nn, c, spp, 0.1])


def test_group_norm(lib):
    n, c, sp, groups, eps = 2, 6, 5, 3, 1e-5
    x, gm, bt = G.uniform((n, c, sp), 24) * 3, G.uniform((c,), 25), G.uniform((c,), 26)
    z = lambda *s: np.zeros(s, np.float32)  # noqa: E731
    cpu_vs_gpu(lib, "group_norm_forward", {"x": x, "g": gm, "b": bt, "xh": z(n, c, sp), "o": z(n, c, sp),
                                           "sd": z(n, groups)},
               ["xh", "o", "sd"], ["x", "g", "b", "xh", "o", "sd", n, c, sp, groups, eps])
    xh, o, sd = z(n, c, sp), z(n, c, sp), z(n, groups)
    oc.ref().check(oc.ref().lib.pxr_be_group_norm_forward(x.ctypes.data, gm.ctypes.data, bt.ctypes.data, xh.ctypes.data,
                                                          o.ctypes.data, sd.ctypes.data, n, c, sp, groups, eps))
    go = G.uniform((n, c, sp), 27)
    cpu_vs_gpu(lib, "group_norm_backward", {"go": go, "g": gm, "xh": xh, "sd": sd, "gi": z(n, c, sp), "gg": z(c),
                                            "bg": z(c)},
               ["gi", "gg", "bg"], ["go", "g", "xh", "sd", "gi", "gg", "bg", n, c, sp, groups])


# ---- recurrent cells -------------------------------------------------------------------------------

# Slots per RecurrentCellOp (device_backend.hpp:75-87): (inputs, outputs); "u" = in (0, 1), "s" =
# signed, "a" = signed away from zero (denominators).
CELLS = {
    0: ("sss", 1),           # RnnBackward: g, dh_next, h -> dz
    1: ("uuuuu", 3),         # LstmForward: i, f, g, o, c_prev -> c, tanh c, h
    2: ("sssuuuuss", 5),     # LstmBackward: g, dh_next, dc_next, i, f, g, o, tanh_c, c_prev -> 5 grads
    3: ("sssuuusa", 2),      # LstmLrp: r, R_h_next, R_c_next, i, f, g, c_prev, c -> R_g, R_c_prev
    4: ("ssuuuss", 5),       # GruBackward: g, dh_next, z, r, n, hn, h_prev -> 5 grads
    5: ("ssuuussaa", 3),     # GruLrp: r, R_h_next, z, r, n, hn, h_prev, h, n_pre -> 3
}


@pytest.mark.parametrize("op", sorted(CELLS))
def test_recurrent_cell(lib, op):
    kinds, nout = CELLS[op]
    n = 1031
    gen = {"u": unit, "s": G.uniform, "a": away}
    ins = [gen[k]((n,), 30 + i) for i, k in enumerate(kinds)]
    outs = [np.zeros(n, np.float32) for _ in range(nout)]
    slots_vs_cpu(lib, "recurrent_cell", op, ins, outs, [1e-6, n], 10, 6)


def test_gru_lrp_hprev(lib):
    rows, hidden = 3, 29
    hp, w, hn = G.uniform((rows, hidden), 40), G.uniform((hidden, hidden), 41), away((rows, hidden), 42)
    rb, direct = G.uniform((rows, hidden), 43), G.uniform((rows, hidden), 44)
    cpu_vs_gpu(lib, "gru_lrp_hprev", {"hp": hp, "w": w, "hn": hn, "rb": rb, "d": direct, "o": np.zeros_like(hp)}, ["o"],
               ["hp", "w", "hn", "rb", "d", "o", rows, hidden, 1e-6])


# ---- Mamba / RWKV / RetNet ---------------------------------------------------------------------------

N_, L_, D_, S_ = 2, 6, 5, 4


def ssm_case(op, seed):
    """(inputs, outputs with their initial contents) of one SsmPassOp at n, l, d, s = 2, 6, 5, 4."""
    n, l, d, s = N_, L_, D_, S_
    k = [seed * 100]

    def u(*shape, kind="s"):
        k[0] += 1
        return {"s": G.uniform, "u": unit, "a": away}[kind](shape, k[0])

    z = lambda *shape: np.zeros(shape, np.float32)  # noqa: E731
    nld, nlds, nls = (n, l, d), (n, l, d, s), (n, l, s)
    if op == 0:  # MambaForward
        A = -unit((d, s), seed)
        return [u(*nld), u(*nld), u(*nls), u(*nls), A, u(d)], [z(*nld), z(*nlds), z(*nlds), z(n, l + 1, d, s), z(*nld)]
    if op == 1:  # MambaBackward
        return ([u(*nld), u(*nld), u(*nld, kind="u"), u(*nld), u(n, l + 1, d, s), u(*nlds, kind="u"), u(*nlds),
                 u(*nls), u(*nls), -unit((d, s), seed), u(d)],
                [z(*nld), z(*nld), z(*nlds), z(*nlds), z(n, d, s)])
    if op == 2:  # MambaGradBC
        return [u(*nld), u(*nld), u(*nld, kind="u"), u(n, l + 1, d, s), u(*nlds)], [z(*nls), z(*nls)]
    if op == 3:  # MambaLrp
        return ([u(*nld), u(*nld, kind="a"), u(*nld), u(n, l + 1, d, s, kind="a"), u(*nlds, kind="u"), u(*nlds),
                 u(*nls), u(d)], [z(*nld), z(n, d, s)])
    if op == 4:  # RwkvTokenShift
        return [u(*nld), u(d, kind="u"), u(d, kind="u"), u(d, kind="u")], [z(*nld), z(*nld), z(*nld)]
    if op == 5:  # RwkvForward
        return ([u(*nld), u(*nld), u(*nld), u(d), u(d, kind="u")],
                [z(*nld), z(*nld), z(*nld), z(*nld), z(*nld), z(*nld), z(n, l + 1, d), z(n, l + 1, d), z(*nld)])
    if op == 6:  # RwkvBackward
        return ([u(*nld), u(*nld, kind="u"), u(*nld), u(*nld, kind="u"), u(*nld, kind="u"), u(*nld),
                 u(*nld, kind="a"), u(n, l + 1, d), u(n, l + 1, d), u(*nld), u(d, kind="u")],
                [z(*nld)] * 5)
    if op == 7:  # RwkvShiftBackward
        return ([u(*nld), u(*nld), u(*nld), u(*nld), u(d, kind="u"), u(d, kind="u"), u(d, kind="u")],
                [z(*nld)] * 4)
    if op == 8:  # RwkvLrp
        return ([u(*nld), u(n, l + 1, d, kind="a"), u(*nld, kind="a"), u(*nld, kind="u"), u(*nld), u(*nld, kind="a"),
                 u(*nld, kind="u"), u(d, kind="u")], [z(*nld)])
    if op == 9:  # RwkvShiftLrp
        return [u(*nld), u(*nld, kind="a"), u(*nld), u(d, kind="u")], [z(*nld)]
    if op == 10:  # StabilizedDiv
        return [u(*nld), u(*nld, kind="a")], [z(*nld)]
    if op == 11:  # RetnetForward
        return [u(*nls), u(*nls), u(*nld)], [z(n, l + 1, s, d), z(*nld)]
    if op == 12:  # RetnetStateGrad
        return [u(*nld), u(*nls)], [z(n, l, s, d)]
    if op == 13:  # RetnetGradQK
        return [u(*nld), u(n, l + 1, s, d), u(n, l, s, d), u(*nld)], [z(*nls), z(*nls)]
    if op == 14:  # RetnetGradV
        return [u(n, l, s, d), u(*nls)], [z(*nld)]
    if op == 15:  # RetnetScores
        return [u(*nls), u(*nls)], [z(n, l, l), z(n, l, l)]
    if op == 16:  # RetnetReadout
        return [u(n, l, l), u(*nld)], [z(*nld)]
    if op == 17:  # RetnetLrpInput
        return ([u(*nld), u(d, s), u(d, s), u(d, d), u(*nls, kind="a"), u(*nls, kind="a"), u(*nld, kind="a"), u(*nls),
                 u(*nls), u(*nld)], [z(*nld)])
    assert op == 18  # ReverseTimeSum
    return [u(*nld)], [z(d)]


@pytest.mark.parametrize("op", range(19))
def test_ssm_pass(lib, op):
    ins, outs = ssm_case(op, op + 1)
    slots_vs_cpu(lib, "ssm_pass", op, ins, outs, [N_, L_, D_, S_, 1e-6, 0.9], 12, 10)


# ---- reinforcement-learning rows ---------------------------------------------------------------------

@pytest.mark.parametrize("op", range(9))
def test_rl_rows(lib, op):
    rows, cols = 37, 11
    r = np.random.RandomState(50 + op)
    idx = r.randint(0, cols, size=rows).astype(np.float32)
    q, v1, v2 = G.uniform((rows, cols), 51) * 3, G.uniform((rows,), 52), G.uniform((rows,), 53)
    z = lambda *s: np.zeros(s, np.float32)  # noqa: E731
    probs = np.exp(q) / np.exp(q).sum(axis=1, keepdims=True)
    exact = ()
    if op == 0:
        ins, outs = [q, idx, v1], [z(rows)]
    elif op == 1:
        ins, outs = [q, idx, v1], [z(rows, cols)]
    elif op == 2:
        ins, outs = [q, idx, v1], [z(rows, cols), z(rows)]
    elif op == 3:
        ins, outs = [probs, idx, v1], [z(rows, cols)]
    elif op == 4:
        ins, outs = [q, idx, -unit((rows,), 54) * 3, v2], [z(rows, cols), z(rows), z(rows), z(rows)]
        exact = (3,)
    elif op == 5:
        ins, outs = [probs, idx, v2, unit((rows,), 55) + 0.5, (r.rand(rows) > 0.3).astype(np.float32)], [z(rows, cols)]
    elif op == 6:
        ins, outs = [q, G.uniform((rows, cols), 56), v1, (r.rand(rows) > 0.7).astype(np.float32)], [z(rows)]
    elif op == 7:
        rows = rows * cols  # one lane per element
        ins, outs = [q.ravel(), G.uniform((rows,), 57)], [z(rows)]
    else:  # token cross-entropy: valid targets, the ignore index, non-integers and out-of-range ids
        t = idx.copy()
        t[:3] = -100.0
        t[3:5] = 2.5
        t[5:7] = [cols, -3.0]
        ins, outs = [q, t], [z(rows, cols), z(rows, 4), z(rows), z(rows)]
        exact = (2, 3)
    slots_vs_cpu(lib, "rl_rows", op, ins, outs, [rows, cols, 0.5, 0.8, 1.2, 0.95, 0.1, -100], 5, 4, exact=exact)
