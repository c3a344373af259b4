"""The drop-in, run: the reference's own modules on MI355XBackend.

oracle/_ref/libpxref_mi355x.so holds the reference's CausalLM, TransformerBlock, LinearModule,
ReluModule, ExplainerContext and LRP::explain (compiled from its sources, against its own
include/pulsatrix/device_backend.hpp) with MI355XBackend as their DeviceBackend, and pxr_be_*, a
shim that calls each DeviceBackend virtual of that backend on device pointers. These tests hold
them to the reference's own fixtures and to the oracle:

  * hf_tiny llama / qwen2 / qwen3 / gemma3 through the reference's CausalLM: transformers logits at
    1e-4, LXT 2.1 relevance (correlation > 0.99999, max relative difference < 1e-4, sums within
    1e-4; tests/attnlrp_parity_test.cpp:28-51);
  * the Zennit 1.0.0 MLP through LRP::explain, every uniform rule and the three composites, at the
    reference's tolerance (tests/lrp_reference_test.cpp:85-91, 285-303);
  * a TransformerBlock at config B and a small CausalLM against the oracle, both epsilon rules;
  * the reference's Hugging Face attention cases (Llama / Qwen2 with padding and a position offset /
    Qwen3 with QK-Norm: forward and input gradient, tests/attention_reference_test.cpp) and its
    independent NumPy AttnLRP block (tests/transformer_block_test.cpp:262-318) at their tolerances;
  * every path virtual against the oracle's restatement of CPUBackend on seeded uniform(-1, 1)
    inputs with non-square shapes, |gpu - cpu| <= 1e-4 (tests/backend_primitive_equivalence_cases.hpp:
    22-75), GEMMs with the K-scaled tolerance of tests/test_kernels_gpu.py.
Where the library was not built the tests fail: the GPU tests are the boundary evidence, and a
missing library must not pass as skipped.
"""
import ctypes

import numpy as np
import pytest

import dropin_cases as dc
import hf_attention_cases as hc
import gpu_util as G
import oracle_ctypes as oc
import rules_cases as rc
from hf_fixtures import hf_tiny, pearson, per_head, sequences
from test_model_gpu import LXT_EPS, argmax_seed, b_config, expect_logits_agree, expect_relevance_agrees

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    G.torch_cuda()
    lib = oc.ref_mi355x()
    if lib is None:
        pytest.fail("oracle/_ref/libpxref_mi355x.so was not built: the boundary evidence needs it "
                    "(__graft_entry__.build() builds it where the reference sources are)")
    assert lib.lib.pxr_be_device() == 2  # DeviceType::Hip (device_backend.hpp:17-21)
    return lib


def be(lib, name, *args):
    """One DeviceBackend virtual through the shim; device buffers are torch tensors."""
    torch = G.torch_cuda()
    torch.cuda.synchronize()  # inputs were written on torch's stream
    conv = [ctypes.c_void_p(a.data_ptr()) if hasattr(a, "data_ptr") else a for a in args]
    lib.check(getattr(lib.lib, "pxr_be_" + name)(*conv))
    lib.check(lib.lib.pxr_be_synchronize())


# ---- the reference's models on MI355XBackend ---------------------------------------------------

@pytest.mark.parametrize("name", sorted(hc.CASES))
def test_reference_attention_on_mi355x_matches_hf_attention_values(lib, name):
    """tests/attention_reference_test.cpp through MI355XBackend: Llama (GQA, right padding), Qwen2
    (MQA, biases, left padding, position offset 3) and Qwen3 (QK-Norm) attention, forward and the
    input gradient, against the values transformers 5.18.0 produced, at 1e-4 * max(1, |x|)."""
    out, grad = hc.run_mha_case(lib, name)
    want_out, want_grad = hc.expected(name)
    hc.assert_matches_reference(out, want_out, name + " forward")
    hc.assert_matches_reference(grad, want_grad, name + " input gradient")


def test_reference_block_on_mi355x_matches_numpy_attnlrp_values(lib):
    """tests/transformer_block_test.cpp:262-318 through MI355XBackend: the independent NumPy AttnLRP
    transcription's forward and LRPRuleConfig{} input relevance, within 1e-4."""
    y, r = hc.run_legacy_block_case(lib)
    v = hc.legacy_block_values()
    assert np.abs(y - np.array(v["expected_y"], np.float32)).max() <= 1e-4
    assert np.abs(r - np.array(v["expected_r_x"], np.float32)).max() <= 1e-4


@pytest.mark.parametrize("name", ["llama", "qwen2", "qwen3", "gemma3"])
def test_reference_causal_lm_on_mi355x_matches_goldens(lib, name):
    cfg, params, golden, ref = hf_tiny(name)
    lm = lib.lm(cfg, params)
    for k in sequences(golden):
        ids = golden["ids.%d" % k].reshape(1, -1)
        logits = lm.forward(ids)[0]
        exp = golden["logits.%d" % k]
        assert np.all(np.abs(logits - exp) <= 1e-4 * np.maximum(1.0, np.abs(exp))), (name, k)
    for k in sequences(ref):
        ids = ref["ids.%d" % k].reshape(1, -1)
        L = ids.shape[1]
        target = int(ref["target.%d" % k][0])
        logits = lm.forward(ids)
        seed = np.zeros_like(logits)
        seed[0, L - 1, target] = logits[0, L - 1, target]
        _, r_tok, key, value = lm.relevance(seed, LXT_EPS, True, want_kv=True)
        expected = ref["relevance.%d" % k]
        assert pearson(r_tok[0], expected) > 0.99999
        assert np.abs(r_tok[0] - expected).max() / np.abs(expected).max() < 1e-4
        assert abs(r_tok.sum() - expected.sum()) <= 1e-4 * abs(expected.sum())
        for i in range(cfg.num_layers):
            assert pearson(per_head(key[i], L, cfg.kv_heads()), ref["key_relevance.%d" % k][i]) > 0.99999
            assert pearson(per_head(value[i], L, cfg.kv_heads()), ref["value_relevance.%d" % k][i]) > 0.99999


@pytest.mark.parametrize("case", dc.explain_cases(), ids=lambda c: c[0])
def test_reference_lrp_explain_on_mi355x_matches_zennit(lib, case):
    name, rule, preset, key = case
    rel, total = oc.mlp_explain(lib, rc.mlp_params(), rc.mlp_input(), rc.MLP_TARGETS, rule, preset)
    rc.expect_reference_close(rel, rc.zennit_values()[key])
    assert abs(total - float(rel.astype(np.float64).sum())) <= 1e-5 * max(1.0, abs(total))


@pytest.mark.parametrize("rule", ["default", "lxt"])
def test_reference_block_on_mi355x_matches_oracle(lib, rule):
    """Config B: the reference's TransformerBlock (d 576, 9/3 heads, FFN 1536, seq 128) on MI355XBackend."""
    cfg = b_config()
    params = oc.synthetic_params(cfg, 2024, block=True)
    x = oc.fill_normal(128 * 576, 7, 1.0).reshape(1, 128, 576)
    ref, gpu = oc.oracle().block(cfg, params), lib.block(cfg, params)
    y_ref, y = ref.forward(x), gpu.forward(x)
    G.assert_close(y, y_ref, 1e-4, "block forward")
    seed = np.zeros_like(y_ref)
    seed[..., 0] = y_ref[..., 0]
    eps, bid = (1e-6, False) if rule == "default" else (LXT_EPS, True)
    expect_relevance_agrees(gpu.relevance(seed, eps, bid), ref.relevance(seed, eps, bid), "block " + rule)


def test_reference_causal_lm_on_mi355x_matches_oracle(lib):
    cfg = oc.model_config(vocab_size=1000, hidden_size=64, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=16,
                          intermediate_size=96, rms_norm_eps=1e-5, rope_theta=100000.0)
    params = oc.synthetic_params(cfg, 99)
    ids = np.random.RandomState(3).randint(0, cfg.vocab_size, size=(2, 37))
    ref, gpu = oc.oracle().lm(cfg, params), lib.lm(cfg, params)
    lr, lg = ref.forward(ids), gpu.forward(ids)
    expect_logits_agree(lg, lr, "logits")
    seed = argmax_seed(lr)
    for eps, bid in ((LXT_EPS, True), (1e-6, False)):
        a = gpu.relevance(seed, eps, bid, want_kv=True)
        b = ref.relevance(seed, eps, bid, want_kv=True)
        for what, x, y in zip(("embedding", "tokens", "keys", "values"), a, b):
            expect_relevance_agrees(x, y, "%s bid=%s" % (what, bid))


@pytest.mark.parametrize("case", rc.all_rules(), ids=lambda c: c[0])
def test_reference_linear_rules_on_mi355x_match_oracle(lib, case):
    """LinearModule::propagate_relevance under every rule (lrp_rules.cpp:72-220) through the
    reference's module on MI355XBackend, against the oracle's restatement."""
    name, rule = case[0], case[1]
    # as tests/test_rules_gpu.py: inputs inside ZBox's box, weights scaled by 1/sqrt(in)
    rng = np.random.RandomState(17)
    x = rng.uniform(-1, 1, (40, 24)).astype(np.float32)
    w = (rng.uniform(-1, 1, (24, 33)) / np.sqrt(24)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, 33).astype(np.float32)
    r = rng.uniform(-1, 1, (40, 33)).astype(np.float32)
    pre, _ = oc.linear_forward(x, w, b)
    expected = oc.linear_relevance_rule(x, w, b, pre, r, rule)
    out = np.empty((40, 24), np.float32)
    fp = oc.fptr
    lib.check(lib.lib.pxr_linear_relevance_rule(fp(x), fp(w), fp(b), fp(r), 40, 24, 33, ctypes.byref(rule), fp(out)))
    expect_relevance_agrees(out, expected, name)


# ---- each DeviceBackend virtual through the shim --------------------------------------------------

def gemm_tol(k):
    return 1e-4 * max(1.0, k / 1024.0)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,k,n,beta", [(5, 7, 3, 0.0), (130, 70, 33, 1.0), (257, 129, 131, 0.0)])
def test_virtual_gemm_ex(lib, ta, tb, m, k, n, beta):
    a = G.uniform((k, m) if ta else (m, k), 1)
    b = G.uniform((n, k) if tb else (k, n), 2)
    c0 = G.uniform((m, n), 3)
    ref = c0.copy()
    G.oracle_call("pxo_gemm_ex", a, ta, b, tb, ref, m, k, n, beta)
    out = G.dev(c0)
    be(lib, "gemm_ex", G.dev(a), ta, G.dev(b), tb, out, m, k, n, beta)
    G.assert_close(G.host(out), ref, gemm_tol(k), "gemm_ex")
    if not ta and not tb and beta == 0.0:
        out2 = G.empty((m, n))
        be(lib, "gemm", G.dev(a), G.dev(b), out2, m, k, n)
        G.assert_close(G.host(out2), ref, gemm_tol(k), "gemm")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_virtual_gemm_strided_batched(lib, ta, tb):
    """The reference's default is a loop of gemm_ex over the batch (device_backend.hpp:372-383);
    strides here are larger than the matrices (padded slices) and beta accumulates."""
    batch, m, k, n, beta = 3, 37, 50, 29, 1.0
    sa, sb, so = m * k + 11, k * n + 5, m * n + 7
    a = G.uniform((batch * sa,), 1)
    b = G.uniform((batch * sb,), 2)
    c = G.uniform((batch * so,), 3)
    ref = c.copy()
    for i in range(batch):
        ai = np.ascontiguousarray(a[i * sa:i * sa + m * k])
        bi = np.ascontiguousarray(b[i * sb:i * sb + k * n])
        ci = np.ascontiguousarray(ref[i * so:i * so + m * n])
        G.oracle_call("pxo_gemm_ex", ai, ta, bi, tb, ci, m, k, n, beta)
        ref[i * so:i * so + m * n] = ci
    out = G.dev(c)
    be(lib, "gemm_strided_batched", G.dev(a), ta, sa, G.dev(b), tb, sb, out, so, m, k, n, batch, beta)
    G.assert_close(G.host(out), ref, gemm_tol(k), "gemm_strided_batched")


def test_virtual_lrp_linear(lib):
    rows, i, o = 45, 70, 33
    x, w, z, r = G.uniform((rows, i), 1), G.uniform((i, o), 2), G.uniform((rows, o), 3), G.uniform((rows, o), 4)
    ref = np.empty((rows, i), np.float32)
    G.oracle_call("pxo_lrp_linear", x, w, z, r, ref, rows, i, o, 1e-6)
    out = G.empty((rows, i))
    be(lib, "lrp_linear", G.dev(x), G.dev(w), G.dev(z), G.dev(r), out, rows, i, o, 1e-6)
    G.assert_close(G.host(out), ref, 1e-4, "lrp_linear")


@pytest.mark.parametrize("bt", [0, 1])
def test_virtual_lrp_bilinear_matmul(lib, bt):
    """Eq. 15 for O = A B per slice, B stored (p, q) or transposed (q, p); O = A B computed here."""
    s, m, p, q = 3, 17, 12, 23
    a = G.uniform((s, m, p), 1)
    b = G.uniform((s, q, p) if bt else (s, p, q), 2)
    bm = np.transpose(b, (0, 2, 1)) if bt else b
    o = np.einsum("smp,spq->smq", a.astype(np.float64), bm.astype(np.float64)).astype(np.float32)
    r = G.uniform((s, m, q), 3)
    ra, rb = np.empty_like(a), np.empty_like(b)
    G.oracle_call("pxo_lrp_bilinear_matmul", a, b, o, r, ra, rb, s, m, p, q, 1e-6, bt)
    ga, gb = G.empty(a.shape), G.empty(b.shape)
    be(lib, "lrp_bilinear_matmul", G.dev(a), G.dev(b), G.dev(o), G.dev(r), ga, gb, s, m, p, q, 1e-6, bt)
    expect_relevance_agrees(G.host(ga), ra, "r_a")
    expect_relevance_agrees(G.host(gb), rb, "r_b")


def test_virtual_softmax_rows_and_rule(lib):
    rows, cols = 37, 129
    x, r = G.uniform((rows, cols), 1) * 4, G.uniform((rows, cols), 2)
    y = np.empty_like(x)
    G.oracle_call("pxo_softmax_rows", x, y, rows, cols)
    gy = G.empty((rows, cols))
    be(lib, "softmax_rows", G.dev(x), gy, rows, cols)
    G.assert_close(G.host(gy), y, 1e-4, "softmax_rows")
    ref = np.empty_like(x)
    G.oracle_call("pxo_lrp_softmax_rows", x, y, r, ref, rows, cols)
    out = G.empty((rows, cols))
    be(lib, "lrp_softmax_rows", G.dev(x), G.dev(y), G.dev(r), out, rows, cols)
    G.assert_close(G.host(out), ref, 1e-4, "lrp_softmax_rows")


@pytest.mark.parametrize("half", [1, 0])
def test_virtual_rope_rotate_and_rule(lib, half):
    slices, L, D = 6, 19, 16
    cs, sn = np.empty((L, D // 2), np.float32), np.empty((L, D // 2), np.float32)
    oc.oracle().lib.pxo_rope_tables(D, 10000.0, L, 0, oc.fptr(cs), oc.fptr(sn))
    x, r = G.uniform((slices, L, D), 1), G.uniform((slices, L, D), 2)
    for inverse in (0, 1):
        ref = np.empty_like(x)
        G.oracle_call("pxo_rope_rotate", x, cs, sn, ref, slices, L, D, inverse, half)
        out = G.empty(x.shape)
        be(lib, "rope_rotate", G.dev(x), G.dev(cs), G.dev(sn), out, slices, L, D, inverse, half)
        G.assert_close(G.host(out), ref, 1e-5, "rope_rotate")
    y = np.empty_like(x)
    G.oracle_call("pxo_rope_rotate", x, cs, sn, y, slices, L, D, 0, half)
    ref = np.empty_like(x)
    G.oracle_call("pxo_lrp_rope", x, y, r, cs, sn, ref, slices, L, D, 1e-6, half)
    out = G.empty(x.shape)
    be(lib, "lrp_rope", G.dev(x), G.dev(y), G.dev(r), G.dev(cs), G.dev(sn), out, slices, L, D, 1e-6, half)
    expect_relevance_agrees(G.host(out), ref, "lrp_rope")


def test_virtual_permute_mask_gather_copy2d_accumulate(lib):
    x = G.uniform((2, 5, 3, 7), 1)
    ref = np.empty((2, 3, 5, 7), np.float32)
    G.oracle_call("pxo_permute_0213", x, ref, 2, 5, 3, 7)
    out = G.empty(ref.shape)
    be(lib, "permute_0213", G.dev(x), out, 2, 5, 3, 7)
    assert np.array_equal(G.host(out), ref)
    for causal, window, keep in ((1, 0, None), (0, 0, True), (1, 4, True)):
        s = G.uniform((2, 3, 9, 9), 2)
        kp = (np.random.RandomState(5).rand(2, 9) > 0.3).astype(np.float32) if keep else None
        ref = s.copy()
        G.oracle_call("pxo_attention_mask_fill", ref, kp, 2, 3, 9, 9, causal, 0, window, -7.0)
        out = G.dev(s)
        be(lib, "attention_mask_fill", out, G.dev(kp) if keep else None, 2, 3, 9, 9, causal, 0, window, -7.0)
        assert np.array_equal(G.host(out), ref), (causal, window, keep)
    table, idx = G.uniform((11, 24), 3), np.array([3, 0, 10, 3, 7], np.float32)
    ref = np.empty((5, 24), np.float32)
    G.oracle_call("pxo_gather_rows", table, idx, ref, 5, 24)
    out = G.empty((5, 24))
    be(lib, "gather_rows", G.dev(table), G.dev(idx), out, 5, 24)
    assert np.array_equal(G.host(out), ref)
    src, dst = G.uniform((6, 10), 4), G.uniform((6, 16), 5)
    ref = dst.copy()
    G.oracle_call("pxo_copy_2d", ref, 16, src, 10, 6, 10)
    out = G.dev(dst)
    be(lib, "copy_2d", out, 16, G.dev(src), 10, 6, 10)
    assert np.array_equal(G.host(out), ref)
    acc = G.uniform((10,), 6)
    ref = acc.copy()
    G.oracle_call("pxo_accumulate_rows", src, ref, 6, 10)
    out = G.dev(acc)
    be(lib, "accumulate_rows", G.dev(src), out, 6, 10)
    G.assert_close(G.host(out), ref, 1e-5, "accumulate_rows")


H2D, D2H, D2D, H2H = 0, 1, 2, 3  # CopyDirection (device_backend.hpp:24-29)


def test_virtual_copy_directions_and_odd_sizes(lib):
    """copy() in every direction with byte counts that are not a multiple of 4 (hip_backend.hip:83-111)."""
    torch = G.torch_cuda()
    src = np.random.RandomState(1).randint(0, 256, size=4099).astype(np.uint8)
    dev = G.keep(torch.zeros(4112, dtype=torch.uint8, device="cuda"))
    for nbytes in (1, 3, 4, 7, 4096, 4099):
        dev.zero_()
        torch.cuda.synchronize()
        lib.check(lib.lib.pxr_be_copy(dev.data_ptr(), src.ctypes.data, nbytes, H2D))
        back = np.zeros(4112, np.uint8)
        lib.check(lib.lib.pxr_be_copy(back.ctypes.data, dev.data_ptr(), nbytes, D2H))
        assert np.array_equal(back[:nbytes], src[:nbytes]) and not back[nbytes:].any(), nbytes
        dev2 = G.keep(torch.zeros(4112, dtype=torch.uint8, device="cuda"))
        torch.cuda.synchronize()
        lib.check(lib.lib.pxr_be_copy(dev2.data_ptr() + 1, dev.data_ptr(), nbytes, D2D))  # unaligned destination
        lib.check(lib.lib.pxr_be_synchronize())
        got = dev2.cpu().numpy()
        assert np.array_equal(got[1:1 + nbytes], src[:nbytes]) and not got[1 + nbytes:].any(), nbytes
        host2 = np.zeros(4112, np.uint8)
        lib.check(lib.lib.pxr_be_copy(host2.ctypes.data, src.ctypes.data, nbytes, H2H))
        assert np.array_equal(host2[:nbytes], src[:nbytes])
    assert lib.lib.pxr_be_copy(None, None, 0, D2D) == 0  # zero bytes: nothing to do


def test_virtual_reductions_and_rows(lib):
    torch = G.torch_cuda()
    n = 100003
    a, b = G.uniform((n,), 1), G.uniform((n,), 2)
    got = ctypes.c_float()
    lib.check(lib.lib.pxr_be_sum(G.dev(a).data_ptr(), n, ctypes.byref(got)))
    G.assert_close(got.value, G.oracle_call("pxo_sum", a, n), 1e-4, "sum")
    lib.check(lib.lib.pxr_be_dot(G.dev(a).data_ptr(), G.dev(b).data_ptr(), n, ctypes.byref(got)))
    ref_dot = G.oracle_call("pxo_dot", a, b, n)
    G.assert_close(got.value, ref_dot, 1e-4, "dot")
    slot = G.empty((1,))
    be(lib, "dot_into", G.dev(a), G.dev(b), n, slot)
    G.assert_close(G.host(slot)[0], ref_dot, 1e-4, "dot_into")
    rows, cols = 33, 70
    x, row = G.uniform((rows, cols), 3), G.uniform((cols,), 4)
    ref = np.empty_like(x)
    G.oracle_call("pxo_add_row_vector", x, row, ref, rows, cols)
    out = G.empty(x.shape)
    be(lib, "add_row_vector", G.dev(x), G.dev(row), out, rows, cols)
    assert np.array_equal(G.host(out), ref)
    acc = G.uniform((cols,), 5)
    ref = acc.copy()
    G.oracle_call("pxo_column_sums", x, ref, rows, cols, 0.5)
    out = G.dev(acc)
    be(lib, "column_sums", G.dev(x), out, rows, cols, 0.5)
    G.assert_close(G.host(out), ref, 1e-5, "column_sums")
    g = G.uniform((cols,), 6)
    ref, rms = np.empty_like(x), np.empty((rows,), np.float32)
    G.oracle_call("pxo_rms_norm_forward", x, g, ref, rms, rows, cols, 1e-5)
    out, grms = G.empty(x.shape), G.empty((rows,))
    be(lib, "rms_norm_forward", G.dev(x), G.dev(g), out, grms, rows, cols, 1e-5)
    G.assert_close(G.host(out), ref, 1e-5, "rms_norm")
    G.assert_close(G.host(grms), rms, 1e-5, "row_rms")
    del torch


def test_virtual_elementwise_family(lib):
    n = 1000
    a, b, r = G.uniform((n,), 1), G.uniform((n,), 2), G.uniform((n,), 3)
    for op in range(8):  # ElementwiseOp: Relu, Neg, Tanh, Sigmoid, Silu, Exp, GeluTanh, Gelu
        ref = np.empty_like(a)
        G.oracle_call("pxo_elementwise", op, a, ref, n)
        out = G.empty((n,))
        be(lib, "elementwise", op, G.dev(a), out, n)
        G.assert_close(G.host(out), ref, 1e-5, "elementwise %d" % op)
    for name in ("add", "mul"):
        ref = np.empty_like(a)
        G.oracle_call("pxo_" + name, a, b, ref, n)
        out = G.empty((n,))
        be(lib, name, G.dev(a), G.dev(b), out, n)
        assert np.array_equal(G.host(out), ref), name
    for beta in (0.0, -0.25):
        ref = np.empty_like(a)
        G.oracle_call("pxo_axpby", 1.5, a, beta, b, ref, n)
        out = G.empty((n,))
        y = G.dev(b) if beta != 0.0 else G.empty((n,))  # beta 0 never reads y: NaN there must not leak
        be(lib, "axpby", 1.5, G.dev(a), beta, y, out, n)
        G.assert_close(G.host(out), ref, 1e-6, "axpby %g" % beta)  # the GPU may fuse a x + b y into an FMA
    ra, rb = np.empty_like(a), np.empty_like(a)
    G.oracle_call("pxo_lrp_residual_split", a, b, r, ra, rb, n, 1e-6)
    ga, gb = G.empty((n,)), G.empty((n,))
    be(lib, "lrp_residual_split", G.dev(a), G.dev(b), G.dev(r), ga, gb, n, 1e-6)
    expect_relevance_agrees(G.host(ga), ra, "residual split a")
    expect_relevance_agrees(G.host(gb), rb, "residual split b")
    ref = np.empty_like(a)
    G.oracle_call("pxo_lrp_bilinear_elementwise", a, b, r, ref, n, 1e-9)
    out = G.empty((n,))
    be(lib, "lrp_bilinear_elementwise", G.dev(a), G.dev(b), G.dev(r), out, n, 1e-9)
    expect_relevance_agrees(G.host(out), ref, "bilinear elementwise")
    for mode in (0, 1, 2):
        ref = np.empty_like(a)
        G.oracle_call("pxo_lrp_stabilized_divide", r, a, b, ref, n, 1e-6, mode)
        out = G.empty((n,))
        be(lib, "lrp_stabilized_divide", G.dev(r), G.dev(a), G.dev(b), out, n, 1e-6, mode)
        expect_relevance_agrees(G.host(out), ref, "stabilized divide %d" % mode)
    out = G.empty((n,))
    be(lib, "fill", out, 2.5, n)
    assert np.all(G.host(out) == 2.5)


def test_virtual_allocation_contract(lib):
    """allocate(0) is nullptr, a nonzero request never is, free(nullptr) is safe (device_backend.hpp:262-276)."""
    p = ctypes.c_void_p(1)
    lib.check(lib.lib.pxr_be_allocate(0, ctypes.byref(p)))
    assert p.value is None
    lib.check(lib.lib.pxr_be_allocate(1000, ctypes.byref(p)))
    assert p.value
    lib.lib.pxr_be_free(p)
    lib.lib.pxr_be_free(None)


# ---- training and non-LLM row / element virtuals: MI355XBackend against the reference CPUBackend ----

def cpu_vs_gpu(lib, name, arrays, outs, args, rel=1e-5, exact=()):
    """Runs pxr_be_<name> on the reference CPUBackend (oracle/_ref/libpxref.so, host arrays) and on
    MI355XBackend (device copies of the same arrays); `args` names arrays by key and passes scalars
    through. Compares each array in `outs` (exactly for the keys in `exact`)."""
    cpu = oc.ref()
    if cpu is None:
        pytest.fail("oracle/_ref/libpxref.so was not built: the boundary evidence needs it "
                    "(__graft_entry__.build() builds it where the reference sources are)")
    host = {k: np.ascontiguousarray(v).copy() for k, v in arrays.items()}
    dev = {k: G.dev(v) for k, v in arrays.items()}
    cpu.check(getattr(cpu.lib, "pxr_be_" + name)(*[host[a].ctypes.data if isinstance(a, str) else a for a in args]))
    be(lib, name, *[dev[a] if isinstance(a, str) else a for a in args])
    for k in outs:
        got, exp = G.host(dev[k]), host[k]
        if k in exact:
            assert np.array_equal(got, exp, equal_nan=True), (name, k)
        else:
            G.assert_close(got, exp, rel, "%s %s" % (name, k))


def test_virtual_backward_rows_against_reference_and_oracle(lib):
    """elementwise_backward (every op), softmax_rows_backward and rms_norm_backward
    (device_backend.hpp:428, 462, 557): against the compiled reference, and the trio's oracle
    restatement (pinned bit for bit to it on the CPU) at the same tolerance."""
    n, rows, cols = 100003, 70, 300
    x, g = G.uniform((n,), 1) * 3, G.uniform((n,), 2)
    for op in range(8):
        cpu_vs_gpu(lib, "elementwise_backward", {"x": x, "g": g, "o": np.zeros_like(x)}, ["o"], [op, "x", "g", "o", n],
                   exact=("o",) if op in (0, 1) else ())
        ref = np.empty_like(x)
        G.oracle_call("pxo_elementwise_backward", op, x, g, ref, n)
        out = G.empty((n,))
        be(lib, "elementwise_backward", op, G.dev(x), G.dev(g), out, n)
        G.assert_close(G.host(out), ref, 1e-5, "elementwise_backward %d vs oracle" % op)
    y = np.exp(G.uniform((rows, cols), 3))
    y /= y.sum(axis=1, keepdims=True)
    dy = G.uniform((rows, cols), 4)
    cpu_vs_gpu(lib, "softmax_rows_backward", {"y": y, "dy": dy, "dx": np.zeros_like(y)}, ["dx"],
               ["y", "dy", "dx", rows, cols])
    xin, gamma = G.uniform((rows, cols), 5), G.uniform((cols,), 6)
    rms = np.sqrt((xin.astype(np.float64) ** 2).mean(axis=1) + 1e-5).astype(np.float32)
    cpu_vs_gpu(lib, "rms_norm_backward", {"g": dy, "gamma": gamma, "x": xin, "rms": rms, "gx": np.zeros_like(xin),
                                          "gt": np.zeros_like(xin)}, ["gx", "gt"],
               ["g", "gamma", "x", "rms", "gx", "gt", rows, cols])


def test_virtual_layer_norm_logsumexp_scatter(lib):
    rows, cols = 45, 257
    x, gamma, beta, gy = G.uniform((rows, cols), 1) * 2, G.uniform((cols,), 2), G.uniform((cols,), 3), \
        G.uniform((rows, cols), 4)
    z = np.zeros_like(x)
    cpu_vs_gpu(lib, "layer_norm_forward", {"x": x, "gamma": gamma, "beta": beta, "xhat": z, "out": z,
                                           "sd": np.zeros(rows, np.float32)}, ["xhat", "out", "sd"],
               ["x", "gamma", "beta", "xhat", "out", "sd", rows, cols, 1e-5])
    xhat = (x - x.mean(axis=1, keepdims=True)) / np.sqrt(x.var(axis=1, keepdims=True) + 1e-5)
    sd = np.sqrt(x.astype(np.float64).var(axis=1) + 1e-5).astype(np.float32)
    cpu_vs_gpu(lib, "layer_norm_backward", {"g": gy, "gamma": gamma, "xhat": xhat.astype(np.float32), "sd": sd,
                                            "gx": z}, ["gx"], ["g", "gamma", "xhat", "sd", "gx", rows, cols])
    cpu_vs_gpu(lib, "logsumexp_rows", {"x": x * 5, "o": np.zeros(rows, np.float32)}, ["o"], ["x", "o", rows, cols])
    # repeated indices accumulate in source order; the reference sums the same way per column
    idx = np.array([3, 0, 3, 7, 3, 1, 0], np.float32)
    src, table = G.uniform((7, 33), 5), G.uniform((8, 33), 6)
    cpu_vs_gpu(lib, "scatter_add_rows", {"src": src, "idx": idx, "t": table}, ["t"], ["src", "idx", "t", 7, 33],
               exact=("t",))


def test_virtual_optimizer_dropout_losses_policy_topk(lib):
    n = 10007
    p, g, m, v = G.uniform((n,), 1), G.uniform((n,), 2), G.uniform((n,), 3) * 0.1, np.abs(G.uniform((n,), 4)) * 0.1
    cpu_vs_gpu(lib, "adam_step", {"p": p, "g": g, "m": m, "v": v}, ["p", "m", "v"],
               ["p", "g", "m", "v", n, 1e-3, 0.9, 0.999, 1e-8, 0.1, 0.001], rel=1e-6)
    x = G.uniform((n,), 5)
    z = np.zeros_like(x)
    cpu_vs_gpu(lib, "dropout_forward", {"x": x, "o": z, "mask": z}, ["o", "mask"],
               ["x", "o", "mask", n, 0.3, 1.0 / 0.7, 1234, 99], exact=("o", "mask"))
    y = (G.uniform((n,), 6) > 0).astype(np.float32)
    xl = x * 30  # both tails of the stable forms
    cpu_vs_gpu(lib, "bce_with_logits", {"x": xl, "y": y, "o": z}, ["o"], ["x", "y", "o", n], rel=1e-6)
    cpu_vs_gpu(lib, "bce_with_logits_grad", {"x": xl, "y": y, "o": z}, ["o"], ["x", "y", "o", n, 0.5], rel=1e-6)
    rows, cols = 33, 6
    mean, ls, e = G.uniform((rows, cols), 7), G.uniform((rows, cols), 8) * 0.5, G.uniform((rows, cols), 9)
    zz = np.zeros((rows, cols), np.float32)
    cpu_vs_gpu(lib, "tanh_gaussian_forward", {"mean": mean, "ls": ls, "e": e, "a": zz, "sd": zz,
                                              "lp": np.zeros(rows, np.float32)}, ["a", "sd", "lp"],
               ["mean", "ls", "e", "a", "sd", "lp", rows, cols, 1e-6, 0.9189385332046727], rel=1e-5)
    a, sd = np.tanh(mean + np.exp(ls) * e).astype(np.float32), np.exp(ls).astype(np.float32)
    ga, glp = G.uniform((rows, cols), 10), G.uniform((rows, cols), 11)
    cpu_vs_gpu(lib, "tanh_gaussian_backward", {"a": a, "sd": sd, "e": e, "ga": ga, "glp": glp, "gm": zz, "gls": zz},
               ["gm", "gls"], ["a", "sd", "e", "ga", "glp", "gm", "gls", rows * cols, 1e-6], rel=1e-5)
    vals = G.uniform((19, 50), 12)
    vals[3, 7] = np.nan
    vals[5, :10] = 0.25  # ties keep the lower column
    k = 6
    for largest in (1, 0):
        cpu_vs_gpu(lib, "top_k_rows", {"x": vals, "v": np.zeros((19, k), np.float32), "i": np.zeros((19, k), np.float32)},
                   ["v", "i"], ["x", "v", "i", 19, 50, k, largest], exact=("v", "i"))


@pytest.mark.parametrize("tied", [1, 0])
def test_reference_causal_lm_backward_on_mi355x_matches_cpu_backend(lib, tied):
    """The backward pass through the drop-in: the reference's CausalLM::backward (causal_lm.cpp:82-92:
    the head, the final RMSNorm, every block's SwiGLU, attention with RoPE and GQA, and the
    embedding's scatter-add) on MI355XBackend against the same code on its CPUBackend; every
    parameter's gradient within 1e-4 of the gradient's scale."""
    cpu = oc.ref()
    if cpu is None:
        pytest.fail("oracle/_ref/libpxref.so was not built: the boundary evidence needs it "
                    "(__graft_entry__.build() builds it where the reference sources are)")
    cfg = oc.model_config(vocab_size=300, hidden_size=64, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=16,
                          intermediate_size=96, rms_norm_eps=1e-5, rope_theta=10000.0, tie_word_embeddings=tied)
    params = oc.synthetic_params(cfg, 21)
    ids = np.random.RandomState(2).randint(0, cfg.vocab_size, size=(2, 13))
    grad = G.uniform((2, 13, cfg.vocab_size), 3)
    got = []
    for L in (cpu, lib):
        lm = L.lm(cfg, params)
        lm.forward(ids)
        out = np.empty_like(params)
        L.lib.pxr_lm_backward.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.check(L.lib.pxr_lm_backward(lm.h, grad.ctypes.data, out.ctypes.data))
        got.append(out)
        del lm
    ref_g, gpu_g = got
    assert np.all(np.isfinite(gpu_g)) and np.abs(ref_g).max() > 0
    off = 0
    for name, shape in oc.lm_layout(cfg):
        size = int(np.prod(shape))
        a, b = gpu_g[off:off + size], ref_g[off:off + size]
        scale = max(float(np.abs(b).max()), 1e-12)
        assert np.abs(a - b).max() <= 1e-4 * scale, (name, float(np.abs(a - b).max()), scale)
        off += size
