"""Throughput of the causal-LM forward + AttnLRP path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode graph|eager] [--no-cpu-baseline]
    python bench.py --op-sweep        # raw op sweep: GEMM shapes, elementwise 2^26, RMSNorm 32768 x 2048
    python bench.py --kernel-probe    # 256 MiB copy + LM-head relevance GEMM, for rocprofv3 --pmc runs
    python bench.py --rule gamma      # the same step under Zennit's Gamma(0.25) (or zplus, alpha2beta1, zbox)
    python bench.py --decode          # Gemma-3-270m shape: batched KV-cached greedy decode + AttnLRP per token
    python bench.py --l1b             # Llama-3.2-1B shape, batch 8 x 1024: the explain step at large shapes
    python bench.py --block           # config B: one TransformerBlock, GPU and reference CPUBackend

Workload: the SmolLM2-135M-shaped causal LM (30 layers, hidden 576, 9 query / 3 KV heads of 64,
SwiGLU FFN 1536, vocab 49152, tied embeddings, RMSNorm eps 1e-5, RoPE theta 100000), fp32,
random init N(0, 0.02) from a seed with every RMSNorm gamma 1, batch 1 x 512 uniform-random token
ids. One step: forward logits, the argmax of the last position's logits seeded with its value
(on device), the AttnLRP relevance pass (LXT settings: epsilon 1e-9, bias in the denominator) back
to the embeddings, and per-token relevance sums. The ids are resident in HBM before the timed
region; every step launches the whole path (a HIP graph of it in graph mode).

Prints one JSON line. Per-kernel times come from the step's own launches (recorded in one eager step,
replayed in order with HIP events on the backend's stream): `gemm_pct_peak` is the sum of 2MNK over
the step's GEMM launches over their summed time against MI355X's 157.3 TFLOP/s dense fp32 matrix
peak, and `roofline` is the kernel variant with the most time per step.
`cpu_baseline` times the reference CPUBackend (oracle/_ref where built, else the oracle
restatement) on the host cores: the median of three complete passes of the same 30-layer model
after a full-depth warm-up.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_MFMA_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0
LXT_EPS = 1e-9

# HBM bytes per launch of the step's kernels, by launch-log name: FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0
# KiB (the factors a 256 MiB copy reads for the two counters), the median over a launch name's
# launches, from rocprofv3 --pmc runs of this bench summarised by `bench.py --pmc-table`
# (profiles/explain_s512_step_counters.md). A launch's kernels add up (the split-K GEMM and its
# reduce); the o and down projections share one name. The roofline line carries the figure of its
# kernel when that kernel was measured under this plan.
STEP_KERNEL_TRAFFIC = {name: kib * 1024 for name, kib in {
    "gemm 32x64d NN pro2 epi9 split1": 14094,  # q|k|v projection (norm folded, RoPE epilogue)
    "attn_fwd": 8240,  # fused attention forward, statistics form (ctx and per-row softmax statistics)
    "gemm 32x48d NN pro0 epi2 split1": 17649,  # o and down projections (median of both)
    "gemm 32x64 NN pro2 epi10 split1": 28750,  # gate|up projection (norm folded, SwiGLU epilogue)
    "gemm 128x128 NT pro0 epi0 split1": 228592,  # LM head forward
    "head_seeded_relevance": 2554,
    "gemm 32x48 NT pro0 epi7 split1": 24936,  # down relevance (SwiGLU rule epilogue)
    "gemm 32x48 NT pro0 epi8 split4": 38806,  # gate|up relevance + its split-K reduce and residual split
    "gemm 32x48d NT pro0 epi4 split1": 9856,  # o relevance (s_pv epilogue)
    "attn_rel_q": 22324,  # q side, recomputing raw and P; writes s and P for the key side
    "attn_rel_kv": 19364,  # key / value side
    "gemm 32x48d NT pro0 epi8 split1": 19934,  # q|k|v relevance (residual split)
    "gemm 32x48d NT pro0 epi3 split1": 16014,  # q|k|v relevance of block 0
}.items()}
# The same for the decode step's tied head (4 x 640 x 262144, skinny NT; `bench.py --decode-probe`,
# profiles/decode_head_gemm_traffic.md): FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0 of the median dispatch.
DECODE_HEAD_TRAFFIC = {"plan": (7, 1), "bytes": (327831.8 * 2.0 + 4096) * 1024}

S_CONFIG = dict(vocab_size=49152, hidden_size=576, num_layers=30, num_heads=9, num_kv_heads=3, head_dim=64,
                intermediate_size=1536, rms_norm_eps=1e-5, rope_theta=100000.0, use_rope=1, rope_rotate_half=1,
                causal=1, qkv_bias=0, out_bias=0, mlp_bias=0, tie_word_embeddings=1, reserved=0)
BATCH, SEQ, SEED = 1, 512, 1234

# Llama-3.2-1B's shape (random init), batch 8 x 1024: the large-shape GEMM and attention regime. The
# CPU baseline runs a bounded sample of it, one sequence of L1B_CPU_SEQ tokens at the full depth.
L1B_CONFIG = dict(S_CONFIG, vocab_size=128256, hidden_size=2048, num_layers=16, num_heads=32, num_kv_heads=8,
                  head_dim=64, intermediate_size=8192, rope_theta=500000.0)
L1B_BATCH, L1B_SEQ, L1B_CPU_SEQ = 8, 1024, 128

# Config B: one block at the SmolLM2 widths, theta 10000, seq 128.
B_CONFIG = dict(hidden_size=576, num_heads=9, num_kv_heads=3, head_dim=64, intermediate_size=1536, rms_norm_eps=1e-5,
                rope_theta=10000.0)
B_SEQ = 128

# The rules --rule selects (LRPRuleConfig fields; LRPRule order 0 Epsilon, 1 Gamma, 2 AlphaBeta, 3 ZBox):
# LXT's AttnLRP (the default, and the headline metric) and Zennit's affine rules at their usual settings.
RULES = {
    "lxt": dict(rule=0, epsilon=LXT_EPS, bias_in_denominator=True),
    "eps": dict(rule=0, epsilon=1e-6),
    "gamma": dict(rule=1, epsilon=1e-6, gamma=0.25),
    "zplus": dict(rule=2, epsilon=1e-6, alpha=1.0, beta=0.0),
    "alpha2beta1": dict(rule=2, epsilon=1e-6, alpha=2.0, beta=1.0),
    "zbox": dict(rule=3, epsilon=1e-6, low=-3.0, high=3.0),
}


# Gemma-3-270m's shape (random init): 18 layers, hidden 640, 4 query / 1 KV heads of 256, GeGLU FFN
# 2048, vocab 262144, tied; Gemma 3's (1 + w) and sandwich norms, QK-Norm, embeddings x sqrt(640),
# query_pre_attn_scalar 256, RoPE 1e6 on the full layers (every sixth) and 1e4 on the sliding ones
# (window 512).
GEMMA_270M = dict(vocab_size=262144, hidden_size=640, num_layers=18, num_heads=4, num_kv_heads=1, head_dim=256,
                  intermediate_size=2048, rms_norm_eps=1e-6, rope_theta=1e6, use_rope=1, rope_rotate_half=1, causal=1,
                  qkv_bias=0, out_bias=0, mlp_bias=0, tie_word_embeddings=1, reserved=0, hidden_act=1, qk_norm=1,
                  post_norms=1, norm_weight_offset=1.0, embed_scale=float(np.float32(np.sqrt(640.0))),
                  query_pre_attn_scalar=256.0, rope_local_base=10000.0, sliding_window=512,
                  sliding_layers=sum(1 << i for i in range(18) if i % 6 != 5))
DECODE_BATCH, DECODE_PROMPT, DECODE_NEW = 4, 64, 256

# GEMM work of one Linear's relevance relative to its forward GEMM, per rule: epsilon one transposed
# GEMM; Gamma and AlphaBeta the reference's eight (four denominators, four backward products: here a
# 2in x 2out stacked GEMM each way); ZBox two backward products (its denominator reuses x W).
LINEAR_RELEVANCE_GEMMS = {"lxt": 1, "eps": 1, "gamma": 8, "zplus": 8, "alpha2beta1": 8, "zbox": 2}


def gemm_flops_per_sequence(c, L, causal_effective, linear_factor=1):
    """Algorithmic GEMM FLOPs of one forward + AttnLRP pass (dense L^2 attention squares, as the
    reference computes them; causal_effective counts only the lower triangle); linear_factor scales
    each Linear's and the head's relevance GEMMs (LINEAR_RELEVANCE_GEMMS)."""
    d, H, Hkv, D, F, V, layers = (c["hidden_size"], c["num_heads"], c["num_kv_heads"], c["head_dim"],
                                  c["intermediate_size"], c["vocab_size"], c["num_layers"])
    qd, kvd = H * D, Hkv * D
    proj = 2 * L * d * (qd + 2 * kvd) + 2 * L * qd * d
    mlp = 2 * L * d * 2 * F + 2 * L * F * d
    att = 2 * (2 * H * L * L * D)  # Q K^T and P V
    if causal_effective:
        att = att * (L + 1) / (2 * L)
    head = 2 * L * d * V
    fwd = layers * (proj + mlp + att) + head
    # Linear-relevance GEMMs; both bilinear shares of each attention product
    rel = layers * (linear_factor * (proj + mlp) + 2 * att) + linear_factor * head
    return fwd + rel


def attention_executed_flops(c, L, n):
    """MFMA work the fused attention kernels of one explain step execute: every L x L x D product over
    the visible 16 x 16 tiles of the causal triangle (nrb (nrb + 1) / 2 tiles per head): the forward's
    two (Q K^T, P V), the q side's three (Q K^T again, s_pv V^T, s K) and the key side's two (s^T Q,
    P^T s_pv), per query head and sequence."""
    H, D, layers = c["num_heads"], c["head_dim"], c["num_layers"]
    nrb = (L + 15) // 16
    per_product = nrb * (nrb + 1) // 2 * 2.0 * 16 * 16 * D
    return layers * n * H * 7 * per_product


def time_cpu_baseline(cfg_fields, seq, rule_name="lxt", batch=1, timed=3):
    """Reference CPUBackend (oracle/_ref where built, else the oracle restatement) on the host cores:
    the model built once, one full-depth warm-up pass (threads, page faults), then `timed` complete
    forward + argmax seed + relevance passes at the full depth; the median is reported."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_ctypes as oc

    rule = oc.lrp_rule(**RULES[rule_name])
    lib, kind = oc.ref(), "reference"
    if lib is None:
        lib, kind = oc.oracle(), "port"
        lib.lib.pxo_set_split_threads(1)  # CPUBackend runs lrp_linear and the bilinear rule on one thread
    ids = np.random.RandomState(SEED).randint(0, cfg_fields["vocab_size"], size=(batch, seq))
    cfg = oc.model_config(**cfg_fields)
    lm = lib.lm(cfg, oc.synthetic_params(cfg, SEED))

    def one_pass():
        t0 = time.perf_counter()
        logits = lm.forward(ids)
        seed = np.zeros_like(logits)
        for b in range(batch):
            t = int(np.argmax(logits[b, -1]))
            seed[b, -1, t] = logits[b, -1, t]
        lm.relevance_rule(seed, rule)
        return time.perf_counter() - t0

    warm = one_pass()
    runs = [one_pass() for _ in range(timed)]
    med = float(np.median(runs))
    cores = oc.oracle().lib.pxo_get_threads()
    return {
        "value": round(batch * seq / med, 3),
        "unit": "tokens/s",
        "cores": int(cores),
        "kind": kind,
        "sample": "%d sequence(s) x %d tokens, the full %d-layer model: median of %d timed forward + argmax seed + "
                  "relevance passes (%s s) after one full-depth warm-up pass (%.1f s); GEMMs on %d std::threads "
                  "(cpu_backend.cpp:38-59), everything else single-threaded"
                  % (batch, seq, cfg_fields["num_layers"], timed, ", ".join("%.1f" % r for r in runs), warm, cores),
        "cpu_model": cpu_model(),
        "nproc": os.cpu_count(),
    }


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def summarize_launches(launches):
    """Groups the launch log of one step by kernel variant: calls, seconds, flops and bytes per
    step, sorted by time; plus totals per family ("gemm", "attention", "rows")."""
    kernels, families = {}, {}
    for r in launches:
        for table, key in ((kernels, r["kernel"]), (families, r["family"])):
            e = table.setdefault(key, {"kernel": key, "family": r["family"], "calls": 0, "seconds": 0.0, "flops": 0.0,
                                       "bytes": 0.0})
            e["calls"] += 1
            e["seconds"] += r["seconds"]
            e["flops"] += r["flops"]
            e["bytes"] += r["bytes"]
    ordered = sorted(kernels.values(), key=lambda e: -e["seconds"])
    return {"kernels": ordered, "families": families, "seconds": sum(r["seconds"] for r in launches)}


def kernel_row(k, traffic=STEP_KERNEL_TRAFFIC):
    row = {"kernel": k["kernel"], "calls_per_step": k["calls"], "avg_us": round(k["seconds"] / k["calls"] * 1e6, 2),
           "us_per_step": round(k["seconds"] * 1e6, 1)}
    if k["flops"] > 0:
        tf = k["flops"] / k["seconds"] / 1e12
        row.update(tflops=round(tf, 2), frac=round(tf / FP32_MFMA_PEAK_TFLOPS, 4))
    elif k["bytes"] > 0:
        gbs = k["bytes"] / k["seconds"] / 1e9
        row.update(gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4))
    if k["bytes"] > 0:
        row["algorithmic_mb"] = round(k["bytes"] / k["calls"] / 1e6, 2)
    if k["kernel"] in traffic:
        row["hbm_mb"] = round(traffic[k["kernel"]] / 1e6, 2)
    return row


def time_kernel(torch, stream, launch, reps):
    """Average duration of `launch()` over reps, HIP events recorded on `stream`."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    launch()
    e0.record(stream)
    for _ in range(reps):
        launch()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps * 1e-3  # seconds


def head_relevance_gemm(torch, N, c, L):
    """The LM head's relevance GEMM exactly as TiedLMHeadModule::run_relevance launches it:
    r_in (L x d) = x * ((R / stab(logits)) E), K = vocab, split-K."""
    V, d = c["vocab_size"], c["hidden_size"]
    g = torch.Generator(device="cuda").manual_seed(1)
    R = torch.zeros(L, V, device="cuda")
    R[-1, 7] = 3.0
    Z = torch.randn(L, V, device="cuda", generator=g)
    E = torch.randn(V, d, device="cuda", generator=g) * 0.02
    X = torch.randn(L, d, device="cuda", generator=g)
    out = torch.empty(L, d, device="cuda")
    desc = N.GemmDesc()
    desc.m, desc.n, desc.k, desc.batch, desc.inner, desc.kgroups = L, d, V, 1, 1, 1
    desc.prologue, desc.epilogue, desc.eps = N.PRO_DIV_STAB, N.EPI_MUL_X, LXT_EPS
    desc.a = N.operand(R.data_ptr(), V)
    desc.z = N.operand(Z.data_ptr(), V)
    desc.b = N.operand(E.data_ptr(), d)
    desc.c = N.operand(out.data_ptr(), d)
    desc.x = N.operand(X.data_ptr(), d)
    ws_bytes = N.gemm_workspace(desc)
    ws = torch.empty(max(ws_bytes // 4, 1), device="cuda")
    desc.workspace, desc.workspace_bytes = ws.data_ptr(), ws_bytes
    keep = (R, Z, E, X, out, ws)
    return desc, 2.0 * L * V * d, keep


def decode_head_gemm(torch, N, c, n):
    """The tied head of a decode step as TiedLMHeadModule::run_forward launches it: logits (n x V) =
    h (n x d) E^T with E stored (V, d), the skinny NT kernel."""
    V, d = c["vocab_size"], c["hidden_size"]
    g = torch.Generator(device="cuda").manual_seed(3)
    H = torch.randn(n, d, device="cuda", generator=g)
    E = torch.randn(V, d, device="cuda", generator=g) * 0.02
    out = torch.empty(n, V, device="cuda")
    desc = N.GemmDesc()
    desc.m, desc.n, desc.k, desc.batch, desc.inner, desc.kgroups = n, V, d, 1, 1, 1
    desc.trans_b = 1
    desc.a = N.operand(H.data_ptr(), d)
    desc.b = N.operand(E.data_ptr(), d)
    desc.c = N.operand(out.data_ptr(), V)
    return desc, 4.0 * (V * d + n * d + n * V), (H, E, out)


def kernel_probe(torch, N, models):
    """Counter-collection workload: 5 copies of 256 MiB (the counters' calibration) and 5 launches of
    the LM-head relevance GEMM, on the backend's stream."""
    st = models.stream()
    n = 64 * 1024 * 1024
    src, dst = torch.rand(n, device="cuda"), torch.empty(n, device="cuda")
    torch.cuda.synchronize()
    for _ in range(5):
        N.call("pxk_copy_2d", dst.data_ptr(), 1 << 20, src.data_ptr(), 1 << 20, 64, 1 << 20, st)
    desc, _, keep = head_relevance_gemm(torch, N, S_CONFIG, SEQ)
    for _ in range(5):
        N.gemm(desc, st)
    models.synchronize()
    print("kernel probe: copy 256 MiB x5, LM-head relevance GEMM x5 (plan tile %d, split-K %d)" % N.gemm_plan(desc))
    del keep


def decode_probe(torch, N, models):
    """Counter-collection workload for the decode line: 5 copies of 256 MiB (the calibration) and 5
    launches of the decode step's tied head (4 x 640 x 262144, skinny NT), on the backend's stream."""
    st = models.stream()
    n = 64 * 1024 * 1024
    src, dst = torch.rand(n, device="cuda"), torch.empty(n, device="cuda")
    torch.cuda.synchronize()
    for _ in range(5):
        N.call("pxk_copy_2d", dst.data_ptr(), 1 << 20, src.data_ptr(), 1 << 20, 64, 1 << 20, st)
    desc, _, keep = decode_head_gemm(torch, N, GEMMA_270M, DECODE_BATCH)
    for _ in range(5):
        N.gemm(desc, st)
    models.synchronize()
    print("decode probe: copy 256 MiB x5, decode-step tied head x5 (plan tile %d, split-K %d)" % N.gemm_plan(desc))
    del keep


# The raw DeviceBackend op sweep: GEMM shapes M x K x N (forward), seeded uniform(-1, 1) data.
SWEEP_GEMMS = [(512, 576, 1536), (512, 1536, 576), (4096, 2048, 8192), (512, 576, 49152)]
SWEEP_ELEMENTS = 1 << 26
SWEEP_RMS_ROWS, SWEEP_RMS_COLS = 32768, 2048


def sweep_gemm(torch, N, M, K, Nn, orient):
    """One sweep GEMM: "NN" C = A B (forward, M x K x N); "NT" the Linear relevance form
    r_in (M x K) = x * ((R / stab(z)) W^T) against the stored (K x N) W (lrp_rules.cpp:197-215,
    device_backend.hpp:627-628); "TN" C (K x N) = A^T S, the weight-side share of a bilinear
    product (lrp_math.hpp:57-86). All three do 2 M K N FLOPs."""
    g = torch.Generator(device="cuda").manual_seed(M + 3 * K + 7 * Nn)
    u = lambda *s: torch.rand(*s, device="cuda", generator=g) * 2 - 1
    desc = N.GemmDesc()
    desc.batch, desc.inner, desc.kgroups = 1, 1, 1
    if orient == "NN":
        A, B, C = u(M, K), u(K, Nn), torch.empty(M, Nn, device="cuda")
        desc.m, desc.n, desc.k = M, Nn, K
        desc.a, desc.b, desc.c = N.operand(A.data_ptr(), K), N.operand(B.data_ptr(), Nn), N.operand(C.data_ptr(), Nn)
        keep = (A, B, C)
    elif orient == "NT":
        R, Z, W, X, C = u(M, Nn), u(M, Nn), u(K, Nn), u(M, K), torch.empty(M, K, device="cuda")
        desc.m, desc.n, desc.k, desc.trans_b = M, K, Nn, 1
        desc.prologue, desc.epilogue, desc.eps = N.PRO_DIV_STAB, N.EPI_MUL_X, 1e-6
        desc.a, desc.z = N.operand(R.data_ptr(), Nn), N.operand(Z.data_ptr(), Nn)
        desc.b, desc.c, desc.x = N.operand(W.data_ptr(), Nn), N.operand(C.data_ptr(), K), N.operand(X.data_ptr(), K)
        keep = (R, Z, W, X, C)
    else:
        A, S, C = u(M, K), u(M, Nn), torch.empty(K, Nn, device="cuda")
        desc.m, desc.n, desc.k, desc.trans_a = K, Nn, M, 1
        desc.a, desc.b, desc.c = N.operand(A.data_ptr(), K), N.operand(S.data_ptr(), Nn), N.operand(C.data_ptr(), Nn)
        keep = (A, S, C)
    ws_bytes = N.gemm_workspace(desc)
    ws = torch.empty(max(ws_bytes // 4, 1), device="cuda")
    desc.workspace, desc.workspace_bytes = ws.data_ptr(), ws_bytes
    return desc, keep + (ws,)


def timed_reps(torch, stream, launch, target_s=0.02):
    """Average launch duration over enough repetitions for about target_s of GPU time."""
    once = time_kernel(torch, stream, launch, 1)
    return time_kernel(torch, stream, launch, int(min(500, max(5, target_s / max(once, 1e-6)))))


def op_sweep(torch, N, models):
    """The op sweep: GEMM TFLOP/s against the fp32 MFMA peak, elementwise and RMSNorm GB/s
    against HBM, each kernel timed with HIP events on the backend's stream."""
    raw_st = models.stream()
    stream = torch.cuda.ExternalStream(raw_st)
    rows = []
    tile_name = {N.TILE_128x128: "128x128", N.TILE_64x64: "64x64", N.TILE_32x64: "32x64", N.TILE_32x32: "32x32",
                 N.TILE_32x64_DIRECT: "32x64d", N.TILE_32x32_DIRECT: "32x32d", N.TILE_32x48_DIRECT: "32x48d",
                 N.TILE_32x48: "32x48"}
    for (M, K, Nn) in SWEEP_GEMMS:
        for orient in ("NN", "NT", "TN"):
            desc, keep = sweep_gemm(torch, N, M, K, Nn, orient)
            t = timed_reps(torch, stream, lambda: N.gemm(desc, raw_st))
            tile, splits = N.gemm_plan(desc)
            tf = 2.0 * M * K * Nn / t / 1e12
            rows.append({"op": "gemm %s" % orient, "shape": "%dx%dx%d" % (M, K, Nn), "plan": "%s/%d" % (tile_name[tile],
                         splits), "avg_us": round(t * 1e6, 2), "tflops": round(tf, 2),
                         "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)})
            del keep
    n = SWEEP_ELEMENTS
    g = torch.Generator(device="cuda").manual_seed(5)
    a, b, r = [torch.rand(n, device="cuda", generator=g) * 2 - 1 for _ in range(3)]
    o1, o2 = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    P = lambda x: x.data_ptr()
    ew = [
        ("add", 12, lambda: N.call("pxk_add", P(a), P(b), P(o1), n, raw_st)),
        ("mul", 12, lambda: N.call("pxk_mul", P(a), P(b), P(o1), n, raw_st)),
        ("relu", 8, lambda: N.call("pxk_elementwise", 0, P(a), P(o1), n, raw_st)),
        ("epsilon-divide", 12, lambda: N.call("pxk_lrp_stabilized_divide", P(a), P(b), None, P(o1), n, 1e-6, 0, raw_st)),
        ("epsilon-divide gated", 16,
         lambda: N.call("pxk_lrp_stabilized_divide", P(a), P(b), P(r), P(o1), n, 1e-6, 1, raw_st)),
        ("residual split", 20, lambda: N.call("pxk_lrp_residual_split", P(a), P(b), P(r), P(o1), P(o2), n, 1e-6, raw_st)),
        ("bilinear elementwise", 16,
         lambda: N.call("pxk_lrp_bilinear_elementwise", P(a), P(b), P(r), P(o1), n, 1e-6, raw_st)),
    ]
    for name, bpe, launch in ew:
        t = timed_reps(torch, stream, launch)
        gbs = bpe * n / t / 1e9
        rows.append({"op": name, "shape": "2^26", "bytes_per_element": bpe, "avg_us": round(t * 1e6, 2),
                     "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
    del a, b, r, o1, o2
    R, C = SWEEP_RMS_ROWS, SWEEP_RMS_COLS
    x = torch.rand(R, C, device="cuda", generator=g) * 2 - 1
    gamma, y, rms = torch.rand(C, device="cuda", generator=g), torch.empty(R, C, device="cuda"), torch.empty(R, device="cuda")
    t = timed_reps(torch, stream, lambda: N.call("pxk_rms_norm_forward", P(x), P(gamma), P(y), P(rms), R, C, 1e-5, raw_st))
    nbytes = 8 * R * C + 4 * R + 4 * C
    rows.append({"op": "rms_norm", "shape": "%dx%d" % (R, C), "bytes_per_element": 8, "avg_us": round(t * 1e6, 2),
                 "gbs": round(nbytes / t / 1e9, 1), "frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)})
    print(json.dumps({"sweep": "raw DeviceBackend op sweep, fp32, seeded uniform(-1,1) data", "peak_tflops":
                      FP32_MFMA_PEAK_TFLOPS, "peak_gbs": HBM_PEAK_GBS, "ops": rows}), flush=True)


def decode_bench(args, torch, N, models):
    """The Gemma-3-270m-shaped decode workload: batch 4, 64-token uniform-random prompts, 256 greedy
    tokens through the KV caches (one HIP graph replay per token), then every generated token
    explained by AttnLRP (LXT settings) over its prefix. A step is the whole job."""
    cfg = N.model_config(**GEMMA_270M)
    t_setup = time.perf_counter()
    lm = models.CausalLM(cfg, seed=SEED, std=0.02)
    n, p, T = DECODE_BATCH, DECODE_PROMPT, DECODE_NEW
    ld = p + T
    prompts = np.random.RandomState(SEED).randint(0, cfg.vocab_size, size=(n, p)).astype(np.float32)
    ids = torch.full((n, ld), -1.0, device="cuda")
    ids[:, :p] = torch.from_numpy(prompts).cuda()
    picked = torch.zeros(n, ld, device="cuda")
    W = p + T - 1
    rel = torch.empty(T, n, W, device="cuda")
    rule = N.lrp_rule(**RULES["lxt"])
    stream = torch.cuda.ExternalStream(models.stream())
    torch.cuda.synchronize()

    def job():
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record(stream)
        lm.generate_device(ids.data_ptr(), n, p, T, ld, picked.data_ptr())
        e[1].record(stream)
        lm.explain_generated_device(ids.data_ptr(), n, p, T, ld, rule, rel.data_ptr())
        e[2].record(stream)
        return e

    for _ in range(max(1, args.warmup)):
        job()
    models.synchronize()
    setup_s = time.perf_counter() - t_setup
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    events = [job() for _ in range(args.steps)]
    models.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dec_s = sum(e[0].elapsed_time(e[1]) for e in events) * 1e-3 / args.steps
    exp_s = sum(e[1].elapsed_time(e[2]) for e in events) * 1e-3 / args.steps
    out_ids = ids.cpu().numpy()
    r = rel.cpu().numpy()
    if not (np.all(np.isfinite(r)) and np.all(out_ids[:, p:] >= 0)):
        print("bench.py: decode produced non-finite relevance or missing ids", file=sys.stderr)
        sys.exit(1)
    tokens = n * T * args.steps
    out = {
        "metric": "KV-cached greedy decode + per-token AttnLRP tokens/s, Gemma-3-270m shape, batch 4, 64 -> 256",
        "value": round(tokens / wall, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: random-init N(0,0.02) weights from seed %d, uniform-random prompt ids" % SEED,
        "config": {"workload": "Gemma-3-270m-shaped causal LM (18 layers, hidden 640, 4/1 heads of 256, GeGLU FFN "
                               "2048, vocab 262144, sliding window 512 on 5 of every 6 layers): batch 4, 64-token "
                               "prompts, 256 greedy tokens through KV caches, each generated token explained by "
                               "AttnLRP (LxtAttnLrpConfig) over its prefix",
                   "global_batch": n, "prompt": p, "new_tokens": T, "parallelism": "single GPU"},
        "decode_ms": round(dec_s * 1e3, 3),
        "decode_tokens_per_s": round(n * T / dec_s, 1),
        "decode_ms_per_step": round(dec_s * 1e3 / T, 4),
        "explain_ms": round(exp_s * 1e3, 3),
        "explained_tokens_per_s": round(n * T / exp_s, 1),
        "setup_s": round(setup_s, 1),
    }
    # ---- roofline: the decode step's largest launch, the tied head over the vocabulary ------------
    desc, nbytes, keep = decode_head_gemm(torch, N, GEMMA_270M, n)
    ker_s = time_kernel(torch, stream, lambda: N.gemm(desc, models.stream()), 20)
    assert N.gemm_plan(desc) == (N.TILE_SKINNY, 1)
    achieved = nbytes / ker_s / 1e9
    out["roofline"] = {
        "kernel": "pxk_gemm NT skinny (decode-step tied head %d x %d x %d: skinny_nt_kernel)" %
                  (n, GEMMA_270M["hidden_size"], GEMMA_270M["vocab_size"]),
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": DECODE_HEAD_TRAFFIC["bytes"] if N.gemm_plan(desc) == DECODE_HEAD_TRAFFIC["plan"] else None,
        "traffic_unit": "bytes per launch",
        "avg_launch_us": round(ker_s * 1e6, 2),
        "algorithmic_bytes_per_launch": int(nbytes),
    }
    del keep
    if not args.no_cpu_baseline:
        # One explanation at the generation's mean prefix length (the bulk of the job), 1 sequence.
        mean_prefix = p + T // 2
        cb = time_cpu_baseline(GEMMA_270M, mean_prefix, "lxt")
        cb["sample"] = "one generated token explained at the mean prefix length (%d): %s" % (mean_prefix, cb["sample"])
        cb["unit"] = "explained tokens/s (1 sequence; decode itself excluded)"
        cb["value"] = round(cb["value"] / mean_prefix, 5)
        out["cpu_baseline"] = cb
    print(json.dumps(out), flush=True)


def pmc_table(names_path, dbs):
    """Per-launch counters of the step from rocprofv3 --pmc databases of `bench.py --steps 1
    --warmup 1 --mode eager --profile-reps 1 --launch-names NAMES` (one counter group per run). That
    run ends with one timed replay of the recorded step, so the last dispatches of each database are
    that replay's, launch by launch as NAMES lists them (a launch dispatching two kernels, a split-K
    GEMM and its reduce, adds both). Per launch name and counter: the median over its launches of the
    counter summed over their dispatches. Derived columns where their counters are present: HBM MB =
    (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0) KiB (the factors a 256 MiB copy reads: bench.py
    --kernel-probe); MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs / (duration x 2.4 GHz); waves
    per CU = SQ_WAVE_CYCLES x 4 / (duration x 2.4 GHz) / 256, with the launch's duration as that run
    measured it (counter collection slows kernels by 10-15%)."""
    import sqlite3
    names = []
    with open(names_path) as f:
        for line in f:
            name, disp = line.rstrip("\n").rsplit("\t", 1)
            names.append((name, int(disp)))
    need = sum(d for _, d in names)
    per = {}  # counter -> {launch name: [value per launch]}; "duration ns" per database

    def assign(counter, vals):
        if len(vals) < need:
            raise SystemExit("%d dispatches with %s, the step's replay needs %d" % (len(vals), counter, need))
        tail, at = vals[len(vals) - need:], 0
        table = per.setdefault(counter, {})
        for name, d in names:
            table.setdefault(name, []).append(sum(tail[at:at + d]))
            at += d

    for db in dbs:
        c = sqlite3.connect(db)
        rows = c.execute("select dispatch_id, counter_name, sum(counter_value), max(duration) from pmc_events "
                         "group by dispatch_id, counter_name order by dispatch_id").fetchall()
        counters = sorted({r[1] for r in rows})
        for counter in counters:
            assign(counter, [v for _, cn, v, _ in rows if cn == counter])
        if "SQ_WAVE_CYCLES" in counters or "SQ_VALU_MFMA_BUSY_CYCLES" in counters:
            assign("duration ns", [dur for _, cn, _, dur in rows if cn == counters[0]])
    med = lambda name, counter: float(np.median(per[counter][name])) if name in per.get(counter, {}) else None
    order = []
    for n, _ in names:
        if n not in order:
            order.append(n)
    counters = [k for k in sorted(per) if k != "duration ns"]
    derived = []
    if "FETCH_SIZE" in per and "WRITE_SIZE" in per:
        derived.append(("HBM MB (F x 2 + W)", lambda n: (2.0 * med(n, "FETCH_SIZE") + med(n, "WRITE_SIZE")) * 1024 / 1e6))
    if "duration ns" in per:
        ghz = lambda n: med(n, "duration ns") * 2.4
        if "SQ_VALU_MFMA_BUSY_CYCLES" in per:
            derived.append(("MFMA busy %", lambda n: 100.0 * med(n, "SQ_VALU_MFMA_BUSY_CYCLES") / 1024 / ghz(n)))
        if "SQ_WAVE_CYCLES" in per:
            derived.append(("waves / CU", lambda n: med(n, "SQ_WAVE_CYCLES") * 4 / ghz(n) / 256))
        counters = ["duration ns"] + counters
    print("| launch | per step | " + " | ".join(counters + [d for d, _ in derived]) + " |")
    print("|---|---:|" + "---:|" * (len(counters) + len(derived)))
    for n in order:
        vals = ["%.0f" % med(n, k) if med(n, k) is not None else "-" for k in counters]
        vals += ["%.2f" % fn(n) for _, fn in derived]
        print("| %s | %d | %s |" % (n, sum(1 for x, _ in names if x == n), " | ".join(vals)))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--mode", choices=("graph", "eager"), default="graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--layers", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--l1b", action="store_true",
                    help="the Llama-3.2-1B-shaped explain step (16 layers, hidden 2048, 32/8 heads, FFN 8192, vocab "
                         "128256, theta 500000) over batch 8 x 1024 instead of the headline S workload")
    ap.add_argument("--block", action="store_true",
                    help="config B: one TransformerBlock forward + epsilon-LRP relevance at seq 128, GPU and "
                         "reference CPUBackend (2 warm-ups, median of 10)")
    ap.add_argument("--profile-reps", type=int, default=5,
                    help="replays of the step's recorded launches for the per-kernel times (default 5)")
    ap.add_argument("--kernel-probe", action="store_true",
                    help="only launch a 256 MiB copy and the LM-head relevance GEMM, 5 times each (for rocprofv3 --pmc)")
    ap.add_argument("--decode-probe", action="store_true",
                    help="only launch a 256 MiB copy and the decode step's tied head, 5 times each (for rocprofv3 --pmc)")
    ap.add_argument("--op-sweep", action="store_true",
                    help="time the raw op sweep (GEMM shapes, elementwise over 2^26, RMSNorm 32768 x 2048) instead")
    ap.add_argument("--decode", action="store_true",
                    help="the Gemma-3-270m decode workload (batch 4, 64 -> 256 tokens, AttnLRP per generated token)")
    ap.add_argument("--rule", choices=sorted(RULES), default="lxt",
                    help="the LRP rule of the relevance pass (default: LXT's AttnLRP epsilon rule, the headline)")
    ap.add_argument("--launch-names", metavar="FILE",
                    help="write the step's launches (name and kernels dispatched, in order) to FILE")
    ap.add_argument("--pmc-table", nargs="+", metavar=("NAMES", "DB"),
                    help="offline: the per-launch HBM traffic of the step from rocprofv3 --pmc FETCH_SIZE / "
                         "WRITE_SIZE databases of a --profile-reps 1 run and its --launch-names file")
    args = ap.parse_args()
    if args.pmc_table:
        pmc_table(args.pmc_table[0], args.pmc_table[1:])
        return
    if args.gpus != 1:
        print("bench.py: this build measures one MI355X (the path runs on one GPU; --gpus %d is not supported)"
              % args.gpus, file=sys.stderr)
        sys.exit(2)

    import torch

    from pulsatrix_amd import models
    from pulsatrix_amd import native as N

    if args.kernel_probe:
        kernel_probe(torch, N, models)
        return
    if args.decode_probe:
        decode_probe(torch, N, models)
        return
    if args.op_sweep:
        op_sweep(torch, N, models)
        return
    if args.decode:
        decode_bench(args, torch, N, models)
        return

    if args.block:
        block_bench(args, N, models)
        return
    if args.l1b:
        explain_bench(args, torch, N, models, dict(L1B_CONFIG, num_layers=args.layers or L1B_CONFIG["num_layers"]),
                      L1B_BATCH, L1B_SEQ, "l1b")
        return
    explain_bench(args, torch, N, models, dict(S_CONFIG, num_layers=args.layers or S_CONFIG["num_layers"]), BATCH,
                  SEQ, "s512")


RULE_TEXT = {"lxt": "LxtAttnLrpConfig: eps 1e-9, bias in denominator",
             "eps": "LRPRuleConfig{1e-6}: the default pre-bias epsilon rule",
             "gamma": "Gamma(0.25) on every Linear and the head, eps 1e-6 elsewhere",
             "zplus": "ZPlus (AlphaBeta 1, 0) on every Linear and the head, eps 1e-6 elsewhere",
             "alpha2beta1": "AlphaBeta(2, 1) on every Linear and the head, eps 1e-6 elsewhere",
             "zbox": "ZBox(-3, 3) on every Linear and the head, eps 1e-6 elsewhere"}


def explain_bench(args, torch, N, models, fields, batch, seq, which):
    """The explain step (forward logits, on-device argmax seed at each sequence's last position, the
    relevance pass, per-token sums, the token relevance to pinned host memory) timed over K steps;
    the per-kernel table from the step's own launches; the CPU baseline on a bounded sample."""
    cfg = N.model_config(**fields)
    t_setup = time.perf_counter()
    lm = models.CausalLM(cfg, seed=SEED, std=0.02)
    ids_host = np.random.RandomState(SEED).randint(0, cfg.vocab_size, size=(batch, seq)).astype(np.float32)
    ids = torch.from_numpy(ids_host).cuda()
    tok = torch.empty(batch * seq, device="cuda")
    tgt = torch.empty(batch, dtype=torch.int64, device="cuda")
    tok_host = torch.empty(batch * seq, pin_memory=True)  # each step's relevance D2H lands here
    torch.cuda.synchronize()
    stream = torch.cuda.ExternalStream(models.stream())

    rule = N.lrp_rule(**RULES[args.rule])

    def eager_step():
        lm.explain_device_rule(ids.data_ptr(), batch, seq, rule, tok.data_ptr(), tgt.data_ptr())

    run = eager_step
    if args.mode == "graph":
        run = lm.replay

    def step():
        run()
        with torch.cuda.stream(stream):  # the token relevance to the host, queued behind the pass
            tok_host.copy_(tok, non_blocking=True)

    for _ in range(max(1, args.warmup)):
        eager_step()
    models.synchronize()
    if args.mode == "graph":
        lm.capture_explain_rule(ids.data_ptr(), batch, seq, rule, tok.data_ptr(), tgt.data_ptr())
        for _ in range(max(1, args.warmup)):
            step()
        models.synchronize()
        torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup

    # ---- timed region: K steps, synchronized on both sides -------------------------------------
    torch.cuda.synchronize()
    models.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    models.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = e0.elapsed_time(e1) * 1e-3
    relevance = tok_host.numpy().copy()
    if not (np.all(np.isfinite(relevance)) and np.array_equal(relevance, tok.cpu().numpy())):
        print("bench.py: non-finite relevance", file=sys.stderr)
        sys.exit(1)

    tokens = batch * seq * args.steps
    value = tokens / wall
    lf = LINEAR_RELEVANCE_GEMMS[args.rule]
    flops_dense = gemm_flops_per_sequence(fields, seq, False, lf) * batch
    flops_causal = gemm_flops_per_sequence(fields, seq, True, lf) * batch

    # ---- per-kernel times of the step's own launches, HIP events on the backend's stream ------
    # One eager step with the launch log open records every launch (kernel variant, arguments,
    # algorithmic work); the recorded launches are then replayed in their order, every dispatch
    # recording its own start and end events, so each kernel runs on the step's own buffers,
    # shapes and cache state and is timed without the gaps between launches.
    launches = models.launch_profile(eager_step, reps=args.profile_reps)
    if args.launch_names:
        with open(args.launch_names, "w") as f:
            for r in launches:
                f.write("%s\t%d\n" % (r["kernel"], r["dispatches"]))
    prof = summarize_launches(launches)
    gemm, attn = prof["families"].get("gemm"), prof["families"].get("attention")
    dom = prof["kernels"][0]  # the most time per step
    dom_bound = "hbm" if dom["family"] == "rows" else "mfma"
    if dom_bound == "mfma":
        achieved, peak, unit = dom["flops"] / dom["seconds"] / 1e12, FP32_MFMA_PEAK_TFLOPS, "TFLOP/s"
    else:
        achieved, peak, unit = dom["bytes"] / dom["seconds"] / 1e9, HBM_PEAK_GBS, "GB/s"
    traffic_table = STEP_KERNEL_TRAFFIC if which == "s512" else {}  # measured for the S step's plans only
    traffic = traffic_table.get(dom["kernel"])
    # Work the step executes: its GEMM launches' 2 M N K plus the attention kernels' MFMA products
    # over the causal tiles (no dense head relevance: the seeded rows alone run).
    attn_exec = attention_executed_flops(fields, seq, batch) if attn is not None else 0.0
    flops_exec = (gemm["flops"] if gemm else 0.0) + attn_exec

    shape = {"s512": "SmolLM2-135M-shaped causal LM", "l1b": "Llama-3.2-1B-shaped causal LM"}[which]
    out = {
        "metric": {"s512": "forward+AttnLRP tokens/s, 135M-shape LM seq 512; GEMM % fp32 MFMA peak",
                   "l1b": "forward+AttnLRP tokens/s, Llama-3.2-1B-shape LM 8 x 1024; GEMM % fp32 MFMA peak"}[which],
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: random-init N(0,0.02) weights from seed %d, uniform-random token ids" % SEED,
        "config": {
            "workload": "%s forward + AttnLRP (%s), argmax seed at the last position of each sequence, batch %d x "
                        "seq %d" % (shape, RULE_TEXT[args.rule], batch, seq),
            "layers": fields["num_layers"], "hidden": fields["hidden_size"],
            "heads": "%d/%d" % (fields["num_heads"], fields["num_kv_heads"]), "head_dim": fields["head_dim"],
            "ffn": fields["intermediate_size"], "vocab": fields["vocab_size"], "tied": True,
            "rope_theta": fields["rope_theta"], "global_batch": batch, "seq_len": seq,
            "parallelism": "single GPU", "mode": args.mode,
        },
        "timing": "value = tokens of K steps / wall time of the K back-to-back steps between synchronisations "
                  "(a mean, not a per-step median); each step is the whole path plus an asynchronous copy of "
                  "the token relevance to pinned host memory",
        "gpu_time_ms_per_step": round(gpu_s / args.steps * 1e3, 4),
        "path_gemm_gflop_per_step": {"dense": round(flops_dense / 1e9, 2), "causal": round(flops_causal / 1e9, 2),
                                     "executed": round(flops_exec / 1e9, 2)},
        "path_tflops_dense": round(flops_dense * args.steps / wall / 1e12, 2),
        "path_tflops_executed": round(flops_exec * args.steps / wall / 1e12, 2),
        "path_flops_note": "dense: the reference's count (every L^2 attention square, the dense head relevance); "
                           "executed: the step's GEMM launches (the head relevance runs on the seeded rows alone) "
                           "plus the attention kernels' MFMA products over the causal tiles",
        "gemm_pct_peak": round(100.0 * gemm["flops"] / gemm["seconds"] / 1e12 / FP32_MFMA_PEAK_TFLOPS, 2),
        "gemm": {"launches_per_step": gemm["calls"], "gflop_per_step": round(gemm["flops"] / 1e9, 2),
                 "ms_per_step": round(gemm["seconds"] * 1e3, 4),
                 "tflops": round(gemm["flops"] / gemm["seconds"] / 1e12, 2),
                 "how": "sum of 2MNK over the step's own GEMM launches / sum of their kernels' durations, each "
                        "dispatch recording its own start and end (hipExtLaunchKernelGGL events) while the step's "
                        "recorded launches are replayed in step order on the step's buffers"},
        "attention": None if attn is None else {
            "launches_per_step": attn["calls"], "gflop_per_step_dense": round(attn["flops"] / 1e9, 2),
            "gflop_per_step_executed": round(attn_exec / 1e9, 2),
            "ms_per_step": round(attn["seconds"] * 1e3, 4), "tflops_dense": round(attn["flops"] / attn["seconds"] / 1e12, 2),
            "tflops_executed": round(attn_exec / attn["seconds"] / 1e12, 2),
            "pct_peak_dense": round(100.0 * attn["flops"] / attn["seconds"] / 1e12 / FP32_MFMA_PEAK_TFLOPS, 2)},
        "launches_per_step": len(launches),
        "kernel_ms_per_step": round(prof["seconds"] * 1e3, 4),
        "roofline": {
            "kernel": dom["kernel"],
            "why": "the kernel variant with the most time per step (%d launches per step)" % dom["calls"],
            "bound": dom_bound,
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": unit,
            "frac": round(achieved / peak, 4),
            "traffic": None if traffic is None else int(traffic),
            "traffic_unit": "HBM bytes per launch (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, copy-calibrated)",
            "avg_launch_us": round(dom["seconds"] / dom["calls"] * 1e6, 2),
            "algorithmic_gflop_per_launch": round(dom["flops"] / dom["calls"] / 1e9, 4),
            "algorithmic_bytes_per_launch": int(dom["bytes"] / dom["calls"]),
        },
        "step_kernels": [kernel_row(k, traffic_table) for k in prof["kernels"][:16]],
        "setup_s": round(setup_s, 1),
    }
    if not args.no_cpu_baseline:
        if which == "s512":
            out["cpu_baseline"] = time_cpu_baseline(fields, seq, args.rule)
        else:
            # A bounded sample: one sequence of L1B_CPU_SEQ tokens at the full depth (the whole
            # 8 x 1024 batch would take the host cores hours).
            cb = time_cpu_baseline(fields, L1B_CPU_SEQ, args.rule, timed=1)
            cb["sample"] = "bounded sample, not the GPU's batch: " + cb["sample"]
            out["cpu_baseline"] = cb
        out["gpu_vs_cpu"] = round(value / out["cpu_baseline"]["value"], 1)
    del lm
    print(json.dumps(out), flush=True)


def block_bench(args, N, models):
    """Config B: one TransformerBlock (hidden 576, 9 / 3 heads of 64, SwiGLU FFN 1536, RMSNorm eps
    1e-5, RoPE theta 10000), weights N(0, 0.02) from a seed with RMSNorm gamma 1, x ~ N(0, 1) of shape
    (1, 128, 576); forward, then epsilon-LRP (LRPRuleConfig{1e-6}) relevance from R_out = y at
    channel 0 (LRPSeed::OutputValue) back to the block input. Host arrays in and out on both sides
    (the block's public forward() / propagate_relevance()). 2 warm-ups, then the median of 10 timed
    runs, on the MI355X path and on the reference CPUBackend."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_ctypes as oc

    cfg = oc.model_config(**B_CONFIG)
    params = oc.synthetic_params(cfg, SEED, block=True)
    x = oc.fill_normal(B_SEQ * B_CONFIG["hidden_size"], SEED + 1, 1.0).reshape(1, B_SEQ, B_CONFIG["hidden_size"])
    gpu = models.Block(N.ModelConfig(**{f: getattr(cfg, f) for f, _ in cfg._fields_}), params)
    lib, kind = oc.ref(), "reference"
    if lib is None:
        lib, kind = oc.oracle(), "port"
    cpu = lib.block(cfg, params)

    def run(block):
        t0 = time.perf_counter()
        y = block.forward(x)
        seed = np.zeros_like(y)
        seed[..., 0] = y[..., 0]
        r = block.relevance(seed, 1e-6, False)
        return time.perf_counter() - t0, y, r

    def timed(block):
        for _ in range(2):
            run(block)
        runs = [run(block) for _ in range(10)]
        return float(np.median([t for t, _, _ in runs])), runs[-1][1], runs[-1][2]

    g_s, g_y, g_r = timed(gpu)
    c_s, c_y, c_r = timed(cpu)
    y_err = float(np.abs(g_y - c_y).max() / max(1.0, np.abs(c_y).max()))
    r_err = float(np.abs(g_r - c_r).max() / np.abs(c_r).max())
    if not (y_err <= 1e-4 and r_err <= 1e-3):
        print("bench.py: config B results differ from the CPU reference (%.2e, %.2e)" % (y_err, r_err), file=sys.stderr)
        sys.exit(1)
    out = {
        "metric": "TransformerBlock forward + epsilon-LRP relevance, config B (seq 128): ms per call, host to host",
        "value": round(g_s * 1e3, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": 10,
        "warmup": 2,
        "higher_is_better": False,
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: N(0,0.02) weights from seed %d (RMSNorm gamma 1), x ~ N(0,1)" % SEED,
        "config": {"workload": "one Llama-style TransformerBlock, hidden 576, 9/3 heads of 64, SwiGLU 1536, "
                               "theta 10000, batch 1 x seq 128; forward, then LRPRuleConfig{1e-6} relevance from "
                               "R_out = y at channel 0 (OutputValue seed)", "parallelism": "single GPU"},
        "timing": "median of 10 calls of forward() + propagate_relevance() after 2 warm-ups; each call copies x "
                  "and R_out from the host and the outputs back, as the block's public API does",
        "tokens_per_s": round(B_SEQ / g_s, 1),
        "parity": {"forward_max_rel": y_err, "relevance_max_rel_to_max": r_err},
        "cpu_baseline": {"value": round(c_s * 1e3, 3), "unit": "ms", "kind": kind,
                         "cores": int(oc.oracle().lib.pxo_get_threads()),
                         "sample": "the same block and inputs: median of 10 calls after 2 warm-ups",
                         "cpu_model": cpu_model(), "nproc": os.cpu_count()},
        "gpu_vs_cpu": round(c_s / g_s, 1),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
