"""bench.py's work accounting on the CPU: the dense and causal GEMM FLOP counts of the S workload
(329.8 and 302.6 GFLOP per 512-token sequence, the path's algorithmic work), the attention kernels'
executed MFMA products over the causal tiles, and the refusal of more than one GPU."""
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_s_workload_flop_counts():
    assert abs(bench.gemm_flops_per_sequence(bench.S_CONFIG, 512, False) / 1e9 - 329.77) < 0.01
    assert abs(bench.gemm_flops_per_sequence(bench.S_CONFIG, 512, True) / 1e9 - 302.6) < 0.1


def test_attention_executed_flops_counts_causal_tiles():
    # 32 row blocks: 528 visible 16 x 16 tiles per head, 7 products of 2 * 16 * 16 * 64 FLOPs each,
    # 9 heads, 30 layers, one sequence.
    assert bench.attention_executed_flops(bench.S_CONFIG, 512, 1) == 30 * 9 * 7 * 528 * 2 * 16 * 16 * 64
    # a ragged length rounds up to whole tiles: 17 tokens are 2 row blocks, 3 tiles
    c = dict(bench.S_CONFIG, num_layers=1, num_heads=1)
    assert bench.attention_executed_flops(c, 17, 2) == 2 * 7 * 3 * 2 * 16 * 16 * 64


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one MI355X" in r.stderr
