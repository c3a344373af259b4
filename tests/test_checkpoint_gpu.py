"""Checkpoint loading to the device: pxk_convert_weight (widening and the (out, in) -> (in, out)
transpose, src/safetensors.cpp:676-740 and src/causal_lm.cpp:257-291) and LoadCausalLM through
pxa_lm_load, on the committed BF16 hf_tiny checkpoints (llama is sharded, qwen2 is one file with
biases and an untied head).

The widening is pinned independently of the kernel's own formula: F16 against numpy's float16,
BF16 against the float32 whose top half it is, F64 against numpy's round-to-nearest cast, and the
two FP8 formats (OCP 8-bit floating point: E4M3 "fn" with bias 7, no infinities and only
S.1111.111 as NaN; E5M2 with bias 15 and IEEE specials) against values the format fixes: the
largest finite, the smallest subnormal and normal, one, negative zero, infinities and NaNs."""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

import gpu_util as G
from hf_fixtures import GOLDEN, hf_tiny, sequences
from pulsatrix_amd import models
from pulsatrix_amd import native as N
from test_model_gpu import to_px

gpu = pytest.mark.gpu
F32, F16, BF16, F64, E4M3, E5M2 = 0, 1, 2, 3, 4, 5


def convert(raw, dtype, rows, cols, transpose):
    src = G.dev(np.frombuffer(raw + b"\0" * (-len(raw) % 4), np.float32))
    out = G.empty((rows * cols,))
    N.call("pxk_convert_weight", G.ptr(src), dtype, rows, cols, int(transpose), G.ptr(out), G.stream())
    return G.host(out)


def same(got, want):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))  # bit-exact, signed zeros too


@gpu
def test_widen_f16_bf16_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint16)
    same(convert(bits.tobytes(), F16, 256, 256, False), bits.view(np.float16).astype(np.float32))
    same(convert(bits.tobytes(), BF16, 256, 256, False), (bits.astype(np.uint32) << 16).view(np.float32))


@gpu
def test_widen_f64_rounds_to_nearest():
    rs = np.random.RandomState(1)
    x = np.concatenate([rs.standard_normal(1000) * 10.0 ** rs.randint(-40, 40, 1000),
                        [1e300, -1e300, 1e-300, 0.0, -0.0, np.inf, -np.inf, np.nan, 1.0 + 2.0 ** -30]])
    same(convert(x.astype(np.float64).tobytes(), F64, 1, x.size, False), x.astype(np.float32))


@gpu
def test_widen_fp8_formats():
    e4m3 = convert(np.arange(256, dtype=np.uint8).tobytes(), E4M3, 16, 16, False)
    assert e4m3[0x7E] == 448.0 and e4m3[0xFE] == -448.0  # largest finite
    assert e4m3[0x01] == 2.0 ** -9 and e4m3[0x08] == 2.0 ** -6 and e4m3[0x07] == 7 * 2.0 ** -9
    assert e4m3[0x38] == 1.0 and e4m3[0x78] == 256.0 and np.signbit(e4m3[0x80]) and e4m3[0x80] == 0.0
    assert np.isnan(e4m3[0x7F]) and np.isnan(e4m3[0xFF]) and np.isnan(e4m3).sum() == 2  # no infinities
    e5m2 = convert(np.arange(256, dtype=np.uint8).tobytes(), E5M2, 16, 16, False)
    assert e5m2[0x7B] == 57344.0 and e5m2[0x01] == 2.0 ** -16 and e5m2[0x04] == 2.0 ** -14
    assert e5m2[0x3C] == 1.0 and e5m2[0x7C] == np.inf and e5m2[0xFC] == -np.inf
    assert np.isnan(e5m2[0x7D]) and np.isnan(e5m2[0x7F]) and np.isnan(e5m2).sum() == 6
    # every finite value is sign * significand * 2^k for the format, and the order is monotone
    fin = e4m3[:0x7F]
    assert np.all(np.diff(fin) > 0)
    fin = e5m2[:0x7C]
    assert np.all(np.diff(fin) > 0)


@gpu
@pytest.mark.parametrize("rows,cols", [(37, 70), (64, 32), (1, 5), (130, 129)])
def test_convert_transposes(rows, cols):
    x = G.uniform((rows, cols), rows + cols)
    bf = (x.view(np.uint32) >> 16).astype(np.uint16)
    want = (bf.astype(np.uint32) << 16).view(np.float32)
    same(convert(bf.tobytes(), BF16, rows, cols, True).reshape(cols, rows), want.T)
    same(convert(x.tobytes(), F32, rows, cols, True).reshape(cols, rows), x.T)


@gpu
@pytest.mark.parametrize("name", ["llama", "qwen2"])
def test_load_causal_lm_matches_host_loaded_model(name):
    """pxa_lm_load on the BF16 checkpoint gives the same model as the host-side loader: identical
    logits and relevance, and the transformers logits at 1e-4."""
    cfg, params, golden, _ = hf_tiny(name)
    loaded = models.CausalLM.load(os.path.join(GOLDEN, "hf_tiny", name))
    host = models.CausalLM(to_px(cfg), params)
    for k in sequences(golden):
        ids = golden["ids.%d" % k].reshape(1, -1)
        a, b = loaded.forward(ids), host.forward(ids)
        assert np.array_equal(a, b), k
        exp = golden["logits.%d" % k]
        assert np.all(np.abs(a[0] - exp) <= 1e-4 * np.maximum(1.0, np.abs(exp)))
        seed = np.zeros_like(a)
        seed[0, -1, int(np.argmax(a[0, -1]))] = a[0, -1].max()
        host.forward(ids)
        assert np.array_equal(loaded.relevance(seed, 1e-9, True)[1], host.relevance(seed, 1e-9, True)[1])


def write_safetensors(path, tensors):
    header, blobs, off = {}, [], 0
    for name, (dtype, arr) in tensors.items():
        b = arr.tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))


@gpu
def test_load_rejects_bad_checkpoints(tmp_path):
    """Config and checkpoint validation happens before any device write."""
    src = os.path.join(GOLDEN, "hf_tiny", "qwen2")
    cfg = json.load(open(os.path.join(src, "config.json")))

    def load(d):
        h = N.host().pxa_lm_load(str(d).encode(), None)
        assert not h
        return N.host().pxa_last_error().decode()

    assert "cannot open" in load(tmp_path) and "config.json" in load(tmp_path)
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    assert "no model.safetensors" in load(tmp_path)
    bad = dict(cfg, rope_scaling={"rope_type": "yarn", "factor": 8.0})  # linear and llama3 are supported
    (tmp_path / "config.json").write_text(json.dumps(bad))
    write_safetensors(tmp_path / "model.safetensors", {"x": ("F32", np.zeros(2, np.float32))})
    assert "rope_scaling \"yarn\"" in load(tmp_path)
    (tmp_path / "config.json").write_text(json.dumps(dict(cfg, hidden_act="relu")))
    assert "hidden_act \"relu\"" in load(tmp_path)
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    assert "has no tensor \"model.embed_tokens.weight\"" in load(tmp_path)
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", 1 << 40))
    assert "header length" in load(tmp_path)
