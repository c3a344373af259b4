"""Every address the attention forward's K / V tile loads (and the recomputing q side's, which read
V with K's lane layout, and the GQA-shared kernels' 16-byte row pieces, a subset of K's layout)
can touch, checked on the host.

attn_fwd_kernel reads each 16-key tile of a KV head through a buffer resource whose range is
pxk_attention_kv_tile_records(l, key0, ld, head_dim) bytes from the tile's first row of the head's
column segment; a load whose bytes fall past the range reads 0 without touching memory. Each lane's
byte offsets are fixed by the kernel's layout (restated below from attention.hip): K as 16-byte
rows (c * ld + 4 g + 16 t), V as 4-byte columns ((4 g + st) * ld + c + 16 t), for lanes c < 16,
g < 4, st < 4 and the DT = ceil16(head_dim) column tiles. For every tile, head and sequence of the
operand layouts the module uses (K from the rotated q|k rows or the packed q|k|v rows, V from the
packed rows, or tight K / V matrices), every dword inside the range must lie inside the operand's
allocation. head_dim 8, 24 and 40 leave columns past head_dim in the last 16-wide tile; the range
must cut those off on the sequence's last row. The range this kernel used before (ending qd floats
past the packed buffer for the last sequence) is checked too, as a negative control: it admits reads
past the allocation at head_dim 8, which is the out-of-bounds read behind a GPU memory fault in a
tiny-model test."""
import ctypes

import numpy as np

from pulsatrix_amd import native as N


def dt_of(d):
    return 1 if d <= 16 else 2 if d <= 32 else 4 if d <= 64 else 8


def lane_dwords(ld, dt):
    """Element offsets (relative to the resource base) of every dword the K and V tile loads read."""
    c = np.arange(16)[:, None, None, None]
    g = np.arange(4)[None, :, None, None]
    t = np.arange(dt)[None, None, :, None]
    e = np.arange(4)[None, None, None, :]  # the 4 dwords of a 16-byte K load / the 4 V rows st
    k = (c * ld + 4 * g + 16 * t + e).ravel()
    v = ((4 * g + e) * ld + c + 16 * t).ravel()
    return k, v


def layouts(n, l, heads, kv_heads, d):
    qd, kvd = heads * d, kv_heads * d
    w3 = qd + 2 * kvd
    rows = n * l
    # (name, K column offset, K row stride, K buffer floats, V column offset, V row stride, V buffer floats)
    yield "rope", qd, qd + kvd, rows * (qd + kvd), qd + kvd, w3, rows * w3
    yield "packed", qd, w3, rows * w3, qd + kvd, w3, rows * w3
    yield "tight", 0, kvd, rows * kvd, 0, kvd, rows * kvd


def max_reach(records_fn, n, l, kv_heads, d, col, ld, size, patterns=(0, 1)):
    """The largest element index inside the range, over every sequence, KV head and tile, relative to
    the operand allocation (must be < size), and the smallest (must be >= 0). patterns: the lane
    layouts read (0: 16-byte rows, 1: 4-byte columns)."""
    dt = dt_of(d)
    k_off, v_off = lane_dwords(ld, dt)
    hi, lo = -1, 1 << 62
    for key0 in range(0, l, 16):
        for hk in range(kv_heads):
            records = records_fn(l, key0, ld, d, hk)
            for offs in [(k_off, v_off)[i] for i in patterns]:
                inside = offs[offs * 4 < records]
                if inside.size == 0:
                    continue
                for b in range(n):
                    base = col + b * l * ld + hk * d + key0 * ld
                    hi, lo = max(hi, base + int(inside.max())), min(lo, base + int(inside.min()))
    return hi, lo


def library_records():
    fn = N.pxk().pxk_attention_kv_tile_records
    fn.argtypes = [ctypes.c_int64] * 4
    fn.restype = ctypes.c_int64
    return lambda l, key0, ld, d, hk=0: fn(l, key0, ld, d)


def previous_records(l, key0, ld, d, hk):
    """The range the kernel used before, for KV head hk: ((l - key0) * ld - hk * d) * 4."""
    return ((l - key0) * ld - hk * d) * 4


SHAPES = [(n, l, h, hkv, d) for n in (1, 2) for l in (1, 5, 16, 17, 40) for (h, hkv) in ((4, 2), (9, 3), (2, 1))
          for d in (4, 8, 12, 16, 24, 40, 64, 68)]


def test_forward_kv_tile_loads_stay_inside_their_operands():
    rec = library_records()
    for n, l, h, hkv, d in SHAPES:
        for name, kc, kld, ksize, vc, vld, vsize in layouts(n, l, h, hkv, d):
            for what, col, ld, size in (("K", kc, kld, ksize), ("V", vc, vld, vsize)):
                hi, lo = max_reach(rec, n, l, hkv, d, col, ld, size)
                assert 0 <= lo and hi < size, (name, what, n, l, h, hkv, d, hi, size)


def test_q_side_v_tile_loads_stay_inside_their_operand():
    """attn_rel_q2_kernel reads its V tiles with K's lane layout (16-byte rows, c * ld + 4 g + 16 t)
    through the same range: every dword inside it must lie inside the V operand too."""
    rec = library_records()
    for n, l, h, hkv, d in SHAPES:
        for name, _, _, _, vc, vld, vsize in layouts(n, l, h, hkv, d):
            hi, lo = max_reach(rec, n, l, hkv, d, vc, vld, vsize, patterns=(0,))
            assert 0 <= lo and hi < vsize, (name, n, l, h, hkv, d, hi, vsize)


def test_range_ends_with_the_heads_values_of_the_last_row():
    rec = library_records()
    for l, ld, d in ((5, 48, 8), (16, 48, 8), (512, 768, 64), (1024, 2560, 64), (33, 100, 40)):
        for key0 in range(0, l, 16):
            assert rec(l, key0, ld, d) == ((l - 1 - key0) * ld + d) * 4
    assert rec(0, 0, 8, 8) == -1 and rec(5, 5, 8, 8) == -1 and rec(5, 0, 4, 8) == -1
    assert rec(1 << 20, 0, 1 << 10, 8) == -1  # past the 32-bit byte count


def test_previous_range_reads_past_the_packed_buffer_at_head_dim_8():
    """Negative control on the CPU: the former range lets the last row's columns 8..15 of the last KV
    head be read past the allocation when K comes from the rotated q|k rows (head_dim 8)."""
    n, l, h, hkv, d = 1, 16, 4, 2, 8
    _, kc, kld, ksize, _, _, _ = next(layouts(n, l, h, hkv, d))
    hi, _ = max_reach(previous_records, n, l, hkv, d, kc, kld, ksize)
    assert hi >= ksize
