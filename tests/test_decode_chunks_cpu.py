"""The key ranges of pxk_decode_attention's 64-key chunks, checked on the host through the kernel's
own definition (pxk_decode_chunk_keys): every chunk stays inside its 64 keys, the cache and the
visible positions, and the chunks together cover exactly the window [lo, p] a query at position p
sees (attention_masked, row_math.hpp:117-126) -- with whole chunks before lo empty, a partly
windowed first chunk, positions past the cache clamped, and windows of 1, 63, 64, 65 and wider
than the cache."""
import ctypes

from pulsatrix_amd import native as N


def test_decode_chunk_key_ranges_stay_in_bounds_and_tile_the_window():
    fn = N.pxk().pxk_decode_chunk_keys
    i64 = ctypes.c_int64
    fn.argtypes = [i64, i64, i64, i64, ctypes.POINTER(i64), ctypes.POINTER(i64)]
    fn.restype = ctypes.c_int
    j0, j1 = i64(), i64()
    for max_keys in (1, 63, 64, 65, 130, 300):
        chunks = (max_keys + 63) // 64
        for window in (0, 1, 5, 63, 64, 65, 100, 128, 1000):
            for pos in range(-2, max_keys + 3):
                p = min(max(pos, 0), max_keys - 1)
                lo = p + 1 - window if 0 < window < p + 1 else 0
                covered = []
                for c in range(chunks):
                    assert fn(pos, max_keys, window, c, ctypes.byref(j0), ctypes.byref(j1)) == 0
                    a, b = j0.value, j1.value
                    if b <= a:
                        continue
                    assert 64 * c <= a and b <= 64 * c + 64, (max_keys, window, pos, c, a, b)
                    assert 0 <= a and b <= p + 1 <= max_keys
                    covered += range(a, b)
                assert covered == list(range(lo, p + 1)), (max_keys, window, pos)
    assert fn(0, 0, 0, 0, ctypes.byref(j0), ctypes.byref(j1)) != 0  # an empty cache is rejected
