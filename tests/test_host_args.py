"""Argument checks of the Python binding (CPU only: no library call).

The library writes Q * K * 4 bytes into each result array and reads R (or,
for a dual-channel search, L) entry ids from the caller's draw, so the
binding rejects arrays of another shape, type or layout before the call.
"""
import numpy as np
import pytest

from garfield_amd import _lib


def test_out_arrays_fresh_and_checked():
    ids, d = _lib._out_arrays(None, 5, 10)
    assert ids.shape == (5, 10) and ids.dtype == np.uint32 and d.dtype == np.float32
    good = (np.zeros((5, 10), np.uint32), np.zeros((5, 10), np.float32))
    assert _lib._out_arrays(good, 5, 10)[0] is good[0]
    bad = [
        (np.zeros((4, 10), np.uint32), good[1]),            # too few rows
        (good[0], np.zeros((5, 10), np.float64)),           # wrong type
        (np.zeros((10, 5), np.uint32).T, good[1]),          # not C-contiguous
        (good[0], np.zeros((5, 9), np.float32)),            # K mismatch
        ([[0] * 10] * 5, good[1]),                          # not an array
    ]
    ro = np.zeros((5, 10), np.uint32)
    ro.flags.writeable = False
    bad.append((ro, good[1]))
    for out in bad:
        with pytest.raises(ValueError):
            _lib._out_arrays(out, 5, 10)


def test_entry_points_length():
    assert _lib._entry_arg(None, 32, "R") is None
    e = _lib._entry_arg(np.arange(32), 32, "R")
    assert e.dtype == np.uint32 and e.size == 32
    with pytest.raises(ValueError, match="R = 32"):
        _lib._entry_arg(np.arange(16), 32, "R")
    # a cell-by-cell draw (R ids) passed to a dual-channel search (L ids)
    with pytest.raises(ValueError, match="L"):
        _lib._entry_arg(np.arange(32), 600, "L (dual-channel)")
