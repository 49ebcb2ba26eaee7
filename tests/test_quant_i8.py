"""The int8 per-dimension quantised vector mode (GF_VEC_I8Q), on the CPU.

The quantiser restates the reference loader's host rules
(indexsearch/production_adapter.cuh:113-165); oracle.quantise_i8 is pinned
by hand-derived known answers that each planted mistake of it fails, and the
library's gf_quantise_i8 (host code) must equal it bit for bit.  The oracle's
distance for the mode (garfield_oracle.cpp canon_dist, vdtype 3) is pinned
by the special case scale 1, zero point 0, where it must equal the u8 mode's
distance bit for bit (same 16-element chunks, the same term q - x), and by
the float64 distance to the dequantised vectors elsewhere.
"""
import numpy as np
import pytest

import garfield_amd._lib as gl
from garfield_amd import synth
from oracle import oracle as orc


def _known_answers():
    """(column, alpha, q, scale, zero) derived by hand:
    - [0 .. 255]: scale 1, zero -128, q = x - 128.
    - [0, 3, 5, 510]: scale 2, zero -128; 3 / 2 = 1.5 and 5 / 2 = 2.5 round
      away from zero to 2 and 3.
    - [-127.5, 1.5, 127.5]: scale 1, zero round(-0.5) = -1; 1.5 -> 2 - 1.
    - [150000, 355000]: min stays at its start value 100000, so scale
      255000 / 255 = 1000 and zero round(-228) clamps to -128; 150 - 128 =
      22 and 355 - 128 clamps to 127.
    - [-355000, -150000]: max stays at -100000, scale 1000, zero round(227)
      clamps to 127; -355 + 127 clamps to -128, -150 + 127 = -23.
    - [7, 7, 7]: constant, scale 1, zero round(-135) clamps to -128, q = -121.
    - [0, 255] with alpha 2: values 0, 510, scale 2, zero -128."""
    return [
        (np.arange(256), 1.0, np.arange(256) - 128, 1.0, -128),
        ([0, 3, 5, 510], 1.0, [-128, -126, -125, 127], 2.0, -128),
        ([-127.5, 1.5, 127.5], 1.0, [-128, 1, 127], 1.0, -1),
        ([150000, 355000], 1.0, [22, 127], 1000.0, -128),
        ([-355000, -150000], 1.0, [-128, -23], 1000.0, 127),
        ([7, 7, 7], 1.0, [-121, -121, -121], 1.0, -128),
        ([0, 255], 2.0, [-128, 127], 2.0, -128),
    ]


@pytest.mark.parametrize("impl", ["oracle", "library"])
def test_quantise_known_answers(impl):
    for col, alpha, q, s, z in _known_answers():
        x = np.asarray(col, np.float32)[:, None]
        got = orc.quantise_i8(x, alpha) if impl == "oracle" else gl.quantise_i8(x, alpha)
        assert got[0][:, 0].tolist() == list(q), (col, got[0][:, 0])
        assert got[1][0] == np.float32(s) and got[2][0] == z, (col, got[1], got[2])


@pytest.mark.parametrize("mutation", [1, 2])
def test_quantise_mutations_fail(mutation):
    wrong = 0
    for col, alpha, q, s, z in _known_answers():
        x = np.asarray(col, np.float32)[:, None]
        got = orc.quantise_i8(x, alpha, mutation=mutation)
        wrong += got[0][:, 0].tolist() != list(q) or got[1][0] != np.float32(s) or got[2][0] != z
    assert wrong > 0


def test_library_quantiser_matches_oracle():
    rng = np.random.default_rng(11)
    cases = [
        (rng.standard_normal((500, 48)).astype(np.float32), 1.0),
        ((rng.standard_normal((300, 32)) * 1e3 + 5e3).astype(np.float32), 1.0),
        (rng.integers(-300, 300, (257, 16)).astype(np.float32) * 0.5, 0.01),
        (np.zeros((1, 16), np.float32), 1.0),
    ]
    x = rng.standard_normal((200, 16)).astype(np.float32)
    x[:, 3] = 2.5                         # a constant dimension
    x[:7, 5] = np.float32(1e6)            # values beyond the start values
    cases.append((x, 1.0))
    for x, alpha in cases:
        want = orc.quantise_i8(x, alpha)
        got = gl.quantise_i8(x, alpha)
        for w, g in zip(want, got):
            assert w.dtype == g.dtype and np.array_equal(w, g)


def test_dequantised_within_half_step():
    """Where neither the zero point nor q clamps, scale * (q - zero) is
    within half a step of the value (C round's error), up to fp32 rounding."""
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((400, 32)) * rng.uniform(0.1, 50, 32)).astype(np.float32)
    q, s, z = orc.quantise_i8(x)
    mn = np.minimum(100000.0, x.min(axis=0))
    zr = orc._round_half_away(np.float32(-128.0) - mn.astype(np.float32) / s)
    free = (zr >= -128) & (zr <= 127)
    assert free.any()
    err = np.abs(s * (q.astype(np.float64) - z) - x)
    inside = (q > -128) & (q < 127) & free[None, :]
    bound = np.broadcast_to(s[None, :] * (0.5 + 1e-4), err.shape)
    assert inside.sum() > 1000 and np.all(err[inside] <= bound[inside])


def _oracle(x, **kw):
    N = x.shape[0]
    pid = np.random.default_rng(3).integers(0, 4, N).astype(np.uint32)
    members = synth.cell_members(pid, 4)
    graphs = np.concatenate([np.zeros((len(m), 4), np.uint32) for m in members])
    return orc.OracleIndex(x, np.zeros((N, 1), np.float32), pid, 4, graphs, np.zeros((N, 4), np.uint32), **kw)


def test_i8q_distance_unit_scale_equals_u8_mode():
    """Integers in [-128, 127] with both ends present in every dimension:
    scale 1, zero 0, q = x, and the mode's distance equals the u8 mode's
    (16-element chunks, term query - x) bit for bit, for fractional queries."""
    rng = np.random.default_rng(5)
    N, D = 120, 64
    x = rng.integers(-128, 128, (N, D)).astype(np.float32)
    x[0], x[1] = -128, 127
    q8, s, z = orc.quantise_i8(x)
    assert np.all(s == 1.0) and np.all(z == 0) and np.array_equal(q8.astype(np.float32), x)
    A = _oracle(q8.astype(np.float32), i8q=(s, z))
    B = _oracle(x, u8=True)
    for t in range(4):
        qf = (rng.standard_normal(D) * 60).astype(np.float32)
        for g in range(0, N, 7):
            da, db = A.distance(qf, g), B.distance(qf, g)
            assert np.float32(da).view(np.uint32) == np.float32(db).view(np.uint32)


def test_i8q_distance_against_float64():
    """General scales and zero points: within the fp32 bound of the float64
    distance to the dequantised row scale * (q - zero)."""
    rng = np.random.default_rng(6)
    N, D = 150, 96
    x = (rng.standard_normal((N, D)) * rng.uniform(0.2, 3, D) + rng.uniform(-2, 2, D)).astype(np.float32)
    q8, s, z = orc.quantise_i8(x)
    O = _oracle(q8.astype(np.float32), i8q=(s, z))
    deq = s.astype(np.float64) * (q8.astype(np.float64) - z)
    for t in range(3):
        qf = (rng.standard_normal(D) * 1.5).astype(np.float32)
        for g in range(0, N, 5):
            ref = np.sum((qf.astype(np.float64) - deq[g]) ** 2)
            assert abs(O.distance(qf, g) - ref) <= 2e-6 * ref + 1e-6, (t, g)
