"""Repeated rows on the float MFMA brute force.  Groups of 48 rows share one
vector and its attributes, and every query lies close to one group, so an
item keeps 32 keys at one distance, all within the query's limit: it flags
the query, and k_bf_f16_final scans that query exactly with the gather
kernel's code (bf_scan_query).  The kept keys' merge also sees equal keys.

Bar: ids, distances and counters bit for bit against the oracle's brute
force, for binary16 and fp32 rows; and some queries took the exact scan
(their DIST counts every passing point, as the oracle's does)."""
import numpy as np
import pytest

from conftest import _float_index_device
from test_gpu_parity import _assert_same, _print_case, _traversal_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def world_dups():
    from garfield_amd import synth
    N, G, M, Q = 6000, 40, 48, 64
    vec = synth.gaussian_unit_vectors(N, 96, 80)
    att = synth.zipf_attrs(N, 3, 81, hi=400)
    for g in range(G):
        vec[g * M:(g + 1) * M] = vec[g * M]
        att[g * M:(g + 1) * M] = att[g * M]
    rng = np.random.default_rng(82)
    heads = (np.arange(Q) % G) * M
    qv = vec[heads] + rng.normal(0.0, 0.01, (Q, 96)).astype(np.float32)
    qv = (qv / np.linalg.norm(qv, axis=1, keepdims=True)).astype(np.float32)
    r = rng.integers(5, 200, (Q, 3)).astype(np.int32)
    lo = (att[heads] - r).astype(np.int32)
    hi = (att[heads] + r).astype(np.int32)
    cfg = dict(vectors=vec, attrs=att, grid=[4, 4, 4], R=32, E=2, C=16, queries=qv, lo=lo, hi=hi)
    ix = synth.build_index(vec, att, cfg["grid"], 32, 2, 16, seed=83, device=_float_index_device())
    return cfg, ix


@pytest.mark.parametrize("vec_dtype", [1, 0])
def test_repeated_rows_flag_and_scan(world_dups, vec_dtype):
    cfg, ix = world_dups
    _print_case("float-bf-dups", vec_dtype=vec_dtype)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 32, prefilter=1.0, vec_dtype=vec_dtype)
    assert st.bf_mfma == 2 and st.q_bruteforce == len(cfg["queries"])
    rows = octr[:, 7] == 2
    scanned = rows & (ctr[:, 1] == octr[:, 1]) & (octr[:, 1] > 48)
    assert np.sum(scanned) > 0
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
