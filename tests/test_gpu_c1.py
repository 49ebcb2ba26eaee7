"""Config C1 at its stated size, on the GPU: 100k x 128 vectors of integers
uniform in [0, 255], 2 attributes uniform in [0, 10000) on a 4x4 grid, per-cell
graphs of degree 16 and 2 cross edges per point (built on the GPU by the
library's builder), 1000 queries at about 30 % selectivity, k = 10.

Checked against a brute-force filtered kNN on the CPU (oracle.ground_truth),
and bit for bit (ids, distances, counters) against the oracle's own search on
the same index: the filtered brute force (prefilter 1.0, the int8 MFMA route),
the cell-by-cell traversal and the dual-channel traversal.
"""
import numpy as np
import pytest

from garfield_amd import synth
from test_gpu_parity import _assert_same, _print_case, _traversal_case

pytestmark = pytest.mark.gpu

_RECALL = {}


@pytest.fixture(scope="module")
def c1_world():
    from oracle import oracle as orc
    cfg = synth.config_small()
    assert cfg["vectors"].shape == (100_000, 128) and cfg["queries"].shape[0] == 1000
    ix = synth.build_index(cfg["vectors"], cfg["attrs"], cfg["grid"], cfg["R"], cfg["E"], cfg["C"], seed=5,
                           device="hip")
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    gt = orc.ground_truth(ix["vectors"], ix["attrs"], cfg["queries"], lo, hi, 10)
    return cfg, ix, gt


def _recall(ids, gt):
    from oracle import oracle as orc
    return orc.recall(ids, gt[0], gt[1])


def test_c1_shape(c1_world):
    cfg, ix, _ = c1_world
    assert ix["P"] == 16 and ix["R"] == 16 and ix["cross"].shape == (100_000, 16 * 2)
    # about 30 % of the points pass a query's ranges, on average
    a = ix["attrs"]
    frac = np.mean([np.mean(np.all((a >= cfg["lo"][q]) & (a <= cfg["hi"][q]), axis=1)) for q in range(0, 1000, 25)])
    assert 0.2 < frac < 0.4


def test_c1_bruteforce_exact(c1_world):
    cfg, ix, gt = c1_world
    _print_case("c1-bruteforce", prefilter=1.0)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 10, prefilter=1.0)
    assert st.q_bruteforce == 1000 and st.bf_mfma == 1
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert _recall(ids, gt) == 1.0


@pytest.mark.parametrize("L", [32, 128])
def test_c1_traversal_parity(c1_world, L):
    cfg, ix, gt = c1_world
    _print_case("c1-traverse", L=L)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, L)
    assert st.q_traverse == 1000
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    _RECALL[("cell", L)] = _recall(ids, gt)


def test_c1_dual_channel_parity(c1_world):
    cfg, ix, gt = c1_world
    _print_case("c1-dual", L=128)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 128, channels=2)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    _RECALL[("dual", 128)] = _recall(ids, gt)


@pytest.mark.parametrize("channels", [1, 2])
@pytest.mark.parametrize("prefilter", [0.0, 0.3])
@pytest.mark.parametrize("L", [600, 1100, 1700])
def test_c1_operating_point_L_parity(c1_world, L, prefilter, channels):
    """The list lengths the recall target needs (L = 600-1700), where the
    kernels run their largest configurations: a 2048- (L = 600) or 4096-slot
    visited set (L >= 1100), lists past 512 entries and 20-32 KB of LDS per
    workgroup.  Ids, distances and counters bit for bit against the oracle,
    which keeps its visited set as an exact set, so a table that filled up
    (an insert reported as 'seen') would show as a difference.  64 queries of
    the batch; cells of 6,250 points, larger than L."""
    cfg, ix, gt = c1_world
    _print_case("c1-high-L", L=L, prefilter=prefilter, channels=channels, Q=64)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, L, prefilter=prefilter, Q=64,
                                                             channels=channels)
    assert st.q_traverse > 0
    if prefilter == 0.0:
        assert st.q_traverse == 64
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    # some query expanded more than 512 nodes (counter 0; route 1 is the
    # cell-by-cell traversal, 4 the dual-channel one), so lists this long ran
    trav = np.isin(ctr[:, 7], (1, 4))
    assert ctr[trav, 0].max() > 512


def test_c1_recall_grows_with_L(c1_world):
    """Against the CPU ground truth: more candidates give more recall, and the
    dual-channel traversal is not worse than the cell-by-cell one at equal L."""
    if len(_RECALL) < 3:
        pytest.skip("needs the parity tests above")
    print(f"[c1] recall {_RECALL}", flush=True)
    assert _RECALL[("cell", 128)] > _RECALL[("cell", 32)] > 0.1
    assert _RECALL[("dual", 128)] >= _RECALL[("cell", 128)] - 0.02
