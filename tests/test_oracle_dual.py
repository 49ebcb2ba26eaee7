"""Pinning the dual-channel traversal of the oracle (orc_set_channels(2),
oracle/garfield_oracle.cpp), the traversal of the reference's
select_path_contain_attr_filter_V2_without_output_dual_channel_in_turn_with_prefilter
(indexsearch/gpu_graph.cu:6249-6640).

1. Agreement with tests/kernel_model.py (KernelModel.search_dual), a second
   restatement that follows the reference kernel's own arrays: top_M_Cand of
   TOPM + 2 DEGREE ids carrying explored bits 31 and 30, `turn`,
   `main_channel`, `cur_visit_p`, merge_top's bisection ranks: ids,
   distances, expansions, distance evaluations and switch slots, on random
   small worlds with 1 to 4 cells, E = 1 and 2, L = 7, 20, 71, entry ids
   beyond the cell sizes, and an epoch cap of 5.
2. A closed form: two cells with complete graphs, every entry on the point
   of its channel's cell farthest from the query.  Each point found then
   pushes out an entry copy, so the result is the filtered brute force of
   both cells, and every point is evaluated (L entries plus the other 58
   points at least; an entry point whose copies were all pushed out is
   found again after each visited-set reset).
3. Every planted mistake (orc_set_dual_mutation) turns 1 or 2 red.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from kernel_model import KernelModel

SENT = 0xFFFFFFFF


@pytest.fixture(autouse=True)
def _reset_oracle():
    orc.set_channels(2)
    orc.set_dual_mutation(0)
    orc.set_max_iter(0)
    orc.set_tie_mode(0)
    yield
    orc.set_channels(1)
    orc.set_dual_mutation(0)
    orc.set_max_iter(0)


def _random_world(seed, N=400, D=8, P=4, R=8, E=2, vmax=256):
    rng = np.random.default_rng(seed)
    v = rng.integers(0, vmax, (N, D)).astype(np.uint8)
    pid = rng.integers(0, P, N).astype(np.uint32)
    att = rng.integers(0, 100, (N, 2)).astype(np.float32)
    g = orc.knn_cell_graphs(v, pid, P, R)
    x = orc.cross_graph(v, pid, P, E)
    return v.astype(np.float32), att, pid, g, x


def _search(O, q, lo, hi, cells, ent, L, P=4):
    cl = np.zeros((1, P), np.uint32)
    cl[0, :len(cells)] = cells
    cnt = np.array([len(cells)], np.uint32)
    ids, dist, ctr = O.search(q[None], lo[None], hi[None], cl, cnt, np.zeros(1, np.uint32), ent, L, nthreads=1)
    return ids[0], dist[0], ctr[0]


_CASES = None


def _cases():
    global _CASES
    if _CASES is not None:
        return _CASES
    worlds = [_random_world(0), _random_world(1, E=1), _random_world(2, vmax=16), _random_world(3, R=5)]
    cases = []
    for w, (vec, att, pid, g, x) in enumerate(worlds):
        M = KernelModel(vec, att, pid, 4, g, x, tie=0)
        rng = np.random.default_rng(500 + w)
        for qi in range(8):
            q = rng.integers(0, 256 if w != 2 else 16, 8).astype(np.float32)
            lo = rng.integers(0, 50, 2).astype(np.float32)
            hi = lo + rng.integers(10, 60, 2).astype(np.float32)
            cells = [int(c) for c in rng.permutation(4)[:rng.integers(1, 5)]]
            for L, cap in ((7, 10000), (20, 10000), (71, 10000), (21, 5)):
                ent = rng.integers(0, 62500, L).astype(np.uint32)
                cases.append((w, cap, q, lo, hi, cells, ent, L,
                              M.search_dual(q, lo, hi, cells, ent, L, max_iter=cap)))
    _CASES = (worlds, cases)
    return _CASES


def check_model():
    worlds, cases = _cases()
    idx = [orc.OracleIndex(v, a, p, 4, g, x) for v, a, p, g, x in worlds]
    bad = 0
    for w, cap, q, lo, hi, cells, ent, L, m in cases:
        orc.set_max_iter(cap)
        ids, dist, ctr = _search(idx[w], q, lo, hi, cells, ent, L)
        same = (ids.tolist() == m[0] and dist.tolist() == [float(np.float32(d)) for d in m[1]]
                and int(ctr[0]) == m[2] and int(ctr[1]) == m[3] and int(ctr[3]) == m[4] and int(ctr[7]) == 4)
        bad += not same
    orc.set_max_iter(0)
    return bad, len(cases)


def test_dual_agrees_with_kernel_model():
    bad, n = check_model()
    assert bad == 0, f"{bad} of {n} cases differ"


def test_model_cases_reach_every_branch():
    """The cases above move channels across cells (switch slots filled), end
    with both channels in one cell, and stop at the epoch cap."""
    _, cases = _cases()
    assert sum(m[4] > 0 for *_, m in cases) > 20
    assert any(len(c[5]) == 1 for c in cases) and any(len(c[5]) == 4 for c in cases)
    assert any(c[1] == 5 for c in cases)


def _closed_form_world():
    """Two cells of 30 points, complete per-cell graphs (R = 29), E = 2."""
    rng = np.random.default_rng(9)
    n, D = 30, 8
    v = rng.integers(0, 256, (2 * n, D)).astype(np.float32)
    pid = np.repeat(np.arange(2, dtype=np.uint32), n)
    att = rng.integers(0, 100, (2 * n, 2)).astype(np.float32)
    g = np.zeros((2 * n, n - 1), np.uint32)
    for r in range(n):
        g[r] = [t for t in range(n) if t != r]
        g[n + r] = g[r]
    x = orc.cross_graph(v.astype(np.uint8), pid, 2, 2)
    return v, att, pid, g, x, n


def check_closed_form():
    v, att, pid, g, x, n = _closed_form_world()
    O = orc.OracleIndex(v, att, pid, 2, g, x)
    rng = np.random.default_rng(10)
    ok = True
    for t in range(6):
        q = rng.integers(0, 256, 8).astype(np.float32)
        lo = np.array([0, 0], np.float32) + t * 5
        hi = np.array([70, 90], np.float32)
        d = ((v.astype(np.float64) - q) ** 2).sum(1)
        far = [int(np.argmax(d[:n])), int(np.argmax(d[n:]))]
        L = 80
        ent = np.array([far[0]] * 40 + [far[1]] * 40, np.uint32)
        ids, dist, ctr = _search(O, q, lo, hi, [0, 1], ent, L, P=2)
        keep = np.nonzero(np.all((att >= lo) & (att <= hi), axis=1))[0]
        order = keep[np.lexsort((keep, d[keep]))][:10]
        want = order.tolist() + [0x7FFFFFFF] * (10 - len(order))
        ok &= ids.tolist() == want
        ok &= int(ctr[1]) >= L + 2 * n - 2 and int(ctr[0]) >= 2
    return bool(ok)


def test_closed_form_two_complete_cells():
    assert check_closed_form()


@pytest.mark.parametrize("mutation", [1, 2, 3, 4, 5, 6])
def test_planted_mistakes_are_caught(mutation):
    orc.set_dual_mutation(mutation)
    try:
        bad, _ = check_model()
        caught = bad > 0 or not check_closed_form()
    finally:
        orc.set_dual_mutation(0)
    assert caught, f"dual mutation {mutation} went unnoticed"
