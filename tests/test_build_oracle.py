"""Index builder, CPU side: the oracle's restatements of the reference's
build scripts pinned by hand-computed cases and by a brute force of a
different form (Python tuple sorts), the library's grid (host code) against
the oracle, and the builder's argument checks (which run before any device
call)."""
import numpy as np
import pytest

from garfield_amd import _lib
from garfield_amd._lib import GarfieldError
from oracle import oracle
from oracle import oracle as orc


# ---------------------------------------------------------------- grid
def test_oracle_grid_hand_case():
    # N = 5, g = 2: avg = 3; stable order of (5, 1, 3, 1, 2) is ids 1, 3, 4, 2, 0
    att = np.array([[5, 0], [1, 1], [3, 0], [1, 1], [2, 0]])
    l_q, r_q, pl, gp = oracle.grid_scatter(att, [2, 2])
    assert list(pl[0]) == [1, 0, 1, 0, 0]
    assert list(l_q[0]) == [1, 3] and list(r_q[0]) == [2, 5]
    # attribute 1 (0, 1, 0, 1, 0): stable ranks put ids 0, 2, 4 first
    assert list(pl[1]) == [0, 1, 0, 1, 0]
    assert list(l_q[1]) == [0, 1] and list(r_q[1]) == [0, 1]
    # row-major, last attribute fastest
    assert list(gp) == [2, 1, 2, 1, 0]


def test_oracle_grid_three_attributes_factors():
    rng = np.random.default_rng(3)
    att = rng.integers(0, 50, (200, 3))
    _, _, pl, gp = oracle.grid_scatter(att, [2, 3, 4])
    assert np.array_equal(gp, pl[0] * 12 + pl[1] * 4 + pl[2])
    # every run but the last holds ceil(N / g) points
    for d, g in enumerate([2, 3, 4]):
        cnt = np.bincount(pl[d], minlength=g)
        avg = -(-200 // g)
        assert np.all(cnt[:-1] == avg) and cnt[-1] == 200 - avg * (g - 1)


@pytest.mark.parametrize("n,grid,hi,seed", [(1000, [4, 4], 10000, 1), (777, [3, 5], 20, 2),
                                            (64, [2, 2, 2], 3, 3), (10, [1], 5, 4), (300, [7], 1, 5)])
def test_library_grid_matches_oracle(n, grid, hi, seed):
    rng = np.random.default_rng(seed)
    att = rng.integers(0, hi, (n, len(grid))).astype(np.float32)
    l_q, r_q, pl, gp = _lib.grid_scatter(att, grid)
    ol, orr, opl, ogp = oracle.grid_scatter(att, grid)
    for d in range(len(grid)):
        assert np.array_equal(l_q[d], ol[d]) and np.array_equal(r_q[d], orr[d])
        assert np.array_equal(pl[d], opl[d])
    assert np.array_equal(gp, ogp)


def test_library_grid_signed_values_and_zeros():
    # negative values, -0.0 next to +0.0 (equal: they keep point-id order)
    rng = np.random.default_rng(6)
    att = rng.integers(-5, 6, (400, 2)).astype(np.float32)
    att[rng.random((400, 2)) < 0.2] = -0.0
    l_q, r_q, pl, gp = _lib.grid_scatter(att, [3, 4])
    ol, orr, opl, ogp = oracle.grid_scatter(att, [3, 4])
    assert all(np.array_equal(pl[d], opl[d]) for d in range(2)) and np.array_equal(gp, ogp)
    assert all(np.array_equal(l_q[d], ol[d]) and np.array_equal(r_q[d], orr[d]) for d in range(2))


def test_library_grid_rejects_unfillable_grid():
    # N = 5, g = 4: avg = 2 and the last run would start at rank 6
    with pytest.raises(GarfieldError) as e:
        _lib.grid_scatter(np.arange(5, dtype=np.float32)[:, None], [4])
    assert e.value.status == 1


# ---------------------------------------------------------------- graphs
def _brute_graph(v, gpid, P, R):
    rows = []
    for c in range(P):
        mem = [i for i in range(len(gpid)) if gpid[i] == c]
        for i, p in enumerate(mem):
            cand = sorted((int(((v[p].astype(int) - v[q].astype(int)) ** 2).sum()), j)
                          for j, q in enumerate(mem) if j != i)
            ids = [j for _, j in cand[:R]]
            if not ids:
                ids = [i]
            rows.append(ids + [ids[0]] * (R - len(ids)))
    return np.array(rows, np.uint32)


def _brute_cross(v, gpid, P, E):
    out = np.zeros((len(gpid), P * E), np.uint32)
    for c in range(P):
        mem = [i for i in range(len(gpid)) if gpid[i] == c]
        if not mem:
            continue
        for p in range(len(gpid)):
            cand = sorted((int(((v[p].astype(int) - v[q].astype(int)) ** 2).sum()), j) for j, q in enumerate(mem))
            ids = [j for _, j in cand[:E]]
            out[p, c * E:(c + 1) * E] = ids + [ids[0]] * (E - len(ids))
    return out


def test_oracle_graph_line_hand_case():
    # one cell, points on a line at 0, 1, 3, 7
    v = np.array([[0], [1], [3], [7]], np.uint8)
    g = oracle.knn_cell_graphs(v, np.zeros(4, np.int64), 1, 2)
    assert g.tolist() == [[1, 2], [0, 2], [1, 0], [2, 1]]
    # the same points as a second cell's members, interleaved with cell 0's
    v2 = np.array([[0], [50], [1], [60], [3], [7]], np.uint8)
    gp = np.array([1, 0, 1, 0, 1, 1])
    g2 = oracle.knn_cell_graphs(v2, gp, 2, 2)
    assert g2.tolist() == [[1, 1], [0, 0], [1, 2], [0, 2], [1, 0], [2, 1]]
    x = oracle.cross_graph(v2, gp, 2, 2)
    # point 0 (value 0): cell 0 = (50, 60) -> 0, 1; cell 1 = (0, 1, 3, 7) -> 0, 1
    assert x[0].tolist() == [0, 1, 0, 1]
    # point 3 (value 60): cell 0 -> 1 (itself), 0; cell 1 -> 3, 2
    assert x[3].tolist() == [1, 0, 3, 2]


def test_oracle_graph_ties_and_tiny_cells():
    rng = np.random.default_rng(9)
    v = rng.integers(0, 2, (40, 8)).astype(np.uint8)   # many equal distances
    gp = np.zeros(40, np.int64)
    gp[30:37] = 2            # cell 2: 7 points
    gp[37] = 3               # cell 3: alone
    gp[38:] = 4              # cell 4: 2 points; cell 1: empty
    for R in (1, 3, 8):
        assert np.array_equal(oracle.knn_cell_graphs(v, gp, 5, R), _brute_graph(v, gp, 5, R))
    for E in (1, 2, 5):
        assert np.array_equal(oracle.cross_graph(v, gp, 5, E), _brute_cross(v, gp, 5, E))


def test_oracle_graph_random_brute_force():
    rng = np.random.default_rng(11)
    v = rng.integers(0, 256, (60, 16)).astype(np.uint8)
    gp = rng.integers(0, 3, 60)
    assert np.array_equal(oracle.knn_cell_graphs(v, gp, 3, 5), _brute_graph(v, gp, 3, 5))
    assert np.array_equal(oracle.cross_graph(v, gp, 3, 3), _brute_cross(v, gp, 3, 3))


def test_oracle_rows_match_full():
    rng = np.random.default_rng(12)
    v = rng.integers(0, 4, (300, 32)).astype(np.uint8)
    gp = rng.integers(0, 5, 300)
    gp[gp == 3] = 4          # cell 3 empty
    gp[7] = 3                # ... but for one point
    rows = [0, 7, 50, 299, 123]
    full_g = oracle.knn_cell_graphs(v, gp, 5, 6)
    order = np.argsort(gp, kind="stable")
    pos = np.empty(300, np.int64)
    pos[order] = np.arange(300)   # cell-major row of each point
    assert np.array_equal(oracle.graph_rows(v, gp, 5, 6, rows), full_g[pos[rows]])
    assert np.array_equal(oracle.cross_rows(v, gp, 5, 3, rows), oracle.cross_graph(v, gp, 5, 3)[rows])


# ---------------------------------------------------------------- k-means labels
def _brute_kmeans(v, C, iters, init):
    x = [list(map(int, r)) for r in v]
    cen = [list(x[i]) for i in init]
    for it in range(iters + 1):
        lab = []
        for p in x:
            best = min(range(C), key=lambda c: (sum((a - b) ** 2 for a, b in zip(p, cen[c])), c))
            lab.append(best)
        if it == iters:
            return np.array(lab), np.array(cen)
        for c in range(C):
            mem = [x[i] for i in range(len(x)) if lab[i] == c]
            if mem:
                n = len(mem)
                cen[c] = [(2 * sum(col) + n) // (2 * n) for col in zip(*mem)]


def test_oracle_kmeans_hand_cases():
    v = np.array([[0], [1], [2], [10], [11], [12]], np.uint8)
    lab, cen = oracle.kmeans(v, 2, 2, [0, 3])
    assert lab.tolist() == [0, 0, 0, 1, 1, 1] and cen.ravel().tolist() == [1, 11]
    # a mean of 0.5 rounds up; a point between two centres takes the smaller index
    lab, cen = oracle.kmeans(np.array([[0], [1]], np.uint8), 1, 1, [0])
    assert cen.ravel().tolist() == [1]
    lab, _ = oracle.kmeans(np.array([[0], [2], [1]], np.uint8), 2, 0, [0, 1])
    assert lab.tolist() == [0, 1, 0]
    # equal initial centres: the second cluster stays empty in the first
    # assignment and keeps its centre (3); the update moves the first to
    # floor((2 * 17 + 3) / 6) = 6, and the final assignment takes 3 back
    lab, cen = oracle.kmeans(np.array([[3], [5], [9]], np.uint8), 2, 1, [0, 0])
    assert lab.tolist() == [1, 0, 0] and cen.ravel().tolist() == [6, 3]


def test_oracle_kmeans_brute_force():
    rng = np.random.default_rng(21)
    v = rng.integers(0, 6, (50, 5)).astype(np.uint8)
    init = rng.choice(50, 6, replace=False)
    lab, cen = oracle.kmeans(v, 6, 4, init)
    blab, bcen = _brute_kmeans(v, 6, 4, init)
    assert np.array_equal(lab, blab) and np.array_equal(cen, bcen)


# ---------------------------------------------------------------- argument checks (no device call)
def test_builder_rejects_bad_input_before_device():
    v = np.zeros((10, 64), np.float32)
    gp = np.zeros(10, np.uint32)
    v[3, 5] = 0.5
    with pytest.raises(GarfieldError) as e:
        _lib.build_graphs(v, gp, 1, 64, 2)
    assert e.value.status == 6   # GF_E_UNSUPPORTED: float data (not integers in [0, 255]) with R above 63
    with pytest.raises(GarfieldError) as e:
        _lib.build_graphs(np.zeros((10, 64), np.uint8), gp, 1, 72, 2)
    assert e.value.status == 6   # R + 1 above 72
    with pytest.raises(GarfieldError) as e:
        _lib.build_graphs(np.zeros((10, 1100), np.uint8), gp, 1, 4, 2)
    assert e.value.status == 6   # dimension above 1024
    with pytest.raises(GarfieldError) as e:
        _lib.build_graphs(np.zeros((10, 64), np.uint8), gp + 1, 1, 4, 2)
    assert e.value.status == 1   # a cell id >= P

    with pytest.raises(GarfieldError) as e:
        _lib.kmeans(np.zeros((10, 64), np.uint8), 3, 2, init_ids=[0, 1, 10])
    assert e.value.status == 1   # an initial centre id >= N
    with pytest.raises(GarfieldError) as e:
        _lib.kmeans(np.zeros((10, 64), np.uint8), 11, 2, init_ids=list(range(10)) + [0])
    assert e.value.status == 1   # more centres than points


def test_graph_optimisation_hand_case():
    """Points 0, 1, 2, 3 on a line, one cell, exact 3-NN rows by (distance, id):
    [1 2 3] [0 2 3] [1 3 0] [2 1 0].  Detours (an earlier neighbour listing
    the target at an earlier rank): row 0 -> 3 through 2 (2 lists 3 at rank 1
    < 2); row 3 -> 1 through 2 (rank 0 < 1) and 3 -> 0 through 1 (rank 0 < 2):
    counts [0 0 1] [0 0 1] [0 0 1] [0 1 1].  With R = 2 each row keeps its
    first edge; reverse lists (rank 0 edges in row order, then rank 1):
    rev[0] = [1], rev[1] = [0, 2], rev[2] = [3, 0], rev[3] = [2]; rows
    [1 2] (rev 1 repeats, then the reordered rest), [0 2], [1 3], [2 1]."""
    g = np.array([[1, 2, 3], [0, 2, 3], [1, 3, 0], [2, 1, 0]])
    o, det = orc.detour_order(g)
    assert det.tolist() == [[0, 0, 1], [0, 0, 1], [0, 0, 1], [0, 1, 1]]
    assert o.tolist() == g.tolist()
    assert orc.optimize_graphs(g, [4], 2).tolist() == [[1, 2], [0, 2], [1, 3], [2, 1]]


def test_detour_counts_brute_force():
    """detour_order against the definition evaluated by plain loops."""
    rng = np.random.default_rng(8)
    for n, I in ((30, 8), (12, 11), (50, 16)):
        g = np.array([rng.choice([x for x in range(n) if x != a], I, replace=False) for a in range(n)])
        o, det = orc.detour_order(g)
        for a in range(n):
            row = g[a].tolist()
            for k, d in enumerate(row):
                cnt = sum(1 for j in range(k) if d in g[row[j]].tolist()[:k])
                assert det[a, k] == cnt
            keyed = sorted(range(I), key=lambda k: (det[a, k], k))
            assert o[a].tolist() == [row[k] for k in keyed]


def test_optimised_graph_properties():
    """Every row holds R distinct in-cell ids without itself, its first R/2
    ids are its first R/2 reordered edges, and every node with an incoming
    pruned edge among the first R ranks is reachable."""
    rng = np.random.default_rng(9)
    x = rng.integers(0, 256, (600, 16)).astype(np.uint8)
    pid = rng.integers(0, 3, 600).astype(np.uint32)
    knn = orc.knn_cell_graphs(x, pid, 3, 24)
    sizes = np.bincount(pid, minlength=3)
    out = orc.optimize_graphs(knn, sizes, 12)
    start = 0
    for c, n in enumerate(sizes):
        o, _ = orc.detour_order(knn[start:start + n])
        for a in range(n):
            row = out[start + a].tolist()
            assert len(set(row)) == 12 and a not in row and max(row) < n
            assert row[:6] == o[a, :6].tolist()
        start += n


# ------------------------------------------------------------ float data
def test_quantise_u8_known_answers():
    # s = 1: rint(x), halves to even (127.5 -> 128, 0.5 -> 0, 2.5 -> 2)
    v = np.array([[0.0, 255.0, 127.5, 0.5, 2.5]], np.float32)
    assert list(orc.quantise_u8(v)[0]) == [0, 255, 128, 0, 2]
    assert list(orc.quantise_u8(np.full((2, 3), 7.0, np.float32)).ravel()) == [0] * 6
    v = np.array([[-2.0, 2.0, 0.0]], np.float32)
    assert list(orc.quantise_u8(v)[0]) == [0, 255, 128]


def test_canon_dists_close_to_float64():
    rng = np.random.default_rng(4)
    X = rng.standard_normal((64, 768)).astype(np.float32)
    d = orc.canon_dists(X[0], X)
    ref = ((X.astype(np.float64) - X[0]) ** 2).sum(1)
    assert d[0] == 0.0
    assert np.allclose(d, ref, rtol=1e-5)


def _exact_rows(v, gp, P, K, rows, cross):
    """Brute force in float64: (distance, local id) order, a different form
    (Python tuple sorts) from the oracle's re-rank."""
    v64 = np.asarray(v, np.float64)
    mem = [np.nonzero(gp == c)[0] for c in range(P)]
    out = []
    for p in rows:
        cells = range(P) if cross else [gp[p]]
        row = []
        for c in cells:
            m = mem[c]
            items = sorted((float(((v64[x] - v64[p]) ** 2).sum()), l) for l, x in enumerate(m)
                           if cross or x != p)
            row.append([l for _, l in items[:K]])
        out.append(row)
    return out


@pytest.mark.parametrize("D,mut", [(96, 0), (96, 1), (200, 0)])
def test_float_rows_are_exact_neighbours(D, mut):
    """On Gaussian, L2-normalised data (config 3's kind) the re-ranked rows
    are the exact float64 nearest neighbours, except between distances within
    1e-6 of each other; without the re-rank (mutation 1, the quantised order)
    they are not."""
    rng = np.random.default_rng(D)
    N, P, R, E = 1200, 4, 16, 3
    v = rng.standard_normal((N, D)).astype(np.float32)
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    gp = rng.integers(0, P, N).astype(np.uint32)
    rows = rng.choice(N, 40, replace=False)
    g = orc.float_graph_rows(v, gp, P, R, rows, mutation=mut)
    ex = _exact_rows(v, gp, P, R, rows, False)
    v64 = v.astype(np.float64)
    mem = [np.nonzero(gp == c)[0] for c in range(P)]
    bad = 0
    for i, p in enumerate(rows):
        m = mem[gp[p]]
        dg = ((v64[m[g[i]]] - v64[p]) ** 2).sum(1)
        de = ((v64[m[ex[i][0]]] - v64[p]) ** 2).sum(1)
        bad += not np.allclose(dg, de, rtol=0, atol=1e-6)
    if mut:
        assert bad > 0
        return
    assert bad == 0
    x = orc.float_cross_rows(v, gp, P, E, rows[:10])
    exc = _exact_rows(v, gp, P, E, rows[:10], True)
    for i, p in enumerate(rows[:10]):
        for c in range(P):
            m = mem[c]
            dx = ((v64[m[x[i, c * E:(c + 1) * E]]] - v64[p]) ** 2).sum(1)
            de = ((v64[m[exc[i][c]]] - v64[p]) ** 2).sum(1)
            assert np.allclose(dx, de, rtol=0, atol=1e-6), (p, c)


def test_float_rows_short_cells():
    """Cells smaller than the degree: rows repeat their nearest, a point
    alone lists itself, cross edges into an empty cell are 0."""
    rng = np.random.default_rng(9)
    v = rng.standard_normal((7, 32)).astype(np.float32)
    gp = np.array([0, 0, 0, 1, 2, 2, 2], np.uint32)   # cell 3 empty
    g = orc.float_graph_rows(v, gp, 4, 4, [0, 3])
    assert g[1].tolist() == [0, 0, 0, 0]              # alone: itself (local id 0)
    assert len(set(g[0].tolist())) == 2 and g[0][2] == g[0][3] == g[0][0]
    x = orc.float_cross_rows(v, gp, 4, 2, [3])
    assert x[0, 6:8].tolist() == [0, 0]
    assert x[0, 2:4].tolist() == [0, 0]               # cell 1 holds only the point itself
