"""Pins the CPU oracle against library routines, closed forms and brute force.

Each check is chosen so that a plausible mistake in the restatement (a wrong
rounding, an off-by-one cell bound, a swapped index, a dropped tie rule)
fails: numpy's IEEE binary16 conversion for f2h, numpy's MT19937 plus the
published nearly-divisionless bounded draw and glibc's additive-feedback
rand() for the entry points, exhaustive box intersection for the cells, and
exact filtered brute force for the search results.
"""
import numpy as np
import pytest

from garfield_amd import synth
from oracle import oracle as orc


def test_f2h_matches_numpy_binary16():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    edge = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25,
                     2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1e30, -1e30, np.inf, -np.inf], np.float32)
    x = np.concatenate([x, edge])
    for alpha in (1.0, 0.01, 3.0):
        with np.errstate(over="ignore"):
            ref = (x * np.float32(alpha)).astype(np.float16).view(np.uint16)
        assert np.array_equal(orc.f2h(x, alpha), ref)


def test_h2f_all_halves():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    lib = orc.load()
    got = np.array([lib.orc_h2f(int(v)) for v in h[::7]], np.float32)
    r = ref[::7]
    ok = (got == r) | (np.isnan(got) & np.isnan(r))
    assert ok.all()


def test_norms_close_to_fp64():
    rng = np.random.default_rng(1)
    x = orc.f2h(rng.standard_normal((64, 768)).astype(np.float32))
    ref = np.sum(x.view(np.float16).astype(np.float64) ** 2, axis=1)
    got = orc.row_norms_f16(x)
    assert np.all(np.abs(got - ref) <= 768 * 2.0 ** -23 * ref)
    xi = orc.f2h(rng.integers(0, 256, (16, 128)).astype(np.float32))
    assert np.array_equal(orc.row_norms_f16(xi), np.sum(xi.view(np.float16).astype(np.float64) ** 2, 1))


def test_idx_mapper_invariants():
    rng = np.random.default_rng(2)
    pid = rng.integers(0, 9, 5000).astype(np.uint32)
    gi, li, off = orc.idx_mapper(pid, 9)
    assert np.array_equal(np.diff(off), np.bincount(pid, minlength=9))
    assert np.array_equal(np.sort(gi), np.arange(5000))
    for c in range(9):
        seg = gi[off[c]:off[c + 1]]
        assert np.all(np.diff(seg) > 0) and np.all(pid[seg] == c)
        assert np.array_equal(li[seg], np.arange(len(seg)))


def _cells_bruteforce(lo, hi, grid, l_q, r_q):
    a = len(grid)
    offs = np.concatenate([[0], np.cumsum(grid)[:-1]])
    out = []
    for q in range(lo.shape[0]):
        ranges = []
        for d in range(a):
            lq = l_q[offs[d]:offs[d] + grid[d]]
            rq = r_q[offs[d]:offs[d] + grid[d]]
            ranges.append([c for c in range(grid[d]) if rq[c] >= lo[q, d] and lq[c] <= hi[q, d]])
        sel = []
        for idx in np.ndindex(*grid):
            if all(idx[d] in ranges[d] for d in range(a)):
                pid = 0
                for d in range(a):
                    pid = pid * grid[d] + idx[d]
                sel.append(pid)
        out.append(sorted(sel))
    return out


def test_cells_match_box_intersection():
    rng = np.random.default_rng(3)
    att = synth.uniform_attrs(4000, 3, 4, hi=200)
    grid = np.array([3, 4, 2])
    l_q, r_q, _, gpid = synth.grid_scatter(att, grid)
    l_q = np.concatenate(l_q).astype(np.float32)
    r_q = np.concatenate(r_q).astype(np.float32)
    lo, hi = synth.ranges_for_selectivity(300, 3, rng.uniform(0.001, 0.8, 300), 5, hi=200)
    cells, cnt = orc.cells(lo, hi, grid, l_q, r_q)
    ref = _cells_bruteforce(lo, hi, grid, l_q, r_q)
    for q in range(300):
        assert list(cells[q, :cnt[q]]) == ref[q]
    # every point passing a range lies in a selected cell
    for q in range(0, 300, 7):
        ok = np.all((att >= lo[q]) & (att <= hi[q]), axis=1)
        assert set(gpid[ok].tolist()) <= set(cells[q, :cnt[q]].tolist())


def test_cells_out_of_domain_select_nothing():
    att = synth.uniform_attrs(1000, 2, 6, hi=100)
    l_q, r_q, _, _ = synth.grid_scatter(att, [4, 4])
    lo = np.array([[150, 0], [0, -50], [10, 10]], np.float32)
    hi = np.array([[160, 99], [99, -10], [20, 20]], np.float32)
    cells, cnt = orc.cells(lo, hi, np.array([4, 4]), np.concatenate(l_q).astype(np.float32),
                           np.concatenate(r_q).astype(np.float32))
    assert cnt[0] == 0 and cnt[1] == 0 and cnt[2] >= 1


def test_cells_skip_empty_cells():
    att = np.array([[0, 0], [0, 1], [9, 9], [9, 8]], np.int32)   # cells (0,1) and (1,0) stay empty
    l_q, r_q, _, gp = synth.grid_scatter(att, [2, 2])
    sizes = np.bincount(gp, minlength=4).astype(np.uint32)
    assert sizes[1] == 0 and sizes[2] == 0
    lo = np.array([[0, 0]], np.float32)
    hi = np.array([[9, 9]], np.float32)
    lq = np.concatenate(l_q).astype(np.float32)
    rq = np.concatenate(r_q).astype(np.float32)
    full, n_full = orc.cells(lo, hi, np.array([2, 2]), lq, rq)
    skip, n_skip = orc.cells(lo, hi, np.array([2, 2]), lq, rq, sizes)
    assert n_full[0] == 4 and list(skip[0, :n_skip[0]]) == [0, 3]


def test_selectivity_counts_and_threshold():
    rng = np.random.default_rng(7)
    att = rng.integers(0, 1000, (20000, 2)).astype(np.float32)
    lo, hi = synth.ranges_for_selectivity(50, 2, rng.uniform(0.001, 0.5, 50), 8, hi=1000)
    counts = np.arange(50, dtype=np.uint32) % 16 + 1
    sel, little = orc.selectivity(att, lo, hi, 0.05, counts)
    ref = np.array([np.count_nonzero(np.all((att >= lo[q]) & (att <= hi[q]), 1)) for q in range(50)])
    assert np.array_equal(sel, ref)
    prop = (ref / 20000.0).astype(np.float32)
    assert np.array_equal(little, np.where(prop <= np.float32(0.05), counts, 0))


def test_topk_clusters_and_cell_sort():
    rng = np.random.default_rng(9)
    d = rng.integers(0, 50, (40, 30)).astype(np.float32)  # many ties
    d[0, 5] = np.nan
    top = orc.topk_clusters(d, 4)
    for q in range(40):
        key = np.where(np.isnan(d[q]), np.inf, d[q])
        ref = np.lexsort((np.arange(30), key))[:4]
        assert np.array_equal(top[q], ref)
    hist = rng.integers(0, 5, (16, 30)).astype(np.uint32)
    cells = np.tile(np.arange(16, dtype=np.uint32), (40, 1))
    counts = rng.integers(1, 17, 40).astype(np.uint32)
    out = orc.sort_cells(cells, counts, top, hist)
    for q in range(40):
        cl = list(range(counts[q]))
        sc = {c: int(hist[c, top[q]].sum()) for c in cl}
        assert list(out[q, :counts[q]]) == sorted(cl, key=lambda c: (-sc[c], c))


def _glibc_rand_seed1():
    """glibc random() TYPE_3 (additive feedback, deg 31, sep 3) seeded with 1."""
    r = [0] * 34
    r[0] = 1
    for i in range(1, 31):
        hi_, lo_ = divmod(r[i - 1], 127773)
        word = 16807 * lo_ - 2836 * hi_
        if word < 0:
            word += 2147483647
        r[i] = word
    for i in range(31, 34):
        r[i] = r[i - 31]
    i = 34
    while True:
        r.append((r[i - 31] + r[i - 3]) & 0xFFFFFFFF)
        if i >= 344:
            yield r[i] >> 1
        i += 1


def _libstdcxx_draw(urange, want):
    """std::mt19937 (default seed) + uniform_int_distribution<>(0, urange - 1)
    distinct draws, then std::random_shuffle with glibc rand() after srand(1)."""
    # std::mt19937 default seed 5489 == numpy's MT19937 init_genrand(5489)
    mt = np.random.RandomState(5489)
    seen, vals = set(), []
    while len(vals) < want:
        # bounded draw by 64-bit multiply (Lemire 2019), as libstdc++ does
        # for a 32-bit engine and a range below 2^32
        prod = int(mt.randint(0, 2 ** 32, dtype=np.uint64)) * urange
        low = prod & 0xFFFFFFFF
        if low < urange:
            thr = (-urange) % urange
            while low < thr:
                prod = int(mt.randint(0, 2 ** 32, dtype=np.uint64)) * urange
                low = prod & 0xFFFFFFFF
        t = prod >> 32
        if t not in seen:
            seen.add(t)
            vals.append(t)
    rnd = _glibc_rand_seed1()
    for i in range(1, want):       # std::random_shuffle
        j = next(rnd) % (i + 1)
        vals[i], vals[j] = vals[j], vals[i]
    return vals


def test_entry_points_restate_libstdcxx_draws():
    N, P, R = 1_000_000, 16, 32
    avg = (N + P - 1) // P
    rand_max = N - (P - 1) * avg
    assert rand_max == 62500
    assert list(orc.entry_points(N, P, R)) == _libstdcxx_draw(rand_max, R * 10)[:R]


def test_entry_draw_streamed_rule():
    # out-of-core host (big_dataset_adapterV3.cuh:3862-3875): 10 L distinct
    # draws below the smallest cell; a range smaller than 10 L is exhausted
    for rng_, L, R in ((3000, 64, 16), (500, 100, 32), (40, 8, 32)):
        want = min(10 * L, rng_)
        ref = _libstdcxx_draw(rng_, want)
        ref = [ref[j] if j < want else j for j in range(R)]
        assert list(orc.entry_draw(rng_, 10 * L, R)) == ref
    # the resident rule is the same draw over N - (P - 1) ceil(N / P)
    assert np.array_equal(orc.entry_points(100000, 16, 16), orc.entry_draw(100000 - 15 * 6250, 160, 16))


def test_cells_grid_integer_brute_force():
    """Arithmetic-grid cells against exhaustive enumeration of the integer
    values in each range, the area formula against the closed form
    sum over cells = prod_d (hi_d - lo_d) / w_d for ranges inside the grid,
    and every little flag against exact rational arithmetic."""
    from fractions import Fraction
    rng = np.random.default_rng(7)
    for a, grid in ((1, [7]), (2, [4, 5]), (3, [3, 2, 4])):
        P = int(np.prod(grid))
        amin = rng.integers(-50, 50, a).astype(np.float32)
        width = rng.integers(1, 40, a).astype(np.float32)
        Q = 300
        lo = (amin + rng.integers(-60, 200, (Q, a))).astype(np.float32)
        hi = (lo + rng.integers(-5, 120, (Q, a))).astype(np.float32)   # some empty (hi < lo)
        thr = 0.3
        cells, cnt, lit, flags = orc.cells_grid(lo, hi, grid, amin, width, thr)
        for q in range(Q):
            per_dim = []
            for d in range(a):
                m, w, g = int(amin[d]), int(width[d]), grid[d]
                cellof = lambda v: min(max((v - m) // w, 0), g - 1)
                per_dim.append(sorted({cellof(v) for v in range(int(lo[q, d]), int(hi[q, d]) + 1)}))
            want = []
            if all(per_dim):
                idx = np.stack(np.meshgrid(*per_dim, indexing="ij"), -1).reshape(-1, a)
                mult = np.array([int(np.prod(grid[d + 1:])) for d in range(a)])
                want = sorted(int(x) for x in idx @ mult)
            assert cnt[q] == len(want) and list(cells[q, :cnt[q]]) == want, q
            assert np.array_equal(np.nonzero(flags[q] & 1)[0], want)
            areas = []
            for pid in want:
                rem, t = pid, []
                for d in range(a - 1, -1, -1):
                    t.append(rem % grid[d])
                    rem //= grid[d]
                t = t[::-1]
                ar = Fraction(1)
                for d in range(a):
                    m, w = int(amin[d]), int(width[d])
                    lb = max(m + t[d] * w, int(lo[q, d]))
                    rb = min(m + (t[d] + 1) * w, int(hi[q, d]))
                    ar *= Fraction(rb - lb, w)
                areas.append(ar)
                if abs(ar - Fraction(thr)) > Fraction(1, 10 ** 9):
                    assert bool(flags[q, pid] & 2) == (ar <= Fraction(thr)), (q, pid)
            assert lit[q] == int(np.count_nonzero(flags[q] & 2))
            inside = all(lo[q, d] >= amin[d] and hi[q, d] < amin[d] + grid[d] * width[d] and lo[q, d] <= hi[q, d]
                         for d in range(a))
            if inside and want:
                closed = Fraction(1)
                for d in range(a):
                    closed *= Fraction(int(hi[q, d]) - int(lo[q, d]), int(width[d]))
                assert sum(areas) == closed


def test_u8_mode_distance():
    """u8 vector mode: 16-element chunks; exact on integer queries (any
    order), within the fp32 bound of fp64 on fractional ones."""
    rng = np.random.default_rng(3)
    N, D = 200, 128
    x = rng.integers(0, 256, (N, D)).astype(np.float32)
    pid = rng.integers(0, 4, N).astype(np.uint32)
    members = synth.cell_members(pid, 4)
    graphs = np.concatenate([np.zeros((len(m), 4), np.uint32) for m in members])
    O = orc.OracleIndex(x, np.zeros((N, 1), np.float32), pid, 4, graphs, np.zeros((N, 4), np.uint32), u8=True)
    qi = rng.integers(0, 256, D).astype(np.float32)
    qf = (rng.random(D) * 255).astype(np.float32)
    for g in range(0, N, 17):
        assert O.distance(qi, g) == float(np.sum((qi.astype(np.int64) - x[g].astype(np.int64)) ** 2))
        ref = np.sum((qf.astype(np.float64) - x[g]) ** 2)
        assert abs(O.distance(qf, g) - ref) <= 1e-6 * ref + 1e-3


@pytest.fixture(scope="module")
def tiny():
    cfg = synth.config_small(N=4000, Q=120, R=16, C=12, sel=0.25, seed=31)
    ix = synth.build_index(cfg["vectors"], cfg["attrs"], cfg["grid"], 16, 2, 12, seed=2)
    l_q, r_q = synth.quantile_arrays(ix)
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    cells, cnt = orc.cells(lo, hi, ix["grid"], l_q, r_q)
    O = orc.OracleIndex(ix["vectors"], ix["attrs"], ix["global_pid"], 16, ix["cell_graphs"], ix["cross"])
    gt, gtd = orc.ground_truth(ix["vectors"], ix["attrs"], cfg["queries"], lo, hi, 10)
    return cfg, ix, lo, hi, cells, cnt, O, gt, gtd


def test_bruteforce_route_is_exact_topk(tiny):
    cfg, ix, lo, hi, cells, cnt, O, gt, gtd = tiny
    ent = orc.entry_points(4000, 16, 16)
    little = cnt.copy()
    ids, dist, ctr = O.search(cfg["queries"], lo, hi, cells, cnt, little, ent, 32)
    assert orc.recall(ids, gt, gtd) == 1.0
    assert np.all(ctr[:, 7] == 2)
    # distances are the exact squared distances (integer data: fp32 is exact)
    for q in range(0, 120, 11):
        for j in range(10):
            if ids[q, j] != orc.SENTINEL:
                ref = np.sum((cfg["queries"][q].astype(np.float64) - ix["vectors"][ids[q, j]]) ** 2)
                assert dist[q, j] == ref == gtd[q, j]


def test_traversal_invariants_and_recall(tiny):
    cfg, ix, lo, hi, cells, cnt, O, gt, gtd = tiny
    ent = orc.entry_points(4000, 16, 16)
    little = np.zeros_like(cnt)
    recs = []
    for L in (10, 40, 160):
        ids, dist, ctr = O.search(cfg["queries"], lo, hi, cells, cnt, little, ent, L)
        recs.append(orc.recall(ids, gt, gtd))
        for q in range(120):
            row = ids[q][ids[q] != orc.SENTINEL]
            assert len(set(row.tolist())) == len(row)                     # unique
            assert np.all(np.diff(dist[q][:len(row)]) >= 0)                # ascending
            if len(row):
                a = ix["attrs"][row]
                assert np.all((a >= lo[q]) & (a <= hi[q]))                 # filter
            for j, i in enumerate(row):
                assert dist[q, j] == np.sum((cfg["queries"][q].astype(np.float64) - ix["vectors"][i]) ** 2)
        assert np.all(ctr[:, 0] > 0)
    assert recs[0] < recs[1] < recs[2] and recs[2] > 0.85


def test_traversal_deterministic_across_threads(tiny):
    cfg, ix, lo, hi, cells, cnt, O, gt, gtd = tiny
    ent = orc.entry_points(4000, 16, 16)
    z = np.zeros_like(cnt)
    a = O.search(cfg["queries"], lo, hi, cells, cnt, z, ent, 64, nthreads=1)
    b = O.search(cfg["queries"], lo, hi, cells, cnt, z, ent, 64, nthreads=8)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_postfilter_and_empty_routes(tiny):
    """Queries with postfilter or more cells: without a full graph no result
    (the reference's full-graph branch is disabled and its brute force covers
    no cell); with one, the full-graph search: filtered, ascending, distinct,
    exact distances, and a recall that grows with L."""
    cfg, ix, lo, hi, cells, cnt, O, gt, gtd = tiny
    ent = orc.entry_points(4000, 16, 16)
    z = np.zeros_like(cnt)
    pf = int(np.median(cnt))
    O0 = orc.OracleIndex(ix["vectors"], ix["attrs"], ix["global_pid"], 16, ix["cell_graphs"], ix["cross"],
                         full=False)
    ids, dist, ctr = O0.search(cfg["queries"], lo, hi, cells, cnt, z, ent, 32, postfilter=pf)
    routed = cnt >= pf
    assert routed.any() and (~routed).any()
    assert np.all(ids[routed] == orc.SENTINEL) and np.all(ctr[routed, 7] == 0)
    assert np.all(ctr[~routed, 7] == 1)
    assert O.FD == 2 * 16
    recs = []
    for L in (16, 64, 256):
        ids, dist, ctr = O.search(cfg["queries"], lo, hi, cells, cnt, z, ent, L, postfilter=pf)
        assert np.all(ctr[routed, 7] == 3) and np.all(ctr[~routed, 7] == 1)
        assert np.all(ctr[routed, 3] == 0) and np.all(ctr[routed, 0] > 0)
        for q in np.nonzero(routed)[0]:
            row = ids[q][ids[q] != orc.SENTINEL]
            assert len(set(row.tolist())) == len(row)
            assert np.all(np.diff(dist[q][:len(row)]) >= 0)
            if len(row):
                a = ix["attrs"][row]
                assert np.all((a >= lo[q]) & (a <= hi[q]))
            for j, i in enumerate(row):
                assert dist[q, j] == np.sum((cfg["queries"][q].astype(np.float64) - ix["vectors"][i]) ** 2)
        recs.append(orc.recall(ids[routed], gt[routed], gtd[routed]))
    assert recs[0] < recs[2] and recs[2] > 0.5, recs


def test_centres_hist_closed_form():
    """Centres = sequential fp32 sums per label / count (np.add.at sums in index
    order); histogram = label counts per cell, by grid cell or by i / ceil(N/P)."""
    rng = np.random.default_rng(5)
    N, D, C, P = 3000, 24, 7, 16
    x = rng.standard_normal((N, D)).astype(np.float32) * 10
    lab = rng.integers(0, C, N).astype(np.int32)
    pid = rng.integers(0, P, N).astype(np.uint32)
    cen, hist = orc.centres_hist(x, lab, pid, P)
    s = np.zeros((C, D), np.float32)
    np.add.at(s, lab, x)
    cnt = np.bincount(lab, minlength=C).astype(np.float32)
    assert np.array_equal(cen, s / cnt[:, None])
    h = np.zeros((P, C), np.uint32)
    np.add.at(h, (pid, lab), 1)
    assert np.array_equal(hist, h)
    _, hc = orc.centres_hist(x, lab, pid, P, contiguous=True)
    avg = -(-N // P)
    h2 = np.zeros((P, C), np.uint32)
    np.add.at(h2, (np.minimum(np.arange(N) // avg, P - 1), lab), 1)
    assert np.array_equal(hc, h2)


def test_ground_truth_brute_force():
    """Exact filtered kNN: fp64 distances, ties by ascending id, sentinel padding."""
    rng = np.random.default_rng(6)
    N, D, a, Q, K = 700, 16, 2, 40, 10
    x = rng.integers(0, 4, (N, D)).astype(np.float32)        # many distance ties
    att = rng.integers(0, 50, (N, a)).astype(np.float32)
    q = rng.integers(0, 4, (Q, D)).astype(np.float32)
    lo = rng.integers(0, 40, (Q, a)).astype(np.float32)
    hi = lo + rng.integers(0, 12, (Q, a)).astype(np.float32)
    ids, dist = orc.ground_truth(x, att, q, lo, hi, K)
    for i in range(Q):
        ok = np.all((att >= lo[i]) & (att <= hi[i]), axis=1)
        cand = np.nonzero(ok)[0]
        d = np.sum((x[cand].astype(np.float64) - q[i]) ** 2, axis=1)
        order = np.lexsort((cand, d))[:K]
        n = len(order)
        assert np.array_equal(ids[i, :n], cand[order])
        assert np.array_equal(dist[i, :n], d[order])
        assert np.all(ids[i, n:] == orc.SENTINEL) and np.all(np.isinf(dist[i, n:]))


def test_recall_known_answers():
    gt = np.array([[1, 2, 3], [4, 5, 6]], np.uint32)
    gtd = np.array([[1.0, 2.0, 3.0], [1.0, 1.0, 1.0]])
    res = np.array([[3, 2, 9], [6, 7, 8]], np.uint32)
    assert orc.recall(res, gt, gtd) == pytest.approx((2 / 3 + 1 / 3) / 2)
    # tie-aware: id 9 at distance 3.0 (= the 3rd ground-truth distance) counts
    rd = np.array([[3.0, 2.0, 3.0], [1.0, 5.0, 1.0]])
    assert orc.recall(res, gt, gtd, rd, tie_aware=True) == pytest.approx((1.0 + 2 / 3) / 2)
    # an empty ground truth counts as recall 1
    e = np.full((1, 3), orc.SENTINEL, np.uint32)
    assert orc.recall(e, e, np.full((1, 3), np.inf)) == 1.0
