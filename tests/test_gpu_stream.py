"""Streamed (out-of-core) search, the arithmetic-grid stage A and the uint8
vector mode, through the C ABI, against the CPU oracle.

The streamed search is checked bit-exactly (ids, fp32 distances, counters)
against the oracle run batch by batch: for each batch of the plan the
oracle searches the batch's selected cells in plan order (the batch's cells
renumbered to come first, so its tie order is the batch's row order), and
the per-batch top K are merged with the batch's entry first at equal
distance.  With one batch holding every cell it must equal the resident
search on the same cell lists and entry points.
"""
import numpy as np
import pytest

from garfield_amd import synth
import garfield_amd._lib as gl

pytestmark = pytest.mark.gpu

GRID = [4, 4]
AMIN = np.zeros(2, np.float32)
WIDTH = np.full(2, 2500.0, np.float32)


def _print_case(name, **kw):
    print(f"[case] {name} " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.fixture(scope="module")
def world_stream():
    N, D, Q = 24000, 64, 200
    rng = np.random.default_rng(41)
    vec = synth.uniform_int_vectors(N, D, 42)
    att = rng.integers(0, 10000, (N, 2)).astype(np.int32)
    queries = synth.uniform_int_vectors(Q, D, 43)
    sel = synth.log_uniform(Q, 0.02, 0.3, 44)
    lo, hi = synth.ranges_for_selectivity(Q, 2, sel, 45)
    lo[0] = [20000, 20000]          # beyond the grid: the last cell
    hi[0] = [30000, 30000]
    lo[1] = [5000, 100]             # empty on attribute 0
    hi[1] = [4000, 9000]
    lo[2] = [0, 0]                  # everything
    hi[2] = [9999, 9999]
    ix = synth.build_index(vec, att, GRID, 16, 2, 0, arith=(AMIN, WIDTH))
    cfg = dict(queries=queries, lo=lo.astype(np.float32), hi=hi.astype(np.float32))
    return cfg, ix


def _args(ix):
    l_q, r_q = synth.quantile_arrays(ix)
    return (ix["vectors"], ix["attrs"], ix["grid"], l_q, r_q, ix["global_pid"], ix["cell_graphs"], ix["cross"])


def _oracle_stream(ix, plan, cfg, flags, ent, L, K=10, rl=10, mfma=False):
    """Per-batch oracle searches merged into a running top K (see module doc).
    mfma: the brute force ran on MFMA, which evaluates every scanned point
    (its DIST counter is the SCAN counter) and, on a streamed batch, does not
    count passing points (PASS = 0)."""
    from oracle import oracle as orc
    P, E, N = ix["P"], ix["E"], ix["vectors"].shape[0]
    sizes = synth.cell_sizes(ix)
    goff = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    Q = cfg["queries"].shape[0]
    run_ids = run_d = run_c = None
    for batch in plan:
        order = list(batch) + [c for c in range(P) if c not in batch]
        new_of = np.empty(P, np.int64)
        new_of[order] = np.arange(P)
        graphs = np.concatenate([ix["cell_graphs"][goff[c]:goff[c + 1]] for c in order])
        cross = ix["cross"].reshape(N, P, E)[:, order, :].reshape(N, P * E)
        O = orc.OracleIndex(ix["vectors"], ix["attrs"], new_of[ix["global_pid"]].astype(np.uint32), P, graphs,
                            cross, u8=True)
        cells = np.zeros((Q, P), np.uint32)
        cnt = np.zeros(Q, np.uint32)
        lit = np.zeros(Q, np.uint32)
        for q in range(Q):
            mine = [i for i, c in enumerate(batch) if flags[q, c] & 1]
            cells[q, :len(mine)] = mine
            cnt[q] = len(mine)
            lit[q] = len(mine) if mine and all(flags[q, batch[i]] & 2 for i in mine) else 0
        ids, d, c = O.search(cfg["queries"], cfg["lo"], cfg["hi"], cells, cnt, lit, ent, L, K=K, rl=rl)
        c = c.copy()
        if mfma:
            c[c[:, 7] == 2, 1] = c[c[:, 7] == 2, 5]
            c[c[:, 7] == 2, 6] = 0     # the streamed MFMA route does not count passing points
        c[:, 7] = np.where(c[:, 7] == 1, 1, np.where(c[:, 7] == 2, 1 << 16, 0))
        if run_ids is None:
            run_ids, run_d, run_c = ids.copy(), d.copy(), c.astype(np.int64)
            continue
        for q in range(Q):
            oi, od = run_ids[q].copy(), run_d[q].copy()
            i = j = 0
            for t in range(K):
                if od[i] < d[q, j]:
                    run_ids[q, t], run_d[q, t] = oi[i], od[i]
                    i += 1
                else:
                    run_ids[q, t], run_d[q, t] = ids[q, j], d[q, j]
                    j += 1
        run_c += c
    return run_ids, run_d, run_c


def _shuffled_plan(P, per, seed):
    cells = np.random.default_rng(seed).permutation(P)
    return [[int(c) for c in cells[i:i + per]] for i in range(0, P, per)]


def test_cells_grid_matches_oracle(world_stream):
    from oracle import oracle as orc
    cfg, ix = world_stream
    _print_case("cells-grid")
    sizes = synth.cell_sizes(ix)
    dev = gl.Index.from_arrays(*_args(ix), vec_dtype=gl.VEC_U8)
    sdev = gl.Index.create_streamed(*_args(ix), batch_cells=4)
    for thr in (0.0, 0.05, 0.5, 2.0):
        oc, on, ol, of = orc.cells_grid(cfg["lo"], cfg["hi"], GRID, AMIN, WIDTH, thr, sizes)
        for d in (dev, sdev):
            b = d.batch(cfg["queries"], cfg["lo"], cfg["hi"])
            b.mark_cells_grid(AMIN, WIDTH, thr)
            c, n, l, _ = b.get_cells()
            assert np.array_equal(n, on) and np.array_equal(l, ol)
            for q in range(len(n)):
                assert np.array_equal(c[q, :n[q]], oc[q, :on[q]]), q
            assert np.array_equal(b.get_cell_flags(), of)
            b.close()
    assert on[0] == 1 and oc[0, 0] == 15 and on[1] == 0 and on[2] == 16
    sdev.close()
    dev.close()


@pytest.mark.parametrize("L", [32, 100])
def test_u8_resident_traversal_parity(world_stream, L):
    import garfield_amd as gf
    from oracle import oracle as orc
    cfg, ix = world_stream
    _print_case("u8-traverse", L=L)
    dev = gl.Index.from_arrays(*_args(ix), vec_dtype=gl.VEC_U8)
    assert dev.vec_dtype == gl.VEC_U8
    b = dev.batch(cfg["queries"], cfg["lo"], cfg["hi"])
    b.mark_cells_grid(AMIN, WIDTH, 0.0)
    gc, gn, gl_, _ = b.get_cells()
    ent = gf.entry_points(ix["vectors"].shape[0], ix["P"], ix["R"])
    ids, dists, st = b.search(L=L, K=10, rl=10, entry_points=ent)
    ctr = b.get_counters()
    O = orc.OracleIndex(ix["vectors"], ix["attrs"], ix["global_pid"], ix["P"], ix["cell_graphs"], ix["cross"],
                        u8=True)
    oids, od, oc = O.search(cfg["queries"], cfg["lo"], cfg["hi"], gc, gn, gl_, ent, L)
    assert np.array_equal(ids, oids)
    assert np.array_equal(dists.view(np.uint32), od.view(np.uint32))
    if st.bf_mfma:
        # the MFMA brute force evaluates every scanned point, the oracle only the passing ones
        rows = oc[:, 7] == 2
        oc[rows, 1] = oc[rows, 5]
    assert np.array_equal(ctr, oc)
    b.close()
    dev.close()


def test_u8_resident_gather_bruteforce(world_stream):
    """K = 20 (above the MFMA route's 16): the gather brute force on u8 rows."""
    import garfield_amd as gf
    from oracle import oracle as orc
    cfg, ix = world_stream
    _print_case("u8-bruteforce")
    dev = gl.Index.from_arrays(*_args(ix), vec_dtype=gl.VEC_U8)
    b = dev.batch(cfg["queries"], cfg["lo"], cfg["hi"])
    b.mark_cells_grid(AMIN, WIDTH, 0.0)
    gc, gn, _, _ = b.get_cells()
    b.set_cells(gc, gn, gn)     # every query on the brute-force route
    ent = gf.entry_points(ix["vectors"].shape[0], ix["P"], ix["R"])
    ids, dists, st = b.search(L=32, K=20, rl=10, entry_points=ent)
    assert st.bf_mfma == 0
    O = orc.OracleIndex(ix["vectors"], ix["attrs"], ix["global_pid"], ix["P"], ix["cell_graphs"], ix["cross"],
                        u8=True)
    oids, od, oc = O.search(cfg["queries"], cfg["lo"], cfg["hi"], gc, gn, gn, ent, 32, K=20)
    assert np.array_equal(ids, oids)
    assert np.array_equal(dists.view(np.uint32), od.view(np.uint32))
    assert np.array_equal(b.get_counters(), oc)
    b.close()
    dev.close()


def test_stream_one_batch_equals_resident(world_stream):
    import garfield_amd as gf
    cfg, ix = world_stream
    _print_case("stream-one-batch")
    P = ix["P"]
    res = gl.Index.from_arrays(*_args(ix), vec_dtype=gl.VEC_U8)
    sx = gl.Index.create_streamed(*_args(ix), plan=[list(range(P))])
    ent = gf.entry_points(ix["vectors"].shape[0], P, ix["R"])
    out = []
    for d in (res, sx):
        b = d.batch(cfg["queries"], cfg["lo"], cfg["hi"])
        b.mark_cells_grid(AMIN, WIDTH, 0.02)
        c, n, l, _ = b.get_cells()
        l = np.where(np.arange(len(n)) % 3 == 0, n, 0).astype(np.uint32)   # every third query: brute force
        b.set_cells(c, n, l)
        ids, dists, st = b.search(L=64, K=10, rl=10, entry_points=ent)
        out.append((ids, dists, b.get_counters(), l, n))
        b.close()
    (i0, d0, c0, l0, n0), (i1, d1, c1, _, _) = out
    assert np.array_equal(i0, i1)
    assert np.array_equal(d0.view(np.uint32), d1.view(np.uint32))
    trav = (l0 == 0) & (n0 > 0)
    assert trav.any() and (l0 > 0).any()
    assert np.array_equal(c0[trav, :7], c1[trav, :7]) and np.all(c1[trav, 7] == 1)
    assert np.all(c1[l0 > 0, 7] == 1 << 16)
    sx.close()
    res.close()


@pytest.mark.parametrize("L,thr,per,K", [(16, 0.02, 4, 10), (64, 0.1, 3, 10), (100, 0.0, 16, 10),
                                         (32, 0.1, 4, 20), (48, 1.0, 5, 10), (48, 1.0, 5, 20)])
def test_stream_batches_match_oracle(world_stream, L, thr, per, K):
    from oracle import oracle as orc
    cfg, ix = world_stream
    _print_case("stream-batches", L=L, thr=thr, per=per, K=K)
    P = ix["P"]
    plan = _shuffled_plan(P, per, seed=L)
    import garfield_amd as gf
    sx = gl.Index.create_streamed(*_args(ix), plan=plan)
    assert sx.streamed and sx.nbatch == len(plan)
    b = sx.batch(cfg["queries"], cfg["lo"], cfg["hi"])
    gf.intersection_area_mark_little_seg_batch_process(b, AMIN, WIDTH, thr)
    flags = b.get_cell_flags()
    ids, dists, st = gf.batch_graph_search_gpu_with_prefilter_batch_process_compressed_graph_T_dataset_resident_u8(
        b, L, K=K)
    ctr = b.get_counters()
    assert 0 < st.n_batches <= len(plan) and st.bytes_h2d > 0
    assert st.bf_mfma == (K <= 16)
    sizes = synth.cell_sizes(ix)
    ent = orc.entry_draw(int(sizes[sizes > 0].min()), 10 * L, ix["R"])
    oids, od, oc = _oracle_stream(ix, plan, cfg, flags, ent, L, K=K, mfma=bool(st.bf_mfma))
    bad = np.nonzero(np.any(ids != oids, axis=1))[0]
    assert bad.size == 0, f"{bad.size} queries differ, first {bad[:5]}: {ids[bad[0]]} vs {oids[bad[0]]}"
    assert np.array_equal(dists.view(np.uint32), od.view(np.uint32))
    assert np.array_equal(ctr.astype(np.int64), oc)
    # a second search on the same batch (state reuse), smaller L
    ids2, _, _ = b.search(L=max(8, L // 2), K=K, rl=10)
    ent2 = orc.entry_draw(int(sizes[sizes > 0].min()), 10 * max(8, L // 2), ix["R"])
    oids2, _, _ = _oracle_stream(ix, plan, cfg, flags, ent2, max(8, L // 2), K=K)
    assert np.array_equal(ids2, oids2)
    b.close()
    sx.close()


def test_stream_under_device_budget(world_stream):
    """A budget below half the resident index: the streamed index fits it and
    still returns the resident brute-force results (recall 1 on the exact
    route), with its device memory within the budget."""
    cfg, ix = world_stream
    _print_case("stream-budget")
    P = ix["P"]
    res = gl.Index.from_arrays(*_args(ix), vec_dtype=gl.VEC_U8)
    budget = res.device_bytes // 2
    sx = gl.Index.create_streamed(*_args(ix), plan=_shuffled_plan(P, 2, seed=9), device_budget=budget)
    assert sx.device_bytes <= budget
    out = []
    for d in (res, sx):
        b = d.batch(cfg["queries"], cfg["lo"], cfg["hi"])
        b.mark_cells_grid(AMIN, WIDTH, 10.0)       # every cell little: exact brute force
        ids, dists, st = b.search(L=32, K=10, rl=10)
        out.append((ids, dists))
        b.close()
    (i0, d0), (i1, d1) = out
    assert np.array_equal(d0.view(np.uint32), d1.view(np.uint32))
    # ids agree wherever the distance is not tied (batches merge ties in plan order)
    for q in range(i0.shape[0]):
        vals, cnt = np.unique(d0[q], return_counts=True)
        single = np.isin(d0[q], vals[cnt == 1]) & (d0[q] != d0[q, -1])
        assert np.array_equal(i0[q, single], i1[q, single]), q
    sx.close()
    res.close()


def test_stream_bruteforce_overflow_rerun():
    """One cell of 80000 points (81 sub-cells) and full-range queries: the
    brute-force pairs outgrow the initial buffers (64 per query), the
    streamed search grows them and runs the brute force again; results are
    the exact filtered top K (resident path and CPU ground truth)."""
    from oracle import oracle as orc
    _print_case("stream-overflow")
    rng = np.random.default_rng(77)
    N, D, Q, R = 80000, 64, 64, 8
    vec = rng.integers(0, 256, (N, D)).astype(np.float32)
    att = rng.integers(0, 10000, (N, 2)).astype(np.float32)
    graphs = rng.integers(0, N, (N, R)).astype(np.uint32)     # any graph: every query takes brute force
    cross = rng.integers(0, N, (N, 2)).astype(np.uint32)
    args = (vec, att, np.array([1, 1], np.uint32), np.array([0, 0], np.float32),
            np.array([9999, 9999], np.float32), np.zeros(N, np.uint32), graphs, cross)
    queries = rng.integers(0, 256, (Q, D)).astype(np.float32)
    lo = np.zeros((Q, 2), np.float32)
    hi = np.full((Q, 2), 9999.0, np.float32)
    lo[::3, 0] = 5000.0                                       # some narrower ranges too
    gt, gtd = orc.ground_truth(vec, att, queries, lo, hi, 10)
    out = []
    for make in (lambda: gl.Index.from_arrays(*args, vec_dtype=gl.VEC_U8),
                 lambda: gl.Index.create_streamed(*args, plan=[[0]])):
        dev = make()
        b = dev.batch(queries, lo, hi)
        b.set_cells(np.zeros((Q, 1), np.uint32), np.ones(Q, np.uint32), np.ones(Q, np.uint32))
        ids, dists, st = b.search(L=16, K=10, rl=10)
        assert st.bf_mfma == 1
        out.append((ids, dists))
        b.close()
        dev.close()
    for ids, dists in out:
        assert np.array_equal(dists, gtd.astype(np.float32))
    assert np.array_equal(out[0][0], out[1][0])


def test_c5_shaped_stream_matches_oracle():
    """Config 5's own shape at 100k points: 128-d u8 vectors uniform in
    [0, 255], 2 uniform attributes in [0, 10000) on a 16x16 arithmetic grid
    (256 cells), R = 32 exact per-cell graphs and E = 2 cross edges (built by
    the library's int8 MFMA builder, which test_gpu_build pins bit for bit),
    queries with selectivity log-U[0.5 %, 20 %], the reference's plan of 16
    consecutive cells per batch (bigdataset_experiment.cu:271-277), streamed
    under a device budget below half the resident index.  Ids, distances and
    counters against the oracle run batch by batch; the same routes mixed as
    the out-of-core driver's little-cell threshold gives them."""
    import garfield_amd as gf
    from oracle import oracle as orc
    N, D, Q, L = 100_000, 128, 160, 48
    grid = [16, 16]
    amin = np.zeros(2, np.float32)
    width = np.full(2, 625.0, np.float32)
    _print_case("c5-shaped", N=N, P=256, R=32)
    vec = synth.uniform_int_vectors(N, D, 501).astype(np.uint8)
    att = np.random.default_rng(502).integers(0, 10000, (N, 2)).astype(np.int32)
    queries = synth.uniform_int_vectors(Q, D, 503).astype(np.float32)
    sel = synth.log_uniform(Q, 0.005, 0.2, 504)
    lo, hi = synth.ranges_for_selectivity(Q, 2, sel, 505)
    ix = synth.build_index(vec, att, grid, 32, 2, 0, device="hip", arith=(amin, width))
    ix["vectors"] = vec.astype(np.float32)
    cfg = dict(queries=queries, lo=lo.astype(np.float32), hi=hi.astype(np.float32))
    res = gl.Index.from_arrays(*_args(ix), vec_dtype=gl.VEC_U8)
    budget = res.device_bytes // 2
    res.close()
    sx = gl.Index.create_streamed(*_args(ix), batch_cells=16, device_budget=budget)
    assert sx.streamed and sx.nbatch == 16 and sx.device_bytes <= budget
    b = sx.batch(cfg["queries"], cfg["lo"], cfg["hi"])
    b.mark_cells_grid(amin, width, 0.3)
    flags = b.get_cell_flags()
    ids, dists, st = b.search(L=L, K=10, rl=10)
    ctr = b.get_counters()
    assert st.q_traverse > 0 and st.q_bruteforce > 0
    sizes = synth.cell_sizes(ix)
    ent = orc.entry_draw(int(sizes[sizes > 0].min()), 10 * L, ix["R"])
    plan = [list(range(16 * i, 16 * i + 16)) for i in range(16)]
    oids, od, oc = _oracle_stream(ix, plan, cfg, flags, ent, L, mfma=bool(st.bf_mfma))
    bad = np.nonzero(np.any(ids != oids, axis=1))[0]
    assert bad.size == 0, f"{bad.size} queries differ, first {bad[:5]}"
    assert np.array_equal(dists.view(np.uint32), od.view(np.uint32))
    assert np.array_equal(ctr.astype(np.int64), oc)
    b.close()
    sx.close()


@pytest.mark.parametrize("thr,L", [(0.05, 48), (1.0, 32)])
def test_planned_stream_matches_oracle(world_stream, thr, L):
    """A plan made by gf_stream_plan_cells from the batch's own stage A cell
    lists (at most 4 cells per batch): the streamed search over it is
    bit-exact against the oracle run batch by batch, and the search's count
    of active (query, batch) pairs is the planner's objective, at most the
    static 2x2-block plan's (a partition the planner also considers)."""
    from oracle import oracle as orc
    cfg, ix = world_stream
    _print_case("stream-planned", thr=thr, L=L)
    P = ix["P"]
    sizes = synth.cell_sizes(ix)
    active = {}
    plans = {"block": synth.block_plan(GRID, 2)}
    probe = gl.Index.create_streamed(*_args(ix), plan=plans["block"])
    b = probe.batch(cfg["queries"], cfg["lo"], cfg["hi"])
    b.mark_cells_grid(AMIN, WIDTH, thr)
    c, n, _, _ = b.get_cells()
    plans["planned"], active["planned"] = gl.plan_cells(c, n, GRID, sizes, max_cells=4)
    _, _, st = b.search(L=L, K=10, rl=10)
    active["block"] = st.n_active
    b.close()
    probe.close()
    assert sorted(x for bt in plans["planned"] for x in bt) == [x for x in range(P) if sizes[x]]
    assert all(len(bt) <= 4 for bt in plans["planned"])
    assert active["planned"] <= active["block"], active
    sx = gl.Index.create_streamed(*_args(ix), plan=plans["planned"])
    b = sx.batch(cfg["queries"], cfg["lo"], cfg["hi"])
    b.mark_cells_grid(AMIN, WIDTH, thr)
    flags = b.get_cell_flags()
    ids, dists, st = b.search(L=L, K=10, rl=10)
    ctr = b.get_counters()
    assert st.n_active == active["planned"]
    ent = orc.entry_draw(int(sizes[sizes > 0].min()), 10 * L, ix["R"])
    oids, od, oc = _oracle_stream(ix, plans["planned"], cfg, flags, ent, L, mfma=bool(st.bf_mfma))
    bad = np.nonzero(np.any(ids != oids, axis=1))[0]
    assert bad.size == 0, f"{bad.size} queries differ, first {bad[:5]}"
    assert np.array_equal(dists.view(np.uint32), od.view(np.uint32))
    assert np.array_equal(ctr.astype(np.int64), oc)
    b.close()
    sx.close()


@pytest.mark.parametrize("thr,L,K", [(0.05, 48, 10), (1.0, 32, 10), (0.1, 32, 20)])
def test_plans_on_one_index(world_stream, thr, L, K):
    """One streamed index, four plans in turn on one query batch, with no
    re-pack: the build-time plan (shuffled, 4 cells per batch), the plan
    gf_batch_plan_stream makes from the batch's own cell lists, an explicit
    plan with a batch of 10 cells (larger than any build-time batch: the
    device buffers grow), and the build-time plan again.  Each search is
    bit-exact (ids, distances, counters) against the oracle run batch by
    batch over that plan; the planned plan's active (query, batch) pairs, as
    the planner counts them, are the search's."""
    import garfield_amd as gf
    from oracle import oracle as orc
    cfg, ix = world_stream
    _print_case("plans-one-index", thr=thr, L=L, K=K)
    P = ix["P"]
    plan0 = _shuffled_plan(P, 4, seed=3)
    sx = gl.Index.create_streamed(*_args(ix), plan=plan0)
    bytes0 = sx.device_bytes
    b = sx.batch(cfg["queries"], cfg["lo"], cfg["hi"])
    gf.intersection_area_mark_little_seg_batch_process(b, AMIN, WIDTH, thr)
    flags = b.get_cell_flags()
    sizes = synth.cell_sizes(ix)
    ent = orc.entry_draw(int(sizes[sizes > 0].min()), 10 * L, ix["R"])
    assert b.stream_plan() == plan0

    def check(plan, tag):
        ids, dists, st = b.search(L=L, K=K, rl=10)
        ctr = b.get_counters()
        assert st.bf_mfma == (K <= 16)
        oids, od, oc = _oracle_stream(ix, plan, cfg, flags, ent, L, K=K, mfma=bool(st.bf_mfma))
        bad = np.nonzero(np.any(ids != oids, axis=1))[0]
        assert bad.size == 0, f"{tag}: {bad.size} queries differ, first {bad[:5]}"
        assert np.array_equal(dists.view(np.uint32), od.view(np.uint32)), tag
        assert np.array_equal(ctr.astype(np.int64), oc), tag
        return ids, dists, st

    r0 = check(plan0, "build-time")
    planned, active, ms = b.plan_stream(max_cells=4)
    assert ms > 0 and b.stream_plan() == planned
    assert sorted(c for bt in planned for c in bt) == [c for c in range(P) if sizes[c]]
    assert all(len(bt) <= 4 for bt in planned)
    _, _, st = check(planned, "planned")
    assert st.n_active == active
    big = [[0, 1, 2, 5], [3, 4], [6, 7, 8, 9, 10, 11, 12, 13, 14, 15]]
    b.set_stream_plan(big)
    assert b.stream_plan() == big
    check(big, "explicit")
    assert sx.device_bytes > bytes0      # the turn buffers grew for the 10-cell batch
    b.set_stream_plan(None)
    assert b.stream_plan() == plan0
    r3 = check(plan0, "build-time again")
    assert np.array_equal(r0[0], r3[0])
    b.close()
    sx.close()


def test_plan_over_budget_refused(world_stream):
    """A plan whose largest batch does not fit the index's device budget is
    refused (GF_E_UNSUPPORTED) and the batch keeps its previous plan."""
    cfg, ix = world_stream
    _print_case("plan-over-budget")
    P = ix["P"]
    plan0 = _shuffled_plan(P, 2, seed=9)
    probe = gl.Index.create_streamed(*_args(ix), plan=plan0)
    budget = probe.device_bytes + 4096
    probe.close()
    sx = gl.Index.create_streamed(*_args(ix), plan=plan0, device_budget=budget)
    b = sx.batch(cfg["queries"], cfg["lo"], cfg["hi"])
    b.mark_cells_grid(AMIN, WIDTH, 0.05)
    with pytest.raises(gl.GarfieldError) as e:
        b.set_stream_plan([list(range(P))])
    assert e.value.status == 6
    assert b.stream_plan() == plan0
    with pytest.raises(gl.GarfieldError):
        b.plan_stream(max_cells=16)          # one batch of every cell: over the budget
    ids, _, st = b.search(L=32, K=10, rl=10)
    assert st.n_batches > 0 and sx.device_bytes <= budget
    b.close()
    sx.close()
