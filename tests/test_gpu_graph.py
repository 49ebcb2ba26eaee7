"""The resident query path's stages replayed as HIP graphs give the eager bits.

A batch's second and later searches run the stage (schedule, traversal,
brute force, merges, statistics, result copies) as one captured graph, and
the second and later stage A and B calls with the same arguments replay
theirs.  Each case runs the stages once eagerly (GARFIELD_NO_GRAPH=1), then
replays them several times with other eager work on the stream in between
(reading the cells back, exact selectivity counts), and compares every
replay's cells, ids, distances and counters with the eager run; a change of
options recaptures.
"""
import numpy as np
import pytest

from garfield_amd import synth

pytestmark = pytest.mark.gpu


def _print_case(name, **kw):
    print(f"[case] {name} " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _replays(monkeypatch, cfg, ix, prefilter, Ls, reps=3, **dev_kw):
    dev = synth.open_device_index(ix, **dev_kw)
    b = dev.batch(cfg["queries"], cfg["lo"].astype(np.float32), cfg["hi"].astype(np.float32))
    b.mark_cells(prefilter)
    if ix["labels"] is not None:
        b.order_cells(4)
    try:
        for L in Ls:
            monkeypatch.setenv("GARFIELD_NO_GRAPH", "1")
            ids0, d0, st0 = b.search(L=L, K=10, rl=10)
            c0 = b.get_counters()
            assert (st0.graph & 1) == 0
            monkeypatch.delenv("GARFIELD_NO_GRAPH")
            for r in range(reps):
                ids, d, st = b.search(L=L, K=10, rl=10)
                c = b.get_counters()
                assert st.graph & 1, f"L={L} run {r}: the search did not run as a graph"
                assert np.array_equal(ids, ids0), f"L={L} replay {r}: ids differ"
                assert np.array_equal(d.view(np.uint32), d0.view(np.uint32)), f"L={L} replay {r}: distances differ"
                assert np.array_equal(c, c0), f"L={L} replay {r}: counters differ"
                assert (st.q_traverse, st.q_bruteforce, st.q_empty) == (st0.q_traverse, st0.q_bruteforce,
                                                                         st0.q_empty)
                # eager work on the stream between replays
                b.mark_cells(prefilter)
                if ix["labels"] is not None:
                    b.order_cells(4)
                b.get_cells()
    finally:
        b.close()
        dev.close()


@pytest.mark.parametrize("prefilter", [1.0, 0.05])
def test_graph_replay_mfma_bruteforce(monkeypatch, world_sub2, prefilter):
    """Integer data: the MFMA brute force with its three launches and merges
    (prefilter 1), or mixed with traversal (0.05)."""
    cfg, ix = world_sub2
    _print_case("graph-mfma", prefilter=prefilter)
    _replays(monkeypatch, cfg, ix, prefilter, [32, 48])


def test_graph_replay_traversal(monkeypatch, world32):
    """Traversal only (prefilter 0), two L values (the second recaptures)."""
    cfg, ix = world32
    _print_case("graph-traverse")
    _replays(monkeypatch, cfg, ix, 0.0, [40, 100])


def test_graph_replay_gather_bruteforce(monkeypatch, world_gauss):
    """Non-integer data: the gather brute force and traversal mixed."""
    cfg, ix = world_gauss
    _print_case("graph-gather")
    _replays(monkeypatch, cfg, ix, 0.05, [32])


def test_graph_replay_into_page_locked_arrays(monkeypatch, world_sub2):
    """Result arrays in page-locked memory receive the device copies
    directly (no staging); every replay gives the eager bits, and a switch
    between pageable and page-locked arrays recaptures."""
    from garfield_amd import pinned_empty
    cfg, ix = world_sub2
    _print_case("graph-pinned-out")
    dev = synth.open_device_index(ix)
    b = dev.batch(cfg["queries"], cfg["lo"].astype(np.float32), cfg["hi"].astype(np.float32))
    Q = cfg["queries"].shape[0]
    pinned = (pinned_empty((Q, 10), np.uint32), pinned_empty((Q, 10), np.float32))
    try:
        b.mark_cells(1.0)
        monkeypatch.setenv("GARFIELD_NO_GRAPH", "1")
        ids0, d0, _ = b.search(L=32, K=10, rl=10)
        monkeypatch.delenv("GARFIELD_NO_GRAPH")
        for r in range(4):
            out = pinned if r % 2 == 0 else None
            if out is not None:
                # a replay must overwrite every entry of the caller's arrays
                out[0].fill(0xFFFFFFFF)
                out[1].fill(np.nan)
            ids, d, st = b.search(L=32, K=10, rl=10, out=out)
            assert st.graph & 1
            assert np.array_equal(ids, ids0), f"run {r}: ids differ"
            assert np.array_equal(d.view(np.uint32), d0.view(np.uint32)), f"run {r}: distances differ"
            if out is not None:
                assert ids is out[0] or np.shares_memory(ids, out[0])
            b.mark_cells(1.0)
    finally:
        b.close()
        dev.close()


def test_reused_batch_switches_entries_and_channels(world32):
    """One batch searched with the index's entry draw, the dual-channel
    traversal (its own draw of L entries), caller-given entry points and the
    draw again, in that order and replayed: every search equals the same
    search on a fresh batch (ids, distances, counters, statistics sums), so a
    skipped entry-point copy never leaves stale entries behind."""
    import garfield_amd as gf
    cfg, ix = world32
    lo, hi = cfg["lo"].astype(np.float32), cfg["hi"].astype(np.float32)
    dev = synth.open_device_index(ix)
    N, P, R = ix["vectors"].shape[0], ix["P"], ix["R"]
    rng = np.random.default_rng(5)
    own = rng.integers(0, 10**6, R).astype(np.uint32)
    plan = [dict(L=64, channels=1), dict(L=33, channels=2), dict(L=64, channels=1, entry_points=own),
            dict(L=64, channels=1), dict(L=33, channels=2), dict(L=64, channels=1)]

    def fresh(kw):
        b = dev.batch(cfg["queries"], lo, hi)
        try:
            b.mark_cells(0.0)
            b.order_cells(4)
            ids, d, st = b.search(K=10, rl=10, **kw)
            return ids, d, b.get_counters(), (st.n_expand, st.n_dist, st.q_traverse, st.q_bruteforce)
        finally:
            b.close()

    want = [fresh(kw) for kw in plan]
    b = dev.batch(cfg["queries"], lo, hi)
    try:
        b.mark_cells(0.0)
        b.order_cells(4)
        for rep in range(2):
            for i, kw in enumerate(plan):
                _print_case("reuse", rep=rep, step=i, L=kw["L"], channels=kw["channels"])
                ids, d, st = b.search(K=10, rl=10, **kw)
                w = want[i]
                assert np.array_equal(ids, w[0]), (rep, i)
                assert np.array_equal(d.view(np.uint32), w[1].view(np.uint32)), (rep, i)
                assert np.array_equal(b.get_counters(), w[2]), (rep, i)
                assert (st.n_expand, st.n_dist, st.q_traverse, st.q_bruteforce) == w[3], (rep, i)
    finally:
        b.close()
        dev.close()
    # the caller's entries and the draw give different trajectories, so the
    # comparison above would see a stale copy
    assert not np.array_equal(want[2][2], want[3][2])
    assert gf.entry_points(N, P, R).shape == (R,)


@pytest.mark.parametrize("prefilters", [(1.0, 0.05), (0.0, 0.05)])
def test_stage_a_b_graph_replays(monkeypatch, world_sub2, world32, prefilters):
    """Stages A (with and without the exact selectivity counts) and B as
    replayed graphs: the cell lists, counts, routing and the searches equal
    the eager run on every replay; timed and untimed calls alternate, the
    reported stage times are positive, and switching the prefilter
    recaptures stage A."""
    cfg, ix = world32 if prefilters[0] == 0.0 else world_sub2
    _print_case("graph-stage-ab", prefilters=prefilters)
    dev = synth.open_device_index(ix)
    b = dev.batch(cfg["queries"], cfg["lo"].astype(np.float32), cfg["hi"].astype(np.float32))
    labels = ix["labels"] is not None
    try:
        want = {}
        monkeypatch.setenv("GARFIELD_NO_GRAPH", "1")
        for pf in prefilters:
            b.mark_cells(pf, timed=False)
            if labels:
                b.order_cells(4, timed=False)
            cells = b.get_cells()
            ids, d, st = b.search(L=40, K=10, rl=10)
            assert st.graph == 0
            want[pf] = (cells, ids, d, b.get_counters())
        monkeypatch.delenv("GARFIELD_NO_GRAPH")
        for r in range(4):
            for pf in prefilters:
                timed = (r + int(pf * 100)) % 2 == 0
                ms_a = b.mark_cells(pf, timed=timed)
                ms_b = b.order_cells(4, timed=not timed) if labels else None
                ids, d, st = b.search(L=40, K=10, rl=10)
                cells = b.get_cells()
                w = want[pf]
                for k, (x, y) in enumerate(zip(cells, w[0])):
                    assert np.array_equal(x, y), f"replay {r} prefilter {pf}: cell array {k} differs"
                assert np.array_equal(ids, w[1]), f"replay {r} prefilter {pf}: ids differ"
                assert np.array_equal(d.view(np.uint32), w[2].view(np.uint32)), f"replay {r} prefilter {pf}: dists"
                assert np.array_equal(b.get_counters(), w[3]), f"replay {r} prefilter {pf}: counters differ"
                # from the second round on, stage A (and B) replay their graphs
                if r >= 1:
                    assert st.graph & 2, f"replay {r} prefilter {pf}: stage A did not replay"
                    if labels:
                        assert st.graph & 4, f"replay {r} prefilter {pf}: stage B did not replay"
                assert st.ms_stage_a > 0.0
                if labels:
                    assert st.ms_stage_b > 0.0
                if timed:
                    assert ms_a is not None and ms_a > 0.0
                elif labels:
                    assert ms_b is not None and ms_b > 0.0
    finally:
        b.close()
        dev.close()


def test_recorded_stage_calls_keep_their_order(world32):
    """Stage calls without ms are recorded and run later (at the next search,
    or first thing in a call that reads the stage buffers), in the order they
    were made: every sequence of calls made without ms gives the cells, ids
    and counters of the same sequence made with ms (each call run at once),
    here with the reference's tie order (ref_ties)."""
    cfg, ix = world32
    lo, hi = cfg["lo"].astype(np.float32), cfg["hi"].astype(np.float32)
    dev = synth.open_device_index(ix, ref_ties=True)
    seqs = [["A", "B", "B", "cells"],
            ["A", "B", "A", "B", "B", "search", "cells"],
            ["A", "B", "search", "B", "search", "cells"],
            ["A", "A", "B", "cells", "B", "cells", "search"]]
    try:
        for n, seq in enumerate(seqs):
            _print_case("recorded-order", seq=n)
            got = {}
            for timed in (True, False):
                b = dev.batch(cfg["queries"], lo, hi)
                out = []
                try:
                    for op in seq:
                        if op == "A":
                            b.mark_cells(0.05, timed=timed)
                        elif op == "B":
                            b.order_cells(4, timed=timed)
                        elif op == "cells":
                            out.append(b.get_cells()[:3])
                        else:
                            ids, d, _ = b.search(L=48, K=10, rl=10)
                            out.append((ids.copy(), d.view(np.uint32).copy(), b.get_counters()))
                finally:
                    b.close()
                got[timed] = out
            for i, (x, y) in enumerate(zip(got[True], got[False])):
                for k, (u, v) in enumerate(zip(x, y)):
                    assert np.array_equal(u, v), f"sequence {n} ({seq}): output {i} part {k} differs"
    finally:
        dev.close()
