"""Batch planning for the streamed index (gf_stream_plan_cells), on the CPU.

The planner is host code.  It groups a grid's cells into batches so that few
queries are active per batch (the out-of-core pipeline's cell scheduling,
README.md:5; the shipped driver fixes its batches by hand,
indexsearch/bigdataset/bigdataset_experiment.cu:271-277, 746-756): the best
guillotine partition of the grid into boxes that fit a batch, by dynamic
programming over boxes.  The oracle restates it as a memoised recursion
(oracle.plan_cells); these tests pin the restatement by a hand-derived plan,
a closed form, the brute-force optimum over every box partition of 2 x n
grids (all of which are guillotine) and an independent recount of the
objective, and then require the library's plan to equal it.  Each planted
mistake of the restatement (oracle.plan_cells(mutation=...)) turns the
brute-force comparison red.
"""
import numpy as np
import pytest

import garfield_amd._lib as gl
from oracle import oracle as orc


def _box_cells(grid, lo, hi):
    """Row-major ids (last axis fastest) of the cells of the box [lo, hi]."""
    axes = [np.arange(l, h + 1) for l, h in zip(lo, hi)]
    mesh = np.meshgrid(*axes, indexing="ij")
    return sorted(int(c) for c in np.ravel_multi_index([m.ravel() for m in mesh], grid))


def _random_boxes(rng, grid, Q, maxw=None):
    sets = []
    for _ in range(Q):
        lo, hi = [], []
        for g in grid:
            w = int(rng.integers(1, (maxw or g) + 1))
            w = min(w, g)
            l = int(rng.integers(0, g - w + 1))
            lo.append(l)
            hi.append(l + w - 1)
        sets.append(_box_cells(grid, lo, hi))
    return sets


def _lists(sets, P):
    """Query cell sets -> (Q x P cell lists, counts) as gf_batch_get_cells gives them."""
    Q = len(sets)
    cells = np.zeros((Q, P), np.uint32)
    counts = np.zeros(Q, np.uint32)
    for q, s in enumerate(sets):
        cells[q, :len(s)] = sorted(s)
        counts[q] = len(s)
    return cells, counts


def _active(plan, sets):
    """The objective, recounted: sum over batches of the queries selecting one of its cells."""
    return sum(sum(1 for s in sets if set(s) & set(batch)) for batch in plan)


def _box_partitions(grid, fits):
    """Every partition of a 2-d grid into boxes that fit (by fits(box cells)):
    the first uncovered cell in row-major order is the top-left corner of
    its box."""
    R, Cn = grid
    covered = np.zeros(grid, bool)

    def rec():
        free = np.argwhere(~covered)
        if free.size == 0:
            yield []
            return
        r0, c0 = free[0]
        for r1 in range(r0, R):
            for c1 in range(c0, Cn):
                if covered[r0:r1 + 1, c0:c1 + 1].any():
                    break
                box = [r * Cn + c for r in range(r0, r1 + 1) for c in range(c0, c1 + 1)]
                if not fits(box):
                    continue
                covered[r0:r1 + 1, c0:c1 + 1] = True
                for rest in rec():
                    yield [box] + rest
                covered[r0:r1 + 1, c0:c1 + 1] = False

    yield from rec()


def test_hand_plan_1d():
    """Four unit cells in a row, two per batch.  Queries: {0,1} three times,
    {2,3}, {1,2}.  Cutting after cell 1 splits only {1,2} (cost 1), after
    cell 0 splits the three {0,1} and leaves 1..3 to cut again, after cell 2
    splits {2,3} and leaves 0..2 to cut again: [[0,1],[2,3]], active
    3 + 1 + 2 = 6."""
    sets = [[0, 1]] * 3 + [[2, 3], [1, 2]]
    cells, counts = _lists(sets, 4)
    plan, act = orc.plan_cells(cells, counts, [4], np.ones(4, np.uint32), max_cells=2)
    assert plan == [[0, 1], [2, 3]] and act == 6


def test_chain_closed_form():
    """g unit cells in a row, m per batch, one query per adjacent pair: each
    batch boundary splits exactly one query, so the optimum uses the fewest
    batches, ceil(g / m), and its objective is (g - 1) + ceil(g / m) - 1."""
    for g, m in ((7, 2), (9, 3), (10, 4), (5, 5), (6, 1)):
        sets = [[i, i + 1] for i in range(g - 1)]
        cells, counts = _lists(sets, g)
        plan, act = orc.plan_cells(cells, counts, [g], np.ones(g, np.uint32), max_cells=m)
        nb = -(-g // m)
        assert len(plan) == nb and act == (g - 1) + nb - 1, (g, m, plan)
        assert sorted(c for b in plan for c in b) == list(range(g))


@pytest.mark.parametrize("mutation", [0, 1, 2])
def test_dp_equals_brute_force_on_2xn_grids(mutation):
    """(objective, batches) of the plan equal the minimum over every box
    partition of 2 x 4 and 2 x 5 grids (cells of random sizes, some empty;
    box-shaped queries; cell and point limits).  Mutations 1 and 2 must
    lose this on some case."""
    rng = np.random.default_rng(5)
    mismatch = 0
    for trial in range(40):
        grid = [2, int(rng.choice([4, 5]))]
        P = grid[0] * grid[1]
        sizes = rng.integers(0, 4, P).astype(np.uint32)
        sizes[rng.integers(0, P)] = 2
        sets = _random_boxes(rng, grid, int(rng.integers(1, 12)), maxw=3)
        cells, counts = _lists(sets, P)
        max_cells = int(rng.choice([2, 3]))
        max_points = int(rng.choice([0, 6]))

        def fits(box):
            ne = [c for c in box if sizes[c]]
            return (len(box) == 1 or (len(ne) <= max_cells and (max_points == 0 or sizes[ne].sum() <= max_points)))

        best = None
        for part in _box_partitions(grid, fits):
            batches = [[c for c in b if sizes[c]] for b in part]
            batches = [b for b in batches if b]
            k = (_active(batches, sets), len(batches))
            best = k if best is None or k < best else best
        plan, act = orc.plan_cells(cells, counts, grid, sizes, max_points=max_points, max_cells=max_cells,
                                   mutation=mutation)
        assert act == _active(plan, sets)
        assert sorted(c for b in plan for c in b) == [c for c in range(P) if sizes[c]]
        mismatch += (act, len(plan)) != best
        if mutation == 0:
            assert (act, len(plan)) == best, (trial, grid, sets, plan, best)
    if mutation:
        assert mismatch > 0, f"mutation {mutation} went unnoticed"


def test_block_plan_is_an_upper_bound():
    """The C5-shaped grid (16 x 16 unit cells, 16 per batch) with queries of
    the streamed bench's kind: the 4 x 4 block plan and the 16-consecutive-
    cell plan are guillotine partitions that fit, so the planned objective
    is at most theirs.  Queries that each lie in one row: whole-row batches
    hold every query once (objective Q, the minimum), which blocks cannot."""
    rng = np.random.default_rng(21)
    grid = [16, 16]
    sets = _random_boxes(rng, grid, 3000, maxw=8)
    cells, counts = _lists(sets, 256)
    plan, act = gl.plan_cells(cells, counts, grid, np.full(256, 100, np.uint32), max_cells=16)
    blocks = [[i * 16 + j for i in range(i0, i0 + 4) for j in range(j0, j0 + 4)]
              for i0 in range(0, 16, 4) for j0 in range(0, 16, 4)]
    strips = [list(range(16 * i, 16 * i + 16)) for i in range(16)]
    assert act == _active(plan, sets)
    assert act <= _active(blocks, sets) < _active(strips, sets)
    assert len(plan) == 16 and all(len(b) == 16 for b in plan)
    rows = []
    for _ in range(500):
        r, w = int(rng.integers(0, 16)), int(rng.integers(2, 9))
        c0 = int(rng.integers(0, 17 - w))
        rows.append(_box_cells(grid, [r, c0], [r, c0 + w - 1]))
    cells, counts = _lists(rows, 256)
    plan, act = gl.plan_cells(cells, counts, grid, np.full(256, 100, np.uint32), max_cells=16)
    assert act == len(rows) < _active(blocks, rows)


@pytest.mark.parametrize("grid", [[6], [4, 4], [8, 8], [3, 5], [4, 4, 4], [2, 3, 2]])
def test_library_plan_matches_oracle(grid):
    rng = np.random.default_rng(sum(grid) * 7 + len(grid))
    P = int(np.prod(grid))
    for trial in range(3):
        sets = _random_boxes(rng, grid, int(rng.integers(0, 200)))
        cells, counts = _lists(sets, P)
        sizes = rng.integers(0, 50, P).astype(np.uint32)
        for max_points, max_cells in ((0, 16), (120, 0), (200, 8), (0, 3)):
            want = orc.plan_cells(cells, counts, grid, sizes, max_points=max_points, max_cells=max_cells)
            got = gl.plan_cells(cells, counts, grid, sizes, max_points=max_points, max_cells=max_cells)
            assert got == want, (grid, trial, max_points, max_cells)
            assert got[1] == _active(got[0], sets)


def test_library_plan_rejects_bad_input():
    cells, counts = _lists([[0, 1]], 4)
    cells[0, 1] = 9
    with pytest.raises(gl.GarfieldError):
        gl.plan_cells(cells, counts, [2, 2], np.ones(4, np.uint32))
    with pytest.raises(ValueError):
        gl.plan_cells(cells, counts, [2, 3], np.ones(4, np.uint32))
    P = 64 * 64 * 2
    with pytest.raises(gl.GarfieldError) as e:
        gl.plan_cells(np.zeros((0, P), np.uint32), np.zeros(0, np.uint32), [64, 64, 2], np.ones(P, np.uint32))
    assert e.value.status == 6
