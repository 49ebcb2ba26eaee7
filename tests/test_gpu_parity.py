"""Parity of the HIP path (libgarfield.so through its C ABI) with the CPU oracle.

Bar: bit-exact for ids, cells, counts, routing, counters and fp32 traversal
distances (the oracle restates the kernels' summation order); the MFMA
centroid distances, whose accumulation order is the hardware's, are checked
against an fp64 reference within a stated tolerance, and every stage after
them is checked exactly on the GPU's own distances.
"""
import os

import numpy as np
import pytest

from garfield_amd import synth

pytestmark = pytest.mark.gpu


def _print_case(name, **kw):
    print(f"[case] {name} " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _oracle_pipeline(cfg, ix, prefilter, topc=4, gpu_topk=None):
    from oracle import oracle as orc
    l_q, r_q = synth.quantile_arrays(ix)
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    cells, cnt = orc.cells(lo, hi, ix["grid"], l_q, r_q, synth.cell_sizes(ix))
    sel, little = orc.selectivity(ix["attrs"], lo, hi, prefilter, cnt)
    return lo, hi, cells, cnt, sel, little


def _device(ix, **kw):
    return synth.open_device_index(ix, **kw)


def test_f2h_bit_exact():
    import garfield_amd as gf
    from oracle import oracle as orc
    _print_case("f2h")
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=1 << 18, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 5.96e-8, 2.98e-8,
                                     np.inf, -np.inf, 6.1e-5, 255.0, 0.1], np.float32)])
    x = x[np.isfinite(x) | np.isinf(x)]
    for alpha in (1.0, 0.01, 3.0):
        g = gf.f2h(x, alpha)
        o = orc.f2h(x, alpha)
        bad = np.nonzero(g != o)[0]
        assert bad.size == 0, (f"alpha={alpha}: {bad.size} mismatches, first x={x[bad[:4]].tolist()} "
                               f"bits={x[bad[:4]].view(np.uint32).tolist()} gpu={g[bad[:4]].tolist()} "
                               f"oracle={o[bad[:4]].tolist()}")


def test_row_norms_f16_bit_exact():
    import garfield_amd as gf
    from oracle import oracle as orc
    _print_case("norms")
    rng = np.random.default_rng(1)
    for D in (96, 128, 768):
        x = orc.f2h(rng.standard_normal((300, D)).astype(np.float32) * 10)
        assert np.array_equal(gf.row_norms_f16(x), orc.row_norms_f16(x)), D


def test_cells_selectivity_routing(small_world):
    cfg, ix = small_world
    _print_case("cells", N=ix["vectors"].shape[0], Q=cfg["queries"].shape[0])
    dev = _device(ix)
    for prefilter in (0.0, 0.05, 0.3, 1.0):
        lo, hi, cells, cnt, sel, little = _oracle_pipeline(cfg, ix, prefilter)
        b = dev.batch(cfg["queries"], lo, hi)
        b.mark_cells(prefilter)
        gc, gcnt, glit, gsel = b.get_cells()
        assert np.array_equal(gcnt, cnt)
        for q in range(len(cnt)):
            assert np.array_equal(gc[q, :cnt[q]], cells[q, :cnt[q]]), q
        assert np.array_equal(gsel, sel)
        assert np.array_equal(glit, little)
        b.close()
    dev.close()


def test_centroid_order(small_world):
    from oracle import oracle as orc
    cfg, ix = small_world
    _print_case("centroid")
    dev = _device(ix)
    lo, hi, cells, cnt, sel, little = _oracle_pipeline(cfg, ix, 0.0)
    b = dev.batch(cfg["queries"], lo, hi)
    b.mark_cells(0.0)
    b.order_cells(4)
    gdist, gtop = b.get_centroid()
    cen, hist = orc.centres_hist(ix["vectors"], ix["labels"], ix["global_pid"], ix["P"])
    qh = orc.f2h(cfg["queries"])
    ch = orc.f2h(cen)
    ref = orc.centroid_dist_f64(qh, ch)
    qn = (orc.row_norms_f16(qh).astype(np.float64))
    cn = (orc.row_norms_f16(ch).astype(np.float64))
    # fp16 products are exact in fp32; the fp32 accumulation error is bounded
    # by D * 2^-24 * sum|q_i c_i| <= D * 2^-24 * (|q|^2 + |c|^2) / 2, plus the
    # rounding of the final sum.
    tol = (128 * 2.0 ** -24 + 4 * 2.0 ** -24) * (qn[:, None] + cn[None, :]) + 1e-3
    assert np.all(np.abs(gdist.astype(np.float64) - ref) <= tol)
    # exact from here on, on the GPU's distances
    assert np.array_equal(gtop, orc.topk_clusters(gdist, 4))
    gc, gcnt, _, _ = b.get_cells()
    ocells = orc.sort_cells(cells, cnt, gtop, hist)
    for q in range(len(cnt)):
        assert np.array_equal(gc[q, :cnt[q]], ocells[q, :cnt[q]]), q
    b.close()
    dev.close()


def test_centroid_order_reference_ties(small_world):
    """ref_ties: equal cell scores keep the order of the reference's network
    (bitonic_sort_id_by_num_int), bit for bit against the oracle's replay in
    tie mode 1 on the GPU's own nearest centres; the order differs from the
    default (ties by cell id) for some queries."""
    from oracle import oracle as orc
    cfg, ix = small_world
    _print_case("centroid-ref-ties")
    lo, hi, cells, cnt, sel, little = _oracle_pipeline(cfg, ix, 0.0)
    _, hist = orc.centres_hist(ix["vectors"], ix["labels"], ix["global_pid"], ix["P"])
    out = {}
    for ref in (False, True):
        dev = _device(ix, ref_ties=ref)
        b = dev.batch(cfg["queries"], lo, hi)
        b.mark_cells(0.0)
        b.order_cells(4)
        _, gtop = b.get_centroid()
        gc, gcnt, _, _ = b.get_cells()
        orc.set_tie_mode(1 if ref else 0)
        try:
            ocells = orc.sort_cells(cells, cnt, gtop, hist)
        finally:
            orc.set_tie_mode(0)
        for q in range(len(cnt)):
            assert np.array_equal(gc[q, :cnt[q]], ocells[q, :cnt[q]]), (ref, q)
        out[ref] = gc
        b.close()
        dev.close()
    assert any(not np.array_equal(out[False][q, :cnt[q]], out[True][q, :cnt[q]]) for q in range(len(cnt)))


def _traversal_case(cfg, ix, L, prefilter=0.0, vec_dtype=0, f2h_factor=1.0, postfilter=1 << 30, Q=None,
                    channels=1, K=10):
    import garfield_amd as gf
    from oracle import oracle as orc
    dev = _device(ix, vec_dtype=vec_dtype, f2h_factor=f2h_factor)
    lo, hi, cells, cnt, sel, little = _oracle_pipeline(cfg, ix, prefilter)
    queries = cfg["queries"] if Q is None else cfg["queries"][:Q]
    lo, hi = lo[:len(queries)], hi[:len(queries)]
    b = dev.batch(queries, lo, hi)
    b.mark_cells(prefilter)
    if ix["labels"] is not None:
        b.order_cells(4)
    gc, gcnt, glit, _ = b.get_cells()
    ent = gf.entry_points(ix["vectors"].shape[0], ix["P"], L if channels == 2 else ix["R"])
    ids, dists, st = b.search(L=L, K=K, rl=10, postfilter=postfilter, entry_points=ent, channels=channels)
    ctr = b.get_counters()
    # binary16 rows: 1 with fp32 accumulation (the oracle's distance mode
    # 0), 4 with the reference's binary16 arithmetic (mode 1)
    vec16 = orc.f2h(ix["vectors"], f2h_factor) if vec_dtype in (1, 4) else None
    if vec_dtype == 3:
        # the int8 values and per-dimension scales the index holds; queries
        # scaled by f2h_factor as the library scales them
        q8, qs, qz = orc.quantise_i8(ix["vectors"], f2h_factor)
        O = orc.OracleIndex(q8.astype(np.float32), ix["attrs"], ix["global_pid"], ix["P"], ix["cell_graphs"],
                            ix["cross"], i8q=(qs, qz))
        oq = np.asarray(queries, np.float32) * np.float32(f2h_factor)
    else:
        O = orc.OracleIndex(ix["vectors"], ix["attrs"], ix["global_pid"], ix["P"], ix["cell_graphs"],
                            ix["cross"], vec_f16=vec16)
        oq = orc.f2h(queries, f2h_factor) if vec_dtype in (1, 4) else queries
    orc.set_channels(channels)
    orc.set_dist_mode(1 if vec_dtype == 4 else 0)
    try:
        oids, odist, octr = O.search(oq, lo, hi, gc, gcnt, glit, ent, L, K=K, rl=10, postfilter=postfilter)
    finally:
        orc.set_channels(1)
        orc.set_dist_mode(0)
    b.close()
    dev.close()
    dump = os.environ.get("GF_DUMP_DIR")
    if dump and (not np.array_equal(ids, oids) or not np.array_equal(ctr, octr)):
        os.makedirs(dump, exist_ok=True)
        np.savez_compressed(os.path.join(dump, f"parity_L{L}_pf{prefilter}_v{vec_dtype}_Q{len(queries)}.npz"),
                            cells=gc, counts=gcnt, little=glit, ent=ent, ids=ids, ctr=ctr, oids=oids, octr=octr,
                            L=L, postfilter=postfilter)
    return ids, dists, ctr, oids, odist, octr, st


def _assert_same(ids, dists, ctr, oids, odist, octr, st=None):
    if st is not None and st.bf_mfma == 1:
        # the MFMA brute force evaluates every scanned point, the oracle only
        # the passing ones
        octr = octr.copy()
        rows = octr[:, 7] == 2
        octr[rows, 1] = octr[rows, 5]
    if st is not None and st.bf_mfma == 2:
        # the fp16 MFMA brute force evaluates exactly the candidates its
        # error bound keeps, the oracle every passing point
        octr = octr.copy()
        rows = octr[:, 7] == 2
        octr[rows, 1] = ctr[rows, 1]
    bad = np.nonzero(np.any(ids != oids, axis=1))[0]
    assert bad.size == 0, f"{bad.size} queries differ, first q={bad[:5]}: gpu={ids[bad[0]]} oracle={oids[bad[0]]}"
    assert np.array_equal(dists.view(np.uint32), odist.view(np.uint32))
    cbad = np.nonzero(np.any(ctr != octr, axis=1))[0]
    assert cbad.size == 0, f"counters differ for q={cbad[:5]}: gpu={ctr[cbad[0]]} oracle={octr[cbad[0]]}"


@pytest.mark.parametrize("L", [10, 32, 64, 100, 256])
def test_traversal_parity_r16(small_world, L):
    cfg, ix = small_world
    _print_case("traverse-r16", L=L)
    _assert_same(*_traversal_case(cfg, ix, L)[:6])


@pytest.mark.parametrize("L", [16, 80, 200])
def test_traversal_parity_r32_mixed(world32, L):
    cfg, ix = world32
    _print_case("traverse-r32", L=L)
    _assert_same(*_traversal_case(cfg, ix, L)[:6])


def test_traversal_parity_fp16(world32):
    cfg, ix = world32
    _print_case("traverse-fp16")
    _assert_same(*_traversal_case(cfg, ix, 64, vec_dtype=1, f2h_factor=0.01)[:6])


@pytest.mark.parametrize("prefilter", [0.05, 1.0])
def test_bruteforce_parity(world32, prefilter):
    cfg, ix = world32
    _print_case("bruteforce", prefilter=prefilter)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 64, prefilter=prefilter)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.q_bruteforce > 0 and st.bf_mfma == 1


@pytest.mark.parametrize("L", [16, 64, 300])
def test_postfilter_full_graph_parity(small_world, L):
    """Queries with postfilter or more cells run the full-graph search
    (FD = 2 x 16 edges per row), bit-exact against the oracle."""
    cfg, ix = small_world
    _print_case("postfilter-full", L=L)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, L, postfilter=12)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.q_fullgraph > 0 and st.q_traverse > 0
    assert st.q_fullgraph == int(np.sum(octr[:, 7] == 3))


def test_postfilter_full_graph_r32_fp16(world32):
    cfg, ix = world32
    _print_case("postfilter-full-fp16")
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 80, vec_dtype=1, f2h_factor=0.01,
                                                             postfilter=6)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.q_fullgraph > 0


def test_postfilter_full_graph_64_cells(world_gauss):
    """4 x 4 x 4 cells: one edge into each cell, FD = 64 (a full wave); with
    postfilter 1 every query that is not all little takes the full graph."""
    cfg, ix = world_gauss
    _print_case("postfilter-full-64")
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 128, postfilter=1)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.q_fullgraph > 0


def test_recall_against_ground_truth(world32):
    from oracle import oracle as orc
    cfg, ix = world32
    _print_case("recall")
    ids, dists, *_ = _traversal_case(cfg, ix, 200)
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    gt, gtd = orc.ground_truth(ix["vectors"], ix["attrs"], cfg["queries"], lo, hi, 10)
    assert orc.recall(ids, gt, gtd) > 0.8
    # every returned id passes the filter and its distance is the exact one
    for q in range(ids.shape[0]):
        for j in range(10):
            i = ids[q, j]
            if i == 0x7FFFFFFF:
                continue
            a = ix["attrs"][i]
            assert np.all(a >= cfg["lo"][q]) and np.all(a <= cfg["hi"][q])
            d = np.sum((cfg["queries"][q].astype(np.float64) - ix["vectors"][i]) ** 2)
            assert abs(d - dists[q, j]) <= 1e-5 * max(d, 1.0)


@pytest.mark.parametrize("L,prefilter", [(32, 0.0), (100, 0.0), (64, 0.01), (64, 1.0)])
def test_gaussian_parity(world_gauss, L, prefilter):
    """Non-integer 96-d data: canonical fp32 summation order, the fp32 MFMA
    brute force with its exact re-rank, 3 attributes."""
    cfg, ix = world_gauss
    _print_case("gauss", L=L, prefilter=prefilter)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, L, prefilter=prefilter)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.bf_mfma == (2 if st.q_bruteforce else 0)
    if prefilter == 1.0:
        assert st.q_traverse == 0


@pytest.mark.parametrize("K", [5, 10, 16])
def test_f32_mfma_bruteforce(world_gauss, K):
    """fp32 rows (96-d, six chunks of four fp32 MFMA k-steps): the float
    MFMA route for K <= 10, the gather kernel beyond; bit-exact either way."""
    cfg, ix = world_gauss
    _print_case("f32-bf", K=K)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 32, prefilter=1.0, K=K)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.q_bruteforce > 0 and st.bf_mfma == (2 if K <= 10 else 0)


@pytest.mark.parametrize("L,prefilter", [(32, 0.0), (100, 0.0), (64, 0.01), (64, 1.0)])
def test_i8q_parity(world_gauss, L, prefilter):
    """int8 per-dimension quantised rows (GF_VEC_I8Q, the reference loader's
    quantisation): traversal and gather brute force bit-exact against the
    oracle's restatement of the same arithmetic."""
    cfg, ix = world_gauss
    _print_case("i8q", L=L, prefilter=prefilter)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, L, prefilter=prefilter, vec_dtype=3)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.bf_mfma == 0
    if prefilter == 1.0:
        assert st.q_traverse == 0


def test_i8q_768d_and_full_graph(world_c4):
    """768-d rows (one 16-byte chunk per lane), f2h_factor 2, and the full
    graph taking the queries with postfilter."""
    cfg, ix = world_c4
    _print_case("i8q-768")
    _assert_same(*_traversal_case(cfg, ix, 64, vec_dtype=3, f2h_factor=2.0)[:6])
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 80, vec_dtype=3, postfilter=4)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.q_fullgraph > 0


def test_i8q_recall(world_gauss):
    """The quantised index still finds the fp32 neighbours: recall@10 against
    exact fp32 ground truth at L = 200 stays within 0.05 of the fp32 index's."""
    from oracle import oracle as orc
    cfg, ix = world_gauss
    _print_case("i8q-recall")
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    gt, gtd = orc.ground_truth(ix["vectors"], ix["attrs"], cfg["queries"], lo, hi, 10)
    r8 = orc.recall(_traversal_case(cfg, ix, 200, vec_dtype=3)[0], gt, gtd)
    r32 = orc.recall(_traversal_case(cfg, ix, 200)[0], gt, gtd)
    assert r8 >= r32 - 0.05 and r8 > 0.8, (r8, r32)


def test_i8q_rejected_where_unsupported(world_gauss):
    """The no-allocation entry point and the streamed index take no
    GF_VEC_I8Q index (status GF_E_UNSUPPORTED)."""
    import garfield_amd as gf
    cfg, ix = world_gauss
    _print_case("i8q-reject")
    dev = _device(ix, vec_dtype=3)
    assert dev.vec_dtype == 3
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    with pytest.raises(gf.GarfieldError) as e:
        gf.search_noalloc(dev, cfg["queries"][:4], lo[:4], hi[:4], 0.0, L=32, K=10)
    assert e.value.status == 6
    dev.close()
    l_q, r_q = synth.quantile_arrays(ix)
    with pytest.raises(gf.GarfieldError) as e:
        gf.Index.create_streamed(ix["vectors"], ix["attrs"].astype(np.float32), ix["grid"], l_q, r_q,
                                 ix["global_pid"], ix["cell_graphs"], ix["cross"], vec_dtype=3)
    assert e.value.status == 6


@pytest.mark.parametrize("L", [16, 64, 200])
def test_dual_channel_parity_r16(small_world, L):
    """The dual-channel traversal (gf_search_dual): ids, distances and
    counters bit-exact against the oracle's restatement."""
    cfg, ix = small_world
    _print_case("dual-r16", L=L)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, L, channels=2)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert np.sum(octr[:, 7] == 4) == st.q_traverse > 0


@pytest.mark.parametrize("L,prefilter", [(33, 0.0), (100, 0.05)])
def test_dual_channel_parity_r32(world32, L, prefilter):
    """R = 32 (64 expansion slots per epoch), odd L, mixed routes."""
    cfg, ix = world32
    _print_case("dual-r32", L=L, prefilter=prefilter)
    _assert_same(*_traversal_case(cfg, ix, L, prefilter=prefilter, channels=2))


@pytest.mark.parametrize("vec_dtype", [0, 1, 3])
def test_dual_channel_row_types(world_gauss, vec_dtype):
    """fp32, fp16 and int8-quantised rows of non-integer data, 64 cells of 3
    attributes; and the full graph beside it for queries with postfilter."""
    cfg, ix = world_gauss
    _print_case("dual-rows", vec_dtype=vec_dtype)
    f = 0.5 if vec_dtype == 1 else 1.0
    _assert_same(*_traversal_case(cfg, ix, 64, vec_dtype=vec_dtype, f2h_factor=f, channels=2))
    # most of these queries select one cell: postfilter 2 sends the others
    # to the full graph
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 48, vec_dtype=vec_dtype, f2h_factor=f,
                                                             postfilter=2, channels=2)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.q_fullgraph > 0 and np.sum(octr[:, 7] == 4) > 0


def test_dual_channel_recall(world32):
    """Recall@10 of the dual-channel route against exact ground truth at
    L = 200, and every returned distance exact."""
    from oracle import oracle as orc
    cfg, ix = world32
    _print_case("dual-recall")
    ids, dists, *_ = _traversal_case(cfg, ix, 200, channels=2)
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    gt, gtd = orc.ground_truth(ix["vectors"], ix["attrs"], cfg["queries"], lo, hi, 10)
    assert orc.recall(ids, gt, gtd) > 0.8


@pytest.mark.parametrize("prefilter,K", [(1.0, 10), (1.0, 5), (0.05, 10)])
def test_f16_mfma_bruteforce_768d(world_c4, prefilter, K):
    """Binary16 rows (768-d): the fp16 MFMA brute force keeps the candidates
    within its error bound and re-ranks them exactly, so ids, distances and
    counters equal the oracle's brute force (DIST aside: it counts the
    candidates re-ranked)."""
    cfg, ix = world_c4
    _print_case("f16-bf", prefilter=prefilter, K=K)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 32, prefilter=prefilter, vec_dtype=1,
                                                             K=K)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.bf_mfma == 2 and st.q_bruteforce > 0
    rows = octr[:, 7] == 2
    assert np.all(ctr[rows, 1] <= octr[rows, 1])       # never more than the passing points


@pytest.mark.parametrize("prefilter", [1.0, 0.01])
def test_f16_mfma_bruteforce_three_attributes(world_gauss, prefilter):
    """96-d binary16 rows (three k-steps), three attributes (two packed
    words), f2h_factor 0.5."""
    cfg, ix = world_gauss
    _print_case("f16-bf-3a", prefilter=prefilter)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 32, prefilter=prefilter, vec_dtype=1,
                                                             f2h_factor=0.5)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.bf_mfma == 2 and st.q_bruteforce > 0


def test_mfma_bruteforce_all_queries(world32):
    """Every query on the int8 MFMA brute force: exact filtered top-10."""
    from oracle import oracle as orc
    cfg, ix = world32
    _print_case("mfma-bf")
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 10, prefilter=1.0)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)
    assert st.bf_mfma == 1 and st.q_traverse == 0
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    gt, gtd = orc.ground_truth(ix["vectors"], ix["attrs"], cfg["queries"], lo, hi, 10)
    assert orc.recall(ids, gt, gtd) == 1.0


def _bf_case(cfg, ix, K, prefilter=1.0):
    import garfield_amd as gf
    from oracle import oracle as orc
    dev = _device(ix)
    lo, hi, cells, cnt, sel, little = _oracle_pipeline(cfg, ix, prefilter)
    b = dev.batch(cfg["queries"], lo, hi)
    b.mark_cells(prefilter)
    gc, gcnt, glit, gsel = b.get_cells()
    assert np.array_equal(gcnt, cnt) and np.array_equal(gsel, sel) and np.array_equal(glit, little)
    if ix["labels"] is not None:
        b.order_cells(4)
    gc, gcnt, glit, _ = b.get_cells()
    ent = gf.entry_points(ix["vectors"].shape[0], ix["P"], ix["R"])
    ids, dists, st = b.search(L=32, K=K, rl=10, entry_points=ent)
    ctr = b.get_counters()
    O = orc.OracleIndex(ix["vectors"], ix["attrs"], ix["global_pid"], ix["P"], ix["cell_graphs"], ix["cross"])
    oids, odist, octr = O.search(cfg["queries"], lo, hi, gc, gcnt, glit, ent, 32, K=K, rl=10)
    b.close()
    dev.close()
    return ids, dists, ctr, oids, odist, octr, st


@pytest.mark.parametrize("prefilter", [0.0, 0.05, 0.3, 1.0])
def test_subcell_selectivity(world_sub2, prefilter):
    """Sub-cell classification + partial scans give the exact selectivity counts."""
    cfg, ix = world_sub2
    _print_case("subcell-sel", prefilter=prefilter)
    dev = _device(ix)
    lo, hi, cells, cnt, sel, little = _oracle_pipeline(cfg, ix, prefilter)
    b = dev.batch(cfg["queries"], lo, hi)
    b.mark_cells(prefilter)
    gc, gcnt, glit, gsel = b.get_cells()
    assert np.array_equal(gcnt, cnt)
    bad = np.nonzero(gsel != sel)[0]
    assert bad.size == 0, f"selcount differs for q={bad[:5]}: gpu={gsel[bad[:5]]} oracle={sel[bad[:5]]}"
    assert np.array_equal(glit, little)
    b.close()
    dev.close()


@pytest.mark.parametrize("K", [5, 10, 16])
def test_subcell_mfma_bruteforce(world_sub2, K):
    cfg, ix = world_sub2
    _print_case("subcell-bf", K=K)
    ids, dists, ctr, oids, odist, octr, st = _bf_case(cfg, ix, K)
    assert st.bf_mfma == 1 and st.q_traverse == 0
    _assert_same(ids, dists, ctr, oids, odist, octr, st)


@pytest.mark.parametrize("prefilter", [0.05, 1.0])
def test_subcell_three_attributes(world_sub3, prefilter):
    cfg, ix = world_sub3
    _print_case("subcell-a3", prefilter=prefilter)
    ids, dists, ctr, oids, odist, octr, st = _bf_case(cfg, ix, 10, prefilter)
    assert st.bf_mfma == 1
    _assert_same(ids, dists, ctr, oids, odist, octr, st)


@pytest.mark.parametrize("L", [32, 100])
def test_c4_fp16_768d_traversal(world_c4, L):
    """768-d fp16 rows (64 lanes x 2 chunks per lane) in the reference's half
    path with f2h_factor 1."""
    cfg, ix = world_c4
    _print_case("c4-traverse", L=L)
    _assert_same(*_traversal_case(cfg, ix, L, vec_dtype=1, f2h_factor=1.0)[:6])


@pytest.mark.parametrize("K", [10, 16])
def test_c4_fp16_768d_bruteforce_and_order(world_c4, K):
    """The brute force on 768-d fp16 rows (prefilter 1: every query), after
    the cluster-guided order of stage B on 768-d centres: the fp16 MFMA route
    at K = 10, the gather kernel at K = 16 (beyond the MFMA route's K)."""
    cfg, ix = world_c4
    _print_case("c4-bruteforce", K=K)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 32, prefilter=1.0, vec_dtype=1,
                                                             f2h_factor=1.0, K=K)
    assert st.bf_mfma == (2 if K <= 10 else 0) and st.q_bruteforce > 0
    _assert_same(ids, dists, ctr, oids, odist, octr, st)


def test_index_opened_from_files(small_world, tmp_path):
    """gf_index_open on the written index files: stage A matches the oracle and
    the search gives the same bits as the index built from the arrays."""
    import garfield_amd._lib as gl
    cfg, ix = small_world
    _print_case("open-files", N=ix["vectors"].shape[0])
    p = synth.write_index(ix, str(tmp_path / "w"))
    lo, hi, cells, cnt, sel, little = _oracle_pipeline(cfg, ix, 0.05)
    out = []
    for dev in (gl.Index.open(**p, degree=ix["R"]), _device(ix)):
        b = dev.batch(cfg["queries"], lo, hi)
        b.mark_cells(0.05)
        b.order_cells(4)
        gc, gcnt, glit, gsel = b.get_cells()
        assert np.array_equal(gcnt, cnt) and np.array_equal(gsel, sel) and np.array_equal(glit, little)
        ids, dists, _ = b.search(L=64, K=10, rl=10)
        # entries past a query's cell count are not defined
        live = np.arange(gc.shape[1])[None, :] < gcnt[:, None]
        out.append((np.where(live, gc, 0), ids, dists, b.get_counters()))
        b.close()
        dev.close()
    for x, y in zip(out[0], out[1]):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("channels", [1, 2])
def test_cli_matches_library(small_world, tmp_path, channels):
    """garfield_search on the index files: the reference's CSV, and the same
    recall as the library on the same batch (channels 2: the dual-channel
    traversal)."""
    import csv
    import subprocess
    from garfield_amd import formats
    from oracle import oracle as orc
    cfg, ix = small_world
    _print_case("cli", channels=channels)
    p = synth.write_index(ix, str(tmp_path / "w"))
    formats.write_fvecs(str(tmp_path / "q.fvecs"), cfg["queries"])
    formats.write_ranges(str(tmp_path / "q.range"), cfg["lo"], cfg["hi"])
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    gt, gtd = orc.ground_truth(ix["vectors"], ix["attrs"], cfg["queries"], lo, hi, 10)
    formats.write_gt(str(tmp_path / "q.gt"), gt)
    cli = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "garfield_amd", "garfield_search")
    args = [cli, "--data_path", p["data_path"], "--query_path", str(tmp_path / "q.fvecs"), "--range",
            str(tmp_path / "q.range"), "--gt", str(tmp_path / "q.gt"), "--cagra_prefix", p["cagra_prefix"],
            "--cagra_suffix", p["cagra_suffix"], "--global_graph", p["global_graph"], "--grid", p["grid"],
            "--attrs", p["attrs"], "--cluster", p["cluster"], "--result", str(tmp_path / "r.csv"),
            "--prefilter", "0.05", "--f2h_factor", "1.0", "--degree", str(ix["R"]), "--L", "32,64",
            "--vec_dtype", "f32", "--channels", str(channels)]
    r = subprocess.run(args, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    rows = list(csv.DictReader(open(tmp_path / "r.csv")))
    assert [int(x["ef"]) for x in rows] == [32, 64]
    for x in rows:
        tot = float(x["cost1"]) + float(x["cost2"]) + float(x["cost3"])
        assert abs(float(x["total_cost"]) - tot) < 1e-5 and float(x["qps"]) > 0
    # the library on the same files, batch and L gives the same recall
    dev = synth.open_device_index(ix)
    b = dev.batch(cfg["queries"], lo, hi)
    b.mark_cells(0.05)
    b.order_cells(4)
    for x in rows:
        ids, _, _ = b.search(L=int(x["ef"]), K=10, rl=10, channels=channels)
        rec = np.mean([len(set(ids[q]) & set(gt[q][gt[q] != 0x7FFFFFFF])) / max(1, np.sum(gt[q] != 0x7FFFFFFF))
                       if np.any(gt[q] != 0x7FFFFFFF) else 1.0 for q in range(len(gt))])
        assert abs(rec - float(x["recall"])) < 1e-5, (x, rec)
    b.close()
    dev.close()
