"""gf_search_noalloc through the C ABI against the batch pipeline it varies
(gf_batch_create + gf_mark_cells + gf_order_cells + gf_search): the same ids
and fp32 distances, bit for bit, on two calls in a row (the second with fewer
queries, so that it runs on what the first left in the shared scratch array),
and a batch too large for the scratch array is refused before any device work."""
import numpy as np
import pytest

from garfield_amd import synth

pytestmark = pytest.mark.gpu


def _print_case(name, **kw):
    print(f"[case] {name} " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _pipeline(dev, q, lo, hi, prefilter, topc, L, ent, postfilter=1 << 30):
    b = dev.batch(q, lo, hi)
    b.mark_cells(prefilter)
    b.order_cells(topc)
    ids, d, _ = b.search(L, postfilter=postfilter, entry_points=ent)
    b.close()
    return ids, d


@pytest.mark.parametrize("world,prefilter,L,kw", [
    ("world32", 0.05, 48, {}),                                  # MFMA route in the pipeline, gather here
    ("world_gauss", 0.02, 40, {}),                              # non-integer data, 3 attributes, 64 cells
    ("world_c4", 0.3, 32, dict(vec_dtype=1, f2h_factor=1.0)),   # fp16 rows, 768-d
    ("world32", 0.05, 48, dict(postfilter=6)),                  # the full-graph route
])
def test_noalloc_matches_batch_pipeline(request, world, prefilter, L, kw):
    import garfield_amd as gf
    cfg, ix = request.getfixturevalue(world)
    kw = dict(kw)
    pf = kw.pop("postfilter", 1 << 30)
    dev = synth.open_device_index(ix, **kw)
    q = cfg["queries"].astype(np.float32)
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    Q = q.shape[0]
    for call, n in enumerate((Q, Q // 2 + 3)):
        for ent in (None, gf.entry_points(ix["vectors"].shape[0], ix["P"], ix["R"])[::-1].copy()):
            _print_case("noalloc", world=world, call=call, Q=n, L=L, entry="ref" if ent is None else "given")
            rids, rd = _pipeline(dev, q[:n], lo[:n], hi[:n], prefilter, 4, L, ent, pf)
            ids = np.full((n, 10), 0xFFFFFFFF, np.uint32)
            d = np.full((n, 10), np.nan, np.float32)
            gids, gd = gf.search_noalloc(dev, q[:n], lo[:n], hi[:n], prefilter, topc=4, L=L, postfilter=pf,
                                         entry_points=ent, out=(ids, d))
            assert gids is ids and gd is d
            assert np.array_equal(ids, rids), (world, call, np.argwhere(ids != rids)[:5])
            assert np.array_equal(d.view(np.uint32), rd.view(np.uint32)), (world, call)
    dev.close()


def test_noalloc_rejects_oversized_batch(world32):
    import garfield_amd as gf
    from garfield_amd._lib import GarfieldError
    cfg, ix = world32
    dev = synth.open_device_index(ix)
    _print_case("noalloc-oversize")
    Q = (gf._lib.NOALLOC_SCRATCH_MB << 20) // (4 * ix["vectors"].shape[1]) + 16
    q = np.zeros((Q, ix["vectors"].shape[1]), np.float32)
    lo = np.zeros((Q, 2), np.float32)
    hi = np.zeros((Q, 2), np.float32)
    with pytest.raises(GarfieldError) as e:
        gf.search_noalloc(dev, q, lo, hi, 1.0)
    assert e.value.status == 6 and "scratch" in str(e.value)
    # the refusal leaves the entry point usable
    n = 40
    rids, rd = _pipeline(dev, cfg["queries"][:n].astype(np.float32), cfg["lo"][:n].astype(np.float32),
                         cfg["hi"][:n].astype(np.float32), 1.0, 4, 32, None)
    ids, d = gf.search_noalloc(dev, cfg["queries"][:n], cfg["lo"][:n], cfg["hi"][:n], 1.0, L=32)
    assert np.array_equal(ids, rids) and np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    dev.close()
