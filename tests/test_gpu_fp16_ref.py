"""The reference's binary16 distance arithmetic on the GPU (GF_VEC_F16_REF):
per 4-element chunk in its 32-lane order, acc = hfma2(q - x, q - x, acc)
rounded to binary16 at every step, the shfl_down hadd2 tree and
float(acc.x) + float(acc.y) (gpu_graph.cu:3394-3403, 3508-3530).

Bar: ids, distances and counters bit for bit against the oracle's REF_HFMA2
mode (orc.set_dist_mode(1), pinned in tests/test_oracle_fp16.py) for both
traversals and the brute force, on the config-4-shaped world (768-d, 6
chunks per lane) and on 128-d integer rows scaled by 0.01 (1 chunk per lane,
values whose squares round in binary16)."""
import numpy as np
import pytest

from test_gpu_parity import _assert_same, _print_case, _traversal_case

pytestmark = pytest.mark.gpu

VEC_F16_REF = 4


@pytest.mark.parametrize("channels", [1, 2])
@pytest.mark.parametrize("L", [32, 128])
def test_ref_hfma2_traversal_c4(world_c4, L, channels):
    cfg, ix = world_c4
    _print_case("f16ref-traverse-c4", L=L, channels=channels)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, L, vec_dtype=VEC_F16_REF, channels=channels)
    assert st.q_traverse > 0
    _assert_same(ids, dists, ctr, oids, odist, octr, st)


def test_ref_hfma2_bruteforce_c4(world_c4):
    cfg, ix = world_c4
    _print_case("f16ref-bruteforce-c4")
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 32, prefilter=1.0, vec_dtype=VEC_F16_REF)
    assert st.q_bruteforce > 0 and st.bf_mfma == 0   # the gather kernel
    _assert_same(ids, dists, ctr, oids, odist, octr, st)


@pytest.mark.parametrize("prefilter", [0.0, 0.05])
def test_ref_hfma2_r32_scaled(world32, prefilter):
    """128-d integer rows times 0.01: squared differences up to 6.5 and sums
    in the hundreds, where binary16 rounds at 2^-4 .. 2^-2."""
    cfg, ix = world32
    _print_case("f16ref-r32", prefilter=prefilter)
    ids, dists, ctr, oids, odist, octr, st = _traversal_case(cfg, ix, 64, prefilter=prefilter,
                                                             vec_dtype=VEC_F16_REF, f2h_factor=0.01)
    _assert_same(ids, dists, ctr, oids, odist, octr, st)


def test_ref_hfma2_differs_from_fp32_accumulation(world32):
    """The two binary16 modes give different distances on the same rows (the
    mode is not a relabelling of the fp32-accumulated route)."""
    cfg, ix = world32
    _print_case("f16ref-vs-f16")
    _, d4, _, _, _, _, _ = _traversal_case(cfg, ix, 64, vec_dtype=VEC_F16_REF, f2h_factor=0.01, Q=64)
    _, d1, _, _, _, _, _ = _traversal_case(cfg, ix, 64, vec_dtype=1, f2h_factor=0.01, Q=64)
    assert not np.array_equal(d4.view(np.uint32), d1.view(np.uint32))
