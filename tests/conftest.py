import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libgarfield.so)")


@pytest.fixture(scope="session")
def small_world():
    """A small config-1-shaped workload and its exact index (built on the CPU)."""
    from garfield_amd import synth
    cfg = synth.config_small(N=6000, Q=256, R=16, C=24, sel=0.3, seed=7)
    ix = synth.build_index(cfg["vectors"], cfg["attrs"], cfg["grid"], cfg["R"], cfg["E"], cfg["C"], seed=3)
    return cfg, ix


@pytest.fixture(scope="session")
def world32():
    """R=32, mixed selectivity, 4x4 grid (config-2-shaped, shrunk)."""
    from garfield_amd import synth
    rng_sel = synth.log_uniform(192, 0.01, 0.5, 21)
    vec = synth.uniform_int_vectors(8000, 128, 20)
    att = synth.uniform_attrs(8000, 2, 22)
    qv = synth.uniform_int_vectors(192, 128, 23)
    lo, hi = synth.ranges_for_selectivity(192, 2, rng_sel, 24)
    cfg = dict(vectors=vec, attrs=att, grid=[4, 4], R=32, E=2, C=32, queries=qv, lo=lo, hi=hi)
    ix = synth.build_index(vec, att, cfg["grid"], 32, 2, 32, seed=4)
    return cfg, ix


def _float_index_device():
    """Non-integer worlds are built by the library's builder where a GPU is
    present (its float-data mode), by torch on the CPU otherwise."""
    import torch
    return "hip" if torch.cuda.is_available() else "cpu"


@pytest.fixture(scope="session")
def world_gauss():
    """Config-3-shaped (shrunk): 96-d Gaussian unit vectors, 3 Zipf attributes on
    4x4x4 cells, selectivity down to 0.1%: non-integer distances exercise the
    canonical summation order and the gather brute force."""
    from garfield_amd import synth
    Q = 128
    vec = synth.gaussian_unit_vectors(6000, 96, 40)
    att = synth.zipf_attrs(6000, 3, 41, hi=400)
    qv = synth.gaussian_unit_vectors(Q, 96, 42)
    sel = synth.log_uniform(Q, 0.001, 0.5, 43)
    lo, hi = synth.ranges_for_selectivity(Q, 3, sel, 44, hi=400)
    cfg = dict(vectors=vec, attrs=att, grid=[4, 4, 4], R=32, E=2, C=16, queries=qv, lo=lo, hi=hi)
    ix = synth.build_index(vec, att, cfg["grid"], 32, 2, 16, seed=6, device=_float_index_device())
    return cfg, ix


@pytest.fixture(scope="session")
def world_c4():
    """Config-4-shaped (shrunk): 768-d Gaussian mixture (1000 components,
    sigma 0.1 around unit centres) stored as fp16 (f2h_factor 1), 2 attributes
    10 * component + U{0..9} on a 4x4 grid, R = 32, queries at 10% selectivity."""
    from garfield_amd import synth
    N, Q, ncomp = 8000, 64, 1000
    vec, comp = synth.gmm_vectors(N, 768, ncomp, 70)
    att = synth.component_attrs(comp, 2, 71)
    qv, _ = synth.gmm_vectors(Q, 768, ncomp, 72)
    lo, hi = synth.ranges_for_selectivity(Q, 2, 0.1, 73, hi=10 * ncomp)
    cfg = dict(vectors=vec, attrs=att, grid=[4, 4], R=32, E=2, C=16, queries=qv, lo=lo, hi=hi)
    ix = synth.build_index(vec, att, cfg["grid"], 32, 2, 16, seed=74, device=_float_index_device())
    return cfg, ix


def _sub_world(N, D, a, grid, hi_attr, Q, seed):
    from garfield_amd import synth
    vec = synth.uniform_int_vectors(N, D, seed)
    att = synth.uniform_attrs(N, a, seed + 1, hi=hi_attr)
    qv = synth.uniform_int_vectors(Q, D, seed + 2)
    sel = synth.log_uniform(Q, 0.002, 0.6, seed + 3)
    lo, hi = synth.ranges_for_selectivity(Q, a, sel, seed + 4, hi=hi_attr)
    # edge cases: an empty range, ranges beyond the domain, one covering all
    lo[0], hi[0] = 5, 4
    lo[1], hi[1] = hi_attr + 10, hi_attr + 20
    lo[2], hi[2] = -50, -1
    lo[3], hi[3] = -5, hi_attr + 5
    cfg = dict(vectors=vec, attrs=att, grid=grid, R=16, E=2, C=16, queries=qv, lo=lo, hi=hi)
    ix = synth.build_index(vec, att, grid, 16, 2, 16, seed=seed + 5)
    return cfg, ix


@pytest.fixture(scope="session")
def world_sub2():
    """Cells of 15k points (16 sub-cells each), 2 attributes, 64-d integer data."""
    return _sub_world(60000, 64, 2, [2, 2], 10000, 160, 60)


@pytest.fixture(scope="session")
def world_sub3():
    """3 attributes (two packed words) with many ties, 2x2x2 cells of 5k points."""
    return _sub_world(40000, 128, 3, [2, 2, 2], 400, 128, 70)
