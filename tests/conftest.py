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
    cfg = dict(vectors=vec, attrs=att, grid=[4, 4, 4], R=16, E=2, C=16, queries=qv, lo=lo, hi=hi)
    ix = synth.build_index(vec, att, cfg["grid"], 16, 2, 16, seed=6)
    return cfg, ix
