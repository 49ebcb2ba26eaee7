"""CPU checks of the boundary: libgarfield.so loads and exports every entry
point include/garfield.h declares, the file formats round-trip, and the C++
loaders reject malformed index files with status codes (no GPU needed: the
files are validated before any device call)."""
import ctypes
import os
import re

import numpy as np
import pytest

from garfield_amd import formats, synth
import garfield_amd._lib as gl

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "garfield.h")).read()
    return sorted(set(re.findall(r"^(?:gf_status|const char\*)\s+(gf_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(gl.lib_path)
    names = _declared()
    assert len(names) >= 18
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(gl._SYMBOLS)


def test_status_strings():
    lib = gl.load()
    assert lib.gf_status_str(0) == b"ok"
    assert lib.gf_status_str(2) == b"i/o error"


def test_entry_points_match_oracle():
    from oracle import oracle as orc
    for N, P, R in ((1_000_000, 16, 32), (100_000, 16, 16), (6000, 16, 16)):
        assert np.array_equal(gl.entry_points(N, P, R), orc.entry_points(N, P, R))


def test_format_round_trips(tmp_path):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((50, 24)).astype(np.float32)
    formats.write_fvecs(tmp_path / "a.fvecs", x)
    assert np.array_equal(formats.read_fvecs(tmp_path / "a.fvecs"), x)
    g = rng.integers(0, 50, (50, 8)).astype(np.uint32)
    formats.write_graph(tmp_path / "g", g)
    assert np.array_equal(formats.read_graph(tmp_path / "g"), g)
    att = synth.uniform_attrs(50, 2, 1, hi=30)
    formats.write_attrs(tmp_path / "at", att)
    assert np.array_equal(formats.read_attrs(tmp_path / "at"), att)
    l_q, r_q, pl, gp = synth.grid_scatter(att, [2, 3])
    formats.write_grid(tmp_path / "grid", [2, 3], l_q, r_q, pl, gp)
    grid, l2, r2, p2, g2 = formats.read_grid(tmp_path / "grid")
    assert list(grid) == [2, 3] and np.array_equal(g2, gp)
    assert all(np.array_equal(u, v) for u, v in zip(l2, l_q))
    lo, hi = synth.ranges_for_selectivity(7, 2, 0.3, 2, hi=30)
    formats.write_ranges(tmp_path / "r", lo, hi)
    l3, h3 = formats.read_ranges(tmp_path / "r", 2)
    assert np.array_equal(l3, lo) and np.array_equal(h3, hi)
    gt = rng.integers(0, 50, (7, 10)).astype(np.uint32)
    formats.write_gt(tmp_path / "gt", gt)
    assert np.array_equal(formats.read_gt(tmp_path / "gt"), gt)
    lab = rng.integers(0, 5, 50).astype(np.int32)
    formats.write_labels(tmp_path / "lab", lab)
    assert np.array_equal(formats.read_labels(tmp_path / "lab"), lab)


def test_grid_matches_reference_layout():
    # grid_scatter_V2: cell j of a dimension holds ranks [j*avg, (j+1)*avg)
    att = np.array([[5, 0], [1, 0], [3, 0], [9, 0], [7, 0]], np.int32)
    l_q, r_q, pl, gp = synth.grid_scatter(att, [2, 1])
    assert list(l_q[0]) == [1, 7] and list(r_q[0]) == [5, 9]
    assert list(pl[0]) == [0, 0, 0, 1, 1]
    assert list(gp) == [0, 0, 0, 1, 1]


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("ix")
    cfg = synth.config_small(N=1200, Q=4, R=8, C=6, sel=0.3, seed=3)
    ix = synth.build_index(cfg["vectors"], cfg["attrs"], [2, 2], 8, 2, 6)
    paths = synth.write_index(ix, str(d / "ix"))
    return d, ix, paths


def _open(paths, **kw):
    try:
        gl.Index.open(**paths, **kw)
    except gl.GarfieldError as e:
        return e.status
    return 0


def test_loader_rejects_missing_and_truncated_files(files):
    d, ix, paths = files
    p = dict(paths)
    p["global_graph"] = str(d / "nope")
    assert _open(p) == 2                                    # GF_E_IO
    raw = open(paths["global_graph"], "rb").read()
    bad = d / "trunc.cross"
    bad.write_bytes(raw[:-12])
    p = dict(paths)
    p["global_graph"] = str(bad)
    assert _open(p) == 3                                    # GF_E_FORMAT (size mismatch)
    assert _open(paths, degree=4) == 3                      # --degree mismatch
    att = formats.read_attrs(paths["attrs"])
    formats.write_attrs(d / "att3", np.concatenate([att, att[:, :1]], 1))
    p = dict(paths)
    p["attrs"] = str(d / "att3")
    assert _open(p) == 3                                    # attribute count differs from grid


def test_loader_rejects_out_of_cell_ids(files):
    d, ix, paths = files
    g = formats.read_graph(paths["cagra_prefix"] + "0" + paths["cagra_suffix"])
    g[3, 2] = g.shape[0] + 5
    formats.write_graph(d / "bad_cell0.graph", g)
    for c in range(1, 4):
        os.link(paths["cagra_prefix"] + f"{c}" + paths["cagra_suffix"], d / f"bad_cell{c}.graph")
    p = dict(paths)
    p["cagra_prefix"] = str(d / "bad_cell")
    assert _open(p) == 3   # GF_E_FORMAT, raised before the device is touched


CLI = os.path.join(ROOT, "garfield_amd", "garfield_search")


def test_cli_usage_and_argument_errors():
    """The driver parses the reference's flags; errors exit 1 before any device call."""
    import subprocess
    assert os.path.exists(CLI), "garfield_search is built with the library"
    r = subprocess.run([CLI, "--help"], capture_output=True, text=True)
    assert r.returncode == 0 and "--prefilter" in r.stdout and "--postfilter" in r.stdout
    r = subprocess.run([CLI, "--data_path", "x"], capture_output=True, text=True)
    assert r.returncode == 1 and "required" in r.stderr
    r = subprocess.run([CLI, "--bogus", "1"], capture_output=True, text=True)
    assert r.returncode == 1 and "unknown flag" in r.stderr
    r = subprocess.run([CLI, "--vec_dtype", "f8"], capture_output=True, text=True)
    assert r.returncode == 1


def test_file_reader_returns_the_written_arrays(files, tmp_path):
    """The C++ index-file reader, built for the CPU, gives back exactly the
    arrays the files were written from (attributes point-major, the grid's
    quantiles as floats, per-cell graphs concatenated in cell order)."""
    import shutil
    import subprocess
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    d, ix, paths = files
    exe = tmp_path / "io_dump"
    subprocess.run([gxx, "-O1", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    os.path.join(ROOT, "tests", "native", "io_dump.cpp"),
                    os.path.join(ROOT, "garfield_amd", "csrc", "gf_io.cpp"), "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe), paths["data_path"][:-len(".fvecs")], str(tmp_path)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    P = int(np.prod(ix["grid"]))
    assert [int(v) for v in r.stdout.split()] == [ix["vectors"].shape[0], ix["vectors"].shape[1],
                                                  ix["attrs"].shape[1], P, ix["R"], ix["cross"].shape[1] // P]
    l_q, r_q = synth.quantile_arrays(ix)
    want = dict(vectors=(ix["vectors"], np.float32), attrs=(ix["attrs"], np.float32), l_q=(l_q, np.float32),
                r_q=(r_q, np.float32), global_pid=(ix["global_pid"], np.uint32),
                cell_graphs=(ix["cell_graphs"], np.uint32), cross=(ix["cross"], np.uint32),
                labels=(ix["labels"], np.int32))
    for name, (ref, t) in want.items():
        got = np.fromfile(tmp_path / name, t)
        np.testing.assert_array_equal(got, np.ascontiguousarray(ref, t).ravel(), err_msg=name)
    # a grid file with trailing bytes is rejected
    bad = tmp_path / "bad"
    for ext in (".fvecs", ".cross", ".attrs", ".cluster"):
        os.link(paths["data_path"][:-len(".fvecs")] + ext, str(bad) + ext)
    for c in range(P):
        os.link(paths["cagra_prefix"] + f"{c}" + paths["cagra_suffix"], f"{bad}_cell{c}.graph")
    open(str(bad) + ".grid", "wb").write(open(paths["grid"], "rb").read() + b"\0\0\0\0")
    r = subprocess.run([str(exe), str(bad), str(tmp_path)], capture_output=True, text=True)
    assert r.returncode == 1 and "trailing" in r.stderr


def test_streamed_plan_validation(files):
    """gf_index_create_streamed rejects bad plans and a device budget below
    two batch images before any device call."""
    d, ix, paths = files
    l_q, r_q = synth.quantile_arrays(ix)
    args = (ix["vectors"], ix["attrs"], ix["grid"], l_q, r_q, ix["global_pid"], ix["cell_graphs"], ix["cross"])

    def status(**kw):
        try:
            gl.Index.create_streamed(*args, **kw)
        except gl.GarfieldError as e:
            return e.status
        return 0

    assert status(plan=[[0, 1], [1, 2]]) == 1          # cell twice
    assert status(plan=[[0, 1], [4]]) == 1             # cell id beyond P = 4
    assert status(plan=[[0, 1], []]) == 1              # empty batch
    assert status(plan=[[0, 1, 2, 3]], device_budget=4096) == 6
    assert status(vec_dtype=gl.VEC_F16) == 6
    bad = ix["vectors"].copy()
    bad[0, 0] = 0.5
    try:
        gl.Index.create_streamed(bad, *args[1:])
        raise AssertionError("non-integer vectors accepted for GF_VEC_U8")
    except gl.GarfieldError as e:
        assert e.status == 1
