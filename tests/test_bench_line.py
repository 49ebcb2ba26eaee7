"""The bench's stdout line stays small enough for the driver to parse.

The driver reads the line back from a ~16 KB tail of the run's combined
stdout and stderr; a line that carries per-L sweep curves (tens of KB) is cut
and lost.  These tests run on the CPU: they import bench.py's line builder
and feed it a line shaped like a real headline run's.
"""
import importlib.util
import json
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def _headline_like():
    cpu = {"value": 434.5, "unit": "queries/s", "cores": 16, "kind": "port", "route": "filtered brute force",
           "host_cpu": "AMD EPYC 9575F 64-Core Processor", "host_nproc": 256,
           "sample": "6138 random queries of the same batch (6138 on the brute force; same cells, routing, L=10, "
                     "prefilter=1.0), search stage only (stages A/B not timed), OpenMP over queries on 16 "
                     "threads (the GPU box's host-core share for one GPU)",
           "note": "x" * 200}
    cands = [{"prefilter": p, "L": 1700, "recall": 0.95123, "route": "traversal", "channels": 2,
              "qps": 123456.7} for p in (1.0, 0.3, 0.3, 0.2, 0.2, 0.1, 0.1, 0.05, 0.05, 0.0, 0.0)]
    roof = {"bound": "mfma", "kernel": "k_bf_i8", "achieved": 540.3, "peak": 5000.0, "unit": "TFLOP/s",
            "op_kind": "int8 MAC x2 (TOP/s)", "frac": 0.108, "traffic": 361234567,
            "traffic_source": "profiles/traffic_C2.md", "ops_per_launch": 320200000000,
            "pairs_passing": 1250000000, "ops_scheduled_per_launch": 400000000000,
            "bytes_per_launch": 361234567, "ms_per_launch": 0.5896,
            "launch": "one search: three k_bf_i8 launches and the two bound merges between them"}
    trav = {"bound": "hbm", "kernel": "k_traverse_dual", "rows": "f32", "channels": 2, "prefilter": 0.3,
            "L": 600, "recall_at_10": 0.9545, "reaches_target": True, "qps": 703943.1, "queries_traversed": 1408,
            "achieved": 3789.2, "peak": 8000.0, "unit": "GB/s", "frac": 0.4737, "bytes_per_launch": 49712345678,
            "ms_per_launch": 13.12, "traffic": 59312345678, "traffic_source": "profiles/traffic_C2.md"}
    return {"metric": "QPS at recall@10≥0.95, 1M×128 fp32, 2-attr range filter, 1 MI355X", "value": 11479970.1,
            "unit": "queries/s", "n_gpus": 1, "steps": 20, "warmup": 5, "ms_per_step": 0.871,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "i8",
            "data": "synthetic (generated in bench.py; index built on the GPU by the library's builder)",
            "config": {"workload": "C2 headline: " + "w" * 300, "route": "filtered brute force (int8 MFMA)",
                       "channels": 1, "rows": "f32", "N": 1000000, "D": 128, "Q": 10000, "K": 10, "L": 10,
                       "prefilter": 1.0, "postfilter": 1 << 30, "f2h_factor": 1.0, "degree": 32, "graph": "cagra",
                       "recall_at_10": 1.0, "recall_at_10_strict": 1.0, "qps_reference_definition": 12738751.2,
                       "ms_stage_a": 0.123, "ms_stage_b": 0.045, "ms_traverse": 0.0, "ms_bruteforce": 0.61,
                       "q_traverse": 0, "q_bruteforce": 10000, "q_empty": 0, "candidates": cands,
                       "curves_file": "gpurun_out/bench_curves.json"},
            "roofline": roof, "traverse_operating_point": trav, "cpu_baseline": cpu,
            "cpu_baseline_traverse": dict(cpu, route="dual-channel traversal")}


def test_headline_line_fits():
    b = _bench()
    s = b.result_line(_headline_like())
    assert len(s.encode()) <= b.MAX_LINE_BYTES
    back = json.loads(s)
    for k in ("metric", "value", "unit", "roofline", "cpu_baseline", "config"):
        assert k in back
    assert "\n" not in s


def test_line_with_curves_is_refused():
    """The round trip that lost a headline: ten 32-point curves in the line."""
    b = _bench()
    out = _headline_like()
    pt = {"L": 1700, "recall": 0.9438, "recall_strict": 0.9438, "qps_step": 25636.0, "ms_traverse": 388.168,
          "ms_bruteforce": 0.051, "traverse_GBs": 2014.0, "traverse_frac": 0.2518, "q_traverse": 10000,
          "q_bruteforce": 0}
    out["traverse_curve"] = {str(i): [pt] * 32 for i in range(10)}
    with pytest.raises(ValueError, match="traverse_curve"):
        b.result_line(out)


def test_curves_side_file(tmp_path):
    b = _bench()
    p = tmp_path / "sub" / "curves.json"
    b.write_curves(str(p), {"0.0": [{"L": 10, "recall": 0.1}]}, {"Q": 1})
    d = json.loads(p.read_text())
    assert d["curves"]["0.0"][0]["L"] == 10 and d["meta"]["Q"] == 1
    b.write_curves("", {}, {})   # '' writes nothing and does not fail
