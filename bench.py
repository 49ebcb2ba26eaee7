#!/usr/bin/env python
"""Headline benchmark: QPS at recall@10 >= 0.95 on the headline config (C2).

Workload (synthetic, generated here): 1M x 128 fp32 integer vectors in
[0,255], 2 uint32 attributes uniform in [0,10000) on a 4x4 rank-quantile grid,
per-cell exact kNN graphs of degree 32 plus 2 exact cross edges per (point,
cell), 1000 k-means centres, 10k queries with range selectivity log-uniform in
[1%, 50%], k = 10.  The index and the exact filtered ground truth are built on
the GPU with torch before any timing (index construction is not the product).

A "step" is one pass of the hot path over the 10k-query batch with inputs
resident in HBM: stage A (cells + prefilter routing), stage B (cluster-guided
cell order) and stage C (traversal / brute force, results copied to the host).
The (L, prefilter) operating point is the one with the highest QPS among the
reference's L sweep (realdataset_search.cu:2757) whose tie-aware recall@10
reaches the target.  Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "QPS at recall@10≥0.95, 1M×128 fp32, 2-attr range filter, 1 MI355X"
L_SWEEP = [10, 15, 20, 25, 30, 35, 40, 45, 50, 55, 60, 70, 80, 90, 100, 120, 140, 160, 180, 200, 250,
           300, 400, 500, 600, 700, 800, 900, 1000, 1100, 1400, 1700]
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
FP16_PEAK_TFLOPS = 2500.0 # MI355X dense fp16 MFMA, 2.5 PFLOP/s
FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA
# The result line is read back from the tail of the run's combined output,
# which holds about 16 KB: the line and everything logged to stderr must fit.
MAX_LINE_BYTES = 6000
DEFAULT_CURVES = os.path.join("gpurun_out", "bench_curves.json")

VERBOSE = False


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def vlog(*a):
    """Per-point progress (every L of a sweep): only with --verbose, so the
    default run's stderr stays a few KB."""
    if VERBOSE:
        log(*a)


def result_line(out):
    """The one stdout JSON line.  Raises if it would not fit the tail the
    driver parses (bulky per-L curves belong in the side file)."""
    s = json.dumps(out, separators=(",", ":"))
    if len(s.encode()) > MAX_LINE_BYTES:
        raise ValueError(f"result line is {len(s.encode())} bytes (> {MAX_LINE_BYTES}); "
                         f"largest keys: {sorted(out, key=lambda k: -len(json.dumps(out[k])))[:3]}")
    return s


def write_curves(path, curves, meta):
    """Full recall / QPS sweeps, keyed like the operating points, to a side
    file (created with its folder)."""
    if not path:
        return
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    with open(path, "w") as f:
        json.dump({"meta": meta, "curves": curves}, f)
    log(f"sweep curves written to {path}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", choices=["headline", "small", "c3", "c4"], default="headline",
                    help="headline: C2 (the metric's config); c3, c4: the non-integer configs, each with its own "
                         "metric string (the fp32 and fp16 distance paths)")
    ap.add_argument("--workload", choices=["resident", "stream", "build"], default="resident",
                    help="stream: the C5-shaped out-of-core workload; build: the index builder on the "
                         "headline index (each its own JSON line, not the headline)")
    ap.add_argument("--stream-n", type=int, default=1_000_000)
    ap.add_argument("--stream-q", type=int, default=10_000)
    ap.add_argument("--stream-budget-mb", type=int, default=64)
    ap.add_argument("--stream-thresholds", default="1.0,0.25,0.0")
    ap.add_argument("--cross-search-ef", type=int, default=32,
                    help="build workload: list length of the search-based cross edges timed beside the exact ones")
    ap.add_argument("--stream-plan", choices=["best", "planned", "static"], default="best",
                    help="stream workload: the plan of the headline value; both are timed on one index (planned: "
                         "batches planned per step from the query batch's cell lists, gf_batch_plan_stream; static: "
                         "the reference's 16 consecutive cells per batch); best: the faster")
    ap.add_argument("--recall", type=float, default=0.95)
    ap.add_argument("--prefilters", default="1.0,0.3,0.2,0.1,0.05,0.0",
                    help="1.0 = every query to the filtered brute force; below 1, queries whose "
                         "selectivity is at most the value take the brute force, the rest traverse")
    ap.add_argument("--postfilter", type=int, default=1 << 30)
    ap.add_argument("--L", type=int, default=0, help="fixed L (skip the sweep)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--graph", choices=["knn", "cagra"], default="cagra",
                    help="per-cell graphs: exact kNN, or optimised (pruned + reverse edges) as cagra.build returns")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traverse", action="store_true", help="skip the traversal roofline line")
    ap.add_argument("--traverse-L", type=int, default=100)
    ap.add_argument("--channels", default="1,2",
                    help="traversals swept: 1 cell-by-cell (gf_search), 2 dual-channel (gf_search_dual)")
    ap.add_argument("--rows", choices=["auto", "f32", "u8", "f16", "f16ref"], default="auto",
                    help="row storage of the resident index (auto: f16 for c4, else f32; u8 is exact for the "
                         "integer-valued configs C1 and C2; f16ref: binary16 rows with the reference's "
                         "binary16 distance arithmetic)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="after the run, stream this many MiB through y = x + 1 (fp32) three times: a kernel "
                         "of known traffic (reads and writes that many bytes) to scale rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--curves-out", default=DEFAULT_CURVES,
                    help="file for the full per-L sweep curves ('' = do not write)")
    ap.add_argument("--verbose", action="store_true", help="log every point of the sweeps to stderr")
    args = ap.parse_args()
    global VERBOSE
    VERBOSE = args.verbose
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the query path shards over "
              "queries with no exchange between GPUs", file=sys.stderr)
        sys.exit(2)

    import torch
    import garfield_amd as gf
    from garfield_amd import synth
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.workload == "stream":
        return stream_bench(args)
    if args.workload == "build":
        return build_bench(args)

    t0 = time.time()
    if args.config == "headline":
        cfg = synth.config_headline()
        workload = ("C2 headline: 1M x 128 fp32 (integers 0-255), 2 uint32 attrs on a 4x4 grid, "
                    f"R=32 per-cell graphs ({'exact 64-NN optimised to 32 (pruned + reverse edges)' if args.graph == 'cagra' else 'exact 32-NN'})"
                    " + E=2 exact cross edges, C=1000, 10k queries, selectivity log-U[1%,50%], k=10")
    elif args.config == "c3":
        cfg = synth.config_c3()
        workload = ("C3: 1M x 96 fp32 Gaussian unit vectors, 3 Zipf(1.1) attrs on a 4x4x4 grid, R=32 per-cell "
                    "graphs (exact 48-NN of the builder's float mode optimised to 32) + E=2 cross edges, C=1000, "
                    "10k queries, selectivity log-U[0.1%,50%], k=10")
    elif args.config == "c4":
        cfg = synth.config_c4()
        workload = ("C4: 1M x 768 Gaussian mixture (1000 components, sigma 0.1) stored as fp16 (f2h_factor 1), "
                    "2 attrs 10*component+U{0..9} on 4x4, R=32 per-cell graphs (exact 48-NN of the builder's "
                    "float mode optimised to 32) + E=2 cross edges, C=1000, 10k queries at 10%, k=10")
    else:
        cfg = synth.config_small()
        workload = "C1: 100k x 128 fp32 (integers 0-255), 2 attrs on 4x4, R=16, E=2, C=100, 1k queries at 30%, k=10"
    metric = {"c3": "QPS at recall@10≥0.95, 1M×96 fp32, 3-attr range filter, 1 MI355X",
              "c4": "QPS at recall@10≥0.95, 1M×768 fp16, 2-attr range filter, 1 MI355X"}.get(args.config, METRIC)
    floatcfg = args.config in ("c3", "c4")
    # C1 / C2 hold integers in [0, 255]: u8 rows (--rows u8) give the same
    # distances as fp32 rows bit for bit (every partial sum is an integer
    # below 2^24) at a quarter of the bytes per row gather
    rows = args.rows if args.rows != "auto" else ("f16" if args.config == "c4" else "f32")
    vec_dtype = {"f32": gf.VEC_F32, "u8": gf.VEC_U8, "f16": gf.VEC_F16, "f16ref": gf.VEC_F16_REF}[rows]
    N, D = cfg["vectors"].shape
    Q = cfg["queries"].shape[0]
    log(f"data generated N={N} D={D} Q={Q} ({time.time() - t0:.1f}s)")
    t1 = time.time()
    # float data: the builder's candidate lists hold at most 63 entries
    ix = synth.build_index(cfg["vectors"], cfg["attrs"], cfg["grid"], cfg["R"], cfg["E"], cfg["C"],
                           device="hip", graph=args.graph, inter=48 if floatcfg else 64)
    log(f"index built on GPU in {time.time() - t1:.1f}s ({args.graph} graphs)")
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    t1 = time.time()
    gt_ids, gt_dist = synth.ground_truth_torch(cfg["vectors"], cfg["attrs"], cfg["queries"], lo, hi, 10)
    # the tie test compares float64 distances: the ground truth's own in
    # float64 too (exact for integer data either way)
    gt_dist = synth.exact_result_dist(cfg["vectors"], cfg["queries"], gt_ids)
    log(f"ground truth in {time.time() - t1:.1f}s")
    torch.cuda.empty_cache()

    t1 = time.time()
    dev = synth.open_device_index(ix, vec_dtype=vec_dtype, f2h_factor=1.0)
    b = dev.batch(cfg["queries"], lo, hi)
    log(f"library index resident ({dev.device_bytes / 2**30:.2f} GiB) in {time.time() - t1:.1f}s")

    # page-locked result arrays: the search copies into them directly
    out = (gf.pinned_empty((Q, 10), np.uint32), gf.pinned_empty((Q, 10), np.float32))

    def step(prefilter, L, ch=1):
        # Stages A and B are enqueued without waiting; the search reports
        # their device times after its one synchronisation.  The result
        # arrays are reused from step to step, page-locked, so the search's
        # device-to-host copies land in them directly.
        b.mark_cells(prefilter, timed=False)
        b.order_cells(4, timed=False)
        ids, dists, st = b.search(L=L, K=10, rl=10, postfilter=args.postfilter, out=out, channels=ch)
        return ids, dists, st, st.ms_stage_a, st.ms_stage_b

    def recall(ids):
        ex = synth.exact_result_dist(cfg["vectors"], cfg["queries"], ids)
        return synth.recall_at_k(ids, ex, gt_ids, gt_dist)

    def recall_by_selectivity(ids):
        """Tie-aware recall of the queries in each band of their selectivity."""
        ex = synth.exact_result_dist(cfg["vectors"], cfg["queries"], ids)
        _, tie = synth.recall_at_k(ids, ex, gt_ids, gt_dist, per_query=True)
        sel = np.asarray(cfg["sel"])
        edges = [0.0, 0.02, 0.05, 0.1, 0.2, 1.0]
        out = []
        for a, b in zip(edges[:-1], edges[1:]):
            m = (sel >= a) & (sel < b)
            if m.any():
                out.append(f"sel[{a:g},{b:g}):{tie[m].mean():.3f}(n={int(m.sum())})")
        return " ".join(out)

    def timed(prefilter, L, steps, warmup, ch=1):
        """steps timed passes after warmup; sums of the device times and the
        algorithmic work the search statistics report."""
        for _ in range(warmup):
            step(prefilter, L, ch)
        torch.cuda.synchronize()
        acc = dict(a=0.0, b=0.0, tr=0.0, bf=0.0, bfk=0.0, btr=0.0, bbf=0.0, obf=0.0)
        t = time.perf_counter()
        for _ in range(steps):
            ids, dists, st, ms_a, ms_b = step(prefilter, L, ch)
            acc["a"] += ms_a
            acc["b"] += ms_b
            acc["tr"] += st.ms_traverse
            acc["bf"] += st.ms_bruteforce
            acc["bfk"] += st.ms_bf_kernel
            acc["btr"] += st.bytes_traverse
            acc["bbf"] += st.bytes_bruteforce
            acc["obf"] += st.ops_bruteforce
        torch.cuda.synchronize()
        acc["elapsed"] = time.perf_counter() - t
        return ids, st, acc

    # Operating points.  The brute-force route (prefilter 1: every query to
    # the filtered brute force, exact at any L) and, for each traversal
    # prefilter, the smallest L of the reference's sweep reaching the target,
    # read off a full sweep (no early stop), which is reported as the
    # traversal curve.
    # Traversal curves are keyed by prefilter, with "dual:" before the
    # prefilter for the dual-channel traversal.
    channels = [int(x) for x in args.channels.split(",")]
    candidates = []
    curves = {}
    for pf, ch in [(float(x), c) for x in args.prefilters.split(",") for c in channels]:
        if pf >= 1.0:
            if ch != channels[0]:
                continue
            ids, dists, st, _, _ = step(pf, 10)
            strict, tie = recall(ids)
            log(f"prefilter={pf}: recall={tie:.4f} (strict {strict:.4f}) q_bf={st.q_bruteforce}")
            if tie >= args.recall:
                candidates.append(dict(prefilter=pf, L=10, recall=tie, strict=strict, route="bruteforce",
                                       channels=1))
            continue
        curve = []
        for L in ([args.L] if args.L else L_SWEEP):
            t = time.perf_counter()
            ids, dists, st, ms_a, ms_b = step(pf, L, ch)
            wall = time.perf_counter() - t
            strict, tie = recall(ids)
            gbs = st.bytes_traverse / max(st.ms_traverse, 1e-9) / 1e6
            curve.append({"L": L, "recall": round(tie, 4), "recall_strict": round(strict, 4),
                          "qps_step": round(Q / wall, 1), "ms_traverse": round(st.ms_traverse, 3),
                          "ms_bruteforce": round(st.ms_bruteforce, 3), "traverse_GBs": round(gbs, 1),
                          "traverse_frac": round(gbs / HBM_PEAK_GBS, 4), "q_traverse": st.q_traverse,
                          "q_bruteforce": st.q_bruteforce})
            vlog(f"{'dual ' if ch == 2 else ''}prefilter={pf} L={L}: recall={tie:.4f} (strict {strict:.4f}) step={wall * 1e3:.1f}ms "
                 f"trav={st.ms_traverse:.1f}ms ({gbs:.0f} GB/s) bf={st.ms_bruteforce:.1f}ms A={ms_a:.2f}ms "
                 f"B={ms_b:.2f}ms q_trav={st.q_traverse} q_bf={st.q_bruteforce}")
            if VERBOSE and pf == 0.0 and "sel" in cfg and L in (100, 600, 1100, 1700):
                vlog(f"  recall by selectivity: {recall_by_selectivity(ids)}")
        curves[("dual:" if ch == 2 else "") + str(pf)] = curve
        reach = [c for c in curve if c["recall"] >= args.recall]
        sel = [c for c in curve if c["L"] in (100, 600, 1100, 1700)]
        log(f"sweep channels={ch} prefilter={pf}: " +
            " ".join(f"L{c['L']}:{c['recall']:.3f}@{c['traverse_frac']:.2f}HBM" for c in sel) +
            (f"; target at L={reach[0]['L']}" if reach else "; target not reached"))
        if reach:
            c = reach[0]
            candidates.append(dict(prefilter=pf, L=c["L"], recall=c["recall"], strict=c["recall_strict"],
                                   route="traversal", channels=ch))
    if not candidates:
        raise SystemExit("no operating point reached the recall target")
    for c in candidates:
        _, _, acc = timed(c["prefilter"], c["L"], max(3, args.steps // 4), 1, c["channels"])
        c["qps"] = Q * max(3, args.steps // 4) / acc["elapsed"]
        log(f"candidate {c['route']} channels={c['channels']} prefilter={c['prefilter']} L={c['L']}: "
            f"{c['qps']:.0f} QPS")
    best = max(candidates, key=lambda c: c["qps"])
    pf, L, bch = best["prefilter"], best["L"], best["channels"]
    log(f"operating point: {best['route']} channels={bch} prefilter={pf} L={L} recall={best['recall']:.4f}")

    ids, last, acc = timed(pf, L, args.steps, args.warmup, bch)
    elapsed = acc["elapsed"]
    K = args.steps
    strict, tie = recall(ids)
    qps = Q * K / elapsed
    ms_per_step = elapsed * 1e3 / K
    ms_a_sum, ms_b_sum, ms_tr, ms_bf, ms_bfk = acc["a"], acc["b"], acc["tr"], acc["bf"], acc["bfk"]
    qps_ref = Q / ((ms_a_sum + ms_b_sum + ms_tr + ms_bf) / K / 1e3)
    # Dominant kernel: the one with the larger device time in the timed steps.
    traffic = profiled_traffic() if args.config == "headline" else {}
    if ms_tr >= ms_bf:
        dom, dom_bytes, dom_ms, mfma = ("k_traverse_dual" if bch == 2 else "k_traverse"), acc["btr"], ms_tr, False
    else:
        mfma = bool(last.bf_mfma)
        # the MFMA kernel alone (its schedule and the final merge are timed in ms_bruteforce)
        dom = {1: "k_bf_i8", 2: "k_bf_f16" if vec_dtype == gf.VEC_F16 else "k_bf_f32"}.get(int(last.bf_mfma),
                                                                                         "k_bruteforce")
        dom_bytes, dom_ms = acc["bbf"], (ms_bfk if mfma else ms_bf)
    if mfma:
        # Algorithmic work of the int8 brute force: D multiply-adds (2 D ops)
        # per (query, point) pair that passes the query's filter.  The
        # kernel evaluates every point of every sub-cell a range reaches
        # (ops_scheduled); the pairs that pass come from the exact counts,
        # made once after the timed steps (with prefilter >= 1 stage A routes
        # without them).
        ctr = b.get_counters()
        n_pass = int(ctr[ctr[:, 7] == 2, 6].sum(dtype=np.int64))
        ops_alg = 2.0 * D * n_pass
        achieved = ops_alg / (dom_ms / K / 1e3) / 1e12 if dom_ms > 0 else 0.0
        tr = traffic.get(dom)
        f16 = dom in ("k_bf_f16", "k_bf_f32")
        peak = {"k_bf_f16": FP16_PEAK_TFLOPS, "k_bf_f32": FP32_PEAK_TFLOPS}.get(dom, INT8_PEAK_TOPS)
        roofline = {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                    "peak": peak, "unit": "TFLOP/s",
                    "op_kind": {"k_bf_f16": "fp16 MAC x2 (TFLOP/s)", "k_bf_f32": "fp32 MAC x2 (TFLOP/s)"}.get(
                        dom, "int8 MAC x2 (TOP/s)"),
                    "frac": round(achieved / peak, 4),
                    "traffic": tr["bytes"] if tr else None,
                    "traffic_source": tr["source"] if tr else None,
                    "ops_per_launch": round(ops_alg), "pairs_passing": n_pass,
                    "ops_scheduled_per_launch": round(acc["obf"] / K),
                    "bytes_per_launch": round(dom_bytes / K), "ms_per_launch": round(dom_ms / K, 4),
                    "launch": (f"one search: one {dom} launch (the exact re-rank k_bf_f16_final is not in it)"
                               if f16 else
                               "one search: three k_bf_i8 launches and the two bound merges between them")}
        dom_desc = f"{achieved:.1f} {'TFLOP/s' if f16 else 'TOP/s'}"
    else:
        achieved = (dom_bytes / K) / (dom_ms / K / 1e3) / 1e9 if dom_ms > 0 else 0.0
        tr = traffic.get(dom)
        roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": tr["bytes"] if tr else None, "traffic_source": tr["source"] if tr else None,
                    "bytes_per_launch": round(dom_bytes / K), "ms_per_launch": round(dom_ms / K, 4)}
        dom_desc = f"{achieved:.0f} GB/s"
    log(f"timed: {qps:.0f} QPS end-to-end, {qps_ref:.0f} QPS (reference definition), "
        f"{dom} {dom_ms / K:.2f} ms at {dom_desc}")

    # The traversal route at its own operating point (the smallest L reaching
    # the target with prefilter 0, else with the other traversal prefilter),
    # timed, with k_traverse priced against HBM.
    trav = None
    if not args.no_traverse:
        tc = [c for c in candidates if c["route"] == "traversal"]
        if tc:
            tp = max(tc, key=lambda c: c["qps"])
            tpf, tL, trec, tch = tp["prefilter"], tp["L"], tp["recall"], tp["channels"]
        else:
            tpf, tL, trec, tch = 0.0, args.traverse_L, None, 1
        tsteps = max(3, args.steps // 4)
        tids, stt, tacc = timed(tpf, tL, tsteps, 1, tch)
        ms_t = tacc["tr"] / tsteps
        gbs = tacc["btr"] / tsteps / (ms_t / 1e3) / 1e9 if ms_t > 0 else 0.0
        tkern = "k_traverse_dual" if tch == 2 else "k_traverse"
        tr = traffic.get(f"{tkern}@{tpf}:{tL}" + ("" if rows == "f32" else f":{rows}"))
        trav = {"bound": "hbm", "kernel": tkern, "rows": rows, "channels": tch, "prefilter": tpf, "L": tL,
                "recall_at_10": round(recall(tids)[1], 4), "reaches_target": trec is not None,
                "qps": round(Q * tsteps / tacc["elapsed"], 1), "queries_traversed": stt.q_traverse,
                "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": round(tacc["btr"] / tsteps),
                "ms_per_launch": round(ms_t, 4), "traffic": tr["bytes"] if tr else None,
                "traffic_source": tr["source"] if tr else None}
        log(f"traversal route: channels={tch} prefilter={tpf} L={tL}: {trav['qps']:.0f} QPS, recall "
            f"{trav['recall_at_10']}, {tkern} {ms_t:.2f} ms, {gbs:.0f} GB/s algorithmic "
            f"({gbs / HBM_PEAK_GBS:.1%} of HBM)")

    cpu = cpu_trav = None
    if not args.no_cpu:
        f16 = vec_dtype in (gf.VEC_F16, gf.VEC_F16_REF)
        ref16 = vec_dtype == gf.VEC_F16_REF
        cpu = cpu_baseline(cfg, ix, b, L, pf, args, bch, f16, ref16)
        if trav is not None and best["route"] != "traversal":
            cpu_trav = cpu_baseline(cfg, ix, b, trav["L"], trav["prefilter"], args, trav["channels"], f16, ref16)

    out = {
        "metric": metric,
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8" if (last.bf_mfma == 1 and ms_bf > ms_tr) else (
            "f16" if vec_dtype in (gf.VEC_F16, gf.VEC_F16_REF) else "f32"),
        "data": "synthetic (generated in bench.py; index built on the GPU by the library's builder)",
        "config": {
            "workload": workload,
            "route": ({1: "filtered brute force (int8 MFMA query-batch kernel)",
                       2: "filtered brute force (float MFMA query-batch kernel, candidates re-ranked exactly)"}.get(
                           int(last.bf_mfma), "filtered brute force (gather kernel)") if best["route"] == "bruteforce"
                      else ("dual-channel" if bch == 2 else "cell-by-cell") +
                      " graph traversal (queries at or below the prefilter selectivity to filtered brute force)"),
            "channels": bch,
            "rows": rows,
            "N": N, "D": D, "Q": Q, "K": 10, "L": L,
            "prefilter": pf, "postfilter": args.postfilter, "f2h_factor": 1.0, "degree": cfg["R"],
            "graph": args.graph,
            "recall_at_10": round(tie, 4), "recall_at_10_strict": round(strict, 4),
            "qps_reference_definition": round(qps_ref, 1),
            "ms_stage_a": round(ms_a_sum / K, 3), "ms_stage_b": round(ms_b_sum / K, 3),
            "ms_traverse": round(ms_tr / K, 3), "ms_bruteforce": round(ms_bf / K, 3),
            "q_traverse": last.q_traverse, "q_bruteforce": last.q_bruteforce, "q_empty": last.q_empty,
            "candidates": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in c.items()
                            if k != "strict"} for c in candidates],
            "curves_file": args.curves_out or None,
        },
        "roofline": roofline,
        "traverse_operating_point": trav,
        "cpu_baseline": cpu,
        "cpu_baseline_traverse": cpu_trav,
    }
    write_curves(args.curves_out, curves, {"config": args.config, "graph": args.graph, "rows": rows,
                                           "recall_target": args.recall, "Q": Q})
    print(result_line(out), flush=True)
    if args.calib_copy_mb:
        n = args.calib_copy_mb * (1 << 20) // 4
        x = torch.zeros(n, dtype=torch.float32, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            torch.add(x, 1.0, out=y)
        torch.cuda.synchronize()
        log(f"calibration: 3 x y = x + 1 over {args.calib_copy_mb} MiB (reads and writes {n * 4} bytes each)")


def profiled_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE, then
    WRITE_SIZE, each scaled by a copy kernel of known size) and committed in
    profiles/traffic_C2.md as lines `traffic <kernel> <bytes>`; bench.py
    cannot read hardware counters from inside its own process."""
    path = os.path.join(ROOT, "profiles", "traffic_C2.md")
    out = {}
    if not os.path.exists(path):
        return out
    for line in open(path):
        parts = line.split()
        if len(parts) == 3 and parts[0] == "traffic":
            out[parts[1]] = {"bytes": int(float(parts[2])), "source": "profiles/traffic_C2.md"}
    return out


PCIE_PEAK_GBS = 64.0   # PCIe 5.0 x16, one direction


def build_bench(args):
    """Index build of the headline index (1M x 128 u8, 4x4 rank-quantile
    cells, R = 32, E = 2): a step is gf_grid_scatter plus gf_build_graphs from
    host arrays to host arrays (uploads, int8 tiles, per-cell graphs, cross
    edges, downloads), plus gf_kmeans labels (C = 1000, 8 rounds).  The roofline is the cross-edge kernel's int8 MFMA rate
    on its algorithmic work: D multiply-adds (2 D ops) per (point, candidate)
    pair, N * N pairs."""
    import garfield_amd._lib as gl
    from garfield_amd import synth
    cfg = synth.config_headline()
    v = cfg["vectors"].astype(np.uint8)
    att = cfg["attrs"].astype(np.float32)
    N, D = v.shape
    R, E, P = cfg["R"], cfg["E"], int(np.prod(cfg["grid"]))

    def step():
        _, _, _, gp = gl.grid_scatter(att, cfg["grid"])
        g, x, st = gl.build_graphs(v, gp, P, R, E)
        lab, _, ms_km = gl.kmeans(v, cfg["C"], 8, seed=5)
        return gp, g, x, st, ms_km

    for _ in range(args.warmup):
        step()
    acc = dict(tiles=0.0, graph=0.0, cross=0.0, prep=0.0, upload=0.0, run=0.0, download=0.0, total=0.0)
    ms_kmeans = 0.0
    t = time.perf_counter()
    for _ in range(args.steps):
        gp, g, x, st, ms_km = step()
        ms_kmeans += ms_km
        for k in acc:
            acc[k] += getattr(st, "ms_" + k)
    elapsed = time.perf_counter() - t
    K = args.steps
    ms_cross = acc["cross"] / K
    tops = 2.0 * st.dim * st.pairs_cross / (ms_cross * 1e-3) / 1e12
    tops_g = 2.0 * st.dim * st.pairs_graph / (acc["graph"] / K * 1e-3) / 1e12
    log(f"build: {elapsed * 1e3 / K:.1f} ms per step; kernels: tiles {acc['tiles'] / K:.2f} ms, graphs "
        f"{acc['graph'] / K:.2f} ms ({tops_g:.0f} TOP/s), cross {ms_cross:.2f} ms ({tops:.0f} TOP/s); "
        f"gf_build_graphs {acc['total'] / K:.1f} ms = prep {acc['prep'] / K:.1f} + upload {acc['upload'] / K:.1f} "
        f"+ run {acc['run'] / K:.1f} + download {acc['download'] / K:.1f}; gf_kmeans (C={cfg['C']}, 8 rounds) "
        f"{ms_kmeans / K:.1f} ms")
    # Cross edges by per-cell graph search (global_graph_build.py's method,
    # the route to indexes too large for N x N distances), on the same graphs:
    # time and the share of the exact edges it finds.
    from garfield_amd.global_graph import global_graph_build
    t0 = time.perf_counter()
    xs = global_graph_build(v, gp, P, g, E, ef=args.cross_search_ef, batch=1 << 17)
    ms_xs = (time.perf_counter() - t0) * 1e3
    samp = np.random.default_rng(1).choice(N, 2000, replace=False)
    found = np.mean([len(set(xs[p, c * E:(c + 1) * E]) & set(x[p, c * E:(c + 1) * E])) / E
                     for p in samp for c in range(P)])
    log(f"cross edges by per-cell search (ef={args.cross_search_ef}): {ms_xs:.0f} ms, "
        f"{found:.4f} of the exact edges found")
    cpu = None
    if not args.no_cpu:
        # the oracle's exact rows (numpy, float64 BLAS dot products) for a
        # sample of points: each row is the same work as in the full build
        from oracle import oracle as orc
        rng = np.random.default_rng(3)
        S, t_cpu, done = 16, 0.0, 0
        while t_cpu < args.cpu_seconds and done < 4096:
            rows = rng.choice(N, S, replace=False)
            t0 = time.perf_counter()
            orc.cross_rows(v, gp, P, E, rows)
            orc.graph_rows(v, gp, P, R, rows)
            t_cpu += time.perf_counter() - t0
            done += S
            S *= 2
        cpu = {"value": round(done / t_cpu, 1), "unit": "points/s", "cores": os.cpu_count(),
               "kind": "port", "sample": f"{done} random points' cross-edge and graph rows (oracle, numpy + BLAS)"}
    out = {
        "metric": "index build throughput, headline index (grid, exact per-cell kNN + cross edges, k-means labels), 1 MI355X",
        "value": round(N * K / elapsed, 1), "unit": "points/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(elapsed * 1e3 / K, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (generated in bench.py; host arrays in and out, PCIe included)",
        "config": {"workload": f"build: {N} x {D} u8 (integers 0-255), 2 attrs on a 4x4 rank-quantile grid, "
                               f"R={R} exact per-cell kNN, E={E} cross edges, k-means labels C={cfg['C']}",
                   "N": N, "D": D, "P": P, "R": R, "E": E,
                   "ms_tiles": round(acc["tiles"] / K, 3), "ms_graph": round(acc["graph"] / K, 3),
                   "ms_cross": round(ms_cross, 3), "pairs_cross": st.pairs_cross, "pairs_graph": st.pairs_graph,
                   "ms_call": round(acc["total"] / K, 3), "ms_host_prep": round(acc["prep"] / K, 3),
                   "ms_upload": round(acc["upload"] / K, 3), "ms_download": round(acc["download"] / K, 3),
                   "C": cfg["C"], "kmeans_rounds": 8, "ms_kmeans": round(ms_kmeans / K, 3),
                   "cross_by_search": {"ef": args.cross_search_ef, "ms": round(ms_xs, 1),
                                       "exact_edges_found": round(float(found), 4),
                                       "searches": N * P}},
        "roofline": {"bound": "mfma", "kernel": "k_knn_i8 (cross edges)", "achieved": round(tops, 1),
                     "peak": INT8_PEAK_TOPS, "unit": "TOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                     "traffic": None, "ms_per_launch": round(ms_cross, 4)},
        "cpu_baseline": cpu,
    }
    print(result_line(out), flush=True)


def stream_bench(args):
    """C5-shaped out-of-core search on one GPU: the index is streamed from
    pinned host memory under a device budget far below its size (config
    synth.config_stream).  One streamed index serves two batch plans without
    a re-pack, timed the same way: the reference's static plan of 16
    consecutive cells per batch (the index's build-time plan) and the batches
    planned from each query batch's own stage A cell lists
    (gf_batch_plan_stream, inside the timed step).  A step is stage A on the
    arithmetic grid, the planning (planned plan), and the streamed search of
    the whole query batch (every batch image crosses PCIe once per step).
    The headline is the faster plan (--stream-plan picks one instead)."""
    import torch
    import garfield_amd._lib as gl
    from garfield_amd import synth
    t0 = time.time()
    cfg = synth.config_stream(N=args.stream_n, Q=args.stream_q)
    N, D = cfg["vectors"].shape
    Q = cfg["queries"].shape[0]
    amin, width = cfg["attr_min"], cfg["attr_width"]
    ix = synth.build_index(cfg["vectors"], cfg["attrs"], cfg["grid"], cfg["R"], cfg["E"], 0, device="hip",
                           arith=(amin, width))
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    gt_ids, gt_dist = synth.ground_truth_torch(cfg["vectors"], cfg["attrs"], cfg["queries"], lo, hi, 10)
    torch.cuda.empty_cache()
    log(f"stream workload built in {time.time() - t0:.1f}s: N={N} D={D} Q={Q} P={ix['P']}")
    P = ix["P"]
    block = [list(range(i, min(P, i + 16))) for i in range(0, P, 16)]   # bigdataset_experiment.cu:271-277
    l_q, r_q = synth.quantile_arrays(ix)
    budget = args.stream_budget_mb << 20
    sizes = synth.cell_sizes(ix)
    # planned batches hold at most 16 cells and the static plan's largest
    # batch's points, so that the same device buffers hold them
    maxpts = max(int(sizes[bt].sum()) for bt in block)

    t1 = time.time()
    sx = gl.Index.create_streamed(ix["vectors"], ix["attrs"], ix["grid"], l_q, r_q, ix["global_pid"],
                                  ix["cell_graphs"], ix["cross"], plan=block, device_budget=budget,
                                  vec_dtype=gl.VEC_U8)
    resident_bytes = N * (D + ix["R"] * 4 + 2 * 4 + 8 + ix["P"] * ix["E"] * 4)
    log(f"streamed index made in {time.time() - t1:.1f}s: build-time plan {len(block)} batches, device "
        f"{sx.device_bytes / 2**20:.1f} MiB (budget {args.stream_budget_mb} MiB; a resident copy needs "
        f"{resident_bytes / 2**30:.2f} GiB)")
    b = sx.batch(cfg["queries"], lo, hi)
    kinds = {"static": "16 consecutive cells per batch (bigdataset_experiment.cu:271-277), the index's build-time plan",
             "planned": (f"planned per step from the query batch's cell lists (gf_batch_plan_stream, <= 16 cells and "
                         f"{maxpts} points per batch)")}

    def step(thr, L, plan):
        ms_a = b.mark_cells_grid(amin, width, thr)
        ms_p = 0.0
        if plan:
            _, _, ms_p = b.plan_stream(max_points=maxpts, max_cells=16)
        ids, dists, st = b.search(L=L, K=10, rl=10)
        return ids, st, ms_a, ms_p

    def recall(ids):
        ex = synth.exact_result_dist(cfg["vectors"], cfg["queries"], ids)
        return synth.recall_at_k(ids, ex, gt_ids, gt_dist)

    # the operating point (on the build-time plan; planning changes which
    # batch a cell is searched in, not what is searched)
    points = []
    for thr in [float(x) for x in args.stream_thresholds.split(",")]:
        for L in ([args.L] if args.L else L_SWEEP):
            t = time.perf_counter()
            ids, st, ms_a, _ = step(thr, L, False)
            wall = time.perf_counter() - t
            strict, tie = recall(ids)
            vlog(f"threshold={thr} L={L}: recall={tie:.4f} step={wall * 1e3:.1f}ms total={st.ms_total:.1f}ms "
                f"h2d={st.ms_h2d:.1f}ms ({st.bytes_h2d / max(st.ms_h2d, 1e-9) / 1e6:.1f} GB/s) "
                f"trav={st.ms_traverse:.1f}ms bf={st.ms_bruteforce:.1f}ms")
            if tie >= args.recall or args.L:
                points.append(dict(thr=thr, L=L, recall=tie, strict=strict, wall=wall))
                break
            if points and wall > 2 * min(p["wall"] for p in points):
                break
    if not points:
        raise SystemExit("no operating point reached the recall target")
    best = min(points, key=lambda p: p["wall"])
    thr, L = best["thr"], best["L"]

    def timed(plan, thr_, L_, steps):
        if not plan:
            b.set_stream_plan(None)
        for _ in range(args.warmup):
            step(thr_, L_, plan)
        torch.cuda.synchronize()
        acc = dict(a=0.0, plan=0.0, total=0.0, h2d=0.0, bytes=0.0, tr=0.0, bf=0.0, btr=0.0)
        t_ = time.perf_counter()
        for _ in range(steps):
            ids_, st_, ms_a, ms_p = step(thr_, L_, plan)
            acc["a"] += ms_a
            acc["plan"] += ms_p
            acc["total"] += st_.ms_total
            acc["h2d"] += st_.ms_h2d
            acc["bytes"] += st_.bytes_h2d
            acc["tr"] += st_.ms_traverse
            acc["bf"] += st_.ms_bruteforce
            acc["btr"] += st_.bytes_traverse
        torch.cuda.synchronize()
        el = time.perf_counter() - t_
        strict_, tie_ = recall(ids_)
        r = {k: v / steps for k, v in acc.items()}
        r.update(elapsed=el, qps=Q * steps / el, strict=strict_, recall=tie_, n_active=st_.n_active,
                 nbatch=st_.n_batches)
        return r

    def brief(r, thr_, L_):
        return {"little_threshold": thr_, "L": L_, "qps": round(r["qps"], 1), "recall_at_10": round(r["recall"], 4),
                "n_active": r["n_active"], "nbatch": r["nbatch"], "ms_plan": round(r["plan"], 3),
                "ms_search": round(r["total"], 3), "ms_h2d": round(r["h2d"], 3), "ms_traverse": round(r["tr"], 3)}

    K = args.steps
    res = {k: timed(k == "planned", thr, L, K) for k in ("static", "planned")}
    for k, r in res.items():
        log(f"{k} plan: {r['qps']:.0f} QPS; per step: planning {r['plan']:.2f} ms, search {r['total']:.2f} ms, "
            f"copies {r['h2d']:.2f} ms at {r['bytes'] / max(r['h2d'], 1e-9) / 1e6:.1f} GB/s, brute force "
            f"{r['bf']:.2f} ms, {r['nbatch']} batches, {r['n_active']} active (query, batch) pairs")
    # the traversal route (every query traverses), where each active (query,
    # batch) pair restarts a traversal
    trav_L = args.traverse_L
    trav = {k: brief(timed(k == "planned", 0.0, trav_L, max(2, K // 2)), 0.0, trav_L) for k in ("static", "planned")}
    log(f"traversal at L={trav_L}: {trav}")
    head = args.stream_plan if args.stream_plan != "best" else max(res, key=lambda k: res[k]["qps"])
    other = "planned" if head == "static" else "static"
    r = res[head]
    device_bytes = sx.device_bytes
    b.close()
    sx.close()
    h2d_gbs = r["bytes"] / (r["h2d"] / 1e3) / 1e9
    trav_gbs = r["btr"] / (r["tr"] / 1e3) / 1e9 if r["tr"] > 0 else 0.0
    out = {
        "metric": "QPS at recall@10≥0.95, C5-shaped out-of-core streaming (scaled), 1 MI355X",
        "value": round(r["qps"], 1), "unit": "queries/s", "n_gpus": 1, "steps": K, "warmup": args.warmup,
        "ms_per_step": round(r["elapsed"] * 1e3 / K, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u8",
        "data": "synthetic (generated in bench.py; exact kNN index built on the GPU, streamed from pinned host memory)",
        "config": {
            "workload": (f"C5-shaped, scaled: {N} x {D} u8 (integers 0-255), 2 uint32 attrs on a 16x16 arithmetic "
                         f"grid, R={ix['R']} exact per-cell kNN + E=2 cross edges, {Q} queries, selectivity "
                         f"log-U[0.5%,20%], k=10, batches {kinds[head]}, device budget {args.stream_budget_mb} MiB"),
            "plan": head, "nbatch": r["nbatch"], "n_active": r["n_active"],
            "other_plan": {"plan": other, "kind": kinds[other], **brief(res[other], thr, L)},
            "traversal": trav,
            "N": N, "D": D, "Q": Q, "K": 10, "L": L, "little_threshold": thr,
            "recall_at_10": round(r["recall"], 4), "recall_at_10_strict": round(r["strict"], 4),
            "device_bytes": device_bytes, "resident_index_bytes": resident_bytes,
            "ms_stage_a": round(r["a"], 3), "ms_plan": round(r["plan"], 3), "ms_search": round(r["total"], 3),
            "ms_h2d": round(r["h2d"], 3), "bytes_h2d": round(r["bytes"]),
            "ms_traverse": round(r["tr"], 3), "ms_bruteforce": round(r["bf"], 3),
        },
        "roofline": {"bound": "pcie", "kernel": "batch image copies (DMA + k_stream_gather)",
                     "achieved": round(h2d_gbs, 2), "peak": PCIE_PEAK_GBS, "unit": "GB/s",
                     "frac": round(h2d_gbs / PCIE_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": round(r["bytes"]), "ms_per_launch": round(r["h2d"], 4)},
        "roofline_traverse": {"bound": "hbm", "kernel": "k_traverse (u8, summed over batches)",
                              "achieved": round(trav_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(trav_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                              "ms_per_launch": round(r["tr"], 4)},
        "cpu_baseline": None,
    }
    print(result_line(out), flush=True)


def cpu_baseline(cfg, ix, batch, L, prefilter, args, channels=1, f16=False, ref16=False):
    """The oracle's traversal / brute force (OpenMP over queries) on a sample of
    the same batch, same routing, same L, same traversal and row type (f16:
    binary16 rows and queries; ref16: with the reference's binary16
    arithmetic), on the host's cores."""
    from oracle import oracle as orc
    import garfield_amd as gf
    batch.mark_cells(prefilter)          # the operating point's cells and routing
    batch.order_cells(4)
    cells, counts, little, _ = batch.get_cells()
    O = orc.OracleIndex(ix["vectors"], ix["attrs"], ix["global_pid"], ix["P"], ix["cell_graphs"], ix["cross"],
                        vec_f16=orc.f2h(ix["vectors"], 1.0) if f16 else None)
    queries = orc.f2h(cfg["queries"], 1.0) if f16 else cfg["queries"]
    ent = gf.entry_points(ix["vectors"].shape[0], ix["P"], L if channels == 2 else ix["R"])
    orc.set_channels(channels)
    orc.set_dist_mode(1 if ref16 else 0)
    # The GPU box allots 16 host cores to its one GPU (OMP_NUM_THREADS is
    # set to that share there); os.cpu_count() sees the whole host.
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(os.cpu_count() or 1, 16)
    lo = cfg["lo"].astype(np.float32)
    hi = cfg["hi"].astype(np.float32)
    Q = cfg["queries"].shape[0]
    rng = np.random.default_rng(0)
    order = rng.permutation(Q)
    n = min(64, Q)
    while True:
        sel = np.sort(order[:n])
        t = time.perf_counter()
        O.search(queries[sel], lo[sel], hi[sel], cells[sel], counts[sel], little[sel], ent, L,
                 postfilter=args.postfilter, nthreads=threads)
        dt = time.perf_counter() - t
        if dt >= args.cpu_seconds or n >= Q:
            break
        n = min(Q, max(n * 2, int(n * args.cpu_seconds / max(dt, 1e-3) * 1.1)))
    orc.set_channels(1)
    orc.set_dist_mode(0)
    routed = int(np.sum((little[sel] == counts[sel]) & (counts[sel] > 0)))
    log(f"cpu baseline (prefilter {prefilter}, L {L}, channels {channels}): {n} queries in {dt:.1f}s on "
        f"{threads} threads")
    return {"value": round(n / dt, 1), "unit": "queries/s", "cores": threads, "kind": "port",
            "route": "filtered brute force" if prefilter >= 1.0 else
                     ("dual-channel " if channels == 2 else "") + "traversal (+ brute force below the prefilter)",
            "host_cpu": host_cpu_model(), "host_nproc": os.cpu_count(),
            "sample": f"{n} random queries of the same batch ({routed} on the brute force; same cells, routing, "
                      f"L={L}, prefilter={prefilter}), search stage only (stages A/B not timed), OpenMP over "
                      f"queries on {threads} threads (the GPU box's host-core share for one GPU)",
            "note": "the oracle: plain C++ (-O3 -march=x86-64-v3 -ffp-contract=off, no hand vectorisation, "
                    "one query per thread), a checker rather than an optimised CPU index, so the GPU/CPU ratio "
                    "is not a measure of kernel quality"}


def host_cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


if __name__ == "__main__":
    main()
