"""Synthetic workloads and GMG index construction for tests and bench.py.

The reference builds its index with cuVS (CAGRA per cell, CAGRA search for
cross edges, k-means), which is not available here; this module builds the
same files from exact nearest neighbours instead (a stronger stand-in):

- grid: rank-quantile cells per attribute, row-major global cell id
  (grid_scatter_V2, indexbuild/tools.py:88-125);
- per-cell graph: exact R nearest neighbours inside the cell, self excluded,
  cell-local ids (cagra_build.py:94-127 writes the same layout);
- cross-cell graph: for every point and every cell, the E nearest points of
  that cell (global_graph_build.py:106-176);
- labels: Lloyd k-means (clustering.py:68-87 writes per-point labels).

Distances run as torch matrix products in fp32 (exact for the integer-valued
configs) on whatever device is given: "cpu" in the tests, "cuda" on the GPU
box for the 1M-point bench.  This is index *construction*, outside the query
path the library implements.
"""
import math

import numpy as np

DOMAIN = 10000  # attribute values are integers in [0, DOMAIN)


def _torch():
    import torch
    return torch


# ------------------------------------------------------------------ data
def uniform_int_vectors(n, d, seed, hi=256):
    rng = np.random.default_rng(seed)
    return rng.integers(0, hi, size=(n, d)).astype(np.float32)


def gaussian_unit_vectors(n, d, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, d)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    return x


def gmm_vectors(n, d, ncomp, seed, sigma=0.1):
    """Config C4's vectors: a mixture of ncomp Gaussians (sigma around unit-norm
    centres); returns the vectors and each point's component."""
    rng = np.random.default_rng(seed)
    cen = rng.standard_normal((ncomp, d))
    cen /= np.linalg.norm(cen, axis=1, keepdims=True)
    comp = rng.integers(0, ncomp, size=n)
    x = (cen[comp] + sigma * rng.standard_normal((n, d))).astype(np.float32)
    return x, comp


def component_attrs(comp, a, seed):
    """Config C4's attributes: 10 * component + U{0..9} on every attribute."""
    rng = np.random.default_rng(seed)
    return (10 * np.asarray(comp)[:, None] + rng.integers(0, 10, size=(len(comp), a))).astype(np.int32)


def uniform_attrs(n, a, seed, hi=DOMAIN):
    rng = np.random.default_rng(seed)
    return rng.integers(0, hi, size=(n, a)).astype(np.int32)


def zipf_attrs(n, a, seed, s=1.1, hi=DOMAIN):
    rng = np.random.default_rng(seed)
    return np.minimum(rng.zipf(s, size=(n, a)) - 1, hi - 1).astype(np.int32)


def ranges_for_selectivity(q, a, sel, seed, hi=DOMAIN):
    """Closed integer ranges whose per-attribute width is sel**(1/a) of the domain."""
    rng = np.random.default_rng(seed)
    sel = np.broadcast_to(np.asarray(sel, np.float64), (q,))
    w = np.clip(np.round(hi * sel ** (1.0 / a)), 1, hi).astype(np.int64)
    lo = np.empty((q, a), np.int64)
    for d in range(a):
        lo[:, d] = (rng.random(q) * (hi - w + 1)).astype(np.int64)
    hi_ = lo + w[:, None] - 1
    return lo.astype(np.int32), hi_.astype(np.int32)


def ranges_for_selectivity_ranked(attrs, q, sel, seed):
    """Closed ranges that each hold a sel**(1/a) fraction of the points'
    values on every attribute (a random window of the sorted values), for
    skewed attributes; equal values at a window's ends widen it."""
    rng = np.random.default_rng(seed)
    n, a = attrs.shape
    sel = np.broadcast_to(np.asarray(sel, np.float64), (q,))
    w = np.clip(np.round(n * sel ** (1.0 / a)), 1, n).astype(np.int64)
    lo = np.empty((q, a), np.int64)
    hi = np.empty((q, a), np.int64)
    for d in range(a):
        s = np.sort(attrs[:, d])
        r0 = (rng.random(q) * (n - w + 1)).astype(np.int64)
        lo[:, d] = s[r0]
        hi[:, d] = s[r0 + w - 1]
    return lo.astype(np.int32), hi.astype(np.int32)


def log_uniform(q, lo, hi, seed):
    rng = np.random.default_rng(seed)
    return np.exp(rng.uniform(math.log(lo), math.log(hi), size=q))


# ------------------------------------------------------------------ grid
def grid_scatter(attrs, grid):
    """grid_scatter_V2: stable rank quantiles per attribute (indexbuild/tools.py:88-125)."""
    attrs = np.asarray(attrs)
    n, a = attrs.shape
    l_q, r_q, pid_lists = [], [], []
    for d in range(a):
        col = attrs[:, d]
        order = np.argsort(col, kind="stable")
        srt = col[order]
        g = int(grid[d])
        avg = (n + g - 1) // g
        left = [j * avg for j in range(g)]
        right = [((j + 1) * avg - 1) if j < g - 1 else (n - 1) for j in range(g)]
        idx = np.zeros(n, np.int32)
        for j in range(g):
            idx[order[j * avg:((j + 1) * avg if j < g - 1 else n)]] = j
        l_q.append(srt[left].astype(np.int32))
        r_q.append(srt[right].astype(np.int32))
        pid_lists.append(idx)
    factors = np.ones(a, np.int64)
    for d in range(a - 2, -1, -1):
        factors[d] = factors[d + 1] * int(grid[d + 1])
    global_pid = np.zeros(n, np.int64)
    for d in range(a):
        global_pid += factors[d] * pid_lists[d]
    return l_q, r_q, pid_lists, global_pid.astype(np.int32)


def grid_scatter_arith(attrs, grid, attr_min, attr_width):
    """Arithmetic grid (the out-of-core driver's cells: width = ceil((max - min) / g), bigdataset_experiment.cu:63-70):
    cell of v on attribute d = min(max(floor((v - min_d) / width_d), 0), g_d - 1).
    l_q / r_q hold each cell's value interval [min + j w, min + (j + 1) w - 1]."""
    attrs = np.asarray(attrs)
    n, a = attrs.shape
    l_q, r_q, pid_lists = [], [], []
    for d in range(a):
        g = int(grid[d])
        m, w = float(attr_min[d]), float(attr_width[d])
        idx = np.clip(np.floor((attrs[:, d].astype(np.float64) - m) / w), 0, g - 1).astype(np.int32)
        l_q.append(np.array([m + j * w for j in range(g)]).astype(np.int32))
        r_q.append(np.array([m + (j + 1) * w - 1 for j in range(g)]).astype(np.int32))
        pid_lists.append(idx)
    factors = np.ones(a, np.int64)
    for d in range(a - 2, -1, -1):
        factors[d] = factors[d + 1] * int(grid[d + 1])
    global_pid = np.zeros(n, np.int64)
    for d in range(a):
        global_pid += factors[d] * pid_lists[d]
    return l_q, r_q, pid_lists, global_pid.astype(np.int32)


def cell_sizes(ix):
    return np.bincount(ix["global_pid"], minlength=ix["P"]).astype(np.uint32)


def cell_members(global_pid, P):
    """Point ids of each cell in ascending id order (cell-local id = position)."""
    order = np.argsort(global_pid, kind="stable")
    sizes = np.bincount(global_pid, minlength=P)
    bounds = np.concatenate([[0], np.cumsum(sizes)])
    return [order[bounds[c]:bounds[c + 1]] for c in range(P)]


# ------------------------------------------------------------------ graphs
def _sqdist(torch, x, y, ynorm):
    xn = (x * x).sum(1, keepdim=True)
    return (xn + ynorm[None, :] - 2.0 * (x @ y.T)).clamp_min_(0.0)


def knn_cell_graphs(vectors, members, R, device="cpu", chunk=4096):
    """Exact R nearest neighbours within each cell, self excluded (cell-local ids)."""
    torch = _torch()
    out = []
    for mem in members:
        if len(mem) == 0:
            continue
        xc = torch.as_tensor(vectors[mem], device=device)
        n = xc.shape[0]
        k = min(R + 1, n)
        yn = (xc * xc).sum(1)
        g = torch.empty((n, R), dtype=torch.int64, device=device)
        for s in range(0, n, chunk):
            e = min(n, s + chunk)
            d = _sqdist(torch, xc[s:e], xc, yn)
            ar = torch.arange(s, e, device=device)
            d[ar - s, ar] = float("inf")
            idx = torch.topk(d, k, dim=1, largest=False, sorted=True).indices[:, :R]
            if idx.shape[1] < R:  # tiny cells: pad by repeating the nearest
                idx = torch.cat([idx, idx[:, :1].expand(-1, R - idx.shape[1])], 1)
            g[s:e] = idx
        out.append(g.cpu().numpy().astype(np.uint32))
    return np.concatenate(out, 0)


def cross_edges(vectors, members, E, device="cpu", chunk=8192):
    """For every point and every cell, the E nearest points of that cell (local ids)."""
    torch = _torch()
    N = vectors.shape[0]
    P = len(members)
    out = np.zeros((N, P * E), np.uint32)
    xall = torch.as_tensor(vectors, device=device)
    for c, mem in enumerate(members):
        if len(mem) == 0:   # empty cell: edges into it are never followed
            continue
        yc = torch.as_tensor(vectors[mem], device=device)
        yn = (yc * yc).sum(1)
        k = min(E, yc.shape[0])
        for s in range(0, N, chunk):
            e = min(N, s + chunk)
            d = _sqdist(torch, xall[s:e], yc, yn)
            idx = torch.topk(d, k, dim=1, largest=False, sorted=True).indices
            if k < E:
                idx = torch.cat([idx, idx[:, :1].expand(-1, E - k)], 1)
            out[s:e, c * E:(c + 1) * E] = idx.cpu().numpy().astype(np.uint32)
    return out


def kmeans_labels(vectors, C, iters, seed, device="cpu", chunk=65536):
    torch = _torch()
    rng = np.random.default_rng(seed)
    x = torch.as_tensor(vectors, device=device)
    N = x.shape[0]
    cen = x[torch.as_tensor(rng.choice(N, size=C, replace=False), device=device)].clone()
    labels = torch.empty(N, dtype=torch.int64, device=device)
    for _ in range(iters):
        cn = (cen * cen).sum(1)
        for s in range(0, N, chunk):
            e = min(N, s + chunk)
            labels[s:e] = _sqdist(torch, x[s:e], cen, cn).argmin(1)
        sums = torch.zeros_like(cen).index_add_(0, labels, x)
        cnt = torch.bincount(labels, minlength=C).to(x.dtype)
        nz = cnt > 0
        cen[nz] = sums[nz] / cnt[nz, None]
    return labels.cpu().numpy().astype(np.int32)


def build_index(vectors, attrs, grid, R, E, C=0, kmeans_iters=8, seed=5, device="cpu", arith=None,
                graph="knn", inter=64):
    """All index arrays, in the layout the files hold.  arith = (attr_min,
    attr_width) builds the cells on an arithmetic grid instead of rank quantiles.
    device "hip": the library's builder (gf_grid_scatter, the int8 MFMA
    gf_build_graphs and gf_kmeans; non-integer data through their u8
    quantisation, graphs re-ranked by exact fp32 distances); else torch on
    that device.  graph "cagra" (device "hip" only): exact kNN graphs of degree
    `inter`, optimised to degree R by gf_optimize_graphs (the graph
    cagra.build returns); "knn": exact kNN graphs of degree R."""
    grid = np.asarray(grid, np.int64)
    P = int(np.prod(grid))
    hip = device == "hip"
    if arith is not None:
        l_q, r_q, pid_lists, global_pid = grid_scatter_arith(attrs, grid, arith[0], arith[1])
    elif hip:
        from ._lib import grid_scatter as lib_grid_scatter
        l_q, r_q, pid_lists, global_pid = lib_grid_scatter(np.asarray(attrs, np.float32), grid)
        global_pid = global_pid.astype(np.int32)
    else:
        l_q, r_q, pid_lists, global_pid = grid_scatter(attrs, grid)
    if graph not in ("knn", "cagra") or (graph == "cagra" and not hip):
        raise ValueError("graph must be 'knn', or 'cagra' with device 'hip'")
    if hip:
        from ._lib import build_graphs, optimize_graphs
        v = vectors if vectors.dtype == np.uint8 else np.asarray(vectors, np.float32)
        if graph == "cagra":
            knn, cross, _ = build_graphs(v, global_pid, P, inter, E)
            sizes = np.bincount(np.asarray(global_pid, np.int64), minlength=P)
            graphs, _ = optimize_graphs(knn, sizes, R)
            del knn
        else:
            graphs, cross, _ = build_graphs(v, global_pid, P, R, E)
    else:
        members = cell_members(global_pid, P)
        graphs = knn_cell_graphs(vectors, members, R, device=device)
        cross = cross_edges(vectors, members, E, device=device)
    if C and hip:
        from ._lib import kmeans
        v = vectors if vectors.dtype == np.uint8 else np.asarray(vectors, np.float32)
        labels = kmeans(v, C, kmeans_iters, seed=seed)[0]
    else:
        labels = kmeans_labels(vectors, C, kmeans_iters, seed, device=device) if C else None
    return dict(vectors=vectors, attrs=attrs, grid=grid.astype(np.int32), l_q=l_q, r_q=r_q,
                pid_lists=pid_lists, global_pid=global_pid, cell_graphs=graphs, cross=cross, labels=labels,
                P=P, R=R, E=E)


def write_index(ix, prefix):
    """Write the index files (formats of README.md:101-170): {prefix}.fvecs, {prefix}_cell{i}.graph, {prefix}.cross, .grid, .attrs, .cluster"""
    from . import formats
    formats.write_fvecs(prefix + ".fvecs", ix["vectors"])
    members = cell_members(ix["global_pid"], ix["P"])
    start = 0
    for c, mem in enumerate(members):
        formats.write_graph(f"{prefix}_cell{c}.graph", ix["cell_graphs"][start:start + len(mem)])
        start += len(mem)
    formats.write_graph(prefix + ".cross", ix["cross"])
    formats.write_grid(prefix + ".grid", ix["grid"], ix["l_q"], ix["r_q"], ix["pid_lists"], ix["global_pid"])
    formats.write_attrs(prefix + ".attrs", ix["attrs"])
    if ix["labels"] is not None:
        formats.write_labels(prefix + ".cluster", ix["labels"])
    return dict(data_path=prefix + ".fvecs", cagra_prefix=prefix + "_cell", cagra_suffix=".graph",
                global_graph=prefix + ".cross", grid=prefix + ".grid", attrs=prefix + ".attrs",
                cluster=prefix + ".cluster" if ix["labels"] is not None else None)


def quantile_arrays(ix):
    """Flattened float l_q / r_q, attribute-major, as the library takes them."""
    return (np.concatenate(ix["l_q"]).astype(np.float32), np.concatenate(ix["r_q"]).astype(np.float32))


def open_device_index(ix, **kw):
    """Index.from_arrays on an index dict from build_index."""
    from ._lib import Index
    l_q, r_q = quantile_arrays(ix)
    return Index.from_arrays(ix["vectors"], ix["attrs"].astype(np.float32), ix["grid"], l_q, r_q,
                             ix["global_pid"], ix["cell_graphs"], ix["cross"], labels=ix["labels"], **kw)


# ------------------------------------------------------------- workloads
def config_small(N=100_000, Q=1000, R=16, C=100, sel=0.3, seed=1):
    """Config C1 (optionally shrunk): 128-d integer vectors, 2 attributes, 4x4 grid."""
    vec = uniform_int_vectors(N, 128, seed)
    att = uniform_attrs(N, 2, seed + 1)
    qv = uniform_int_vectors(Q, 128, seed + 2)
    lo, hi = ranges_for_selectivity(Q, 2, sel, seed + 3)
    return dict(vectors=vec, attrs=att, grid=[4, 4], R=R, E=2, C=C, queries=qv, lo=lo, hi=hi)


def config_headline(N=1_000_000, Q=10_000, R=32, C=1000, seed=11):
    """Config C2 (headline): 1M x 128 integers, 2 attributes on 4x4, selectivity log-U[1%, 50%]."""
    vec = uniform_int_vectors(N, 128, seed)
    att = uniform_attrs(N, 2, seed + 1)
    qv = uniform_int_vectors(Q, 128, seed + 2)
    sel = log_uniform(Q, 0.01, 0.5, seed + 3)
    lo, hi = ranges_for_selectivity(Q, 2, sel, seed + 4)
    return dict(vectors=vec, attrs=att, grid=[4, 4], R=R, E=2, C=C, queries=qv, lo=lo, hi=hi, sel=sel)


def config_c3(N=1_000_000, Q=10_000, R=32, C=1000, seed=31):
    """Config C3: N x 96 Gaussian unit vectors, 3 Zipf(1.1) attributes on a
    4x4x4 rank grid (64 cells), selectivity log-U[0.1%, 50%] (ranges drawn
    in rank space, as the skewed values need)."""
    vec = gaussian_unit_vectors(N, 96, seed)
    att = zipf_attrs(N, 3, seed + 1)
    qv = gaussian_unit_vectors(Q, 96, seed + 2)
    sel = log_uniform(Q, 0.001, 0.5, seed + 3)
    lo, hi = ranges_for_selectivity_ranked(att, Q, sel, seed + 4)
    return dict(vectors=vec, attrs=att, grid=[4, 4, 4], R=R, E=2, C=C, queries=qv, lo=lo, hi=hi, sel=sel)


def config_c4(N=1_000_000, Q=10_000, R=32, C=1000, ncomp=1000, seed=41):
    """Config C4: N x 768 vectors of a Gaussian mixture (ncomp components,
    sigma 0.1 around unit centres; the queries from the same mixture), 2
    attributes 10 * component + U{0..9} on a 4x4 grid, 10% selectivity."""
    vec, comp = gmm_vectors(N, 768, ncomp, seed)
    att = component_attrs(comp, 2, seed + 1)
    rng = np.random.default_rng(seed)
    cen = rng.standard_normal((ncomp, 768))
    cen /= np.linalg.norm(cen, axis=1, keepdims=True)     # the same centres as gmm_vectors draws
    qr = np.random.default_rng(seed + 2)
    qc = qr.integers(0, ncomp, size=Q)
    qv = (cen[qc] + 0.1 * qr.standard_normal((Q, 768))).astype(np.float32)
    lo, hi = ranges_for_selectivity(Q, 2, 0.1, seed + 3, hi=10 * ncomp)
    return dict(vectors=vec, attrs=att, grid=[4, 4], R=R, E=2, C=C, queries=qv, lo=lo, hi=hi)


def config_stream(N=1_000_000, Q=10_000, R=32, seed=21):
    """Config C5 scaled to one GPU box's build time: N x 128 integer vectors
    (stored as u8), 2 uint32 attributes uniform in [0,10000) on a 16x16
    arithmetic grid (width 625), R=32, E=2, selectivity log-U[0.5%, 20%]."""
    vec = uniform_int_vectors(N, 128, seed)
    att = uniform_attrs(N, 2, seed + 1)
    qv = uniform_int_vectors(Q, 128, seed + 2)
    sel = log_uniform(Q, 0.005, 0.2, seed + 3)
    lo, hi = ranges_for_selectivity(Q, 2, sel, seed + 4)
    width = float((DOMAIN + 15) // 16)
    return dict(vectors=vec, attrs=att, grid=[16, 16], R=R, E=2, C=0, queries=qv, lo=lo, hi=hi, sel=sel,
                attr_min=np.zeros(2, np.float32), attr_width=np.full(2, width, np.float32))


def block_plan(grid, block):
    """Static plan of compact blocks of block x block cells on a 2-d grid (the
    spatially grouped batches of bigdataset_experiment.cu:746-756)."""
    g0, g1 = int(grid[0]), int(grid[1])
    plan = []
    for i0 in range(0, g0, block):
        for j0 in range(0, g1, block):
            plan.append([i * g1 + j for i in range(i0, min(g0, i0 + block)) for j in range(j0, min(g1, j0 + block))])
    return plan


def ground_truth_torch(vectors, attrs, queries, lo, hi, K, device="cuda", chunk=256):
    """Exact filtered kNN (naive_brute_force_with_filter, gpu_graph.cu:10782-10812)
    in fp64 on `device`; returns ids (missing = 0x7FFFFFFF) and squared distances."""
    torch = _torch()
    x = torch.as_tensor(vectors, device=device, dtype=torch.float64)
    xn = (x * x).sum(1)
    at = torch.as_tensor(attrs, device=device)
    Q = queries.shape[0]
    ids = np.full((Q, K), 0x7FFFFFFF, np.uint32)
    dist = np.full((Q, K), np.inf, np.float64)
    for s in range(0, Q, chunk):
        e = min(Q, s + chunk)
        q = torch.as_tensor(queries[s:e], device=device, dtype=torch.float64)
        d = (q * q).sum(1, keepdim=True) + xn[None, :] - 2.0 * (q @ x.T)
        l = torch.as_tensor(lo[s:e], device=device)
        h = torch.as_tensor(hi[s:e], device=device)
        ok = torch.ones_like(d, dtype=torch.bool)
        for j in range(at.shape[1]):
            ok &= (at[None, :, j] >= l[:, None, j]) & (at[None, :, j] <= h[:, None, j])
        d = torch.where(ok, d, torch.full_like(d, float("inf")))
        v, i = torch.topk(d, K, dim=1, largest=False, sorted=True)
        v = v.cpu().numpy()
        i = i.cpu().numpy().astype(np.uint32)
        i[~np.isfinite(v)] = 0x7FFFFFFF
        ids[s:e] = i
        dist[s:e] = v
    return ids, dist


def recall_at_k(res_ids, res_exact_dist, gt_ids, gt_dist, per_query=False):
    """(strict, tie-aware) recall: strict is |res ∩ gt| / |gt| (tools.cuh:384-453,
    1 when the filter passes nothing); tie-aware also counts a result whose exact
    distance is <= the K-th ground-truth distance.  per_query: the two arrays
    of per-query recalls instead of their means."""
    Q, K = gt_ids.shape
    strict = np.empty(Q)
    tie = np.empty(Q)
    for q in range(Q):
        g = gt_ids[q][gt_ids[q] != 0x7FFFFFFF]
        if g.size == 0:
            strict[q] = tie[q] = 1.0
            continue
        r = res_ids[q]
        valid = r != 0x7FFFFFFF
        strict[q] = np.intersect1d(r[valid], g).size / g.size
        kth = gt_dist[q][g.size - 1]
        _, first = np.unique(r, return_index=True)
        uniq = np.zeros(K, bool)
        uniq[first] = True
        tie[q] = min(np.count_nonzero(valid & uniq & (res_exact_dist[q] <= kth)), g.size) / g.size
    if per_query:
        return strict, tie
    return float(strict.mean()), float(tie.mean())


def exact_result_dist(vectors, queries, ids, device="cuda"):
    torch = _torch()
    safe = np.where(ids == 0x7FFFFFFF, 0, ids).astype(np.int64)
    x = torch.as_tensor(vectors, device=device, dtype=torch.float64)
    q = torch.as_tensor(queries, device=device, dtype=torch.float64)
    g = x[torch.as_tensor(safe, device=device)]
    d = ((g - q[:, None, :]) ** 2).sum(-1).cpu().numpy()
    d[ids == 0x7FFFFFFF] = np.inf
    return d
