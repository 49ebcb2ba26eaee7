"""ctypes binding of the CPU oracle (oracle/_build/libgforacle.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it as the checker / CPU baseline; the product package
(garfield_amd) never imports it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libgforacle.so")
NCNT = 8
SENTINEL = 0x7FFFFFFF
_lib = None


def build():
    subprocess.run(["make", "-C", HERE], check=True)


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = C.CDLL(LIB)
        _lib.orc_f2h_one.restype = C.c_uint16
        _lib.orc_f2h_one.argtypes = [C.c_float, C.c_float]
        _lib.orc_h2f.restype = C.c_float
        _lib.orc_h2f.argtypes = [C.c_uint16]
        _lib.orc_distance.restype = C.c_float
        _lib.orc_recall.restype = C.c_double
    return _lib


class _Index(C.Structure):
    _fields_ = [("N", C.c_uint32), ("D", C.c_uint32), ("a", C.c_uint32), ("P", C.c_uint32),
                ("R", C.c_uint32), ("E", C.c_uint32), ("vdtype", C.c_int32),
                ("vec_f32", C.c_void_p), ("qscale", C.c_void_p), ("qzero", C.c_void_p),
                ("vec_f16", C.c_void_p), ("attrs", C.c_void_p),
                ("graph", C.c_void_p), ("offset", C.c_void_p), ("global_idx", C.c_void_p),
                ("local_idx", C.c_void_p), ("cross", C.c_void_p),
                ("FD", C.c_uint32), ("fgraph", C.c_void_p), ("fentry", C.c_void_p)]


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def idx_mapper(global_pid, P):
    pid = _c(global_pid, np.uint32)
    N = pid.size
    gi = np.empty(N, np.uint32)
    li = np.empty(N, np.uint32)
    off = np.empty(P + 1, np.uint32)
    load().orc_idx_mapper(C.c_uint32(N), C.c_uint32(P), _p(pid), _p(gi), _p(li), _p(off))
    return gi, li, off


def f2h(x, alpha=1.0):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    load().orc_f2h(_p(x), C.c_size_t(x.size), C.c_float(alpha), _p(out))
    return out


def row_norms_f16(x):
    x = _c(x, np.uint16)
    out = np.empty(x.shape[0], np.float32)
    load().orc_row_norms_f16(_p(x), C.c_uint32(x.shape[0]), C.c_uint32(x.shape[1]), _p(out))
    return out


def centres_hist(data, labels, global_pid, P, contiguous=False):
    data = _c(data, np.float32)
    labels = _c(labels, np.int32)
    pid = _c(global_pid, np.uint32)
    N, D = data.shape
    Cn = int(labels.max()) + 1
    cen = np.empty((Cn, D), np.float32)
    hist = np.empty((P, Cn), np.uint32)
    load().orc_centres_hist(C.c_uint32(N), C.c_uint32(D), C.c_uint32(Cn), C.c_uint32(P), _p(data),
                            _p(labels), _p(pid), C.c_int32(int(contiguous)), _p(cen), _p(hist))
    return cen, hist


def cells(lo, hi, grid, l_q, r_q, cell_size=None):
    lo = _c(lo, np.float32)
    hi = _c(hi, np.float32)
    grid = _c(grid, np.uint32)
    Q, a = lo.shape
    P = int(np.prod(grid))
    out = np.zeros((Q, P), np.uint32)
    cnt = np.empty(Q, np.uint32)
    cs = None if cell_size is None else _c(cell_size, np.uint32)
    load().orc_cells(C.c_uint32(Q), C.c_uint32(a), _p(lo), _p(hi), _p(grid), _p(_c(l_q, np.float32)),
                     _p(_c(r_q, np.float32)), _p(cs) if cs is not None else None, _p(out), _p(cnt))
    return out, cnt


def cells_grid(lo, hi, grid, attr_min, attr_width, threshold, cell_size=None):
    """Arithmetic-grid stage A: (cells Q x P, counts, little counts, flags Q x P)."""
    lo = _c(lo, np.float32)
    hi = _c(hi, np.float32)
    grid = _c(grid, np.uint32)
    Q, a = lo.shape
    P = int(np.prod(grid))
    out = np.zeros((Q, P), np.uint32)
    cnt = np.empty(Q, np.uint32)
    lit = np.empty(Q, np.uint32)
    flags = np.empty((Q, P), np.uint8)
    cs = None if cell_size is None else _c(cell_size, np.uint32)
    load().orc_cells_grid(C.c_uint32(Q), C.c_uint32(a), _p(lo), _p(hi), _p(grid), _p(_c(attr_min, np.float32)),
                          _p(_c(attr_width, np.float32)), C.c_double(threshold),
                          _p(cs) if cs is not None else None, _p(out), _p(cnt), _p(lit), _p(flags))
    return out, cnt, lit, flags


def selectivity(attrs, lo, hi, threshold, counts, nthreads=0):
    attrs = _c(attrs, np.float32)
    lo = _c(lo, np.float32)
    hi = _c(hi, np.float32)
    counts = _c(counts, np.uint32)
    Q, a = lo.shape
    sel = np.empty(Q, np.uint32)
    little = np.empty(Q, np.uint32)
    load().orc_selectivity(C.c_uint32(Q), C.c_uint32(attrs.shape[0]), C.c_uint32(a), _p(attrs), _p(lo),
                           _p(hi), C.c_float(threshold), _p(counts), _p(sel), _p(little), C.c_int(nthreads))
    return sel, little


def centroid_dist_f64(qh, ch):
    qh = _c(qh, np.uint16)
    ch = _c(ch, np.uint16)
    out = np.empty((qh.shape[0], ch.shape[0]), np.float64)
    load().orc_centroid_dist_f64(C.c_uint32(qh.shape[0]), C.c_uint32(ch.shape[0]), C.c_uint32(qh.shape[1]),
                                 _p(qh), _p(ch), _p(out))
    return out


def topk_clusters(dist, k):
    dist = _c(dist, np.float32)
    out = np.empty((dist.shape[0], k), np.uint32)
    load().orc_topk_clusters(C.c_uint32(dist.shape[0]), C.c_uint32(dist.shape[1]), C.c_uint32(k), _p(dist),
                             _p(out))
    return out


def sort_cells(cells_, counts, topk, hist):
    cells_ = _c(cells_, np.uint32).copy()
    counts = _c(counts, np.uint32)
    topk = _c(topk, np.uint32)
    hist = _c(hist, np.uint32)
    Q, P = cells_.shape
    load().orc_sort_cells(C.c_uint32(Q), C.c_uint32(P), C.c_uint32(hist.shape[1]), C.c_uint32(topk.shape[1]),
                          _p(cells_), _p(counts), _p(topk), _p(hist))
    return cells_


def entry_points(N, P, R):
    out = np.empty(R, np.uint32)
    load().orc_entry_points(C.c_uint32(N), C.c_uint32(P), C.c_uint32(R), _p(out))
    return out


def entry_points_pair(N, P, R, FD):
    """The R traversal entries and the FD full-graph entries (point ids) of
    one generator, as the reference draws them (gpu_graph.cu:12503-12539)."""
    out = np.empty(R, np.uint32)
    outf = np.empty(max(FD, 1), np.uint32)
    load().orc_entry_points_pair(C.c_uint32(N), C.c_uint32(P), C.c_uint32(R), C.c_uint32(FD), _p(out), _p(outf))
    return out, outf[:FD]


def entry_draw(range_, ndraw, R):
    out = np.empty(R, np.uint32)
    load().orc_entry_draw(C.c_uint32(range_), C.c_uint32(ndraw), C.c_uint32(R), _p(out))
    return out


class OracleIndex:
    """The index in the reference's representation (point-id order + idx mapper)."""

    def __init__(self, vectors, attrs, global_pid, P, cell_graphs, cross, vec_f16=None, u8=False, full=True,
                 i8q=None):
        """u8=True: the HIP path's uint8 vector mode (vectors hold the integer values).
        i8q=(scale, zero): the int8 per-dimension quantised mode (vectors hold
        the int8 values q of scale * (q - zero), quantise_i8); queries are
        then given times the index's f2h_factor.
        full=True: the full graph of the library's resident index (P <= 64
        cells, FE = min(E, R, 64 // P) edges into each cell, entries from the
        second draw), used by queries with postfilter or more cells; without
        it they return no result."""
        self.vectors = _c(vectors, np.float32)
        self.vec_f16 = None if vec_f16 is None else _c(vec_f16, np.uint16)
        self.attrs = _c(attrs, np.float32)
        self.graph = _c(cell_graphs, np.uint32)
        self.cross = _c(cross, np.uint32)
        self.P = P
        self.gidx, self.lidx, self.offset = idx_mapper(global_pid, P)
        N, D = self.vectors.shape
        vdt = (2 if u8 else 0) if self.vec_f16 is None else 1
        self.qscale = self.qzero = None
        if i8q is not None:
            vdt = 3
            self.qscale = _c(i8q[0], np.float32)
            self.qzero = _c(i8q[1], np.int32)
        self.s = _Index(N, D, self.attrs.shape[1], P, self.graph.shape[1], self.cross.shape[1] // P,
                        vdt, _p(self.vectors), None if self.qscale is None else _p(self.qscale),
                        None if self.qzero is None else _p(self.qzero),
                        None if self.vec_f16 is None else _p(self.vec_f16), _p(self.attrs), _p(self.graph),
                        _p(self.offset), _p(self.gidx), _p(self.lidx), _p(self.cross), 0, None, None)
        R, E = self.graph.shape[1], self.cross.shape[1] // P
        avg = (N + P - 1) // P
        if full and P <= 64 and E > 0 and N > (P - 1) * avg and N >= min(E, R, 64 // P) * P:
            self.FE = min(E, R, 64 // P)
            self.FD = self.FE * P
            self.fgraph = np.empty((N, self.FD), np.uint32)
            load().orc_full_graph(C.byref(self.s), C.c_uint32(self.FE), _p(self.fgraph))
            _, self.fentry = entry_points_pair(N, P, R, self.FD)
            self.fentry = _c(self.fentry, np.uint32)
            self.s.FD = self.FD
            self.s.fgraph = _p(self.fgraph)
            self.s.fentry = _p(self.fentry)
        else:
            self.FE = self.FD = 0

    def search(self, queries, lo, hi, cells_, counts, little, entry, L, K=10, rl=10, postfilter=1 << 30,
               nthreads=0):
        dt = np.uint16 if self.vec_f16 is not None else np.float32
        q = _c(queries, dt)
        lo = _c(lo, np.float32)
        hi = _c(hi, np.float32)
        cells_ = _c(cells_, np.uint32)
        counts = _c(counts, np.uint32)
        little = _c(little, np.uint32)
        entry = _c(entry, np.uint32)
        Q = q.shape[0]
        ids = np.empty((Q, K), np.uint32)
        dist = np.empty((Q, K), np.float32)
        ctr = np.empty((Q, NCNT), np.uint32)
        load().orc_search(C.byref(self.s), _p(q), C.c_uint32(Q), _p(lo), _p(hi), _p(cells_), _p(counts),
                          _p(little), _p(entry), C.c_uint32(L), C.c_uint32(K), C.c_uint32(rl),
                          C.c_uint32(min(int(postfilter), 0xFFFFFFFF)), _p(ids), _p(dist), _p(ctr),
                          C.c_int(nthreads))
        return ids, dist, ctr

    def trace(self, query, lo, hi, cells_, entry, L, K=10, rl=10, cap=100000, full=False):
        """One traversal query over the ordered cells `cells_` (full=True: the
        full-graph search, needs an index with a full graph) with its
        trajectory: (ids, dists, counters, expanded point ids, the cell of each
        expansion, recycle ids, recycle distances)."""
        dt = np.uint16 if self.vec_f16 is not None else np.float32
        q = _c(np.atleast_2d(query), dt)
        lo = _c(np.atleast_2d(lo), np.float32)
        hi = _c(np.atleast_2d(hi), np.float32)
        cl = np.zeros((1, self.P), np.uint32)
        cl[0, :len(cells_)] = cells_
        cnt = np.array([len(cells_)], np.uint32)
        entry = _c(entry, np.uint32)
        ids = np.empty(K, np.uint32)
        dist = np.empty(K, np.float32)
        ctr = np.empty(NCNT, np.uint32)
        ex = np.empty(cap, np.uint32)
        exc = np.empty(cap, np.uint32)
        rid = np.empty(rl, np.uint32)
        rd = np.empty(rl, np.float32)
        n = load().orc_search_trace(C.byref(self.s), _p(q), C.c_uint32(0), _p(lo), _p(hi), _p(cl), _p(cnt),
                                    _p(entry), C.c_uint32(L), C.c_uint32(K), C.c_uint32(rl), _p(ids), _p(dist),
                                    _p(ctr), _p(ex), _p(exc), C.c_uint32(cap), _p(rid), _p(rd),
                                    C.c_uint32(0 if full else 1 << 30))
        n = min(int(n), cap)
        return ids, dist, ctr, ex[:n].copy(), exc[:n].copy(), rid, rd

    def distance(self, query, gid):
        dt = np.uint16 if self.vec_f16 is not None else np.float32
        q = _c(query, dt)
        return load().orc_distance(C.byref(self.s), _p(q), C.c_uint32(gid))


def set_tie_mode(mode):
    """0: equal distances ordered by cell-major position (the HIP kernels'
    rule); 1: the reference's order (distance alone, its sorting networks)."""
    load().orc_set_tie_mode(C.c_int(int(mode)))


def set_dist_mode(mode):
    """fp16 path distances: 0 binary16 values, fp32 accumulation (the HIP
    kernels' arithmetic); 1 REF_HFMA2, the reference's half arithmetic."""
    load().orc_set_dist_mode(C.c_int(int(mode)))


def half_rne(v):
    lib = load()
    lib.orc_half_rne.restype = C.c_uint16
    lib.orc_half_rne.argtypes = [C.c_double]
    return int(lib.orc_half_rne(float(v)))


def hfma2_dist(q, x):
    q = _c(q, np.uint16)
    x = _c(x, np.uint16)
    lib = load()
    lib.orc_hfma2_dist.restype = C.c_float
    return float(lib.orc_hfma2_dist(_p(q), _p(x), C.c_uint32(q.size)))


def set_mutation(m):
    """Plant mistake number m in the traversal (0: none); test use only."""
    load().orc_set_mutation(C.c_int(int(m)))


MUTATIONS = {
    1: "merge ties put the list entry before the incoming one",
    2: "visited set rebuilt every 3 iterations, not 4",
    3: "cross slot i follows candidate i / 2, not i % 64",
    4: "evicted entries kept in the recycle list whether or not they pass the filter",
    5: "the end of a cell leaves the list's explored bits as they are",
    6: "cross edges tried from the last to the first",
    7: "first-cell entries enter the visited set by local id, not point id",
    8: "neighbours seen before are dropped instead of entering at +inf",
    9: "the final list is not filtered",
    10: "the next cell's entries are slots R..2R-1, not 0..R-1",
    11: "recycle merge ties put the recycle entry before the evictee",
    12: "cross slot i follows candidate i % 32 (only the first 32 candidates feed the slots)",
    13: "cross edges read for the current cell instead of the next",
    14: "full graph: the reset re-inserts the list only, not the B region",
    15: "full graph: entry points are not put in the visited set",
    16: "full graph assembly: own-cell edges read from the cross edges",
}


def set_max_iter(n):
    """Per-cell iteration cap of the traversal (0: the reference's 10000)."""
    load().orc_set_max_iter(C.c_uint32(int(n)))


def set_channels(n):
    """Traversal of traversal-routed queries: 1 the cell-by-cell search, 2 the
    dual-channel search (entry points: L ids)."""
    load().orc_set_channels(C.c_int(int(n)))


def set_dual_mutation(m):
    """Plant mistake number m in the dual-channel search (0: none); test use only."""
    load().orc_set_dual_mutation(C.c_int(int(m)))


def bitonic_sort_dis(dis, ids):
    d = _c(dis, np.float32).copy()
    i = _c(ids, np.uint32).copy()
    load().orc_bitonic_sort_dis(_p(d), _p(i), C.c_uint32(d.size))
    return d, i


def warp_sort(key, val):
    k = _c(key, np.float32).copy()
    v = _c(val, np.uint32).copy()
    load().orc_warp_sort(_p(k), _p(v), C.c_uint32(k.size))
    return k, v


def merge_top(d1, i1, d2, i2, tie=1):
    """merge_top on two sorted lists (tie 1: distance alone; 0: ties by id);
    returns the lists' new contents."""
    a = [_c(d1, np.float32).copy(), _c(i1, np.uint32).copy(), _c(d2, np.float32).copy(), _c(i2, np.uint32).copy()]
    load().orc_merge_top(_p(a[0]), _p(a[1]), C.c_uint32(a[0].size), _p(a[2]), _p(a[3]), C.c_uint32(a[2].size),
                         C.c_int(tie))
    return a


def merge_recycle(attrs, lo, hi, dA, iA, dB, iB, dR, iR, tie=1):
    """merge_top_with_recycle_list + the evictee sort and recycle merge:
    returns (A, B, recycle) as (distances, ids) pairs."""
    attrs = _c(attrs, np.float32)
    lo = _c(lo, np.float32)
    hi = _c(hi, np.float32)
    a = [_c(x, dt).copy() for x, dt in ((dA, np.float32), (iA, np.uint32), (dB, np.float32), (iB, np.uint32),
                                         (dR, np.float32), (iR, np.uint32))]
    load().orc_merge_recycle(_p(attrs), C.c_uint32(attrs.shape[1]), _p(lo), _p(hi), _p(a[0]), _p(a[1]),
                             C.c_uint32(a[0].size), _p(a[2]), _p(a[3]), C.c_uint32(a[2].size), _p(a[4]), _p(a[5]),
                             C.c_uint32(a[4].size), C.c_int(tie))
    return (a[0], a[1]), (a[2], a[3]), (a[4], a[5])


def ground_truth(data, attrs, queries, lo, hi, K, nthreads=0):
    data = _c(data, np.float32)
    attrs = _c(attrs, np.float32)
    queries = _c(queries, np.float32)
    lo = _c(lo, np.float32)
    hi = _c(hi, np.float32)
    N, D = data.shape
    Q = queries.shape[0]
    ids = np.empty((Q, K), np.uint32)
    dist = np.empty((Q, K), np.float64)
    load().orc_ground_truth(C.c_uint32(N), C.c_uint32(D), C.c_uint32(attrs.shape[1]), _p(data), _p(attrs),
                            C.c_uint32(Q), _p(queries), _p(lo), _p(hi), C.c_uint32(K), _p(ids), _p(dist),
                            C.c_int(nthreads))
    return ids, dist


def recall(res, gt, gt_dist, res_dist_exact=None, tie_aware=False):
    res = _c(res, np.uint32)
    gt = _c(gt, np.uint32)
    gt_dist = _c(gt_dist, np.float64)
    Q, K = res.shape
    rd = _c(res_dist_exact if res_dist_exact is not None else np.zeros_like(gt_dist), np.float64)
    return load().orc_recall(C.c_uint32(Q), C.c_uint32(K), _p(res), _p(gt), _p(gt_dist), _p(rd),
                             C.c_int(int(tie_aware)))


# ------------------------------------------------------------ index build
# Restatements of the reference's index-build scripts (numpy), the checker
# of gf_grid_scatter / gf_build_graphs.

def grid_scatter(attrs, grid):
    """grid_scatter_V2 (indexbuild/tools.py:88-125): per attribute a stable
    argsort (:98), runs of avg = ceil(N / g) ranks (:100-107; the last run
    takes the rest), quantiles = the sorted values at each run's first and
    last rank (:101-102, :108), global pid = row-major with the last attribute
    fastest (:111-120)."""
    attrs = np.asarray(attrs, np.float64)
    n, a = attrs.shape
    l_q, r_q, pid_lists = [], [], []
    for d in range(a):
        order = np.argsort(attrs[:, d], kind="stable")
        srt = attrs[order, d]
        g = int(grid[d])
        avg = (n + g - 1) // g
        idx = np.zeros(n, np.int64)
        left = [j * avg for j in range(g)]
        right = [(j + 1) * avg - 1 if j < g - 1 else n - 1 for j in range(g)]
        for j in range(g):
            idx[order[left[j]:right[j] + 1]] = j
        l_q.append(srt[left])
        r_q.append(srt[right])
        pid_lists.append(idx)
    factors = np.concatenate([np.cumprod(np.asarray(grid, np.int64)[::-1])[::-1][1:], [1]])
    global_pid = sum(factors[d] * pid_lists[d] for d in range(a))
    return l_q, r_q, pid_lists, global_pid


def _members(global_pid, P):
    order = np.argsort(np.asarray(global_pid), kind="stable")
    bounds = np.concatenate([[0], np.cumsum(np.bincount(global_pid, minlength=P))])
    return [order[bounds[c]:bounds[c + 1]] for c in range(P)]


def _sq(x, y):
    """Exact squared distances of integer-valued rows (int64): the dot
    products run in float64, exact while every partial sum stays below 2^53."""
    xi = x.astype(np.int64)
    yi = y.astype(np.int64)
    dots = np.rint(x.astype(np.float64) @ y.astype(np.float64).T).astype(np.int64)
    return (xi * xi).sum(1)[:, None] + (yi * yi).sum(1)[None, :] - 2 * dots


def knn_cell_graphs(vectors, global_pid, P, R):
    """Per-cell graphs in the layout of cagra_build.py:94-127 (rows of R
    cell-local ids, cells concatenated in cell order, members by ascending
    point id), exact: each point's R nearest other points of its cell by
    (squared distance, local id); fewer than R others repeat the nearest; a
    point alone in its cell lists itself."""
    v = np.asarray(vectors)
    rows = []
    for mem in _members(global_pid, P):
        n = len(mem)
        if n == 0:
            continue
        # (distance, local id) order as one int64 key per pair; self last
        key = _sq(v[mem], v[mem]) * n + np.arange(n)[None, :]
        np.fill_diagonal(key, np.iinfo(np.int64).max)
        o = np.argsort(key, axis=1, kind="stable")[:, :max(0, min(R, n - 1))]
        g = np.empty((n, R), np.uint32)
        if n == 1:
            g[:] = 0
        else:
            g[:, :o.shape[1]] = o
            g[:, o.shape[1]:] = o[:, :1]
        rows.append(g)
    return np.concatenate(rows, 0)


def cross_graph(vectors, global_pid, P, E):
    """Cross-cell graph of global_graph_build.py:106-176 (row p, columns
    c*E .. c*E+E-1: the E nearest points of cell c to point p as cell-local
    ids, p's own cell included), exact by (squared distance, local id);
    a cell with fewer than E points repeats the nearest; edges into an empty
    cell are 0."""
    v = np.asarray(vectors)
    N = v.shape[0]
    out = np.zeros((N, P * E), np.uint32)
    for c, mem in enumerate(_members(global_pid, P)):
        n = len(mem)
        if n == 0:
            continue
        key = _sq(v, v[mem]) * n + np.arange(n)[None, :]
        o = np.argsort(key, axis=1, kind="stable")[:, :min(E, n)]
        out[:, c * E:c * E + o.shape[1]] = o
        out[:, c * E + o.shape[1]:(c + 1) * E] = o[:, :1]
    return out


def graph_rows(vectors, global_pid, P, R, rows):
    """knn_cell_graphs' rows of the points `rows` only (row i = point rows[i])."""
    v = np.asarray(vectors)
    gp = np.asarray(global_pid)
    mem = _members(gp, P)
    out = np.empty((len(rows), R), np.uint32)
    for i, p in enumerate(rows):
        m = mem[gp[p]]
        n = len(m)
        self_lid = int(np.searchsorted(m, p))
        if n == 1:
            out[i] = self_lid
            continue
        key = _sq(v[p:p + 1], v[m])[0] * n + np.arange(n)
        key[self_lid] = np.iinfo(np.int64).max
        o = np.argsort(key, kind="stable")[:min(R, n - 1)]
        out[i, :len(o)] = o
        out[i, len(o):] = o[0]
    return out


def cross_rows(vectors, global_pid, P, E, rows):
    """cross_graph's rows of the points `rows` only."""
    v = np.asarray(vectors)
    out = np.zeros((len(rows), P * E), np.uint32)
    for c, m in enumerate(_members(np.asarray(global_pid), P)):
        n = len(m)
        if n == 0:
            continue
        d = _sq(v[np.asarray(rows)], v[m]) * n + np.arange(n)[None, :]
        o = np.argsort(d, axis=1, kind="stable")[:, :min(E, n)]
        out[:, c * E:c * E + o.shape[1]] = o
        out[:, c * E + o.shape[1]:(c + 1) * E] = o[:, :1]
    return out


def _round_half_away(v):
    """C's round() of fp32 values: half away from zero (exact in float64)."""
    v = np.asarray(v, np.float32).astype(np.float64)
    return np.trunc(v + np.copysign(0.5, v))


def quantise_i8(x, alpha=1.0, mutation=0):
    """The reference's int8 quantisation of its out-of-core loader
    (indexsearch/production_adapter.cuh:113-165), in fp32: x *= alpha; per
    dimension min and max starting from 100000 and -100000; scale = (max -
    min) / 255; zero point round(-128 - min / scale) clamped to [-128, 127];
    q = round(x / scale) + zero point clamped to [-128, 127]; round() half
    away from zero.  A dimension with max == min (the reference divides by
    zero there) takes scale 1.  Returns (q int8, scale fp32, zero int32).
    mutation 1: round half to even; 2: min and max from the data alone."""
    v = np.asarray(x, np.float32) * np.float32(alpha)
    if mutation == 2:
        mn, mx = v.min(axis=0), v.max(axis=0)
    else:
        mn = np.minimum(np.float32(100000.0), v.min(axis=0))
        mx = np.maximum(np.float32(-100000.0), v.max(axis=0))
    s = (mx - mn) / np.float32(255.0)
    s = np.where(s > 0, s, np.float32(1.0)).astype(np.float32)
    rnd = np.rint if mutation == 1 else _round_half_away
    z = np.clip(rnd(np.float32(-128.0) - mn / s), -128, 127).astype(np.int32)
    q = np.clip(rnd(v / s) + z, -128, 127).astype(np.int8)
    return q, s, z


def quantise_u8(vectors):
    """The builder's u8 quantisation of float data for its candidate pass:
    rint((x - min) / s), s = (max - min) / 255, in float64 over all values
    (all 0 when they are equal)."""
    v = np.asarray(vectors, np.float32).astype(np.float64)
    lo, hi = v.min(), v.max()
    s = (hi - lo) / 255.0
    q = np.rint((v - lo) / s) if s > 0 else np.zeros_like(v)
    return np.clip(q, 0, 255).astype(np.uint8)


def canon_dists(q, X):
    """Canonical fp32 distances of query q to the rows of X (the kernels'
    summation order for fp32 rows, garfield_oracle.cpp canon_dist)."""
    lib = load()
    q = np.ascontiguousarray(q, np.float32)
    X = np.ascontiguousarray(X, np.float32)
    out = np.empty(X.shape[0], np.float32)
    lib.orc_canon_dists(_p(q), _p(X), C.c_uint32(X.shape[0]), C.c_uint32(q.size), _p(out))
    return out


def _rerank(q, X, cand, keep, fill):
    """Candidate local ids re-ranked by (canonical fp32 distance, id),
    repeats and ids in `drop` removed; the first `keep`, a short list
    repeating its nearest (or `fill` when empty)."""
    ids = list(dict.fromkeys(int(c) for c in cand))
    if not ids:
        return [fill] * keep
    d = canon_dists(q, X[ids])
    order = sorted(range(len(ids)), key=lambda i: (d[i].view(np.uint32), ids[i]))
    out = [ids[i] for i in order][:keep]
    return out + [out[0]] * (keep - len(out))


FLOAT_MARGIN = 16


def float_graph_rows(vectors, global_pid, P, R, rows, margin=FLOAT_MARGIN, mutation=0):
    """Per-cell graph rows of float data for the points `rows`: the
    candidates are graph_rows of the u8 quantisation (quantise_u8) at degree
    min(R + margin, 63); they are re-ranked by canonical fp32 distance (ties
    by local id), repeats and the point itself dropped, and the first R kept
    (a short row repeats its nearest; a point alone lists itself).
    mutation (tests only): 1 re-ranks by the quantised order (no re-rank)."""
    v = np.asarray(vectors, np.float32)
    gp = np.asarray(global_pid)
    Rk = min(R + margin, 63)
    cand = graph_rows(quantise_u8(v), gp, P, Rk, rows)
    mem = _members(gp, P)
    out = np.empty((len(rows), R), np.uint32)
    for i, p in enumerate(rows):
        m = mem[gp[p]]
        self_lid = int(np.searchsorted(m, p))
        c = [x for x in cand[i] if x != self_lid]
        if mutation == 1:
            c = list(dict.fromkeys(int(x) for x in c))[:R]
            out[i] = (c + [c[0]] * (R - len(c))) if c else [self_lid] * R
            continue
        out[i] = _rerank(v[p], v[m], c, R, self_lid)
    return out


def float_cross_rows(vectors, global_pid, P, E, rows, margin=FLOAT_MARGIN):
    """Cross-cell rows of float data for the points `rows`: for every
    non-empty cell, cross_rows of the u8 quantisation with min(E + margin,
    64) candidates, re-ranked by canonical fp32 distance (ties by local id),
    repeats dropped, the first E kept (a short list repeats its nearest);
    edges into an empty cell are 0."""
    v = np.asarray(vectors, np.float32)
    gp = np.asarray(global_pid)
    Ek = min(E + margin, 64)
    cand = cross_rows(quantise_u8(v), gp, P, Ek, rows)
    out = np.zeros((len(rows), P * E), np.uint32)
    for c, m in enumerate(_members(gp, P)):
        if len(m) == 0:
            continue
        for i, p in enumerate(rows):
            out[i, c * E:(c + 1) * E] = _rerank(v[p], v[m], cand[i, c * Ek:(c + 1) * Ek], E, 0)
    return out


def detour_order(knn_cell):
    """One cell's kNN rows (n x I, local ids) in ascending (detourable
    routes, rank) order, the reordering step of CAGRA's graph optimisation
    (Ootomo et al., ICDE 2024): edge k of row a, to d = g[a, k], has a detour
    through every b = g[a, j], j < k, whose own row lists d at a position
    below k (first occurrence)."""
    g = np.asarray(knn_cell, np.int64)
    n, I = g.shape
    pos = np.full((n, n), I, np.int64)           # pos[b, x]: first position of x in row b
    for j in range(I - 1, -1, -1):
        pos[np.arange(n), g[:, j]] = j
    M = pos[g[:, :, None], g[:, None, :]]        # M[a, j, k] = position of g[a, k] in row g[a, j]
    k = np.arange(I)
    det = ((M < k[None, None, :]) & (k[None, :, None] < k[None, None, :])).sum(axis=1)
    order = np.argsort(det * I + k[None, :], axis=1, kind="stable")
    return np.take_along_axis(g, order, axis=1), det


def optimize_graphs(knn_graphs, cell_sizes, R):
    """gf_optimize_graphs restated: per cell, the detour order, then reverse
    edges (for every rank k < R of the reordered rows, in row order, edge
    a -> b appends a to b's reverse list, at most R, never b itself), then
    each row = its first R // 2 reordered edges, its reverse edges, the rest
    of its reordered row, each id once, padded with its first id."""
    g = np.asarray(knn_graphs, np.int64)
    I = g.shape[1]
    out = np.empty((g.shape[0], R), np.uint32)
    start = 0
    for n in cell_sizes:
        n = int(n)
        if n == 0:
            continue
        o, _ = detour_order(g[start:start + n])
        rev = [[] for _ in range(n)]
        for k in range(R):
            for a in range(n):
                b = int(o[a, k])
                if b != a and len(rev[b]) < R:
                    rev[b].append(a)
        for a in range(n):
            row = []
            for x in list(o[a, :R // 2]) + rev[a] + list(o[a, R // 2:]):
                if len(row) < R and int(x) not in row:
                    row.append(int(x))
            row += [row[0]] * (R - len(row))
            out[start + a] = row
        start += n
    return out


def kmeans(vectors, C, iters, init_ids):
    """gf_kmeans' definition (the reference fits cuVS k-means, absent here,
    clustering.py:68-87): integer Lloyd rounds from the points init_ids;
    assignment = nearest centre by exact squared distance, the smaller centre
    index on ties (np.argmin); update = floor((2 sum + n) / (2 n)) per
    dimension, an empty cluster kept; `iters` rounds, then a final
    assignment.  Returns (labels, centres)."""
    x = np.asarray(vectors).astype(np.int64)
    cen = x[np.asarray(init_ids)].copy()
    for it in range(iters + 1):
        lab = np.argmin(_sq(x, cen), axis=1)
        if it == iters:
            return lab.astype(np.int32), cen.astype(np.uint8)
        n = np.bincount(lab, minlength=C).astype(np.int64)
        sums = np.zeros_like(cen)
        np.add.at(sums, lab, x)
        nz = n > 0
        cen[nz] = (2 * sums[nz] + n[nz, None]) // (2 * n[nz, None])


def plan_cells(cells_, counts, grid, cell_size, max_points=0, max_cells=16, mutation=0):
    """Batch plan for out-of-core streaming from stage A cell lists, restated
    as a memoised recursion over boxes of the grid.  The objective is the
    out-of-core pipeline's cell scheduling (README.md:5: cells grouped so
    that few queries are active per batch; the shipped driver fixes its
    batches by hand, indexsearch/bigdataset/bigdataset_experiment.cu:271-277,
    746-756): the sum over batches of the queries selecting one of the
    batch's cells.  Batches are boxes (at most max_cells non-empty cells and
    max_points points, 0 = no limit) of the best guillotine partition: a box
    that fits is one batch; otherwise it is cut between cells t-1 and t of
    axis d, minimising (queries selecting cells on both sides + the parts'
    costs, then the number of batches), first (d, t) in ascending order on a
    tie.  A query is the bounding box of its cells; grid cells are row-major,
    last axis fastest.  Returns (plan, active) with active recounted from
    the lists.  mutation (tests only): 1 counts a cut's straddling queries
    without testing that they meet the box on the other axes, 2 compares
    (batches, cost) instead of (cost, batches)."""
    grid = [int(g) for g in grid]
    a = len(grid)
    P = int(np.prod(grid))
    sizes = [int(x) for x in cell_size]
    coords = np.array(np.unravel_index(np.arange(P), grid)).T          # P x a
    boxes = []
    for q in range(len(counts)):
        n = int(counts[q])
        if n:
            cc = coords[np.asarray(cells_[q][:n], np.int64)]
            boxes.append((cc.min(0), cc.max(0)))
    qlo = np.array([b[0] for b in boxes], np.int64).reshape(-1, a)
    qhi = np.array([b[1] for b in boxes], np.int64).reshape(-1, a)

    def cells_in(x0, x1):
        return [c for c in range(P) if sizes[c] and all(x0[d] <= coords[c][d] <= x1[d] for d in range(a))]

    def cut(x0, x1, d, t):
        m = (qlo[:, d] <= t - 1) & (qhi[:, d] >= t)
        if mutation != 1:
            for e in range(a):
                if e != d:
                    m &= (qlo[:, e] <= x1[e]) & (qhi[:, e] >= x0[e])
        return int(m.sum())

    memo = {}

    def best(x0, x1):
        key = (x0, x1)
        if key in memo:
            return memo[key]
        inside = cells_in(x0, x1)
        pts = sum(sizes[c] for c in inside)
        unit = all(x0[d] == x1[d] for d in range(a))
        if unit or ((max_cells == 0 or len(inside) <= max_cells) and (max_points == 0 or pts <= max_points)):
            memo[key] = (0, 1 if inside else 0, None)
            return memo[key]
        res = None
        for d in range(a):
            for t in range(x0[d] + 1, x1[d] + 1):
                lo_hi = x1[:d] + (t - 1,) + x1[d + 1:]
                hi_lo = x0[:d] + (t,) + x0[d + 1:]
                ca, la, _ = best(x0, lo_hi)
                cb, lb, _ = best(hi_lo, x1)
                c, l = cut(x0, x1, d, t) + ca + cb, la + lb
                k = (l, c) if mutation == 2 else (c, l)
                if res is None or k < res[0]:
                    res = (k, c, l, (d, t))
        memo[key] = (res[1], res[2], res[3])
        return memo[key]

    plan = []

    def emit(x0, x1):
        _, _, sp = best(x0, x1)
        if sp is None:
            inside = cells_in(x0, x1)
            if inside:
                plan.append(inside)
            return
        d, t = sp
        emit(x0, x1[:d] + (t - 1,) + x1[d + 1:])
        emit(x0[:d] + (t,) + x0[d + 1:], x1)

    emit(tuple([0] * a), tuple(g - 1 for g in grid))
    sets = [set(int(c) for c in cells_[q][:int(counts[q])]) for q in range(len(counts))]
    active = sum(sum(1 for st in sets if st & set(bt)) for bt in plan)
    return plan, active
