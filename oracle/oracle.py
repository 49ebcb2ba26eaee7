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
                ("vec_f32", C.c_void_p), ("vec_f16", C.c_void_p), ("attrs", C.c_void_p),
                ("graph", C.c_void_p), ("offset", C.c_void_p), ("global_idx", C.c_void_p),
                ("local_idx", C.c_void_p), ("cross", C.c_void_p)]


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


def entry_draw(range_, ndraw, R):
    out = np.empty(R, np.uint32)
    load().orc_entry_draw(C.c_uint32(range_), C.c_uint32(ndraw), C.c_uint32(R), _p(out))
    return out


class OracleIndex:
    """The index in the reference's representation (point-id order + idx mapper)."""

    def __init__(self, vectors, attrs, global_pid, P, cell_graphs, cross, vec_f16=None, u8=False):
        """u8=True: the HIP path's uint8 vector mode (vectors hold the integer values)."""
        self.vectors = _c(vectors, np.float32)
        self.vec_f16 = None if vec_f16 is None else _c(vec_f16, np.uint16)
        self.attrs = _c(attrs, np.float32)
        self.graph = _c(cell_graphs, np.uint32)
        self.cross = _c(cross, np.uint32)
        self.P = P
        self.gidx, self.lidx, self.offset = idx_mapper(global_pid, P)
        N, D = self.vectors.shape
        self.s = _Index(N, D, self.attrs.shape[1], P, self.graph.shape[1], self.cross.shape[1] // P,
                        (2 if u8 else 0) if self.vec_f16 is None else 1, _p(self.vectors),
                        None if self.vec_f16 is None else _p(self.vec_f16), _p(self.attrs), _p(self.graph),
                        _p(self.offset), _p(self.gidx), _p(self.lidx), _p(self.cross))

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

    def distance(self, query, gid):
        dt = np.uint16 if self.vec_f16 is not None else np.float32
        q = _c(query, dt)
        return load().orc_distance(C.byref(self.s), _p(q), C.c_uint32(gid))


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
