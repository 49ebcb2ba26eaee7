"""ctypes binding of libgarfield.so (include/garfield.h)."""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
lib_path = os.environ.get("GARFIELD_LIB") or os.path.join(_HERE, "libgarfield.so")

NO_RESULT = 0x7FFFFFFF
NOALLOC_SCRATCH_MB = 32   # GF_NOALLOC_SCRATCH_MB
NCOUNTERS = 8
VEC_F32 = 0
VEC_F16 = 1
VEC_U8 = 2
VEC_I8Q = 3
VEC_F16_REF = 4   # binary16 rows, the reference's binary16 distance arithmetic
COUNTER_NAMES = ("expand", "dist", "attr", "cross", "lrow", "scan", "pass", "route")


class GarfieldError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"garfield status {status}: {msg}")
        self.status = status


class _Paths(C.Structure):
    _fields_ = [("data_path", C.c_char_p), ("cagra_prefix", C.c_char_p), ("cagra_suffix", C.c_char_p),
                ("global_graph", C.c_char_p), ("grid", C.c_char_p), ("attrs", C.c_char_p),
                ("cluster", C.c_char_p)]


class _OpenOpts(C.Structure):
    _fields_ = [("degree", C.c_uint32), ("f2h_factor", C.c_float), ("vec_dtype", C.c_int32),
                ("hist_contiguous", C.c_int32), ("device", C.c_int32), ("ref_ties", C.c_int32)]


class _Host(C.Structure):
    _fields_ = [("N", C.c_uint32), ("D", C.c_uint32), ("a", C.c_uint32), ("P", C.c_uint32),
                ("R", C.c_uint32), ("E", C.c_uint32),
                ("vectors", C.c_void_p), ("attrs", C.c_void_p), ("grid_shape", C.c_void_p),
                ("l_q", C.c_void_p), ("r_q", C.c_void_p), ("global_pid", C.c_void_p),
                ("cell_graphs", C.c_void_p), ("cross", C.c_void_p), ("labels", C.c_void_p)]


class _Info(C.Structure):
    _fields_ = [("N", C.c_uint32), ("D", C.c_uint32), ("a", C.c_uint32), ("P", C.c_uint32),
                ("R", C.c_uint32), ("E", C.c_uint32), ("C", C.c_uint32), ("vec_dtype", C.c_uint32),
                ("f2h_factor", C.c_float), ("device_bytes", C.c_uint64), ("streamed", C.c_uint32),
                ("nbatch", C.c_uint32)]


class _SearchOpts(C.Structure):
    _fields_ = [("L", C.c_uint32), ("K", C.c_uint32), ("rl", C.c_uint32), ("postfilter", C.c_uint32),
                ("entry_points", C.c_void_p)]


class _NoallocOpts(C.Structure):
    _fields_ = [("prefilter", C.c_float), ("topc", C.c_uint32), ("search", _SearchOpts)]


class _StreamPlan(C.Structure):
    _fields_ = [("device_budget", C.c_uint64), ("nbatch", C.c_uint32), ("batch_cells", C.c_uint32),
                ("sizes", C.c_void_p), ("cells", C.c_void_p)]


class SearchStats(C.Structure):
    _fields_ = [("ms_traverse", C.c_double), ("ms_bruteforce", C.c_double), ("ms_total", C.c_double),
                ("q_traverse", C.c_uint32), ("q_bruteforce", C.c_uint32), ("q_empty", C.c_uint32),
                ("n_expand", C.c_uint64), ("n_dist", C.c_uint64), ("n_attr", C.c_uint64),
                ("n_cross", C.c_uint64), ("n_lrow", C.c_uint64), ("n_scan", C.c_uint64),
                ("n_pass", C.c_uint64), ("bytes_traverse", C.c_double), ("bytes_bruteforce", C.c_double),
                ("ops_bruteforce", C.c_double), ("bf_mfma", C.c_uint32), ("ms_bf_kernel", C.c_double),
                ("n_batches", C.c_uint32), ("bytes_h2d", C.c_double), ("ms_h2d", C.c_double),
                ("ms_stage_a", C.c_double), ("ms_stage_b", C.c_double), ("graph", C.c_uint32),
                ("q_fullgraph", C.c_uint32), ("n_active", C.c_uint64)]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


class BuildStats(C.Structure):
    _fields_ = [("ms_tiles", C.c_double), ("ms_graph", C.c_double), ("ms_cross", C.c_double),
                ("pairs_graph", C.c_uint64), ("pairs_cross", C.c_uint64), ("dim", C.c_uint32),
                ("ms_prep", C.c_double), ("ms_upload", C.c_double), ("ms_run", C.c_double),
                ("ms_download", C.c_double), ("ms_total", C.c_double)]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


_SYMBOLS = {
    "gf_index_open": [C.POINTER(_Paths), C.POINTER(_OpenOpts), C.POINTER(C.c_void_p)],
    "gf_index_create": [C.POINTER(_Host), C.POINTER(_OpenOpts), C.POINTER(C.c_void_p)],
    "gf_index_create_streamed": [C.POINTER(_Host), C.POINTER(_OpenOpts), C.POINTER(_StreamPlan),
                                 C.POINTER(C.c_void_p)],
    "gf_index_open_streamed": [C.POINTER(_Paths), C.POINTER(_OpenOpts), C.POINTER(_StreamPlan),
                               C.POINTER(C.c_void_p)],
    "gf_index_close": [C.c_void_p],
    "gf_index_get_info": [C.c_void_p, C.POINTER(_Info)],
    "gf_batch_create": [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p)],
    "gf_batch_free": [C.c_void_p],
    "gf_mark_cells": [C.c_void_p, C.c_float, C.POINTER(C.c_double)],
    "gf_order_cells": [C.c_void_p, C.c_uint32, C.POINTER(C.c_double)],
    "gf_mark_cells_grid": [C.c_void_p, C.c_void_p, C.c_void_p, C.c_double, C.POINTER(C.c_double)],
    "gf_search": [C.c_void_p, C.POINTER(_SearchOpts), C.c_void_p, C.c_void_p, C.POINTER(SearchStats)],
    "gf_search_dual": [C.c_void_p, C.POINTER(_SearchOpts), C.c_void_p, C.c_void_p, C.POINTER(SearchStats)],
    "gf_batch_get_cells": [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p],
    "gf_batch_set_cells": [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p],
    "gf_batch_get_centroid": [C.c_void_p, C.c_void_p, C.c_void_p],
    "gf_batch_get_counters": [C.c_void_p, C.c_void_p],
    "gf_batch_get_cell_flags": [C.c_void_p, C.c_void_p],
    "gf_f2h": [C.c_void_p, C.c_size_t, C.c_float, C.c_void_p],
    "gf_row_norms_f16": [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p],
    "gf_entry_points": [C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p],
    "gf_grid_scatter": [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                        C.c_void_p],
    "gf_build_graphs": [C.c_void_p, C.c_int32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32,
                        C.c_uint32, C.c_int32, C.c_void_p, C.c_void_p, C.POINTER(BuildStats)],
    "gf_optimize_graphs": [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32, C.c_uint32, C.c_int32,
                           C.c_void_p, C.POINTER(C.c_double)],
    "gf_kmeans": [C.c_void_p, C.c_int32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_int32,
                  C.c_void_p, C.c_void_p, C.POINTER(C.c_double)],
    "gf_search_noalloc": [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.POINTER(_NoallocOpts),
                          C.c_void_p, C.c_void_p],
    "gf_stream_plan_cells": [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_uint64,
                             C.c_uint32, C.c_void_p, C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)],
    "gf_batch_plan_stream": [C.c_void_p, C.c_uint64, C.c_uint32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                             C.POINTER(C.c_double)],
    "gf_batch_set_stream_plan": [C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p],
    "gf_batch_get_stream_plan": [C.c_void_p, C.POINTER(C.c_uint32), C.c_void_p, C.c_void_p],
    "gf_quantise_i8": [C.c_void_p, C.c_uint64, C.c_uint32, C.c_float, C.c_void_p, C.c_void_p, C.c_void_p],
    "gf_host_alloc": [C.c_size_t, C.POINTER(C.c_void_p)],
    "gf_host_free": [C.c_void_p],
    "gf_status_str": [C.c_int32],
    "gf_last_error": [],
}

_lib = None


def load():
    """Load libgarfield.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(lib_path):
            raise ImportError(f"{lib_path} is missing: run __graft_entry__.build() "
                              "or python garfield_amd/build.py")
        lib = C.CDLL(lib_path)
        for name, args in _SYMBOLS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = C.c_char_p if name in ("gf_status_str", "gf_last_error") else C.c_int32
        _lib = lib
    return _lib


def _check(status):
    if status != 0:
        lib = load()
        raise GarfieldError(status, lib.gf_last_error().decode(errors="replace"))


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _opts(degree, f2h_factor, vec_dtype, hist_contiguous, device, ref_ties=False):
    return _OpenOpts(degree=degree, f2h_factor=f2h_factor, vec_dtype=vec_dtype,
                     hist_contiguous=int(hist_contiguous), device=device, ref_ties=int(ref_ties))


def _out_arrays(out, Q, K):
    """Result arrays for a search: fresh ones, or the caller's (ids, dists),
    checked to be C-contiguous (Q, K) uint32 and float32, since the library
    writes Q * K * 4 bytes into each."""
    if out is None:
        return np.empty((Q, K), np.uint32), np.empty((Q, K), np.float32)
    ids, dists = out
    for arr, dt in ((ids, np.uint32), (dists, np.float32)):
        if (not isinstance(arr, np.ndarray) or arr.shape != (Q, K) or arr.dtype != dt
                or not arr.flags.c_contiguous or not arr.flags.writeable):
            raise ValueError(f"out arrays must be writeable C-contiguous ({Q}, {K}) uint32 and float32")
    return ids, dists


def _entry_arg(entry_points, n, what):
    """The caller's entry-point draw, which the library reads n ids from
    (R for a cell-by-cell search, L for a dual-channel one)."""
    if entry_points is None:
        return None
    ent = _c(entry_points, np.uint32).reshape(-1)
    if ent.size != n:
        raise ValueError(f"entry_points must hold {what} = {n} ids, got {ent.size}")
    return ent


class Index:
    """A GMG index resident on one GPU."""

    def __init__(self, handle):
        self._h = handle
        info = _Info()
        _check(load().gf_index_get_info(self._h, C.byref(info)))
        self.N, self.D, self.a, self.P = info.N, info.D, info.a, info.P
        self.R, self.E, self.C = info.R, info.E, info.C
        self.vec_dtype, self.f2h_factor = info.vec_dtype, info.f2h_factor
        self.streamed, self.nbatch = bool(info.streamed), info.nbatch

    @classmethod
    def open(cls, data_path, cagra_prefix, cagra_suffix, global_graph, grid, attrs, cluster=None,
             degree=0, f2h_factor=1.0, vec_dtype=VEC_F32, hist_contiguous=False, device=0, ref_ties=False):
        enc = lambda s: None if s is None else str(s).encode()
        paths = _Paths(enc(data_path), enc(cagra_prefix), enc(cagra_suffix), enc(global_graph),
                       enc(grid), enc(attrs), enc(cluster))
        h = C.c_void_p()
        _check(load().gf_index_open(C.byref(paths), C.byref(_opts(degree, f2h_factor, vec_dtype,
                                                                    hist_contiguous, device, ref_ties)),
                                    C.byref(h)))
        return cls(h)

    @classmethod
    def from_arrays(cls, vectors, attrs, grid_shape, l_q, r_q, global_pid, cell_graphs, cross,
                    labels=None, f2h_factor=1.0, vec_dtype=VEC_F32, hist_contiguous=False, device=0,
                    degree=0, ref_ties=False):
        """Arrays as in the files: vectors (N,D) point order, cell_graphs (N,R)
        concatenated per cell in cell order, cross (N, P*E) point order."""
        keep = dict(
            vectors=_c(vectors, np.float32), attrs=_c(attrs, np.float32),
            grid=_c(grid_shape, np.uint32), l_q=_c(l_q, np.float32), r_q=_c(r_q, np.float32),
            pid=_c(global_pid, np.uint32), graphs=_c(cell_graphs, np.uint32), cross=_c(cross, np.uint32),
            labels=None if labels is None else _c(labels, np.int32))
        N, D = keep["vectors"].shape
        a = keep["attrs"].shape[1]
        P = int(np.prod(keep["grid"]))
        R = keep["graphs"].shape[1]
        E = keep["cross"].shape[1] // P
        host = _Host(N, D, a, P, R, E, _ptr(keep["vectors"]), _ptr(keep["attrs"]), _ptr(keep["grid"]),
                     _ptr(keep["l_q"]), _ptr(keep["r_q"]), _ptr(keep["pid"]), _ptr(keep["graphs"]),
                     _ptr(keep["cross"]), _ptr(keep["labels"]))
        h = C.c_void_p()
        _check(load().gf_index_create(C.byref(host), C.byref(_opts(degree, f2h_factor, vec_dtype,
                                                                     hist_contiguous, device, ref_ties)),
                                      C.byref(h)))
        return cls(h)

    @staticmethod
    def _plan(device_budget, plan, batch_cells):
        keep = None
        if plan is None:
            sp = _StreamPlan(int(device_budget), 0, int(batch_cells), None, None)
        else:
            sizes = _c([len(b) for b in plan], np.uint32)
            cells = _c([c for b in plan for c in b], np.uint32)
            keep = (sizes, cells)
            sp = _StreamPlan(int(device_budget), len(plan), int(batch_cells), _ptr(sizes), _ptr(cells))
        return sp, keep

    @classmethod
    def create_streamed(cls, vectors, attrs, grid_shape, l_q, r_q, global_pid, cell_graphs, cross,
                        plan=None, device_budget=0, batch_cells=16, vec_dtype=VEC_U8, device=0, degree=0):
        """A streamed (out-of-core) index: plan is a list of batches of cell
        ids (None: consecutive cells, batch_cells per batch)."""
        keep = dict(
            vectors=_c(vectors, np.float32), attrs=_c(attrs, np.float32),
            grid=_c(grid_shape, np.uint32), l_q=_c(l_q, np.float32), r_q=_c(r_q, np.float32),
            pid=_c(global_pid, np.uint32), graphs=_c(cell_graphs, np.uint32), cross=_c(cross, np.uint32))
        N, D = keep["vectors"].shape
        a = keep["attrs"].shape[1]
        P = int(np.prod(keep["grid"]))
        R = keep["graphs"].shape[1]
        E = keep["cross"].shape[1] // P
        host = _Host(N, D, a, P, R, E, _ptr(keep["vectors"]), _ptr(keep["attrs"]), _ptr(keep["grid"]),
                     _ptr(keep["l_q"]), _ptr(keep["r_q"]), _ptr(keep["pid"]), _ptr(keep["graphs"]),
                     _ptr(keep["cross"]), None)
        sp, _keep = cls._plan(device_budget, plan, batch_cells)
        h = C.c_void_p()
        _check(load().gf_index_create_streamed(C.byref(host), C.byref(_opts(degree, 1.0, vec_dtype, False, device)),
                                               C.byref(sp), C.byref(h)))
        return cls(h)

    @classmethod
    def open_streamed(cls, data_path, cagra_prefix, cagra_suffix, global_graph, grid, attrs, cluster=None,
                      plan=None, device_budget=0, batch_cells=16, degree=0, vec_dtype=VEC_U8, device=0):
        enc = lambda s: None if s is None else str(s).encode()
        paths = _Paths(enc(data_path), enc(cagra_prefix), enc(cagra_suffix), enc(global_graph),
                       enc(grid), enc(attrs), enc(cluster))
        sp, _keep = cls._plan(device_budget, plan, batch_cells)
        h = C.c_void_p()
        _check(load().gf_index_open_streamed(C.byref(paths), C.byref(_opts(degree, 1.0, vec_dtype, False, device)),
                                             C.byref(sp), C.byref(h)))
        return cls(h)

    @property
    def device_bytes(self):
        """Device memory the index holds now (a streamed index's batch
        buffers grow for a query batch's larger plan)."""
        info = _Info()
        _check(load().gf_index_get_info(self._h, C.byref(info)))
        return info.device_bytes

    def close(self):
        if self._h:
            _check(load().gf_index_close(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def batch(self, queries, lo, hi):
        return Batch(self, queries, lo, hi)


class Batch:
    """A query batch (vectors + closed ranges) on the index's GPU."""

    def __init__(self, index, queries, lo, hi):
        self.index = index
        q = _c(queries, np.float32)
        lo = _c(lo, np.float32)
        hi = _c(hi, np.float32)
        if q.ndim != 2 or q.shape[1] != index.D:
            raise ValueError("queries must be (Q, D)")
        if lo.shape != (q.shape[0], index.a) or hi.shape != lo.shape:
            raise ValueError("lo/hi must be (Q, a)")
        self.Q = q.shape[0]
        self._topc = 0
        h = C.c_void_p()
        _check(load().gf_batch_create(index._h, _ptr(q), self.Q, _ptr(lo), _ptr(hi), C.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            _check(load().gf_batch_free(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def mark_cells(self, prefilter, timed=True):
        """Stage A; returns its device time in ms (timed=False: returns None
        without waiting for the stage; the search statistics report it)."""
        ms = C.c_double()
        _check(load().gf_mark_cells(self._h, float(prefilter), C.byref(ms) if timed else None))
        return ms.value if timed else None

    def mark_cells_grid(self, attr_min, attr_width, threshold):
        amin = _c(attr_min, np.float32)
        width = _c(attr_width, np.float32)
        ms = C.c_double()
        _check(load().gf_mark_cells_grid(self._h, _ptr(amin), _ptr(width), float(threshold), C.byref(ms)))
        return ms.value

    def get_cell_flags(self):
        f = np.empty((self.Q, self.index.P), np.uint8)
        _check(load().gf_batch_get_cell_flags(self._h, _ptr(f)))
        return f

    def order_cells(self, topc=4, timed=True):
        """Stage B; returns its device time in ms (timed=False: as mark_cells)."""
        ms = C.c_double()
        _check(load().gf_order_cells(self._h, int(topc), C.byref(ms) if timed else None))
        self._topc = topc
        return ms.value if timed else None

    def search(self, L, K=10, rl=10, postfilter=1 << 30, entry_points=None, out=None, channels=1):
        """out: optional (ids, dists) arrays of shape (Q, K), uint32 and float32,
        C-contiguous, that receive the results (a caller searching in a loop
        reuses them instead of touching fresh pages every call).  channels=2:
        the dual-channel traversal (gf_search_dual; entry_points then holds
        L ids)."""
        ids, dists = _out_arrays(out, self.Q, K)
        ent = _entry_arg(entry_points, L if channels == 2 else self.index.R,
                         "L (dual-channel)" if channels == 2 else "R")
        opts = _SearchOpts(L, K, rl, min(int(postfilter), 0xFFFFFFFF), _ptr(ent))
        st = SearchStats()
        fn = load().gf_search_dual if channels == 2 else load().gf_search
        _check(fn(self._h, C.byref(opts), _ptr(ids), _ptr(dists), C.byref(st)))
        return ids, dists, st

    def get_cells(self):
        P = self.index.P
        cells = np.empty((self.Q, P), np.uint32)
        counts = np.empty(self.Q, np.uint32)
        little = np.empty(self.Q, np.uint32)
        sel = np.empty(self.Q, np.uint32)
        _check(load().gf_batch_get_cells(self._h, _ptr(cells), _ptr(counts), _ptr(little), _ptr(sel)))
        return cells, counts, little, sel

    def set_cells(self, cells, counts, little):
        cells = _c(cells, np.uint32)
        counts = _c(counts, np.uint32)
        little = _c(little, np.uint32)
        _check(load().gf_batch_set_cells(self._h, _ptr(cells), _ptr(counts), _ptr(little)))

    def get_centroid(self):
        dist = np.empty((self.Q, self.index.C), np.float32)
        topk = np.empty((self.Q, self._topc), np.uint32)
        _check(load().gf_batch_get_centroid(self._h, _ptr(dist), _ptr(topk)))
        return dist, topk

    def plan_stream(self, max_points=0, max_cells=0):
        """Streamed index: plan this batch's batches from its stage A cell
        lists (gf_batch_plan_stream); its next searches use the plan.
        Returns (plan, active, ms): the batches of cell ids, the plan's
        active (query, batch) pairs, the call's host wall time."""
        nb = C.c_uint32(0)
        act = C.c_uint64(0)
        ms = C.c_double(0.0)
        _check(load().gf_batch_plan_stream(self._h, int(max_points), int(max_cells), C.byref(nb), C.byref(act),
                                           C.byref(ms)))
        return self.stream_plan(), int(act.value), ms.value

    def set_stream_plan(self, plan):
        """Streamed index: the batches this batch's searches use (a list of
        lists of cell ids); None or [] returns to the index's build-time plan."""
        plan = plan or []
        sizes = _c([len(b) for b in plan] or [0], np.uint32)
        cells = _c([c for b in plan for c in b] or [0], np.uint32)
        _check(load().gf_batch_set_stream_plan(self._h, len(plan), _ptr(sizes), _ptr(cells)))

    def stream_plan(self):
        """The plan this batch's next streamed search uses."""
        P = self.index.P
        nb = C.c_uint32(0)
        sizes = np.zeros(P, np.uint32)
        cells = np.zeros(P, np.uint32)
        _check(load().gf_batch_get_stream_plan(self._h, C.byref(nb), _ptr(sizes), _ptr(cells)))
        plan, k = [], 0
        for i in range(nb.value):
            plan.append([int(c) for c in cells[k:k + sizes[i]]])
            k += int(sizes[i])
        return plan

    def get_counters(self):
        c = np.empty((self.Q, NCOUNTERS), np.uint32)
        _check(load().gf_batch_get_counters(self._h, _ptr(c)))
        return c


def search_noalloc(index, queries, lo, hi, prefilter, topc=4, L=64, K=10, rl=10, postfilter=1 << 30,
                   entry_points=None, out=None):
    """Stages A, B and C in one call that allocates no device memory
    (gf_search_noalloc): the same ids and distances as
    Batch.mark_cells(prefilter) + order_cells(topc) + search(...)."""
    q = _c(queries, np.float32)
    lo = _c(lo, np.float32)
    hi = _c(hi, np.float32)
    if q.ndim != 2 or q.shape[1] != index.D or lo.shape != (q.shape[0], index.a) or hi.shape != lo.shape:
        raise ValueError("queries must be (Q, D) and lo/hi (Q, a)")
    Q = q.shape[0]
    ids, dists = _out_arrays(out, Q, K)
    ent = _entry_arg(entry_points, index.R, "R")
    opts = _NoallocOpts(float(prefilter), int(topc),
                        _SearchOpts(L, K, rl, min(int(postfilter), 0xFFFFFFFF), _ptr(ent)))
    _check(load().gf_search_noalloc(index._h, _ptr(q), Q, _ptr(lo), _ptr(hi), C.byref(opts), _ptr(ids),
                                    _ptr(dists)))
    return ids, dists


def f2h(x, alpha=1.0):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    _check(load().gf_f2h(_ptr(x), x.size, float(alpha), _ptr(out)))
    return out


def row_norms_f16(x):
    x = _c(x, np.uint16)
    out = np.empty(x.shape[0], np.float32)
    _check(load().gf_row_norms_f16(_ptr(x), x.shape[0], x.shape[1], _ptr(out)))
    return out


def entry_points(N, P, R):
    out = np.empty(R, np.uint32)
    _check(load().gf_entry_points(N, P, R, _ptr(out)))
    return out


def quantise_i8(x, alpha=1.0):
    """The int8 quantisation a VEC_I8Q index holds (gf_quantise_i8, host
    code): returns (q (n x D int8), scale (D fp32), zero (D int32)), the
    vector x dequantising to scale * (q - zero)."""
    v = _c(x, np.float32)
    n, D = v.shape
    q = np.empty((n, D), np.int8)
    s = np.empty(D, np.float32)
    z = np.empty(D, np.int32)
    _check(load().gf_quantise_i8(_ptr(v) if n else None, n, D, float(alpha), _ptr(s), _ptr(z),
                                 _ptr(q) if n else None))
    return q, s, z


def plan_cells(cells, counts, grid, cell_size, max_points=0, max_cells=16):
    """Batch plan for a streamed index from stage A cell lists (Q x P rows,
    counts[q] ids each, as Batch.get_cells returns them) on a grid of shape
    `grid` (gf_stream_plan_cells): returns (plan, active), plan a list of
    batches of cell ids (the form Index.create_streamed takes), active the
    plan's sum over batches of active queries."""
    cl = _c(cells, np.uint32)
    cn = _c(counts, np.uint32)
    sz = _c(cell_size, np.uint32)
    g = _c(grid, np.uint32).reshape(-1)
    Q = cn.shape[0]
    P = sz.shape[0]
    if int(np.prod(g)) != P:
        raise ValueError(f"grid {list(g)} does not hold {P} cells")
    if Q and cl.shape != (Q, P):
        raise ValueError(f"cells must be Q x P = {Q} x {P}, got {cl.shape}")
    sizes = np.zeros(P, np.uint32)
    flat = np.zeros(P, np.uint32)
    nb = C.c_uint32(0)
    act = C.c_uint64(0)
    _check(load().gf_stream_plan_cells(_ptr(cl) if Q else None, _ptr(cn) if Q else None, Q, g.shape[0], _ptr(g),
                                       _ptr(sz), int(max_points), int(max_cells), _ptr(sizes), _ptr(flat),
                                       C.byref(nb), C.byref(act)))
    plan, k = [], 0
    for i in range(nb.value):
        plan.append([int(c) for c in flat[k:k + sizes[i]]])
        k += int(sizes[i])
    return plan, int(act.value)


def grid_scatter(attrs, grid):
    """grid_scatter_V2 (indexbuild/tools.py:88-125) in the library: returns
    (l_q, r_q, pid_lists, global_pid); l_q / r_q are lists of per-attribute
    float32 arrays (attribute values are integers held as floats)."""
    att = _c(attrs, np.float32)
    if att.ndim != 2:
        raise GarfieldError(1, "attrs must be N x a")
    n, a = att.shape
    g = _c(grid, np.uint32)
    if g.shape != (a,):
        raise GarfieldError(1, "grid must hold one size per attribute")
    lq = np.empty(int(g.sum()), np.float32)
    rq = np.empty(int(g.sum()), np.float32)
    pl = np.empty((a, n), np.uint32)
    gp = np.empty(n, np.uint32)
    _check(load().gf_grid_scatter(_ptr(att), n, a, _ptr(g), _ptr(lq), _ptr(rq), _ptr(pl), _ptr(gp)))
    cut = np.cumsum(g)[:-1]
    return np.split(lq, cut), np.split(rq, cut), list(pl), gp


def build_graphs(vectors, global_pid, P, R, E, device=0, graphs=True, cross=True):
    """Exact per-cell graphs (N x R, cell-major) and cross-cell graph
    (N x P*E, point-id order) on the GPU; returns (graphs, cross, BuildStats)
    with None for a graph not asked for.  vectors: uint8, or float32 holding
    integers in [0, 255]."""
    v = np.asarray(vectors)
    if v.ndim != 2:
        raise GarfieldError(1, "vectors must be N x D")
    if v.dtype == np.uint8:
        v, vt = np.ascontiguousarray(v), VEC_U8
    else:
        v, vt = _c(v, np.float32), VEC_F32
    n, d = v.shape
    gp = _c(global_pid, np.uint32)
    if gp.shape != (n,):
        raise GarfieldError(1, "global_pid must hold one cell per vector")
    g = np.empty((n, R), np.uint32) if graphs else None
    x = np.empty((n, P * E), np.uint32) if cross else None
    st = BuildStats()
    _check(load().gf_build_graphs(_ptr(v), vt, n, d, _ptr(gp), P, R if graphs else 0, E if cross else 0,
                                  device, _ptr(g), _ptr(x), C.byref(st)))
    return g, x, st


def optimize_graphs(knn_graphs, cell_sizes, R, device=0):
    """gf_optimize_graphs: the kNN graphs (N, I) -> optimised graphs (N, R)
    (rank-based reordering by detourable routes, then reverse edges)."""
    g = _c(knn_graphs, np.uint32)
    sz = _c(cell_sizes, np.uint32)
    N, I = g.shape
    out = np.empty((N, R), np.uint32)
    ms = C.c_double()
    _check(load().gf_optimize_graphs(_ptr(g), N, I, _ptr(sz), sz.size, R, device, _ptr(out), C.byref(ms)))
    return out, ms.value


def kmeans(vectors, ncent, iters, init_ids=None, seed=5, device=0):
    """Cluster labels (gf_kmeans): integer Lloyd rounds from the points
    init_ids (default: ncent distinct points drawn with numpy's
    default_rng(seed)); returns (labels int32[N], centres uint8[ncent, D],
    wall ms)."""
    v = np.asarray(vectors)
    if v.ndim != 2:
        raise GarfieldError(1, "vectors must be N x D")
    if v.dtype == np.uint8:
        v, vt = np.ascontiguousarray(v), VEC_U8
    else:
        v, vt = _c(v, np.float32), VEC_F32
    n, d = v.shape
    if init_ids is None:
        init_ids = np.random.default_rng(seed).choice(n, size=ncent, replace=False)
    ids = _c(init_ids, np.uint32)
    if ids.shape != (ncent,):
        raise GarfieldError(1, "init_ids must hold ncent point ids")
    lab = np.empty(n, np.int32)
    cen = np.empty((ncent, d), np.uint8)
    ms = C.c_double()
    _check(load().gf_kmeans(_ptr(v), vt, n, d, ncent, iters, _ptr(ids), device, _ptr(lab), _ptr(cen),
                            C.byref(ms)))
    return lab, cen, ms.value


def pinned_empty(shape, dtype):
    """An uninitialised numpy array in page-locked host memory (gf_host_alloc),
    freed when the array is collected; Batch.search(out=...) copies into such
    arrays directly."""
    import weakref
    dt = np.dtype(dtype)
    n = int(np.prod(shape)) * dt.itemsize
    ptr = C.c_void_p()
    _check(load().gf_host_alloc(max(n, 1), C.byref(ptr)))
    buf = (C.c_uint8 * max(n, 1)).from_address(ptr.value)
    weakref.finalize(buf, load().gf_host_free, C.c_void_p(ptr.value))
    return np.frombuffer(buf, dtype=dt, count=int(np.prod(shape))).reshape(shape)
