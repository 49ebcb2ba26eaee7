"""Approximate cross-cell graph by per-cell graph search, the method of the
reference's indexbuild/global_graph_build.py:106-176: every point searches
every cell's graph index for its E nearest points there (the reference runs
cagra.search with itopk_size = searchEf and k = edges_num, in batches of
62 500 queries, and stores the cell-local neighbour ids).

Here the search is the library's own traversal (gf_search) restricted to one
cell per query, with no attribute filter: for a cell c every point traverses
c's graph from the entry-point draw with a candidate list of ef and keeps its
E nearest found.  The exact builder (gf_build_graphs) needs N x N distances
for the cross edges; this needs about N x P searches of a few hundred
distances each, the route to indexes of C5's size.
"""
import numpy as np

from . import _lib


def global_graph_build(vectors, global_pid, P, cell_graphs, E, ef=32, batch=65536, vec_dtype=None, device=0):
    """Cross-cell graph (N x P*E, point-id order; row p, columns c*E..c*E+E-1:
    cell-local ids of p's E nearest points found in cell c, own cell
    included) by one single-cell search per (point, cell).  A search that
    finds fewer than E points (a cell smaller than E) repeats its nearest;
    edges into an empty cell are 0.  vec_dtype: the rows the traversal
    reads (default: u8 for u8 input, else fp32)."""
    v = np.ascontiguousarray(vectors)
    N = v.shape[0]
    gp = np.asarray(global_pid, np.int64)
    if vec_dtype is None:
        vec_dtype = _lib.VEC_U8 if v.dtype == np.uint8 else _lib.VEC_F32
    sizes = np.bincount(gp, minlength=P)
    order = np.argsort(gp, kind="stable")
    start = np.concatenate([[0], np.cumsum(sizes)])
    lrow = np.empty(N, np.int64)
    lrow[order] = np.arange(N) - start[gp[order]]          # cell-local id of each point
    # An index of the graphs alone: one attribute that every range below
    # holds, a grid of P cells along it, and no cross edges the single-cell
    # searches would read.
    ix = _lib.Index.from_arrays(v.astype(np.float32), np.zeros((N, 1), np.float32), [P],
                                np.arange(P, dtype=np.float32), np.arange(P, dtype=np.float32), gp,
                                cell_graphs, np.zeros((N, P), np.uint32), vec_dtype=vec_dtype, device=device)
    out = np.zeros((N, P * E), np.uint32)
    try:
        for s in range(0, N, batch):
            e = min(N, s + batch)
            Q = e - s
            b = ix.batch(v[s:e].astype(np.float32), np.full((Q, 1), -1.0, np.float32),
                         np.full((Q, 1), 1.0, np.float32))
            cells = np.zeros((Q, P), np.uint32)
            ones = np.ones(Q, np.uint32)
            zeros = np.zeros(Q, np.uint32)
            try:
                for c in range(P):
                    if not sizes[c]:
                        continue
                    cells[:, 0] = c
                    b.set_cells(cells, ones, zeros)
                    ids, _, _ = b.search(L=ef, K=E, rl=10)
                    found = ids != _lib.NO_RESULT
                    loc = np.where(found, lrow[np.where(found, ids, 0)], 0)
                    loc = np.where(found, loc, loc[:, :1])      # fewer than E: repeat the nearest
                    out[s:e, c * E:(c + 1) * E] = loc
            finally:
                b.close()
    finally:
        ix.close()
    return out
