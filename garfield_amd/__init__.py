"""garfield_amd: MI355X-native Garfield query path (multi-attribute range-filtered ANN).

Python binding of libgarfield.so over its C ABI (include/garfield.h).  The
functions below keep the names and argument meaning of the reference's host
stages (ZJU-DAILY/Garfield indexsearch/):

- ``intersection_area_mark_little_seg_V2``  real_dataset_adapter.cuh:388-519
- ``get_partitions_access_order_V2``        gpu_graph.cu:11742-11845
- ``batch_graph_search_gpu_with_prefilter_and_postfilter``  gpu_graph.cu:12463-12616
- ``intersection_area_mark_little_seg_batch_process``  gpu_graph.cu:12066-12187 (arithmetic grid)
- ``batch_graph_search_gpu_with_prefilter_batch_process_compressed_graph_T_dataset_resident_u8``
  big_dataset_adapterV3.cuh:3719-4117 (out-of-core; the index is ``Index.create_streamed``)

All computation runs in the HIP library; every call raises if the library has
not been built or cannot reach a GPU, and there is no CPU fallback.
"""
from ._lib import (GarfieldError, Index, Batch, SearchStats, BuildStats, lib_path, f2h, row_norms_f16,
                   entry_points, grid_scatter, plan_cells, quantise_i8, build_graphs, optimize_graphs, kmeans, pinned_empty, search_noalloc, NO_RESULT, NCOUNTERS,
                   VEC_F32, VEC_F16, VEC_U8, VEC_I8Q, VEC_F16_REF)


def intersection_area_mark_little_seg_V2(batch, prefilter):
    """Stage A: cells per query and prefilter routing; returns device ms."""
    return batch.mark_cells(prefilter)


def get_partitions_access_order_V2(batch, topc=4):
    """Stage B: cluster-guided cell order; returns device ms."""
    return batch.order_cells(topc)


def batch_graph_search_gpu_with_prefilter_and_postfilter(batch, L, K=10, recycle_list_size=10,
                                                         postfilter=1 << 30, entry_points=None):
    """Stage C: traversal / brute force; returns (ids[Q,K], dists[Q,K], SearchStats)."""
    return batch.search(L=L, K=K, rl=recycle_list_size, postfilter=postfilter,
                        entry_points=entry_points)


def intersection_area_mark_little_seg_batch_process(batch, attr_min, attr_width, little_seg_threshold):
    """Stage A on an arithmetic grid (per-cell overlap areas); returns device ms."""
    return batch.mark_cells_grid(attr_min, attr_width, little_seg_threshold)


def batch_graph_search_gpu_with_prefilter_batch_process_compressed_graph_T_dataset_resident_u8(
        batch, L, K=10, recycle_list_size=10, entry_points=None):
    """Out-of-core stage C on a streamed index (the batch plan is the index's);
    returns (ids[Q,K], dists[Q,K], SearchStats)."""
    if not batch.index.streamed:
        raise GarfieldError(1, "not a streamed index: use batch_graph_search_gpu_with_prefilter_and_postfilter")
    return batch.search(L=L, K=K, rl=recycle_list_size, entry_points=entry_points)


def grid_scatter_V2(attrs, grid):
    """Index build: the rank-quantile grid (indexbuild/tools.py:88-125);
    returns (l_q, r_q, pid_lists, global_pid)."""
    return grid_scatter(attrs, grid)


__all__ = [
    "GarfieldError", "Index", "Batch", "SearchStats", "BuildStats", "lib_path", "f2h", "row_norms_f16",
    "entry_points", "grid_scatter", "grid_scatter_V2", "build_graphs", "kmeans", "pinned_empty", "NO_RESULT", "NCOUNTERS", "VEC_F32", "VEC_F16", "VEC_F16_REF", "VEC_U8",
    "intersection_area_mark_little_seg_V2", "get_partitions_access_order_V2",
    "batch_graph_search_gpu_with_prefilter_and_postfilter",
    "intersection_area_mark_little_seg_batch_process",
    "batch_graph_search_gpu_with_prefilter_batch_process_compressed_graph_T_dataset_resident_u8",
]
