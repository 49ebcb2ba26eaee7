"""garfield_amd: MI355X-native Garfield query path (multi-attribute range-filtered ANN).

Python binding of libgarfield.so over its C ABI (include/garfield.h).  The
functions below keep the names and argument meaning of the reference's host
stages (ZJU-DAILY/Garfield indexsearch/):

- ``intersection_area_mark_little_seg_V2``  real_dataset_adapter.cuh:388-519
- ``get_partitions_access_order_V2``        gpu_graph.cu:11742-11845
- ``batch_graph_search_gpu_with_prefilter_and_postfilter``  gpu_graph.cu:12463-12616

All computation runs in the HIP library; every call raises if the library has
not been built or cannot reach a GPU, and there is no CPU fallback.
"""
from ._lib import (GarfieldError, Index, Batch, SearchStats, lib_path, f2h, row_norms_f16,
                   entry_points, NO_RESULT, NCOUNTERS, VEC_F32, VEC_F16)


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


__all__ = [
    "GarfieldError", "Index", "Batch", "SearchStats", "lib_path", "f2h", "row_norms_f16",
    "entry_points", "NO_RESULT", "NCOUNTERS", "VEC_F32", "VEC_F16",
    "intersection_area_mark_little_seg_V2", "get_partitions_access_order_V2",
    "batch_graph_search_gpu_with_prefilter_and_postfilter",
]
