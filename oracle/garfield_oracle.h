/*
 * CPU oracle for the Garfield query path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is a plain C++ restatement of the reference's query path
 * (ZJU-DAILY/Garfield, indexsearch/) written from the reference source read as
 * text.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only as the checker / CPU baseline: the product path
 * (libgarfield.so) never links or calls it.
 *
 * Each entry point cites the reference function it restates.  Semantics that
 * the reference leaves to thread races or that read out of bounds are replaced
 * by one deterministic rule, shared with the HIP implementation:
 *   - candidates are ordered by (distance, cell-major position) where the
 *     cell-major position of point g is offset[cell(g)] + local_idx[g];
 *     the reference orders equal distances by sorting-network position;
 *   - cross-cell entry slots are filled in slot order 0..127;
 *   - the +inf distance replaces the reference's 1e9 stand-in;
 *   - out-of-bounds reads of the reference (entry ids past a small first cell,
 *     the cross-edge fallback scan to 62500, the ci > L guard, ranges outside
 *     the grid) are
 *     replaced by the in-bounds rule named at each function.
 */
#ifndef GARFIELD_ORACLE_H
#define GARFIELD_ORACLE_H
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

#define ORC_SENTINEL_ID 0x7FFFFFFFu   /* reference's "no result" id (top & 0x7FFFFFFF) */

/* Index in the reference's representation (point-id order, idx mapper). */
typedef struct {
    uint32_t N, D, a, P, R, E;
    int32_t vdtype;               /* 0: fp32 vectors, 1: fp16 bit patterns, 2: u8 values (in vec_f32),
                                     3: int8 values q (in vec_f32) of x = qscale (q - qzero) */
    const float* vec_f32;         /* N*D, point-id order (vdtype 0, 2 and 3) */
    const float* qscale;          /* D (vdtype 3) */
    const int32_t* qzero;         /* D (vdtype 3) */
    const uint16_t* vec_f16;      /* N*D, point-id order, binary16 bits */
    const float* attrs;           /* N*a */
    const uint32_t* graph;        /* N*R, per-cell graphs concatenated in cell order */
    const uint32_t* offset;       /* P+1, cell start rows (graph_start_index / R) */
    const uint32_t* global_idx;   /* N: offset[c]+local -> point id */
    const uint32_t* local_idx;    /* N: point id -> local id in its cell */
    const uint32_t* cross;        /* N*P*E: cell-local ids, point-id order */
    /* The full graph (FD = 0: none; orc_full_graph), point-id order and
     * point ids, and its FD entry point ids (orc_entry_points_pair). */
    uint32_t FD;
    const uint32_t* fgraph;       /* N*FD */
    const uint32_t* fentry;       /* FD */
} orc_index;

/* full_graph_search.cuh:984-997 assemble_edges: row g of the full graph
 * holds, for every cell c in order, FE edges of g into c -- its own graph's
 * first FE edges when c is g's cell, else its first FE cross edges into c --
 * as point ids (local ids reduced modulo |c|; empty cells: 0xFFFFFFFF).
 * out: N*FE*P, point-id order. */
void orc_full_graph(const orc_index* ix, uint32_t FE, uint32_t* out);
/* gpu_graph.cu:12503-12539: the R traversal entries (orc_entry_points) and,
 * from the same generator, FD distinct full-graph entries drawn from [0, N). */
void orc_entry_points_pair(uint32_t N, uint32_t P, uint32_t R, uint32_t FD, uint32_t* out, uint32_t* outf);

/* tools.cuh:862-915 get_idx_mapper */
void orc_idx_mapper(uint32_t N, uint32_t P, const uint32_t* global_pid,
                    uint32_t* global_idx, uint32_t* local_idx, uint32_t* offset /*P+1*/);

/* tools.cuh:308-320 f2h: binary16 round-to-nearest-even of (x*alpha) in fp32 */
uint16_t orc_f2h_one(float x, float alpha);
void orc_f2h(const float* x, size_t n, float alpha, uint16_t* out);
float orc_h2f(uint16_t h);

/* tools.cuh:1561-1586 find_norm, canonical order of the HIP kernel
 * (64 lane-strided fp32 fma partial sums, then an xor butterfly). */
void orc_row_norms_f16(const uint16_t* x, uint32_t n, uint32_t D, float* out);

/* tools.cuh:569-602 load_clustering: fp32 centres (sequential sums, then divide)
 * and the cell x cluster histogram.  contiguous=1 reproduces the reference's
 * i / ceil(N/P) cell assignment (tools.cuh:587-590); 0 uses global_pid. */
void orc_centres_hist(uint32_t N, uint32_t D, uint32_t C, uint32_t P,
                      const float* data, const int32_t* labels,
                      const uint32_t* global_pid, int32_t contiguous,
                      float* centres /*C*D*/, uint32_t* hist /*P*C*/);

/* real_dataset_adapter.cuh:126-216 (+ gpu_graph.cu:10965-10973): selected cells
 * of each query in ascending cell id order.  cells is Q*P (stride P). */
void orc_cells(uint32_t Q, uint32_t a, const float* lo, const float* hi,
               const uint32_t* grid, const float* l_q, const float* r_q,
               const uint32_t* cell_size /* P or NULL: cells with no point are skipped */,
               uint32_t* cells, uint32_t* counts);

/* gpu_graph.cu:11095-11188 intersection_area_batch_mark_little_seg (arithmetic
 * grid): cell index trunc((v - min) / width) in fp32, clamped to [0, g - 1]
 * (the reference clamps only the upper one); little when the product of
 * per-attribute overlaps in cell widths (fp64, unfused) is <= thr.  An empty
 * range (lo > hi) selects nothing.  flags Q*P: 1 selected |
 * 2 little; little[q] = little cells; cells ascending (stride P). */
void orc_cells_grid(uint32_t Q, uint32_t a, const float* lo, const float* hi, const uint32_t* grid,
                    const float* amin, const float* width, double thr, const uint32_t* cell_size,
                    uint32_t* cells, uint32_t* counts, uint32_t* little, uint8_t* flags);

/* real_dataset_adapter.cuh:346-383 prefiltering_tag_elements: exact count of
 * points passing the range, and the routing value little[q]. */
void orc_selectivity(uint32_t Q, uint32_t N, uint32_t a, const float* attrs,
                     const float* lo, const float* hi, float threshold,
                     const uint32_t* counts, uint32_t* selcount, uint32_t* little,
                     int nthreads);

/* Centroid distances (tools.cuh:1493-1559) in fp64 from fp16 operands:
 * |q|^2 + |c|^2 - 2 q.c, the value the MFMA kernel approximates. */
void orc_centroid_dist_f64(uint32_t Q, uint32_t C, uint32_t D,
                           const uint16_t* qh, const uint16_t* ch, double* out);

/* tools.cuh:1398-1491 select_topk_by_reduce_min: the k nearest centres by
 * (distance, index) -- the reference keeps k=4 and breaks ties by thread. */
void orc_topk_clusters(uint32_t Q, uint32_t C, uint32_t k, const float* dist,
                       uint32_t* out);

/* gpu_graph.cu:11343-11396 sort_by_clustering_info_weighted: reorder each
 * query's cells by descending sum of hist[cell][c] over its top clusters;
 * ties by ascending cell id (tie mode 0) or in the order of the reference's
 * network bitonic_sort_id_by_num_int (gpu_graph.cu:123-141) (tie mode 1). */
void orc_sort_cells(uint32_t Q, uint32_t P, uint32_t C, uint32_t k,
                    uint32_t* cells, const uint32_t* counts,
                    const uint32_t* topk, const uint32_t* hist);

/* gpu_graph.cu:12503-12526 entry points: mt19937 (default seed),
 * uniform_int_distribution<>(0, rand_max-1) distinct draws, random_shuffle
 * after srand(1); rand_max = N - (P-1)*ceil(N/P). */
void orc_entry_points(uint32_t N, uint32_t P, uint32_t R, uint32_t* out);
/* The draw itself: min(ndraw, range) distinct values in [0, range), shuffled,
 * the first R (big_dataset_adapterV3.cuh:3862-3875 draws 10 L below the
 * smallest cell). */
void orc_entry_draw(uint32_t range, uint32_t ndraw, uint32_t R, uint32_t* out);

/* Canonical squared L2 distance between query q and point gid (the HIP
 * kernels' summation order). */
float orc_distance(const orc_index* ix, const void* q, uint32_t gid);
/* Canonical fp32 distances (the kernels' summation order for fp32 rows) of
 * query q to the n rows of X (n*D). */
void orc_canon_dists(const float* q, const float* X, uint32_t n, uint32_t D, float* out);

/* gpu_graph.cu:3266-4131 fused kernel (+ host wrapper 12463-12616):
 * cell-by-cell traversal or filtered brute force per query.
 * queries: Q*D fp32 (vdtype 0, 2; vdtype 3: times the index's f2h_factor)
 * or binary16 bits (vdtype 1).
 * cells: Q*P strided, already ordered.  counters: Q*ORC_NCNT. */
#define ORC_NCNT 8
enum { ORC_C_EXPAND = 0, ORC_C_DIST = 1, ORC_C_ATTR = 2, ORC_C_CROSS = 3,
       ORC_C_LROW = 4, ORC_C_SCAN = 5, ORC_C_PASS = 6, ORC_C_ROUTE = 7 };
void orc_search(const orc_index* ix, const void* queries, uint32_t Q,
                const float* lo, const float* hi,
                const uint32_t* cells, const uint32_t* counts, const uint32_t* little,
                const uint32_t* entry, uint32_t L, uint32_t K, uint32_t rl,
                uint32_t postfilter, uint32_t* out_ids, float* out_dist,
                uint32_t* counters, int nthreads);

/* Order of equal distances in orc_search: 0 (default) (distance, cell-major
 * position), the HIP kernels' total order; 1 the reference's -- distance
 * alone, its sorting networks (warpSort gpu_graph.cu:144-159,
 * bitonic_sort_id_by_dis_no_explore :77-101) and merge_top's ranks
 * (:162-222) deciding between equal distances.  Process-wide. */
void orc_set_tie_mode(int mode);
/* Distance arithmetic of the fp16 path (vdtype 1): 0 (default) binary16
 * values accumulated in fp32 in the kernels' canonical order; 1 REF_HFMA2,
 * the reference's half arithmetic (hsub2 / hfma2 in its lane order, hadd2
 * shfl_down tree, gpu_graph.cu:3394-3403) with every half operation rounded
 * once to binary16.  Process-wide. */
void orc_set_dist_mode(int mode);
/* binary16 round-to-nearest-even of a double; the REF_HFMA2 distance of two
 * binary16 rows (D a multiple of 4). */
uint16_t orc_half_rne(double v);
float orc_hfma2_dist(const uint16_t* q, const uint16_t* x, uint32_t D);
/* Plants one numbered mistake in the traversal (0 = none), so that tests can
 * show that their checks catch it; see MUT_* in garfield_oracle.cpp. */
void orc_set_mutation(int m);
/* Per-cell iteration cap of the traversal (0 restores the reference's 10000). */
void orc_set_max_iter(uint32_t n);
/* Traversal of traversal-routed queries: 1 (default) the fused kernel's
 * cell-by-cell search; 2 the dual-channel search of
 * select_path_..._dual_channel_in_turn_with_prefilter (gpu_graph.cu:6249-6640),
 * whose `entry` argument holds L entry ids (route counter 4). */
void orc_set_channels(int n);
/* Planted mistakes of the dual-channel search, for the pinning tests only. */
void orc_set_dual_mutation(int m);
/* One query (no little cells; postfilter as in orc_search: 1 << 30 forces
 * the traversal, 0 the full graph of an index that has one) with its
 * trajectory: the point ids expanded in order and the cell of each expansion
 * (P on the full graph; up to cap), and the recycle list before the final
 * merge.  Returns the expansions. */
uint32_t orc_search_trace(const orc_index* ix, const void* queries, uint32_t qi, const float* lo, const float* hi,
                          const uint32_t* cells, const uint32_t* counts, const uint32_t* entry, uint32_t L,
                          uint32_t K, uint32_t rl, uint32_t* out_ids, float* out_dist, uint32_t* counters,
                          uint32_t* expanded, uint32_t* expanded_cell, uint32_t cap, uint32_t* rec_ids,
                          float* rec_dist, uint32_t postfilter);
/* The oracle's building blocks, for known-answer tests:
 * bitonic_sort_id_by_dis_no_explore (gpu_graph.cu:77-101), warpSort
 * (:144-159), merge_top (:162-222; tie 0 orders equal distances by id) and
 * merge_top_with_recycle_list + the recycle merge (:224-315, 3412-3425). */
void orc_bitonic_sort_dis(float* dis, uint32_t* ids, uint32_t len);
void orc_warp_sort(float* key, uint32_t* val, uint32_t len);
void orc_merge_top(float* d1, uint32_t* i1, uint32_t n, float* d2, uint32_t* i2, uint32_t m, int tie);
void orc_merge_recycle(const float* attrs, uint32_t a, const float* lo, const float* hi, float* dA, uint32_t* iA,
                       uint32_t L, float* dB, uint32_t* iB, uint32_t R, float* dR, uint32_t* iR, uint32_t rl,
                       int tie);

/* gpu_graph.cu:10782-10812 naive_brute_force_with_filter: exact filtered kNN
 * on fp32 (computed in fp64), ascending by (distance, id); missing entries are
 * ORC_SENTINEL_ID with distance +inf. */
void orc_ground_truth(uint32_t N, uint32_t D, uint32_t a, const float* data,
                      const float* attrs, uint32_t Q, const float* queries,
                      const float* lo, const float* hi, uint32_t K,
                      uint32_t* gt_ids, double* gt_dist, int nthreads);

/* tools.cuh:384-453 recall: mean over queries of |res ∩ gt| / |gt| (1 if the
 * gt is empty).  tie_aware: a result also counts if its exact distance is
 * <= the K-th ground-truth distance. */
double orc_recall(uint32_t Q, uint32_t K, const uint32_t* res, const uint32_t* gt,
                  const double* gt_dist, const double* res_dist_exact, int tie_aware);

#ifdef __cplusplus
}
#endif
#endif
