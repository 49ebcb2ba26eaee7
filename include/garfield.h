/*
 * garfield.h -- C ABI of the MI355X-native Garfield query path (libgarfield.so).
 *
 * The reference (ZJU-DAILY/Garfield) has no FFI: its query path sits behind
 * three host C++ functions, a CLI and a set of index files.  This header is the
 * plain-C replacement a binding (ctypes, cgo, JNI) attaches to.  Every entry
 * point names the reference interface it replaces (file:line under
 * indexsearch/ or indexbuild/).
 *
 * Conventions: all pointers are host pointers; sizes are element counts;
 * every call returns a gf_status (0 = success) and never exits the process;
 * gf_last_error() gives a message for the last failure on the calling thread.
 * One gf_index per device; calls on one handle must be serialised by the
 * caller.  Result ids are point ids (positions in the .fvecs file); a missing
 * result is GF_NO_RESULT, as the reference's top & 0x7FFFFFFF sentinel.
 */
#ifndef GARFIELD_H
#define GARFIELD_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t gf_status;
#define GF_OK 0
#define GF_E_ARG 1          /* invalid argument or inconsistent sizes */
#define GF_E_IO 2           /* file cannot be opened or is truncated */
#define GF_E_FORMAT 3       /* file contents violate the index format */
#define GF_E_DEVICE 4       /* HIP runtime error */
#define GF_E_NOMEM 5        /* device or host allocation failed */
#define GF_E_UNSUPPORTED 6  /* valid input outside what this build supports */
#define GF_E_STATE 7        /* call out of order (e.g. search before mark) */

#define GF_NO_RESULT 0x7FFFFFFFu

#define GF_VEC_F32 0        /* traversal distances on fp32 vectors */
#define GF_VEC_F16 1        /* on binary16 copies half(x * f2h_factor), fp32 accumulation */
#define GF_VEC_U8 2         /* on uint8 copies (vectors must be integers in [0, 255], as the
                               reference's u8 datasets, tools.cuh:134-150), fp32 accumulation */
#define GF_VEC_I8Q 3        /* on int8 copies quantised per dimension as the reference's
                               out-of-core loader does (production_adapter.cuh:108-165: scale
                               (max - min) / 255, zero point round(-128 - min / scale), q =
                               round(x / scale) + zero point in [-128, 127], after x *= f2h_factor);
                               distances to the dequantised scale * (q - zero point) in fp32;
                               resident indexes only */
#define GF_VEC_F16_REF 4    /* binary16 copies as GF_VEC_F16, distances in the reference's binary16
                               arithmetic: per 4-element chunk, in its 32-lane chunk order,
                               acc = __hfma2(q - x, q - x, acc) rounded to binary16 at every step,
                               then its shfl_down 16..1 __hadd2 tree and float(acc.x) + float(acc.y)
                               (gpu_graph.cu:3394-3403, 3508-3530); the brute force runs on the
                               gather kernel; resident indexes only */

typedef struct gf_index gf_index;
typedef struct gf_batch gf_batch;

/* Index files: the realdataset_search flags that name them
 * (realdataset_search.cu:2712-2751; formats in README.md:101-170). */
typedef struct {
    const char* data_path;     /* --data_path    .fvecs base vectors */
    const char* cagra_prefix;  /* --cagra_prefix per-cell graph i is prefix + i + suffix */
    const char* cagra_suffix;  /* --cagra_suffix */
    const char* global_graph;  /* --global_graph cross-cell graph */
    const char* grid;          /* --grid         rank-quantile grid */
    const char* attrs;         /* --attrs        per-point attributes */
    const char* cluster;       /* --cluster      per-point k-means labels; NULL = no labels */
} gf_index_paths;

typedef struct {
    uint32_t degree;          /* --degree: per-cell graph degree R; 0 = from the files */
    float f2h_factor;         /* --f2h_factor: scale before fp16 conversion (0 means 1) */
    int32_t vec_dtype;        /* GF_VEC_F32, GF_VEC_F16, GF_VEC_U8, GF_VEC_I8Q or GF_VEC_F16_REF */
    int32_t hist_contiguous;  /* 1: cell x cluster histogram by i / ceil(N/P) as the
                                 reference (tools.cuh:587-590); 0: by grid cell */
    int32_t device;           /* HIP device ordinal */
    int32_t ref_ties;         /* stage B, cells of equal score: 1 keeps the order of the reference's
                                 sorting network (bitonic_sort_id_by_num_int, gpu_graph.cu:123-141,
                                 11389); 0 orders them by ascending cell id */
} gf_open_opts;

/* The same content as the files, in host memory (no files needed). */
typedef struct {
    uint32_t N, D, a, P, R, E;
    const float* vectors;        /* N*D fp32, point-id order */
    const float* attrs;          /* N*a attribute values (integers converted to float) */
    const uint32_t* grid_shape;  /* a cells per attribute; P = product */
    const float* l_q;            /* sum(grid) lower quantile values, attribute-major */
    const float* r_q;            /* sum(grid) upper quantile values */
    const uint32_t* global_pid;  /* N cell of each point (row-major, last attribute fastest) */
    const uint32_t* cell_graphs; /* N*R per-cell graphs concatenated in cell order, cell-local ids */
    const uint32_t* cross;       /* N*(P*E) cross-cell graph rows, cell-local ids, point-id order */
    const int32_t* labels;       /* N k-means labels, or NULL */
} gf_index_host;

typedef struct {
    uint32_t N, D, a, P, R, E, C;  /* C = number of cluster centres (0 without labels) */
    uint32_t vec_dtype;
    float f2h_factor;
    uint64_t device_bytes;         /* device memory held by the index */
    uint32_t streamed;             /* 1: a streamed (out-of-core) index */
    uint32_t nbatch;               /* streamed: batches of its plan */
} gf_index_info;

/* Loaders: load_data (tools.cuh:85-106), get_graph_info (check.cu:406-484),
 * load_result (tools.cuh:205-223), load_grid_infos + load2GPU
 * (real_dataset_adapter.cuh:563-619), load_attrs (tools.cuh:746-765),
 * get_idx_mapper (tools.cuh:862-915), load_clustering (tools.cuh:569-602). */
gf_status gf_index_open(const gf_index_paths* paths, const gf_open_opts* opts, gf_index** out);
gf_status gf_index_create(const gf_index_host* host, const gf_open_opts* opts, gf_index** out);
gf_status gf_index_close(gf_index* ix);
gf_status gf_index_get_info(const gf_index* ix, gf_index_info* out);

/* Streamed (out-of-core) index: the cells' graphs, vectors, attributes and
 * every (cell, cell') slice of cross edges (the reference's "T" layout,
 * big_dataset_adapterV3.cuh:3539-3541) stay in pinned host memory in the
 * resident row order, whatever the batch plan.  gf_search streams the
 * batches of a plan through two device buffers: DMA copies on a side stream
 * assemble each batch's image (a few per run of consecutive cell ids, the
 * cross edges of two runs in one 2-D copy), overlapped with the search of the
 * previous batch.  The plan given here is the index's build-time plan; a
 * query batch may replace it (gf_batch_plan_stream, gf_batch_set_stream_plan)
 * without a re-pack.  Replaces the out-of-core driver's host-pinned loaders
 * (get_graph_info_host, check.cu:572-623; load_result_pined,
 * tools.cuh:241-255), its static batch plan (bigdataset_experiment.cu:271-277,
 * 746-756), its per-slice copies (big_dataset_adapterV3.cuh:3925-3946) and
 * the device buffers it sizes from the largest batch
 * (bigdataset_experiment.cu:776-793).  Host memory: N * (rowbytes + 4 * (2 +
 * a + R + P * E)) bytes plus the sub-cell metadata. */
typedef struct {
    uint64_t device_budget;   /* bytes the two batch buffers may use (the device cap); 0 = no cap */
    uint32_t nbatch;          /* batches in cells/sizes; 0 = consecutive cells, batch_cells per batch */
    uint32_t batch_cells;     /* cells per batch when nbatch == 0 (the reference's MAX_BATCH_SIZE: 16) */
    const uint32_t* sizes;    /* nbatch batch sizes */
    const uint32_t* cells;    /* sum(sizes) cell ids, batch after batch; each cell at most once
                                 (a cell in no batch is never searched) */
} gf_stream_plan;

gf_status gf_index_create_streamed(const gf_index_host* host, const gf_open_opts* opts,
                                   const gf_stream_plan* plan, gf_index** out);
gf_status gf_index_open_streamed(const gf_index_paths* paths, const gf_open_opts* opts,
                                 const gf_stream_plan* plan, gf_index** out);

/* Batch plan for a streamed index from a query batch's stage A cell lists:
 * the out-of-core pipeline's cell scheduling, which groups cells so that few
 * queries are active per batch (README.md:5; the shipped driver writes its
 * batches by hand, bigdataset_experiment.cu:271-277, 746-756).  The grid has
 * a axes of grid_shape[d] cells (P = product, row-major, last axis fastest);
 * cells/counts are gf_batch_get_cells' Q*P lists; cell_size holds the P cell
 * sizes.  The plan is the guillotine partition of the grid into boxes of at
 * most max_cells non-empty cells (0: no limit) and max_points points (0: no
 * limit) that minimises the sum over batches of the queries selecting a cell
 * of the batch (each query read as the bounding box of its cells), then the
 * number of batches.  Writes nbatch batch sizes to sizes (room for P) and
 * the cells batch after batch to plan_cells (room for P), in the form
 * gf_stream_plan takes; empty cells are left out.  *active (may be NULL)
 * receives the plan's objective counted from the lists.  Host only;
 * GF_E_UNSUPPORTED for grids with more than 2^22 (x0, x1) box slots. */
gf_status gf_stream_plan_cells(const uint32_t* cells, const uint32_t* counts, uint32_t Q, uint32_t a,
                               const uint32_t* grid_shape, const uint32_t* cell_size, uint64_t max_points,
                               uint32_t max_cells, uint32_t* sizes, uint32_t* plan_cells, uint32_t* nbatch,
                               uint64_t* active);

/* The batch plan a streamed index's gf_search uses for this query batch,
 * made from the batch's stage A cell lists (the out-of-core pipeline's
 * dynamic cell scheduling, README.md:5; the reference's driver fixes its
 * batches by hand, bigdataset_experiment.cu:271-277, 746-756): each query's
 * bounding box of cells on the device, gf_stream_plan_cells' dynamic program
 * on the host (max_points, max_cells as there), the batches' headers; the
 * plan's active (query, batch) pairs counted on the device.  The index's
 * rows are not re-packed.  The batch keeps the plan for its next searches
 * (until the next call, gf_batch_set_stream_plan or gf_batch_free); a plan
 * whose largest batch needs more device memory than the index's two batch
 * buffers hold grows them within the index's device budget, else
 * GF_E_UNSUPPORTED.  Synchronous; *ms (may be NULL) receives the call's host
 * wall time, *nbatch and *active (may be NULL) the plan's batches and its
 * active pairs.  GF_E_UNSUPPORTED on a resident index, GF_E_STATE before
 * stage A. */
gf_status gf_batch_plan_stream(gf_batch* b, uint64_t max_points, uint32_t max_cells, uint32_t* nbatch,
                               uint64_t* active, double* ms);
/* Sets this query batch's plan explicitly: nbatch batches of sizes[i] cell
 * ids in cells, batch after batch, each cell at most once (a cell in no
 * batch is never searched), the form gf_stream_plan takes; nbatch = 0 goes
 * back to the index's build-time plan.  Buffers grow as for
 * gf_batch_plan_stream. */
gf_status gf_batch_set_stream_plan(gf_batch* b, uint32_t nbatch, const uint32_t* sizes, const uint32_t* cells);
/* The plan this batch's next search uses: *nbatch, then (each may be NULL;
 * room for P) the batch sizes and the cells batch after batch. */
gf_status gf_batch_get_stream_plan(const gf_batch* b, uint32_t* nbatch, uint32_t* sizes, uint32_t* cells);

/* A query batch: Q query vectors (Q*D fp32) and closed ranges lo/hi (Q*a),
 * uploaded to the device (realdataset_search.cu:2198-2245 load + f2h). */
gf_status gf_batch_create(gf_index* ix, const float* queries, uint32_t Q,
                          const float* lo, const float* hi, gf_batch** out);
gf_status gf_batch_free(gf_batch* b);

/* Stage A -- intersection_area_mark_little_seg_V2<A,T>
 * (real_dataset_adapter.cuh:388-519): the cells each range intersects and the
 * prefilter routing: a query whose exact selectivity is <= prefilter is sent
 * to filtered brute force.  With prefilter >= 1 every query is routed there
 * without counting (count / N <= 1 always holds); the exact counts are then
 * made when gf_batch_get_cells asks for selcount or counters are read.
 * ms (may be NULL) receives the device time.  With ms NULL the call only
 * records the stage: the next gf_search runs it at the start of its own HIP
 * graph and gf_search_stats.ms_stage_a reports its device time; a call that
 * reads or writes the stage's outputs (the batch getters, gf_batch_set_cells,
 * gf_mark_cells_grid, gf_batch_plan_stream) runs it first.  The same holds
 * for gf_order_cells. */
gf_status gf_mark_cells(gf_batch* b, float prefilter, double* ms);

/* Stage B -- get_partitions_access_order_V2 (gpu_graph.cu:11742-11845):
 * orders each query's cells by overlap with its topc nearest cluster centres
 * (the reference uses topc = 4).  Without labels the order is left as is. */
gf_status gf_order_cells(gf_batch* b, uint32_t topc, double* ms);

/* Stage A on an arithmetic grid -- intersection_area_mark_little_seg_batch_process
 * (gpu_graph.cu:12066-12187) and its kernel intersection_area_batch_mark_little_seg
 * (gpu_graph.cu:11095-11188), the out-of-core driver's stage A: attribute d
 * has cells of width attr_width[d] from attr_min[d] (the index's grid shape);
 * a selected cell is "little" when its overlap with the range, as a fraction
 * of a cell, is <= threshold.  little[q] = number of little cells. */
gf_status gf_mark_cells_grid(gf_batch* b, const float* attr_min /*a*/, const float* attr_width /*a*/,
                             double threshold, double* ms);

/* Stage C -- batch_graph_search_gpu_with_prefilter_and_postfilter<T>
 * (gpu_graph.cu:12463-12616) and its kernel (gpu_graph.cu:3266-4131).  On a
 * streamed index: batch_graph_search_gpu_with_prefilter_batch_process_compressed_graph_T_dataset_resident_u8
 * (big_dataset_adapterV3.cuh:3719-4117) and its kernel (:2674-3316): per batch,
 * each query searches its selected cells of the batch, in plan order (brute
 * force when all of them are little), from fresh entry points, and its K
 * results merge into a running top-K; postfilter does not apply. */
typedef struct {
    uint32_t L;            /* candidate list length (the reference's ef / TOPM) */
    uint32_t K;            /* results per query (reference: 10) */
    uint32_t rl;           /* recycle list length (reference: 10), <= 16 */
    uint32_t postfilter;   /* --postfilter: queries with >= this many cells (not all
                              little) skip the cell-by-cell traversal; on a resident
                              index of at most 64 cells they search its full graph
                              (the branch gpu_graph.cu:3644-3787, which the reference
                              disables with `&& false`), else they get no result */
    const uint32_t* entry_points;  /* R cell-local entry ids, or NULL for the
                                      reference's mt19937 draw (gpu_graph.cu:12503-12526;
                                      streamed: big_dataset_adapterV3.cuh:3862-3875) */
} gf_search_opts;

#define GF_NCOUNTERS 8  /* per-query counters, same order as the oracle's */
typedef struct {
    double ms_traverse;      /* device time of the traversal kernel (streamed: summed over batches) */
    double ms_bruteforce;    /* device time of the brute-force kernel (streamed: summed over batches) */
    double ms_total;         /* device time of the whole search stage */
    uint32_t q_traverse, q_bruteforce, q_empty;
    uint64_t n_expand, n_dist, n_attr, n_cross, n_lrow, n_scan, n_pass;
    double bytes_traverse;   /* algorithmic HBM bytes of the traversal kernel */
    double bytes_bruteforce; /* algorithmic HBM bytes of the brute-force kernel */
    double ops_bruteforce;   /* arithmetic of the brute-force kernel (int8 MACs x 2 on MFMA) */
    uint32_t bf_mfma;        /* 1 if the brute force ran as the int8 MFMA query-batch kernel */
    double ms_bf_kernel;     /* device time of the MFMA brute-force kernel alone (no schedule, no merge) */
    /* streamed index only */
    uint32_t n_batches;      /* batches searched (a batch none of whose cells a query selects is skipped) */
    double bytes_h2d;        /* bytes copied host -> device (a batch no query traverses: its brute-force sections only) */
    double ms_h2d;           /* sum of the copies' device times */
    /* device times of the batch's latest stage A (gf_mark_cells or
       gf_mark_cells_grid) and stage B (gf_order_cells) calls; 0 if none ran */
    double ms_stage_a;
    double ms_stage_b;
    /* HIP graph replays: bit 0 the search stage (a resident index's second
       and later searches of a batch with the same buffers and options), bit 1
       the latest gf_mark_cells call and bit 2 the latest gf_order_cells call
       (their second and later calls with the same arguments) */
    uint32_t graph;
    /* queries on the full-graph route (postfilter or more cells, not all
       little; a resident index of at most 64 cells); their device time is in
       ms_traverse */
    uint32_t q_fullgraph;
    /* streamed index: sum over the searched batches of the queries that
       select a cell of the batch (each such pair restarts the query's search
       in that batch) */
    uint64_t n_active;
} gf_search_stats;

gf_status gf_search(gf_batch* b, const gf_search_opts* opts, uint32_t* ids /*Q*K*/,
                    float* dists /*Q*K or NULL*/, gf_search_stats* stats /*or NULL*/);

/* gf_search with the dual-channel traversal for the traversal-routed
 * queries (replaces batch_graph_search_gpu, gpu_graph.cu:12223-12300, and
 * the traversal of its kernel select_path_..._dual_channel_in_turn_with_prefilter,
 * gpu_graph.cu:6249-6640): two channels walk two cells of a query's list at
 * once over one candidate list of L entries, the channel in turn expanding
 * its first unexplored entry and the other a partner reached through a
 * cross edge; a channel with nothing left moves to the next cell through
 * 128 cross-edge slots, or joins the other channel.  opts->entry_points
 * holds L cell-local ids (the first ceil(L/2) for the first cell, the rest
 * for the second, each reduced modulo its cell's size), or NULL for the
 * reference's draw of L.  Other routes (brute force, full graph) as
 * gf_search.  Resident indexes with R <= 32; route counter 4. */
gf_status gf_search_dual(gf_batch* b, const gf_search_opts* opts, uint32_t* ids /*Q*K*/,
                         float* dists /*Q*K or NULL*/, gf_search_stats* stats /*or NULL*/);

/* Inspection / injection of the batch's intermediate state, for parity
 * tests and for callers that compute cell lists themselves.
 * cells is Q*P (row q holds counts[q] cell ids), the reference's
 * partition_infos[0..3] without compaction. */
gf_status gf_batch_get_cells(const gf_batch* b, uint32_t* cells, uint32_t* counts,
                             uint32_t* little, uint32_t* selcount);
gf_status gf_batch_set_cells(gf_batch* b, const uint32_t* cells, const uint32_t* counts,
                             const uint32_t* little);
gf_status gf_batch_get_centroid(const gf_batch* b, float* dist /*Q*C*/, uint32_t* topc /*Q*topc*/);
/* Per (query, cell) flags, Q*P bytes: 1 = selected, 2 = little (the
 * reference's partition_is_selected and is_little_seg, gpu_graph.cu:12066-12187).
 * After gf_mark_cells or gf_batch_set_cells the first little[q] cells of a
 * query's list are the little ones. */
gf_status gf_batch_get_cell_flags(const gf_batch* b, uint8_t* flags);
gf_status gf_batch_get_counters(const gf_batch* b, uint32_t* counters /*Q*GF_NCOUNTERS*/);

/* One query batch through stages A, B and C in one call that allocates
 * nothing.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc).  The call is synchronous (it copies the host arrays and waits
 * for its stream), so it cannot be recorded under HIP graph capture.  It runs the kernels of gf_batch_create,
 * gf_mark_cells(prefilter), gf_order_cells(topc) and gf_search(search) on a
 * resident index and returns the same ids and distances; routed queries take
 * the gather brute force, whose results equal the MFMA route's.  Every
 * per-batch buffer is carved from a per-device static array of
 * GF_NOALLOC_SCRATCH_MB MiB that each GPU holds until the process ends; a
 * batch whose buffers do not fit (about Q * (4 D + 4 P + 8 K + 64) bytes, plus
 * 2 D per query with labels) is GF_E_UNSUPPORTED.  The array keeps the last
 * call's contents and is shared by every call on that GPU: calls that overlap
 * on one GPU race.  Host arrays need not be page-locked. */
#define GF_NOALLOC_SCRATCH_MB 32
typedef struct {
    float prefilter;         /* as gf_mark_cells */
    uint32_t topc;           /* as gf_order_cells, 1..4 (unused without labels) */
    gf_search_opts search;   /* as gf_search */
} gf_noalloc_opts;
gf_status gf_search_noalloc(gf_index* ix, const float* queries, uint32_t Q, const float* lo, const float* hi,
                            const gf_noalloc_opts* opts, uint32_t* ids /*Q*K*/, float* dists /*Q*K or NULL*/);

/* Page-locked host memory (hipHostMalloc).  No counterpart in the reference:
 * result arrays allocated here receive gf_search's device-to-host copies
 * directly, without a staging copy on the host.  Free with gf_host_free. */
gf_status gf_host_alloc(size_t bytes, void** out);
gf_status gf_host_free(void* ptr);

/* f2h (tools.cuh:308-320) on the device: out[i] = binary16(x[i]*alpha), RNE. */
gf_status gf_f2h(const float* x, size_t n, float alpha, uint16_t* out);
/* find_norm (tools.cuh:1561-1586) on the device: squared norms of fp16 rows. */
gf_status gf_row_norms_f16(const uint16_t* x, uint32_t n, uint32_t D, float* out);
/* Entry points of the reference's host wrapper (gpu_graph.cu:12503-12526):
 * mt19937 default seed, distinct uniform draws in [0, N-(P-1)*ceil(N/P)),
 * std::random_shuffle after srand(1) (this reseeds the process's rand()). */
gf_status gf_entry_points(uint32_t N, uint32_t P, uint32_t R, uint32_t* out);

/* ---- Index build: the files the reference's indexbuild/ scripts write ---- */

/* grid_scatter_V2 (indexbuild/tools.py:88-125): per attribute, the points in
 * stable ascending order of value are cut into grid_shape[d] runs of
 * ceil(N / g) (the last run takes the rest); l_q / r_q (sum(grid) values,
 * attribute-major, as gf_index_host) hold each run's first and last value,
 * pid_lists (a*N, attribute-major) each point's run, and global_pid the
 * row-major cell id (last attribute fastest).  Host code.  Any output may be
 * NULL.  GF_E_ARG when a last run would start beyond N (the reference's
 * script fails there). */
gf_status gf_grid_scatter(const float* attrs /*N*a*/, uint32_t N, uint32_t a, const uint32_t* grid_shape,
                          float* l_q, float* r_q, uint32_t* pid_lists, uint32_t* global_pid);

typedef struct {
    double ms_tiles;        /* int8 tile build */
    double ms_graph;        /* per-cell graphs (kernel time) */
    double ms_cross;        /* cross-cell graph (kernel time) */
    uint64_t pairs_graph;   /* distances evaluated: sum of |cell|^2 */
    uint64_t pairs_cross;   /* N * sum of |cell| */
    uint32_t dim;           /* dimension as computed (D rounded up to 64) */
    double ms_prep;         /* host: input checks, cell layout, item lists */
    double ms_upload;       /* device set-up, allocations and uploads */
    double ms_run;          /* wall time of the kernels (the graphs' download overlaps the cross pass) */
    double ms_download;     /* the cross edges to the caller's array */
    double ms_total;        /* the whole call */
} gf_build_stats;

/* The per-cell graphs (cagra_build.py:94-127 writes the layout: rows of R
 * cell-local ids, cells concatenated in cell order, members in ascending
 * point id) and the cross-cell graph (global_graph_build.py:106-176: for
 * every point, in point-id order, and every cell c, the E nearest points of
 * c as cell-local ids, the point's own cell included) of the points'
 * cells global_pid, by exact nearest neighbours where the reference uses
 * CAGRA: ordered by (squared L2 distance, cell-local id); a graph row
 * excludes the point itself; a row with fewer candidates than it holds
 * repeats its nearest (a point alone in its cell lists itself); edges into
 * an empty cell are 0.  vectors: N*D in point-id order, GF_VEC_U8 bytes or
 * GF_VEC_F32.  u8 data and floats that are all integers in [0, 255] get
 * exact neighbours from int8 MFMA distances.  Other float data: the same
 * kernels on the u8 quantisation rint((x - min) / s), s = (max - min) / 255
 * over all values, keep 16 more candidates per list (at most 63 per graph
 * row, 64 per cross list), which are then ordered by exact fp32 distance
 * (the traversal's summation order), repeats dropped.  D up to 1024; R + 1
 * and E up to 72 (float data: R up to 63, E up to 64).  cell_graphs (N*R)
 * or cross (N*P*E) may be NULL to skip that graph.  Runs on HIP device
 * `device`; stats may be NULL. */
gf_status gf_build_graphs(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D,
                          const uint32_t* global_pid, uint32_t P, uint32_t R, uint32_t E, int32_t device,
                          uint32_t* cell_graphs, uint32_t* cross, gf_build_stats* stats);

/* The optimised per-cell graphs cagra.build returns (cagra_build.py:94-125
 * saves index.graph; cuVS builds a kNN graph of a larger intermediate degree
 * and optimises it), written from CAGRA's published algorithm (Ootomo et al.,
 * ICDE 2024): each row of the kNN graph knn_graphs (N*I, per-cell graphs
 * concatenated in cell order, cell-local ids, rows ordered by distance, e.g.
 * gf_build_graphs with R = I) is reordered by ascending (number of detourable
 * two-hop routes, rank): the edge at rank k to D has a detour through every
 * B at a rank below k that lists D at a rank below k (GPU).  Then (host) every
 * pruned edge A -> B among the first R adds A to B's reverse list (ranks in
 * order, nodes in order, at most R per list), and the output row keeps the
 * first R/2 reordered edges, then its reverse edges, then the rest of the
 * reordered row, each id once (a row still short repeats its first id).
 * I <= 64, R <= I; ms (wall time of the call) may be NULL. */
gf_status gf_optimize_graphs(const uint32_t* knn_graphs, uint32_t N, uint32_t I, const uint32_t* cell_size,
                             uint32_t P, uint32_t R, int32_t device, uint32_t* graphs /*N*R*/, double* ms);

/* Per-point cluster labels for the index (the .cluster file; the reference
 * fits cuVS k-means and predicts, clustering.py:68-87).  Integer Lloyd
 * iterations: centres start as the points init_ids (C of them); an
 * assignment gives each point its nearest centre by exact squared L2
 * distance (ties to the smaller centre index); an update moves each centre
 * to the rounded mean floor((2 sum + n) / (2 n)) of its n members (an empty
 * cluster keeps its centre).  `iters` assign + update rounds, then a final
 * assignment gives the labels.  D up to 1024; float data that are not all
 * integers in [0, 255] are clustered in gf_build_graphs' u8 quantisation
 * (centres are then in its units).  centres (C*D bytes) may be NULL; ms
 * (wall time of the call) may be NULL. */
gf_status gf_kmeans(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D, uint32_t C, uint32_t iters,
                    const uint32_t* init_ids, int32_t device, int32_t* labels /*N*/, uint8_t* centres /*C*D*/,
                    double* ms);

/* The int8 quantisation a GF_VEC_I8Q index holds (replaces the reference
 * loader's production_adapter.cuh:110-183 load_dataset_return_int8_arr, whose
 * int8 array, scales and zero points it returns): x (n*D) times alpha, per
 * dimension scale (max - min) / 255 with min and max starting from 100000
 * and -100000, zero point round(-128 - min / scale) clamped to [-128, 127],
 * out = round(x / scale) + zero point clamped to [-128, 127], fp32 arithmetic,
 * round() half away from zero; a dimension with max == min takes scale 1.
 * Host only (no device). */
gf_status gf_quantise_i8(const float* x, uint64_t n, uint32_t D, float alpha, float* scale /*D*/,
                         int32_t* zero /*D*/, int8_t* out /*n*D*/);

const char* gf_status_str(gf_status s);
const char* gf_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* GARFIELD_H */
