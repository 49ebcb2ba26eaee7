// Internal declarations shared by the HIP kernels (gf_kernels.hip) and the
// host side of libgarfield.so (gf_host.cpp, gf_io.cpp).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/garfield.h"

namespace gf {

constexpr uint32_t kMaxIter = 10000;  // per-cell iteration cap (gpu_graph.cu:39)
constexpr uint32_t kHashReset = 4;    // visited-set reset period (gpu_graph.cu:34)
constexpr uint32_t kXSlots = 128;     // cross-cell entry slots (gpu_graph.cu:42)
constexpr uint32_t kXStep = 64;       // candidates feeding the slots (gpu_graph.cu:3564)
constexpr uint32_t kOffLds = 1024;    // cell offsets (P + 1) the traversal keeps in LDS

// LDS bytes of the traversal kernel: candidate list, slot scratch, row list,
// visited set of hsize keys, and the P + 1 cell offsets when they fit.
inline bool trav_offsets_in_lds(uint32_t P) { return P + 1 <= kOffLds; }
// Visited-set slots for at most `live` keys between two clears: a load
// factor of at most 0.6 (linear probing then needs about 3.6 probes for a new
// key at the worst load, 1.75 for a present one), a multiple of 64, at least
// 256.  The table never fills, so its set semantics are exact.
inline uint32_t visited_slots(uint32_t live) {
    const uint32_t s = (live * 5u + 2u) / 3u;
    const uint32_t r = (s + 63u) / 64u * 64u;
    return r < 256u ? 256u : r;
}
inline uint32_t trav_lds_bytes(uint32_t Lpad, uint32_t hsize, uint32_t P) {
    return Lpad * 8 + kXSlots * 8 + 128 * 4 + hsize * 4 + (trav_offsets_in_lds(P) ? (P + 1) * 4 : 0);
}
// LDS bytes of the dual-channel traversal: candidate list, switch slots and
// evictees, row list, visited set.
inline uint32_t trav_dual_lds_bytes(uint32_t Lpad, uint32_t hsize) {
    return Lpad * 8 + 2 * kXSlots * 8 + 128 * 4 + hsize * 4;
}
constexpr uint32_t kMaxAttr = 8;      // attributes per point supported
constexpr uint32_t kMaxE = 4;         // cross edges per (point, cell) supported
constexpr uint32_t kSelTile = 1024;   // rows per selectivity tile
constexpr uint32_t kEmpty = 0xFFFFFFFFu;

// Candidate word: high 32 bits = fp32 distance bits (non-negative, so the
// unsigned order is the float order), low 32 bits = row << 2 | explored << 1
// | passes-filter.  Ordering uses the word with the two flag bits cleared,
// i.e. (distance, cell-major row).
constexpr uint32_t kRecSent = 0xFFFFFFFEu;  // row 0x3FFFFFFF, explored, not passing
constexpr uint64_t kCandSent = (uint64_t(0x7F800000u) << 32) | kRecSent;
constexpr uint32_t kRowSent = 0x3FFFFFFFu;

// Per-query counter slots (same order as the oracle's ORC_C_*).
enum { C_EXPAND = 0, C_DIST = 1, C_ATTR = 2, C_CROSS = 3, C_LROW = 4, C_SCAN = 5,
       C_PASS = 6, C_ROUTE = 7 };

// Distance kernel shape for a row of D elements: 16-byte chunks, LPR lanes
// per row (power of two in [8, 64]), CPL chunks per lane.
// Row layout of the distance kernels: vt 0 = fp32, 1 = binary16, 2 = uint8
// vectors; a row is nch 16-byte chunks, LPR lanes per row, cpl chunks per lane.
// Row types stored as binary16 (GF_VEC_F16, GF_VEC_F16_REF).
inline bool half_rows(int vdtype) { return vdtype == GF_VEC_F16 || vdtype == GF_VEC_F16_REF; }

struct RowShape {
    int vt;
    uint32_t nch, lpr, cpl;
};
RowShape row_shape(uint32_t D, int vt);
uint32_t row_shape_max_cpl(int vt);
void quantise_i8(const float* x, uint64_t n, uint32_t D, float alpha, std::vector<float>& scale,
                 std::vector<int32_t>& zero, int8_t* out);

struct TravArgs {
    const char* vec;          // N rows of rowbytes, cell-major
    uint32_t rowbytes, nch;
    const float* attrs;       // N*a, cell-major
    const uint32_t* graph;    // N*R cell-local neighbour ids, cell-major rows
    const uint32_t* cross;    // cell-local ids: edge e of row r into cell c at r*xrow + c*xcell + e
    uint64_t xrow, xcell;     // resident index: P*E, E; a streamed batch ("T" layout): E, rows*E
    const uint32_t* offset;   // P+1
    const uint32_t* gidx;     // row -> point id
    const uint32_t* lrow;     // row -> cell-local id
    const uint32_t* prow;     // point id -> row (dual-channel traversal)
    const char* queries;      // Q rows of qbytes (fp32, or fp16 in f16 mode)
    uint32_t qbytes;
    const float* lo;          // Q*a
    const float* hi;
    const uint32_t* cells;    // Q*P ordered cell lists
    const uint32_t* counts;   // Q
    const uint32_t* little;   // Q
    const uint32_t* sched;    // schedule: traversal queries, then brute-force queries
    const uint32_t* srange;   // device [begin, end) of this launch's queries in sched
    const uint32_t* entry;    // R entry ids
    uint32_t* out_ids;        // Q*K
    float* out_dist;          // Q*K
    uint32_t* counters;       // Q*GF_NCOUNTERS
    uint32_t a, P, R, E, L, K, rl, hsize, Lpad;   // hsize: visited-set slots (visited_slots)
    uint32_t offl;            // 1: the launch's LDS holds the P + 1 cell offsets (trav_lds_bytes)
    // Full-graph route (queries with postfilter or more cells): the graph
    // over every point, FD rows per row (cell-major rows, kEmpty = no edge),
    // its FD entry rows and this launch's query range in sched.
    const uint32_t* fgraph;
    const uint32_t* fentry;
    const uint32_t* frange;
    uint32_t FD;
};

// Sub-cells: per cell a rank grid of attribute bins (host build in
// gf_host.cpp).  Tiles of 16 points are grouped by sub-cell; tile t of the
// tmeta array holds [row x 16][attribute word x 16] x AW (AW = ceil(a/2)
// 32-bit words of two 16-bit offsets from the cell's smallest value).
struct SubArgs {
    const uint32_t* sbase;     // P+1 first sub-cell of each cell
    const uint32_t* scell;     // cell of each sub-cell
    const uint32_t* ssize;     // points per sub-cell
    const uint32_t* stile;     // NS+1 first tile of each sub-cell
    const int32_t* sbox;       // NS*2a: per attribute min, max
    const uint32_t* tmeta;     // per tile: rows, attribute words
    const int32_t* abase;      // P*a smallest attribute value of each cell
    uint32_t a, AW, P, NS;
};

// Query-batch brute force on int8 MFMA (integer data in [0, 255]).  Vectors
// are stored shifted by -128 as int8 in the sub-cell tile order, each tile in
// MFMA operand order: tile t, k-step s holds 64 lanes x 16 bytes, lane l
// carrying bytes [64 s + 16 (l / 16), +16) of point l % 16.  tnorm holds per
// tile [-floor(|x'|^2 / 2) x 16][|x'|^2 x 16].  The brute force reads one
// record per tile (bf_rec_bytes): the D / 64 k-steps, the tile's norms, then
// its meta (rows, AW attribute words x 16), records back to back in tile
// order, so consecutive tiles are one contiguous range.
constexpr uint32_t kBfTile = 16;      // points per tile
constexpr uint32_t kBfKMax = 16;      // largest K of the MFMA route
constexpr uint32_t kBfQB = 64;        // queries per work item
constexpr uint32_t kBfMaxItemTiles = 65536;   // tiles per MFMA work item (keeps buffer offsets below 2^31)
constexpr uint32_t kBfSeedTiles = 16;         // tiles per seed item: a seed sub-cell spreads over several waves
constexpr uint32_t kBfHFirstPass = 4;         // binary16 rows' first pass: sub-cells with grid hash % 4 == 0
constexpr uint32_t kBfHSeedTiles = 128;       // the same for the float MFMA route (measured: C4 5.6 ms at 128, 6.0 at 16)
constexpr size_t kDirectListMax = size_t(64) << 20;   // NS x Q bound of one-pass sub-cell lists (256 MiB)
struct BfItem {
    uint32_t sub, qbase, nq;           // sub-cell, first entry of its query list, queries
    uint32_t tb, te;                   // tiles [tb, te) of the sub-cell
    uint32_t inside;                   // 1: every query's range contains the sub-cell's box
};
__host__ __device__ inline uint32_t bf_rec_bytes(uint32_t D, uint32_t AW) { return (D / 64u) * 1024u + 128u + 64u * (1u + AW); }
// Float tile record of the float MFMA brute force (KS operand chunks of 64
// lanes x 16 bytes in MFMA operand order, then the tile's meta record of
// 16 (1 + AW) words, then its 16 rows' |x|^2 as fp32).
__host__ __device__ inline uint32_t bf_frec_bytes(uint32_t KS, uint32_t AW) { return KS * 1024u + 64u * (2u + AW); }
struct BfGemmArgs {
    SubArgs sa;
    const uint8_t* rec;        // tile records (bf_rec_bytes each)
    const int8_t* q8;          // Q*D queries shifted by -128
    const int32_t* nq;         // |q - 128|^2
    const float* lo;
    const float* hi;
    const BfItem* items;
    const uint32_t* nitems;    // device scalar
    const uint32_t* bq;        // query of each (query, sub-cell) pair, grouped by sub-cell
    const uint32_t* part_off;  // per query: first pair (its partial area holds pairs * K keys)
    uint32_t* pcnt;            // per query: keys appended so far (zeroed before)
    uint64_t* part;            // partial keys: (d << 32) | row
    uint32_t* gbound;          // per query: smallest K-th distance of any item so far
    const uint32_t* ok;        // schedule fits its buffers (else the kernel does nothing)
    // Optional seed items (null: none), run before every other item so that
    // each query's bound is set from one well-filled sub-cell early.
    const BfItem* sitems;
    const uint32_t* nseed;     // device count of seed items
    uint32_t nseed_cap;        // capacity of sitems
    uint32_t K, D;
    // What a launch runs: the seed items if seeds_on, and of the item list
    // all (irange 0), the first *nitems_a (1), the rest (2) or none (3).
    uint32_t seeds_on;
    uint32_t irange;
    const uint32_t* nitems_a;
    uint64_t* stamp = nullptr;   // optional: the device wall clock when the launch starts
};
// Query-batch brute force of float rows on MFMA (k_bf_f16: binary16 rows,
// fp16 MFMA; k_bf_f32: fp32 rows, fp32 MFMA): candidate keys within the
// distances' error bound, re-ranked exactly by k_bf_f16_final.  Items and
// tiles as k_bf_i8's.
constexpr uint32_t kBfHKT = 32;       // keys an item keeps per query
struct BfHArgs {
    SubArgs sa;
    const uint8_t* rec;        // tile records (bf_frec_bytes each)
    const void* q16;           // Q*D queries of the rows' type
    const float* qnorm;        // per query |q|^2
    const float* eps;          // per query bound of |d' - d|
    const float* lo;
    const float* hi;
    const BfItem* items;
    const uint32_t* nitems;
    const uint32_t* bq;
    const uint32_t* part_off;  // per query: first pair (its area holds pairs * kBfHKT keys)
    uint32_t* pcnt;
    uint64_t* part;            // kept keys (d' bits << 32) | row
    uint32_t* gbound;          // per query: bits of the smallest K-th d' of any item so far
    uint32_t* over;            // per query: 1 if an item may have dropped a candidate
    const uint32_t* ok;
    const BfItem* sitems;
    const uint32_t* nseed;
    uint32_t nseed_cap;
    // What a launch runs, as BfGemmArgs: the seed items if seeds_on, and of
    // the item list all (irange 0), the first *nitems_a (1), the rest (2)
    // or none (3).
    uint32_t seeds_on;
    uint32_t irange;
    const uint32_t* nitems_a;
    uint32_t K, D;
};
struct BfHFinal {
    const uint32_t* ok;
    const uint32_t* over;
    const uint32_t* pcnt;
    const uint32_t* part_off;
    const uint64_t* part;
    const float* eps;
    const uint32_t* selcount;
};
// vt 1 (binary16 rows): D in {64, 96, 128, 256, 512, 768}; vt 0 (fp32
// rows): D in {64, 96, 128, 256}; AW 1 or 2; K <= 10.
bool bf_float_supported(int vt, uint32_t D, uint32_t AW, uint32_t K);
hipError_t launch_bf_float(const BfHArgs& a, int vt, uint32_t AW, uint32_t ncu, hipStream_t st);
// Brute-force queries of the schedule range srange in a.sched (binary16 or fp32 rows).
hipError_t launch_bf_f16_final(const RowShape& rs, const TravArgs& a, const BfHFinal& f, uint32_t grid,
                               hipStream_t st);

// Index build: exact nearest neighbours over int8 tiles (k_knn_i8).
constexpr uint32_t kKnnKMax = 72;   // largest K (R + 1 for graphs, E for cross edges)
struct KnnItem {
    uint32_t qtile;   // first of up to four query tiles (64 points) of cell qcell
    uint32_t qcell;
    uint32_t tcell;   // the cell whose points are the candidates
};
struct KnnArgs {
    const int8_t* vt;        // tiles of every cell, cell-major, members in id order
    const int32_t* tnorm;    // per tile [-floor(|x'|^2 / 2) x 16][|x'|^2 x 16]
    const uint32_t* trow;    // per tile row: point id, 0xFFFFFFFF = padding
    const uint32_t* ctile;   // P + 1: first tile of each cell
    const uint32_t* coff;    // P + 1: first member (cell-major position) of each cell
    const KnnItem* items;
    uint32_t nitems;
    uint32_t K;              // keys kept per query
    uint32_t R;              // > 0: graph rows of R ids (K = R + 1); 0: cross edges
    uint32_t P;
    uint32_t* out;           // graph: rows in cell-major order; cross: N x P x K
    // A launch covers tiles [chunk * ctiles, (chunk + 1) * ctiles) of each
    // target cell; the keys found so far carry over in state (graph: N x K,
    // cross: N x P x K, cell-major rows).
    uint32_t chunk, ctiles;
    uint64_t* state;
};
hipError_t launch_knn_i8(const KnnArgs& a, uint32_t KS, uint32_t ncu, hipStream_t st);
uint32_t knn_ks(uint32_t D);    // k-steps of 64 dimensions the kNN kernel runs for D (0: D too large)
uint32_t knn_qt(uint32_t KS);   // query tiles per wave for KS (items group this many)

// Exact fp32 re-rank of kNN candidate lists (float data): one wave per list.
struct RerankArgs {
    const float* vec;         // cell-major fp32 rows of rowbytes, zero padded to whole 16-byte chunks
    uint32_t rowbytes, nch;
    const uint32_t* coff;     // P + 1 cell starts (cell-major rows)
    const uint32_t* rowcell;  // cell of each cell-major row
    const uint32_t* cmrow;    // cell-major row of each point id
    const uint32_t* cand;     // candidate lists of nc cell-local ids
    uint32_t nc, keep, P;
    uint32_t graph;           // 1: list i = cell-major row i's own-cell candidates (itself excluded);
                              // 0: list i = point i / P's candidates in cell i % P
    uint32_t* out;            // keep ids per list
};
hipError_t launch_rerank(const RerankArgs& a, uint32_t D, uint32_t nlists, hipStream_t st);
// Graph optimisation, first step: every row's I neighbours (cell-local ids,
// rows cell-major, offset P + 1) rewritten in ascending (detourable routes,
// rank) order.  I <= 64.
hipError_t launch_prune(const uint32_t* knn, uint32_t N, uint32_t I, const uint32_t* offset, uint32_t P,
                        uint32_t* out, hipStream_t st);
// k-means update: cnt and fill (C each) must start at zero; start (C) and
// mem (N) are scratch; centres (C x Dp u8) are rewritten where a cluster
// has members.
hipError_t launch_kmeans_update(const uint8_t* vec, uint32_t Dp, const uint32_t* lab2, uint32_t N, uint32_t C,
                                uint32_t* cnt, uint32_t* start, uint32_t* fill, uint32_t* mem, uint8_t* centres,
                                hipStream_t st);

struct BfFinalArgs {
    uint32_t* gbound;          // optional: per query the bound the items reached
    const uint32_t* bfq;       // schedule
    const uint32_t* srange;    // device [begin, end) of the brute-force queries in bfq
    const uint32_t* part_off;  // per query: first pair (partial area = pairs * K keys)
    uint32_t* pcnt;            // keys appended for each query (bound_only: reset to the kept keys)
    const uint32_t* ok;
    uint64_t* part;            // bound_only: each query's area compacted to its K smallest keys
    const uint32_t* counts;
    const uint32_t* cells;
    const uint32_t* offset;
    const uint32_t* selcount;
    const uint32_t* gidx;
    uint32_t* out_ids;
    float* out_dist;
    uint32_t* counters;
    uint32_t K, P;
    // Bound only: lower each query's gbound to the K-th smallest key appended
    // so far and leave the keys, results and counters as they are.
    uint32_t bound_only;
    uint64_t* stamp = nullptr;   // optional: the device wall clock when the launch starts
};
// Stage A on sub-cells: one workgroup per sub-cell over all queries.  A point
// that passes a range lies in a cell the range selects, so the relation of a
// range to a sub-cell's attribute box alone decides what the sub-cell adds to
// the query's exact count.
struct SubSelArgs {
    SubArgs sa;
    uint32_t Q;
    const float* lo;
    const float* hi;
    uint32_t* selcount;        // zeroed before; receives atomic sums
};
// Stage C schedule of the MFMA brute force: per sub-cell, the brute-force
// queries whose range reaches it, in query order.
struct BfSchedArgs {
    SubArgs sa;
    uint32_t Q, postfilter;
    const uint32_t* counts;
    const uint32_t* little;
    const float* lo;
    const float* hi;
    uint32_t* nsub;            // pairs per query (pass 1, zeroed before)
    uint32_t* bcnt;            // pairs per sub-cell (pass 1)
    uint32_t* bin;             // of which the range contains the whole sub-cell box (pass 1)
    const uint32_t* bstart;    // exclusive scan of bcnt (pass 2)
    uint32_t* bq;
    const uint32_t* ok;        // bq and part are large enough (pass 2)
    const uint32_t* nbf;       // device count of brute-force queries (0: nothing to do)
    // Optional (null: every sub-cell a range reaches): per (query, cell),
    // stride bP, bit 2 = the cell is one the query's brute force scans.
    const uint8_t* bfm;
    uint32_t bP;
    // Optional (null: queries 0..Q-1): candidate queries qlist[qrange[0] ..
    // qrange[1]) (device range), e.g. the schedule's brute-force queries.
    const uint32_t* qlist;
    const uint32_t* qrange;
    // Items cover at most tch tiles of a sub-cell (0: the whole sub-cell);
    // nsub counts a pair once per such chunk, each of which appends <= K keys.
    uint32_t tch;
    // > 0: one pass writes each sub-cell's list into bq[s * qcap, (s + 1) * qcap)
    // (inside queries from the front, partial ones from the back); 0: count
    // and fill passes at the scan bstart of bcnt.
    uint32_t qcap;
    // Optional (one-pass lists with qlist): the candidate records k_bfseed
    // writes for candidate index ci: its query (kEmpty: not on the
    // brute-force route), seed sub-cell (whose pair is listed, counted and run
    // as a seed item instead) and range (rlo / rhi: attribute d at d * Q + ci);
    // per sub-cell the seeds at the front of its region (scnt).
    const uint32_t* rq;
    const uint32_t* rseed;
    const float* rlo;
    const float* rhi;
    const uint32_t* scnt;
};

// Seed choice (one-pass lists only): per brute-force query, the sub-cell its
// brute force reaches that holds the most points of its range (whole
// sub-cells by size, partial ones by box overlap), listed at the front of
// that sub-cell's region and counted in nsub; also the candidate records
// k_bfsched reads.
struct BfSeedArgs {
    SubArgs sa;
    uint32_t Q, postfilter;
    const uint32_t* counts;
    const uint32_t* little;
    const uint32_t* cells;     // Q x P cell lists
    const float* lo;
    const float* hi;
    const uint8_t* bfm;        // as BfSchedArgs
    uint32_t bP;
    const uint32_t* qlist;
    const uint32_t* qrange;
    uint32_t qcap, tch;        // tch: tiles per seed item
    uint32_t itch;             // tiles per regular item
    uint32_t* scnt;            // zeroed before
    uint32_t* bq;
    uint32_t* nsub;            // written: the query's seed and regular item chunks
    uint32_t* rq;              // candidate records (BfSchedArgs), Q each
    uint32_t* rseed;
    float* rlo;                // a x Q
    float* rhi;
};
// Query schedule (gpu_graph.cu:12485-12493): traversal queries by descending
// cell count, then brute-force queries, then full-graph queries.  tot[0..3] =
// traversal, brute-force, empty, full-graph query counts; ranges[0..3] =
// traversal [begin, end), brute force [begin, end); ranges[4..5] = full graph.
struct SchedArgs {
    uint32_t Q, P, postfilter;
    uint32_t full;            // 1: queries with postfilter or more cells (not all little) take the full graph
    uint32_t* franges;        // ranges[4..5] (null when full is 0)
    const uint32_t* counts;
    const uint32_t* little;
    uint32_t* sched;
    uint32_t* tot;
    uint32_t* ranges;
};
// Sums of the per-query counters and of the brute-force schedule for the
// search statistics: out[0..6] counter sums, out[7] traversal and full-graph DIST, out[8]
// brute-force DIST, out[9] sum of pairs x sub-cell size, out[10] sum of
// items x tiles per item.
struct StatsArgs {
    uint32_t Q, NS;
    const uint32_t* counters;
    const uint32_t* bcnt;      // null without the MFMA schedule
    const uint32_t* bin;       // inside queries of each list, counted apart when split
    const uint32_t* sseed;     // seed queries of each sub-cell (null: none)
    bool split;                // items group inside and partial queries separately
    const uint32_t* ssize;
    const uint32_t* stile;
    unsigned long long* out;   // zeroed before
};

// Kernel launchers (gf_kernels.hip).  All are asynchronous on `st`.
// The search launches take a grid of `grid` workgroups (an upper bound of
// their query range, which is read on the device).
hipError_t launch_traverse(const RowShape& rs, const TravArgs& a, uint32_t lds_bytes, uint32_t grid, hipStream_t st);
// Dual-channel traversal: R <= 32, entry holds L ids, prow set.
hipError_t launch_traverse_dual(const RowShape& rs, const TravArgs& a, uint32_t lds_bytes, uint32_t grid,
                                hipStream_t st);
hipError_t launch_invert_rows(const uint32_t* gidx, uint32_t N, uint32_t* prow, hipStream_t st);
// The full-graph route (fgraph, fentry, frange, FD of a), same LDS layout.
hipError_t launch_fullgraph(const RowShape& rs, const TravArgs& a, uint32_t lds_bytes, uint32_t grid, hipStream_t st);
// The full graph: row r, slot c * FE + e holds edge e of row r into cell c as a
// cell-major row: the per-cell graph's edge e for r's own cell, the cross edge
// e into c otherwise, kEmpty into an empty cell.
hipError_t launch_assemble_full(const uint32_t* graph, const uint32_t* cross, const uint32_t* offset,
                                const uint32_t* rowcell, uint32_t N, uint32_t P, uint32_t R, uint32_t E, uint32_t FE,
                                uint32_t* out, hipStream_t st);
hipError_t launch_bruteforce(const RowShape& rs, const TravArgs& a, uint32_t grid, hipStream_t st);
hipError_t launch_fill_results(uint32_t* ids, float* dist, uint32_t n, hipStream_t st);
hipError_t launch_bf_i8(const BfGemmArgs& a, uint32_t ncu, hipStream_t st);   // grid: ncu x resident workgroups per CU
hipError_t launch_bf_final(const BfFinalArgs& a, uint32_t grid, hipStream_t st);
hipError_t launch_tile_i8(const void* vec_cm, bool u8, uint32_t D, const uint32_t* tmeta, uint32_t AW, uint32_t ntile,
                          int8_t* vt, int32_t* tnorm, hipStream_t st);
// The brute force's tile records (bf_rec_bytes each) from the same inputs.
// Float tile records (bf_frec_bytes) of ntile tiles from cell-major rows of
// type vt (1 binary16, 0 fp32) and their norms.
hipError_t launch_tile_frec(const void* vec, int vt, uint32_t D, const uint32_t* tmeta, const float* xnorm,
                            uint32_t AW, uint32_t ntile, uint8_t* rec, hipStream_t st);
hipError_t launch_tile_rec(const void* vec_cm, bool u8, uint32_t D, const uint32_t* tmeta, uint32_t AW, uint32_t ntile,
                           uint8_t* rec, hipStream_t st);
hipError_t launch_note_bf(const uint32_t* tot, uint32_t* note, hipStream_t st);
hipError_t launch_subsel(const SubSelArgs& a, hipStream_t st);
hipError_t launch_bfsched(const BfSchedArgs& a, bool fill, hipStream_t st);
hipError_t launch_bfsched_direct(const BfSchedArgs& a, hipStream_t st);   // one pass, after k_bfseed
hipError_t launch_bfitems(const uint32_t* bcnt, const uint32_t* bin, const uint32_t* bstart, uint32_t qcap,
                          const uint32_t* stile, uint32_t tch, uint32_t NS, uint32_t* icnt, uint32_t* ioff,
                          BfItem* items, uint32_t* nitems, const uint32_t* ok, bool fill, hipStream_t st,
                          const uint32_t* scnt = nullptr, BfItem* sitems = nullptr, uint32_t* nseed = nullptr,
                          uint32_t scap = 0, const uint32_t* sorder = nullptr, uint32_t ns1 = 0,
                          uint32_t* nitems_a = nullptr, uint32_t stch = 0);
hipError_t launch_bfseed(const BfSeedArgs& a, uint32_t Q, hipStream_t st);
// out[0] = start[n-1] + cnt[n-1] (total of an exclusive scan); out[1] = out[0] <= cap
// (with cap2 != 0 also out[0] * mul <= cap2).
hipError_t launch_sched(const SchedArgs& a, hipStream_t st);
hipError_t launch_stats(const StatsArgs& a, hipStream_t st);
hipError_t launch_total(const uint32_t* cnt, const uint32_t* start, uint32_t n, uint32_t cap, uint32_t mul,
                        uint64_t cap2, uint32_t* out, hipStream_t st);
hipError_t launch_q_i8(const float* q, uint32_t Q, uint32_t D, int8_t* q8, int32_t* nq, hipStream_t st);
hipError_t launch_f2h(const float* x, uint16_t* out, size_t n, float alpha, hipStream_t st);
hipError_t launch_f2h_pad(const float* x, uint32_t rows, uint32_t D, uint16_t* out,
                          uint32_t rows_pad, uint32_t Dp, float alpha, hipStream_t st);
hipError_t launch_norms_f16(const uint16_t* x, uint32_t n, uint32_t D, uint32_t ld, float* out,
                            hipStream_t st);
// Optional parts of stage A's cell kernel: with little (and selcount) also
// the routing of a prefilter >= 1 (selcount 0 and every selected cell little,
// as k_route computes it then); st_entry, the device wall clock when the
// launch starts; st_exit (with ticket, a zeroed counter), when it ends.
struct CellsTail {
    uint32_t* selcount = nullptr;
    uint32_t* little = nullptr;
    uint64_t* st_entry = nullptr;
    uint32_t* ticket = nullptr;
    uint64_t* st_exit = nullptr;
};
hipError_t launch_cells(uint32_t Q, uint32_t a, const float* lo, const float* hi,
                        const uint32_t* grid, const uint32_t* doff, const float* l_q,
                        const float* r_q, uint32_t P, const uint32_t* offset, uint32_t* cells,
                        uint32_t* counts, hipStream_t st, const CellsTail& tl = CellsTail{});
hipError_t launch_cellq_count(uint32_t Q, uint32_t P, const uint32_t* cells,
                              const uint32_t* counts, uint32_t* ccount, hipStream_t st);
hipError_t launch_scan_small(const uint32_t* in, uint32_t n, uint32_t* out_excl, hipStream_t st);
// The scan and launch_total's outputs (tot[0..1]) in one kernel.
hipError_t launch_scan_total(const uint32_t* in, uint32_t n, uint32_t* out_excl, uint32_t cap, uint32_t mul,
                             uint64_t cap2, uint32_t* tot, hipStream_t st);
hipError_t launch_cellq_fill(uint32_t Q, uint32_t P, const uint32_t* cells,
                             const uint32_t* counts, const uint32_t* cstart, uint32_t* cfill,
                             uint32_t* cellq, hipStream_t st);
hipError_t launch_selcount(uint32_t ntiles, const uint32_t* tile_cell, const uint32_t* tile_row0,
                           const uint32_t* tile_n, const float* attrs, uint32_t a,
                           const uint32_t* cstart, const uint32_t* ccount,
                           const uint32_t* cellq, const float* lo, const float* hi,
                           uint32_t* selcount, hipStream_t st);
hipError_t launch_route(uint32_t Q, uint32_t N, float thr, const uint32_t* selcount,
                        const uint32_t* counts, uint32_t* little, hipStream_t st, uint32_t* ticket = nullptr,
                        uint64_t* st_exit = nullptr);   // st_exit: the end of the launch (stamp_exit)
hipError_t launch_cells_grid(uint32_t Q, uint32_t a, const float* lo, const float* hi, const float* amin,
                             const float* width, const uint32_t* grid, uint32_t P, const uint32_t* offset,
                             double thr, uint32_t* cells, uint32_t* counts, uint32_t* little, uint8_t* flags,
                             hipStream_t st);
hipError_t launch_cell_flags(uint32_t Q, uint32_t P, const uint32_t* cells, const uint32_t* counts,
                             const uint32_t* little, uint8_t* flags, hipStream_t st);
hipError_t launch_stream_lists(uint32_t Q, uint32_t P, uint32_t B, const uint32_t* bcell, const uint8_t* flags,
                               uint32_t* lists, uint32_t* counts, uint32_t* little, hipStream_t st);
// Also zeroes scnt (NS entries) and *nseed when given.
hipError_t launch_bf_reset(uint32_t Q, uint32_t* nsub, uint32_t* pcnt, uint32_t* gbound, hipStream_t st,
                          uint32_t NS = 0, uint32_t* scnt = nullptr, uint32_t* nseed = nullptr);
// Also zeroes z[0, nz) (a search's statistics sums, for one kernel less).
// The brute force's per-query state as k_bf_reset sets it (nsub and pcnt
// 0, gbound open; scnt[0..NS) and *nseed 0 when given), for a reset that
// does it too.
struct BfReset {
    uint32_t* nsub = nullptr;
    uint32_t* pcnt = nullptr;
    uint32_t* gbound = nullptr;
    uint32_t NS = 0;
    uint32_t* scnt = nullptr;
    uint32_t* nseed = nullptr;
};
hipError_t launch_reset_results(uint32_t Q, uint32_t K, uint32_t* ids, float* dist, uint32_t* ctr, hipStream_t st,
                                uint32_t* z = nullptr, uint32_t nz = 0, uint64_t* stp = nullptr, uint32_t nst = 0,
                                const BfReset& br = BfReset{});
// stats (16, optional), tot (24) and stamps (12) to page-locked host buffers;
// stamps[2], the search's end, is taken by this kernel when it starts.
hipError_t launch_gather_meta(const unsigned long long* stats, const uint32_t* tot, const uint64_t* stamps,
                              unsigned long long* h_stats, uint32_t* h_tot, uint64_t* h_stamps, hipStream_t st);
hipError_t launch_zero_u32(uint32_t* x, uint32_t n, hipStream_t st);   // a kernel, so that it can sit in a graph
hipError_t launch_stamp(uint64_t* t, hipStream_t st, uint32_t n = 1);   // t[0..n) = device wall clock when it runs
// need: 2 * nbatch entries, the need flags, then the active queries per batch
hipError_t launch_batch_need(uint32_t Q, uint32_t P, uint32_t nbatch, const uint32_t* plan_cells,
                             const uint32_t* plan_off, const uint8_t* flags, uint32_t* need, hipStream_t st);
hipError_t launch_cell_boxes(uint32_t Q, uint32_t P, uint32_t a, const uint32_t* grid, const uint32_t* cells,
                             const uint32_t* counts, uint32_t* box, hipStream_t st);
// One piece of a streamed batch image, read by k_stream_gather from pinned
// host memory: nrow rows of width bytes, source rows spitch apart from byte
// src of the arena (base 0) or of the plan's header block (base 1), image
// rows dpitch apart from byte dst.  mw != 0: tile metadata of mw words per
// tile, whose words w with w % mw < 16 (rows) gain add unless 0xFFFFFFFF.
struct GatherDesc {
    uint64_t src, dst, spitch, dpitch;
    uint32_t width, nrow, base, add, mw;
    uint32_t pad[3];
};
hipError_t launch_stream_gather(const GatherDesc* desc, uint32_t n, const char* arena, const char* head, char* img,
                                hipStream_t st);
hipError_t launch_merge_stream(uint32_t Q, uint32_t K, uint32_t* run_ids, float* run_dist, const uint32_t* ids,
                               const float* dist, uint32_t* run_ctr, const uint32_t* ctr, bool first,
                               hipStream_t st);
hipError_t launch_centroid(const uint16_t* qh, const uint16_t* ch, const float* qn,
                           const float* cn, uint32_t Q, uint32_t C, uint32_t Qp, uint32_t Cp,
                           uint32_t Dp, float* dist, hipStream_t st, uint64_t* st_entry = nullptr);
// chosen: topk already holds each query's topc nearest centres (dist unused).
// ref_ties: equal scores keep the reference's sorting-network order.
hipError_t launch_order(uint32_t Q, uint32_t C, uint32_t P, uint32_t topc, const float* dist,
                        const uint32_t* hist, uint32_t* cells, const uint32_t* counts,
                        uint32_t* topk, hipStream_t st, bool chosen = false, bool ref_ties = false);
// Each query's topc (<= 4) nearest centres without the distance matrix.
hipError_t launch_centroid_top(const uint16_t* qh, const uint16_t* ch, const float* qn, const float* cn, uint32_t Q,
                               uint32_t C, uint32_t Qp, uint32_t Cp, uint32_t Dp, uint32_t topc, uint32_t* topk,
                               hipStream_t st, uint64_t* st_entry = nullptr);

// Host-side file readers (gf_io.cpp).  Each throws gf::Error on failure.
struct Error {
    gf_status code;
    std::string msg;
};
struct HostIndex {
    uint32_t N = 0, D = 0, a = 0, P = 0, R = 0, E = 0;
    std::vector<float> vectors, attrs, l_q, r_q;
    std::vector<uint32_t> grid, global_pid, cell_graphs, cross;
    std::vector<int32_t> labels;
    bool has_labels = false;
};
void read_index_files(const gf_index_paths& p, uint32_t degree, HostIndex& out);

}  // namespace gf
