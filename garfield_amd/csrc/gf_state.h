// Host-side state of libgarfield.so shared by gf_host.cpp (resident
// indexes, the C ABI) and gf_stream.cpp (streamed indexes): owning device
// and pinned host buffers, error macros, and the opaque gf_index / gf_batch.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gf_internal.h"

#define GF_HIP(x)                                                                              \
    do {                                                                                       \
        hipError_t e_ = (x);                                                                   \
        if (e_ != hipSuccess)                                                                  \
            throw gf::Error{GF_E_DEVICE, std::string(#x) + ": " + hipGetErrorString(e_)};          \
    } while (0)

#define GF_REQUIRE(cond, code, msg)                  \
    do {                                             \
        if (!(cond)) throw gf::Error{(code), (msg)};     \
    } while (0)

namespace gf {

// Owning device buffer.
template <typename T>
struct DevBuf {
    T* p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { release(); }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    void alloc(size_t count) {
        if (count == n && p) return;
        release();
        if (count == 0) return;
        hipError_t e = hipMalloc(&p, count * sizeof(T));
        if (e != hipSuccess) {
            p = nullptr;
            throw gf::Error{GF_E_NOMEM, "hipMalloc of " + std::to_string(count * sizeof(T)) + " bytes failed"};
        }
        n = count;
    }
    void upload(const T* src, size_t count) {
        alloc(count);
        if (count) GF_HIP(hipMemcpy(p, src, count * sizeof(T), hipMemcpyHostToDevice));
    }
    void upload(const std::vector<T>& v) { upload(v.data(), v.size()); }
    size_t bytes() const { return n * sizeof(T); }
};

inline uint32_t round_up(uint32_t x, uint32_t m) { return (x + m - 1) / m * m; }

// Owning pinned host buffer (hipHostMalloc): the source of streamed copies.
template <typename T>
struct PinBuf {
    T* p = nullptr;
    size_t n = 0;
    PinBuf() = default;
    PinBuf(const PinBuf&) = delete;
    PinBuf& operator=(const PinBuf&) = delete;
    ~PinBuf() { release(); }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        n = 0;
    }
    void alloc(size_t count, unsigned flags = hipHostMallocDefault) {
        release();
        if (count == 0) return;
        hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&p), count * sizeof(T), flags);
        if (e != hipSuccess) {
            p = nullptr;
            throw gf::Error{GF_E_NOMEM, "hipHostMalloc of " + std::to_string(count * sizeof(T)) + " bytes failed"};
        }
        n = count;
    }
    size_t bytes() const { return n * sizeof(T); }
};

// Sub-cells of every cell, host arrays (compute_subcells).
struct SubHost {
    uint32_t AW = 0, NS = 0, ntile = 0;
    // Brute-force pass order: the ns1 sub-cells of the first pass (about one
    // in eight of each cell's rank grid, spread over it), then the rest.
    // shash: per sub-cell the grid hash that picks them (first_pass_order).
    uint32_t ns1 = 0;
    std::vector<uint32_t> sorder, shash;
    std::vector<uint32_t> sbase, scell, ssize, stile, tmeta;
    std::vector<int32_t> sbox, abase;
};

// A streamed index keeps no per-point array on the device.  Its rows stay in
// pinned host memory, in one arena laid out in the resident row order (cells
// in id order, each cell's rows consecutive), whatever the plan:
//   vec    N x rowbytes
//   gidx   N          point id of each row
//   attrs  N x a      fp32
//   graph  N x R      cell-local neighbour ids
//   lrow   N          cell-local id of each row
//   cross  P x N x E  target-major: edge e of row g into cell c' at
//          (c' * N + g) * E + e.  The rows of one cell into c' are the
//          reference's per-pair "T" slice (big_dataset_adapterV3.cuh:3539-3541),
//          and the slices of a run of consecutive cells into c' are adjacent.
//   sub-cells (MFMA brute force: u8 vectors, D a multiple of 64 up to 256):
//          ssize NS, sbox NS x 2a, tmeta tiles x 16 (1 + AW) with resident rows
// A plan groups cells into batches.  A search assembles each batch's image in
// one of two device buffers ("turns") on a side stream, from pieces: per run
// of consecutive cell ids in the batch one piece of each array it needs, per
// (source run, target run) one two-dimensional piece of cross edges, and the
// batch header, which the plan builds on the host.  The large 1-D pieces
// (rows of vectors and graphs) move by DMA; one k_stream_gather launch reads
// the others from the pinned memory over PCIe.  The image is a small
// index of the batch's cells, the sections the brute force needs first, so
// that a batch none of whose queries traverses moves only a prefix:
//   header offset B + 1 (first row of each batch cell), bcell B (cell ids);
//          with sub-cells sbase B + 1, scell NS, stile NS + 1 (batch-local),
//          abase B x a
//   ssize NS, sbox NS x 2a, tmeta tiles x MW (rows made batch rows on the
//          way: a run's rows all move by the same amount)
//   vec    rows x rowbytes (the batch's cells in plan order)
//   gidx   rows                        <- end of the MFMA brute-force prefix
//   attrs  rows x a                    <- end of the gather brute-force prefix
//   graph  rows x R, lrow rows
//   cross  B x rows x E: edge e of row r into the batch's i-th cell at
//          (i * rows + r) * E + e
// Every section starts on a 256-byte boundary.
struct StreamRun {            // a maximal run of consecutive cell ids in a batch
    uint32_t i0 = 0, n = 0;   // first batch cell, cells
    uint32_t c0 = 0;          // cell id of the first
    uint32_t g0 = 0, r0 = 0, rows = 0;   // first resident row, first batch row, rows
    uint32_t s0 = 0, sb0 = 0, ns = 0;    // first resident / batch sub-cell, sub-cells
    uint32_t t0 = 0, tb0 = 0, nt = 0;    // first resident / batch tile, tiles
};

struct StreamBatch {
    uint32_t B = 0, rows = 0, NS = 0, ntile = 0;
    size_t o_offset = 0, o_bcell = 0, o_sbase = 0, o_scell = 0, o_stile = 0, o_abase = 0;
    size_t head = 0;        // header bytes (image prefix copied from the plan's pinned block)
    size_t o_ssize = 0, o_sbox = 0, o_tmeta = 0, o_vec = 0, o_gidx = 0, o_attrs = 0, o_graph = 0, o_lrow = 0,
           o_cross = 0;
    size_t bytes = 0;       // image size
    size_t bytes_mfma = 0;  // prefix the MFMA brute force reads
    size_t bytes_bf = 0;    // prefix the gather brute force reads
    size_t head_off = 0;    // header in the plan's pinned block
    uint32_t run0 = 0, nrun = 0;   // the batch's runs in StreamPlan::runs
    // its pieces: in StreamPlan::desc from desc0 (k_stream_gather) and in
    // StreamPlan::dma from dma0 (hipMemcpyAsync, the large 1-D ones); the
    // first ndesc[w] and ndma[w], bytes moved[w], make the MFMA brute
    // force's prefix (w = 0), the gather brute force's (1), the image (2)
    uint32_t desc0 = 0, ndesc[3] = {0, 0, 0};
    uint32_t dma0 = 0, ndma[3] = {0, 0, 0};
    size_t moved[3] = {0, 0, 0};
};

struct StreamCopy {   // a 1-D piece of a batch image moved by DMA from the arena
    size_t src, dst, bytes;
};

// A batch plan of a streamed index: the index's build-time plan, or one a
// query batch sets (gf_batch_plan_stream / gf_batch_set_stream_plan).
struct StreamPlan {
    std::vector<std::vector<uint32_t>> cells;
    std::vector<StreamBatch> batches;
    std::vector<StreamRun> runs;
    PinBuf<char> head;         // coherent pinned memory, read by k_stream_gather
    DevBuf<GatherDesc> desc;   // every batch's gathered pieces
    std::vector<StreamCopy> dma;   // every batch's DMA pieces
    // cells batch after batch and the first of each batch, for k_batch_need
    DevBuf<uint32_t> plan_cells, plan_off;
    size_t max_bytes = 0;
    uint32_t Bmax = 0, NSmax = 0, tmax = 0;
};

// The part of the batch planner's dynamic program that depends on the grid,
// the cell sizes and the batch limits only (plan_boxes): the boxes that do
// not fit a batch, ordered so that both parts of any cut of a box come before
// it, and each box's batch count when it is a leaf.
struct PlanFrame {
    uint32_t a = 0;
    std::vector<uint32_t> grid;
    uint64_t max_points = 0;
    uint32_t max_cells = 0;
    uint32_t stride[kMaxAttr] = {}, bstride[kMaxAttr] = {};
    size_t nbox = 0;
    std::vector<uint32_t> order;   // boxes that do not fit
    std::vector<uint8_t> leaf;     // per box: 0 / 1 batches when it is a leaf; 2 = not a leaf
};

struct StreamIndex {
    PinBuf<char> host;   // the arena (coherent pinned memory, read by k_stream_gather)
    size_t arena_bytes = 0;
    size_t a_vec = 0, a_gidx = 0, a_attrs = 0, a_graph = 0, a_lrow = 0, a_cross = 0, a_ssize = 0, a_sbox = 0,
           a_tmeta = 0;
    uint32_t rows = 0;            // N
    std::vector<uint32_t> size;   // points per cell
    SubHost sh;                   // sub-cell offsets (the arena holds ssize, sbox, tmeta)
    std::unique_ptr<PlanFrame> frame;   // the planner's frame for the latest batch limits
    std::unique_ptr<StreamPlan> plan;   // the build-time plan
    DevBuf<char> turn[2];
    uint64_t budget = 0;
    uint32_t min_cell = 0;
    // MFMA brute force: int8 tile records of the batch being searched
    bool i8 = false;
    uint32_t AW = 0;
    size_t trec_tiles = 0;
    DevBuf<uint8_t> trec;
    hipStream_t copy = nullptr;
    hipEvent_t ready[2] = {nullptr, nullptr}, freed[2] = {nullptr, nullptr};
    ~StreamIndex() {
        for (auto& e : ready) if (e) (void)hipEventDestroy(e);
        for (auto& e : freed) if (e) (void)hipEventDestroy(e);
        if (copy) (void)hipStreamDestroy(copy);
    }
};

}  // namespace gf

using gf::DevBuf;

struct gf_index {
    int device = 0;
    hipStream_t stream = nullptr;
    uint32_t N = 0, D = 0, a = 0, P = 0, R = 0, E = 0, C = 0;
    int32_t vdtype = GF_VEC_F32;
    float alpha = 1.0f;
    std::vector<float> qscale;      // GF_VEC_I8Q: per-dimension scale and zero point
    std::vector<int32_t> qzero;
    bool ref_ties = false;   // stage B: equal cell scores in the reference's network order
    gf::RowShape rs{};
    uint32_t rowbytes = 0, Cp = 0, Dp = 0;
    std::vector<uint32_t> offset_h, grid_h;
    DevBuf<char> vec;
    DevBuf<float> attrs, l_q, r_q, cnorm;
    DevBuf<uint32_t> graph, cross, offset, gidx, lrow, grid, doff, hist;
    DevBuf<uint32_t> entry_ref;   // the reference's entry-point draw (resident index: made when it is built)
    DevBuf<uint32_t> entry_dual;  // the same draw of L entries for the dual-channel traversal
    uint32_t entry_gen = 0;       // bumped whenever entry_ref or entry_dual is (re)written
    DevBuf<uint32_t> prow;        // point id -> row (dual-channel traversal, made at its first search)
    // Full-graph route (P <= 64): every row's FE edges into each cell (FD =
    // FE * P rows per row) and the FD entry rows of the reference's second draw.
    uint32_t FE = 0, FD = 0;
    DevBuf<uint32_t> fgraph, fentry;
    DevBuf<uint32_t> tile_cell, tile_row0, tile_n;
    DevBuf<uint16_t> centres;
    uint32_t ntiles = 0;
    // Sub-cells (integer attributes spread by less than 65534 inside every
    // cell, a <= 4): each cell is split by a rank grid of S bins per
    // attribute; tiles of 16 points are grouped by sub-cell and carry the
    // cell-major row and the packed 16-bit attribute offsets of each point.
    bool sub = false;
    uint32_t AW = 0, NS = 0, ntile = 0;
    std::vector<uint32_t> ssize_h, stile_h, shash_h;
    DevBuf<uint32_t> sbase, scell, ssize, stile, tmeta;
    DevBuf<uint32_t> sorder;   // sub-cells of the brute force's first pass (ns1 of them), then the rest
    uint32_t ns1 = 0;
    DevBuf<int32_t> sbox, abase;
    // Query-batch MFMA brute force (additionally: vectors integers in
    // [0, 255], D a multiple of 64 up to 256): int8 tiles and norms.
    bool i8 = false;
    DevBuf<uint8_t> trec;   // MFMA brute force: int8 tile records (gf::bf_rec_bytes each)
    // Float rows with sub-cells (binary16 or fp32, shapes of
    // bf_float_supported) and no int8 route: the MFMA brute force of float
    // rows, with |x|^2 per row and the largest |x| over the index.
    bool hf = false;
    DevBuf<float> xnormf;
    DevBuf<uint8_t> frec;   // its tile records (gf::bf_frec_bytes each)
    double xmaxf = 0.0;
    int ncu = 0;
    int wclk_khz = 100000;   // rate of the device wall clock the search's timestamps read
    // Streamed index (gf_index_create_streamed / gf_index_open_streamed):
    // the per-point arrays above stay empty.
    std::unique_ptr<gf::StreamIndex> sx;
    ~gf_index() {
        sx.reset();
        if (stream) (void)hipStreamDestroy(stream);
    }
    uint64_t device_bytes() const {
        return vec.bytes() + attrs.bytes() + l_q.bytes() + r_q.bytes() + cnorm.bytes() + graph.bytes() +
               cross.bytes() + offset.bytes() + gidx.bytes() + lrow.bytes() + grid.bytes() + doff.bytes() +
               hist.bytes() + tile_cell.bytes() + tile_row0.bytes() + tile_n.bytes() + centres.bytes() +
               sbase.bytes() + scell.bytes() + ssize.bytes() + stile.bytes() + tmeta.bytes() + sbox.bytes() +
               sorder.bytes() + abase.bytes() + trec.bytes() + xnormf.bytes() + frec.bytes() +
               (sx ? sx->turn[0].bytes() + sx->turn[1].bytes() + sx->trec.bytes() : 0);
    }
};

namespace gf {
// One stage of the query path as a HIP graph: captured on its second call
// and replayed while its key (the buffers it touches, the options, the
// route) is unchanged; one launch instead of several, no host gaps between
// the kernels.  If capture or instantiation fails the stage runs eagerly from
// then on.  GARFIELD_NO_GRAPH=1 turns replay off.
struct StageGraph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    std::vector<uint64_t> gkey;
    uint32_t nruns = 0;
    bool off = false, replayed = false;
    StageGraph() = default;
    StageGraph(const StageGraph&) = delete;
    StageGraph& operator=(const StageGraph&) = delete;
    void drop() {
        if (gexec) (void)hipGraphExecDestroy(gexec);
        if (graph) (void)hipGraphDestroy(graph);
        gexec = nullptr;
        graph = nullptr;
        gkey.clear();
    }
    // Enqueues the stage on st: replays the graph, captures and launches a
    // new one, or calls enqueue() directly.  enqueue must not allocate or
    // wait on the host.
    template <class F>
    void run(const std::vector<uint64_t>& key, hipStream_t st, F&& enqueue) {
        replayed = false;
        ++nruns;
        const char* env = std::getenv("GARFIELD_NO_GRAPH");
        if (off || nruns < 2 || (env && env[0] == '1')) {
            enqueue();
            return;
        }
        if (!(gexec && key == gkey)) {
            drop();
            if (hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed) != hipSuccess) {
                (void)hipGetLastError();
                off = true;
                enqueue();
                return;
            }
            bool ok = true;
            try {
                enqueue();
            } catch (...) {
                ok = false;
            }
            hipGraph_t g = nullptr;
            const hipError_t e = hipStreamEndCapture(st, &g);
            if (!ok || e != hipSuccess || !g || hipGraphInstantiate(&gexec, g, nullptr, nullptr, 0) != hipSuccess) {
                if (g) (void)hipGraphDestroy(g);
                gexec = nullptr;
                (void)hipGetLastError();
                off = true;
                enqueue();
                return;
            }
            graph = g;
            gkey = key;
        }
        GF_HIP(hipGraphLaunch(gexec, st));
        replayed = true;
    }
    ~StageGraph() { drop(); }
};
}  // namespace gf

struct gf_batch {
    gf_index* ix = nullptr;
    uint32_t Q = 0, Qp = 0, topc = 0;
    bool marked = false;
    // the latest stage A sent every query to the brute force (prefilter >= 1)
    bool route_bf = false;
    // Stage calls made without ms on a resident index, not yet enqueued:
    // the search enqueues them in its own graph; any other call that reads
    // or writes the stage buffers enqueues them first (flush_stages).
    bool pend_a = false, pend_b = false;
    float pend_pf = 0.0f;
    bool i8 = false;
    DevBuf<int8_t> q8;
    DevBuf<int32_t> nq;
    // brute-force schedule of stage C (tot: device totals and fit flags)
    DevBuf<uint32_t> tot;
    DevBuf<uint32_t> bcnt, bin, bstart, pcnt, bq, nsub, part_off, icnt, ioff, bfq;
    DevBuf<gf::BfItem> items;
    DevBuf<uint64_t> part;
    // Capacity of the schedule in (query, sub-cell) pairs (part holds K
    // partial results per pair) and, when NS x Q lists fit, the capacity of
    // each sub-cell's own list (qcap = Q: k_bfsched fills the lists in one
    // pass); qcap = 0 selects the count-scan-fill scheme with bq of pair_cap.
    size_t pair_cap = 0;
    uint32_t qcap = 0;
    // Seed schedule of a resident index's one-pass lists: candidate records
    // (query, seed sub-cell, range), seeds per sub-cell and the seed items.
    DevBuf<uint32_t> scnt, rq, rseed;
    DevBuf<float> rlo, rhi;
    DevBuf<gf::BfItem> sitems;
    // slots: (sub-cell, tile chunk) combinations, bounding the items beyond
    // one per 64 pairs.
    // The sub-cells and slots (and queries) the buffers were sized for: a
    // schedule over more must call alloc_pairs again.
    uint32_t ns_cap = 0, q_cap = 0;
    size_t slot_cap = 0;
    bool pairs_fit(uint32_t Q, uint32_t NS, size_t slots) const {
        return part.n && Q <= q_cap && NS <= ns_cap && slots <= slot_cap;
    }
    void alloc_pairs(size_t pairs, uint32_t K, uint32_t Q, uint32_t NS, size_t slots) {
        const bool direct = size_t(NS) * Q <= gf::kDirectListMax;
        qcap = direct ? Q : 0u;
        pair_cap = pairs;
        ns_cap = NS;
        q_cap = Q;
        slot_cap = slots;
        const size_t nbq = direct ? size_t(NS) * Q : pairs;
        if (bq.n < nbq) bq.alloc(nbq);
        part.alloc(pairs * K);
        items.alloc(pairs / gf::kBfQB + (direct ? 2 : 1) * slots + 2);
    }
    DevBuf<unsigned long long> stats;
    DevBuf<float> qf32, qnorm, lo, hi, cdist, out_dist;
    DevBuf<uint16_t> q16, q16v;
    DevBuf<float> qi8q;   // GF_VEC_I8Q: query rows [c | s], c_d = fma(s_d, z_d, q_d)
    DevBuf<float> qnf, heps;   // float MFMA brute force: |q|^2 of the query as the rows hold it, bound of |d' - d|
    DevBuf<uint32_t> hover;     // fp16 brute force: queries whose kept keys may miss a candidate
    DevBuf<uint32_t> cells, counts, little, selcount, cellq, ccount, cstart, cfill, topk;
    DevBuf<uint32_t> out_ids, counters, sched, entry, gbound;
    // What entry holds when it is a copy of the index's draw (source buffer,
    // count, generation), so that a search with the same draw skips the copy.
    const uint32_t* entry_src = nullptr;
    uint32_t entry_src_n = 0, entry_src_gen = 0;
    // Per (query, cell) flags, 1 = selected | 2 = little: written by the
    // arithmetic-grid stage A, else derived from the cell lists on use.
    DevBuf<uint8_t> flags;
    bool flags_ready = false;
    // True after gf_mark_cells: every query's list holds every non-empty cell
    // its range reaches and little is 0 or the count, so the MFMA brute force
    // may pair a query with every sub-cell its range reaches; otherwise bfmask
    // (Q*P, bit 2 = a cell the query's brute force scans) restricts it.
    bool bf_all = false;
    DevBuf<uint8_t> bfmask;
    // selcount holds the exact counts (false after gf_mark_cells with
    // prefilter >= 1, which routes without them); pass_pending: the last
    // search's MFMA brute force reported PASS from counts not made yet.
    bool sel_exact = true;
    bool pass_pending = false;
    // Streamed search: per-batch cell lists and results, and the batch plan
    // this query batch set (none: the index's build-time plan).
    DevBuf<uint32_t> slist, scount, slittle, s_ids, s_ctr, note, need;
    DevBuf<float> s_dist;
    std::unique_ptr<gf::StreamPlan> splan;
    DevBuf<uint32_t> qbox;   // per query: bounding box of its cells on the grid (planning)
    // pinned staging of a resident search's results, totals and timestamps
    gf::PinBuf<uint32_t> h_ids, h_tot;
    gf::PinBuf<float> h_dist;
    gf::PinBuf<unsigned long long> h_stats;
    DevBuf<uint64_t> stamps;
    gf::PinBuf<uint64_t> h_stamps;
    // Stage B ran; cdist holds the query x centre matrix of that run.
    bool ordered = false, cdist_ready = false;
    // Device times of the latest stage A and B calls: events sev[0..1]
    // (stage A on an arithmetic grid) or device timestamps in stamps[5..6]
    // (stage A) and stamps[7..8] (stage B), which the search gathers.
    enum : uint8_t { kTimeNone = 0, kTimeEvents = 1, kTimeStamps = 2 };
    // kNStamps gathered; then the zeroed counter of stamp_exit for stage A
    // (kTicketA: a u64 slot holding a u32 counter)
    static constexpr uint32_t kStampA = 5, kStampB = 7, kNStamps = 12, kTicketA = 12;
    hipEvent_t sev[2] = {nullptr, nullptr};
    uint8_t time_a = kTimeNone, time_b = kTimeNone;
    // Records event i of sev (created on first use).
    void stage_event(int i, hipStream_t st) {
        if (!sev[i]) GF_HIP(hipEventCreate(&sev[i]));
        GF_HIP(hipEventRecord(sev[i], st));
    }
    // Device time between sev[0] and sev[1] (waits for the latter).
    double event_ms() {
        GF_HIP(hipEventSynchronize(sev[1]));
        float ms = 0;
        GF_HIP(hipEventElapsedTime(&ms, sev[0], sev[1]));
        return ms;
    }
    void ensure_stamps() {
        if (!stamps.n) {
            stamps.alloc(kNStamps + 4);
            h_stamps.alloc(kNStamps);
            GF_HIP(hipMemset(stamps.p, 0, (kNStamps + 4) * sizeof(uint64_t)));
        }
    }
    uint32_t* ticket(uint32_t i) { return reinterpret_cast<uint32_t*>(stamps.p + i); }
    // Milliseconds between the host copies of stamps i and i + 1.
    double stamp_ms(uint32_t i) const {
        const uint64_t* t = h_stamps.p;
        return t[i + 1] >= t[i] ? double(t[i + 1] - t[i]) / double(ix->wclk_khz) : 0.0;
    }
    // Waits for the stream and copies stamps [i, i + n) to the host.
    void fetch_stamps(uint32_t i, uint32_t n, hipStream_t st) {
        GF_HIP(hipStreamSynchronize(st));
        GF_HIP(hipMemcpy(h_stamps.p + i, stamps.p + i, n * sizeof(uint64_t), hipMemcpyDeviceToHost));
    }
    // Stage A, stage B and the search stage as HIP graphs.
    gf::StageGraph sg[3];
    static constexpr int kGraphA = 0, kGraphB = 1, kGraphSearch = 2;
    bool graph_replayed() const { return sg[kGraphSearch].replayed; }
    template <class F>
    void run_stage(const std::vector<uint64_t>& key, hipStream_t st, F&& enqueue) {
        sg[kGraphSearch].run(key, st, enqueue);
    }
    ~gf_batch() {
        for (auto& e : sev) if (e) (void)hipEventDestroy(e);
    }
};


namespace gf {
inline void set_device(const gf_index* ix) { GF_HIP(hipSetDevice(ix->device)); }
// The message gf_last_error() returns on the calling thread.
void set_last_error(const std::string& msg);
}  // namespace gf

namespace gf {
// Sub-cells of every cell (host arrays; see build_subcells in gf_host.cpp):
// false when the attributes do not allow them (a > 4, non-integer values, or
// a spread of 65534 or more inside a cell).
// The first-pass sub-cells (grid hash divisible by m), then the rest.
void first_pass_order(const std::vector<uint32_t>& shash, uint32_t m, std::vector<uint32_t>& order, uint32_t& ns1);
bool compute_subcells(const gf_index_host& h, const std::vector<uint32_t>& gidx, const std::vector<uint32_t>& size,
                      const std::vector<uint32_t>& offset_h, uint32_t a, uint32_t P, SubHost& out);
// Checks shared by resident and streamed indexes, and the idx mapper
// (tools.cuh:862-915): size[c] points per cell, ix.offset_h, gidx (row ->
// point id), lrow (row -> cell-local id).  Every id the kernels dereference
// is validated here, before any device call.
void map_cells(const gf_index_host& h, const gf_open_opts* opts, gf_index& ix, std::vector<uint32_t>& size,
               std::vector<uint32_t>& gidx, std::vector<uint32_t>& lrow);
// Streamed index (gf_stream.cpp): fills the pinned arena, makes the
// build-time plan and sizes the device buffers; then the streamed stage C.
void build_streamed(const gf_index_host& h, const gf_open_opts* opts, const gf_stream_plan* plan, gf_index& ix);
// A plan of a streamed index over the given batches of cell ids (each cell at
// most once): image layouts, runs and headers; the index's turn buffers and
// tile scratch grow to hold its largest batch within the device budget.
// reuse (may be null): a plan whose host and device buffers the new one may
// take over (it is left without them).
std::unique_ptr<StreamPlan> make_stream_plan(gf_index& ix, std::vector<std::vector<uint32_t>> cells,
                                             StreamPlan* reuse);
// gf_batch_plan_stream (returns the plan's active (query, batch) pairs) and
// gf_batch_set_stream_plan (no batches: back to the build-time plan).
uint64_t stream_plan_batch(gf_batch& b, uint64_t max_points, uint32_t max_cells);
void stream_set_plan(gf_batch& b, std::vector<std::vector<uint32_t>> cells);
void stream_search(gf_batch& b, const gf_search_opts& o, uint32_t* ids, float* dists, gf_search_stats* stats);
uint64_t plan_cells(const uint32_t* cells, const uint32_t* counts, uint32_t Q, uint32_t a, const uint32_t* grid,
                    const uint32_t* cell_size, uint64_t max_points, uint32_t max_cells,
                    std::vector<std::vector<uint32_t>>& plan);
// The planner's dynamic program on query boxes (qlo / qhi: a grid coordinates
// per query, lo <= hi), without the objective count.  cache (may be null):
// a frame kept for these cell sizes, reused when grid and limits match, else
// rebuilt into it.
void plan_boxes(const std::vector<uint32_t>& qlo, const std::vector<uint32_t>& qhi, uint32_t a, const uint32_t* grid,
                const uint32_t* cell_size, uint64_t max_points, uint32_t max_cells,
                std::vector<std::vector<uint32_t>>& plan, std::unique_ptr<PlanFrame>* cache = nullptr);
// Entry-point draws (mt19937 default seed, distinct uniform_int_distribution
// draws in [0, range), std::random_shuffle after srand(1)): the first R.
void entry_points_draw(uint32_t range, uint32_t ndraw, uint32_t R, uint32_t* out);
// The resident search's two draws in one generator sequence
// (gpu_graph.cu:12503-12539): 10 R distinct values below range1, shuffled,
// the first R; then, continuing the same mt19937 and rand() streams, 10 BD
// distinct values below range2, shuffled, the first BD (for the full graph).
void entry_points_pair(uint32_t range1, uint32_t R, uint32_t range2, uint32_t BD, uint32_t* out1, uint32_t* out2);
// Index builder (gf_build.cpp): the rank-quantile grid and the exact graphs.
void grid_scatter(const float* attrs, uint32_t N, uint32_t a, const uint32_t* grid, float* l_q, float* r_q,
                  uint32_t* pid_lists, uint32_t* global_pid);
void build_graphs(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D, const uint32_t* global_pid,
                  uint32_t P, uint32_t R, uint32_t E, int32_t device, uint32_t* cell_graphs, uint32_t* cross,
                  gf_build_stats* stats);
void optimize_graphs(const uint32_t* knn, uint32_t N, uint32_t I, const uint32_t* cell_size, uint32_t P,
                     uint32_t R, int32_t device, uint32_t* graphs, double* ms);
void kmeans_labels(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D, uint32_t C, uint32_t iters,
                   const uint32_t* init_ids, int32_t device, int32_t* labels, uint8_t* centres, double* ms);
}  // namespace gf
