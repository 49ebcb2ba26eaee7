// Streamed (out-of-core) index and search: the reference's out-of-core
// scheduler batch_graph_search_gpu_with_prefilter_batch_process_compressed_graph_T_dataset_resident_u8
// (big_dataset_adapterV3.cuh:3719-4117), rebuilt around a pinned arena and
// per-plan batch images.
//
// The reference issues one cudaMemcpyAsync per cell graph and per (cell,
// cell') cross-edge slice of a batch (big_dataset_adapterV3.cuh:3925-3946),
// then serialises the pipeline with cudaDeviceSynchronize (:4010) and
// re-ranks L candidates per query on 9 host threads (:3741-3797).  Here the
// index's rows sit in one pinned arena in resident row order, the cross
// edges target-major (gf_state.h, StreamIndex), so that a batch's image is
// assembled from a few pieces per run of consecutive cell ids in the batch
// (the cross edges of a pair of runs in one two-dimensional piece), whatever
// the plan: the index's build-time plan, or one a query batch makes from its
// own stage A cell lists, with no re-pack.  Large pieces move by DMA, the
// rest by one gather kernel that reads the pinned memory over PCIe (one DMA
// command per piece would cost more than moving the small ones).  The copies
// run on a side stream into one of two device buffers while the compute
// stream searches the previous batch; events order buffer reuse, and no host synchronisation
// happens inside the loop.  Distances are exact on the device (fp32 or u8
// data), so the per-batch top K merges into a running top K on the device
// instead of a host re-rank.
#include <algorithm>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "gf_state.h"

namespace gf {
namespace {

constexpr size_t kAlign = 256;
constexpr uint32_t kStreamTileChunk = 16;   // tiles per MFMA brute-force item on a streamed batch
constexpr int kCopyCore = 0, kCopyAttrs = 1, kCopyAll = 2;   // sections of a batch image to copy
// 1-D pieces of at least this many bytes move by DMA (a few us of command
// overhead each, no CU time); smaller and 2-D ones by k_stream_gather
constexpr size_t kDmaPiece = size_t(256) << 10;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }


// Runs body(lo, hi) over [0, n) on up to 16 host threads.
template <class F>
void parallel_for(size_t n, size_t grain, F&& body) {
    const size_t hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    const size_t nt = std::min(hw, std::max<size_t>(1, n / std::max<size_t>(grain, 1)));
    if (nt <= 1) {
        body(size_t(0), n);
        return;
    }
    std::vector<std::thread> th;
    for (size_t t = 0; t < nt; ++t) th.emplace_back([&, t] { body(n * t / nt, n * (t + 1) / nt); });
    for (auto& x : th) x.join();
}

// Device bytes a streamed index holds for turn buffers of `turn` bytes and
// tile records for `tiles` tiles.
uint64_t stream_device_need(const gf_index& ix, const StreamIndex& S, size_t turn, size_t tiles) {
    return 2 * uint64_t(turn) + (S.i8 ? uint64_t(tiles) * bf_rec_bytes(ix.D, S.AW) : 0);
}

}  // namespace

std::unique_ptr<StreamPlan> make_stream_plan(gf_index& ix, std::vector<std::vector<uint32_t>> cells,
                                             StreamPlan* reuse) {
    StreamIndex& S = *ix.sx;
    const uint32_t P = ix.P, a = ix.a, E = ix.E, R = ix.R;
    const uint32_t MW = 16 * (1 + S.AW);
    const SubHost& sh = S.sh;
    std::unique_ptr<StreamPlan> pl(new StreamPlan());
    {
        std::vector<char> seen(P, 0);
        for (const auto& bt : cells) {
            GF_REQUIRE(!bt.empty(), GF_E_ARG, "empty batch in the stream plan");
            for (uint32_t c : bt) {
                GF_REQUIRE(c < P, GF_E_ARG, "stream plan cell id out of range");
                GF_REQUIRE(!seen[c], GF_E_ARG, "cell " + std::to_string(c) + " appears twice in the stream plan");
                seen[c] = 1;
            }
        }
    }
    size_t head_total = 0;
    for (const auto& cl : cells) {
        StreamBatch sb;
        sb.B = uint32_t(cl.size());
        uint64_t rows = 0;
        for (uint32_t c : cl) rows += S.size[c];
        sb.rows = uint32_t(rows);
        if (S.i8)
            for (uint32_t c : cl) {
                sb.NS += sh.sbase[c + 1] - sh.sbase[c];
                sb.ntile += sh.stile[sh.sbase[c + 1]] - sh.stile[sh.sbase[c]];
            }
        // runs of consecutive cell ids
        sb.run0 = uint32_t(pl->runs.size());
        uint32_t r = 0, sbi = 0, tbi = 0;
        for (uint32_t i = 0; i < sb.B; ++i) {
            const uint32_t c = cl[i];
            if (i == 0 || c != cl[i - 1] + 1) {
                StreamRun u;
                u.i0 = i;
                u.c0 = c;
                u.g0 = ix.offset_h[c];
                u.r0 = r;
                if (S.i8) {
                    u.s0 = sh.sbase[c];
                    u.sb0 = sbi;
                    u.t0 = sh.stile[u.s0];
                    u.tb0 = tbi;
                }
                pl->runs.push_back(u);
            }
            StreamRun& u = pl->runs.back();
            ++u.n;
            u.rows += S.size[c];
            r += S.size[c];
            if (S.i8) {
                const uint32_t ns = sh.sbase[c + 1] - sh.sbase[c];
                const uint32_t nt = sh.stile[sh.sbase[c + 1]] - sh.stile[sh.sbase[c]];
                u.ns += ns;
                u.nt += nt;
                sbi += ns;
                tbi += nt;
            }
        }
        sb.nrun = uint32_t(pl->runs.size()) - sb.run0;
        // image layout
        size_t o = 0;
        auto take = [&](size_t bytes) {
            const size_t at = o;
            o = align_up(o + bytes);
            return at;
        };
        sb.o_offset = take((size_t(sb.B) + 1) * 4);
        sb.o_bcell = take(size_t(sb.B) * 4);
        if (S.i8) {
            sb.o_sbase = take((size_t(sb.B) + 1) * 4);
            sb.o_scell = take(size_t(sb.NS) * 4);
            sb.o_stile = take((size_t(sb.NS) + 1) * 4);
            sb.o_abase = take(size_t(sb.B) * a * 4);
        }
        sb.head = o;
        if (S.i8) {
            sb.o_ssize = take(size_t(sb.NS) * 4);
            sb.o_sbox = take(size_t(sb.NS) * 2 * a * 4);
            sb.o_tmeta = take(size_t(sb.ntile) * MW * 4);
        }
        sb.o_vec = take(rows * ix.rowbytes);
        sb.o_gidx = take(rows * 4);
        sb.bytes_mfma = o;
        sb.o_attrs = take(rows * a * 4);
        sb.bytes_bf = o;
        sb.o_graph = take(rows * R * 4);
        sb.o_lrow = take(rows * 4);
        sb.o_cross = take(size_t(sb.B) * rows * E * 4);
        sb.bytes = o;
        sb.head_off = head_total;
        head_total += sb.head;
        pl->max_bytes = std::max(pl->max_bytes, sb.bytes);
        pl->Bmax = std::max(pl->Bmax, sb.B);
        pl->NSmax = std::max(pl->NSmax, sb.NS);
        pl->tmax = std::max(pl->tmax, sb.ntile);
        pl->batches.push_back(sb);
    }
    // room on the device for the plan's largest batch (checked before any
    // device call)
    const size_t turn = std::max(S.turn[0].n, pl->max_bytes);
    const size_t tiles = std::max(S.trec_tiles, size_t(std::max(pl->tmax, 1u)));
    const bool grow = turn > S.turn[0].n || (S.i8 && tiles > S.trec_tiles);
    if (grow) {
        const uint64_t need = stream_device_need(ix, S, turn, tiles);
        GF_REQUIRE(S.budget == 0 || need <= S.budget, GF_E_UNSUPPORTED,
                   "the plan's largest batch needs " + std::to_string(need) + " device bytes (two images" +
                       (S.i8 ? std::string(" and its int8 tiles") : std::string()) + "), over the device budget of " +
                       std::to_string(S.budget));
    }
    GF_HIP(hipSetDevice(ix.device));
    // headers (in the previous plan's buffers when they are large enough)
    if (reuse && reuse->head.n >= std::max<size_t>(head_total, 1)) {
        std::swap(pl->head.p, reuse->head.p);
        std::swap(pl->head.n, reuse->head.n);
    } else {
        pl->head.alloc(std::max<size_t>(head_total, 1), hipHostMallocCoherent);
    }
    std::memset(pl->head.p, 0, std::max<size_t>(head_total, 1));
    for (size_t bi = 0; bi < cells.size(); ++bi) {
        const auto& cl = cells[bi];
        const StreamBatch& sb = pl->batches[bi];
        char* h = pl->head.p + sb.head_off;
        uint32_t* offset = reinterpret_cast<uint32_t*>(h + sb.o_offset);
        offset[0] = 0;
        for (uint32_t i = 0; i < sb.B; ++i) offset[i + 1] = offset[i] + S.size[cl[i]];
        std::memcpy(h + sb.o_bcell, cl.data(), cl.size() * 4);
        if (!S.i8) continue;
        uint32_t* sbase = reinterpret_cast<uint32_t*>(h + sb.o_sbase);
        uint32_t* scell = reinterpret_cast<uint32_t*>(h + sb.o_scell);
        uint32_t* stile = reinterpret_cast<uint32_t*>(h + sb.o_stile);
        int32_t* abase = reinterpret_cast<int32_t*>(h + sb.o_abase);
        uint32_t ns = 0, nt = 0;
        for (uint32_t i = 0; i < sb.B; ++i) {
            const uint32_t c = cl[i];
            sbase[i] = ns;
            for (uint32_t d = 0; d < a; ++d) abase[size_t(i) * a + d] = sh.abase[size_t(c) * a + d];
            for (uint32_t s0 = sh.sbase[c]; s0 < sh.sbase[c + 1]; ++s0, ++ns) {
                scell[ns] = i;
                stile[ns] = nt;
                nt += sh.stile[s0 + 1] - sh.stile[s0];
            }
        }
        sbase[sb.B] = ns;
        stile[ns] = nt;
    }
    // The pieces of each batch image (k_stream_gather), checked against the
    // image, the arena and the header block.
    {
        std::vector<GatherDesc> ds;
        pl->dma.clear();
        const size_t arena = S.arena_bytes, rb = ix.rowbytes;
        for (auto& sb : pl->batches) {
            sb.desc0 = uint32_t(ds.size());
            sb.dma0 = uint32_t(pl->dma.size());
            size_t moved = 0;
            auto put = [&](uint32_t base, size_t src, size_t dst, size_t width, uint32_t nrow = 1, size_t spitch = 0,
                           size_t dpitch = 0, uint32_t add = 0, uint32_t mw = 0) {
                if (!width || !nrow) return;
                const size_t send = src + (nrow - 1) * spitch + width, dend = dst + (nrow - 1) * dpitch + width;
                GF_REQUIRE(send <= (base ? head_total : arena) && dend <= sb.bytes && width <= UINT32_MAX, GF_E_STATE,
                           "internal: a streamed batch piece out of bounds");
                moved += width * nrow;
                if (base == 0 && nrow == 1 && !mw && width >= kDmaPiece) {
                    pl->dma.push_back(StreamCopy{src, dst, width});
                    return;
                }
                GatherDesc g{};
                g.src = src; g.dst = dst; g.spitch = spitch; g.dpitch = dpitch;
                g.width = uint32_t(width); g.nrow = nrow; g.base = base; g.add = add; g.mw = mw;
                ds.push_back(g);
            };
            auto level = [&](int w) {
                sb.ndesc[w] = uint32_t(ds.size()) - sb.desc0;
                sb.ndma[w] = uint32_t(pl->dma.size()) - sb.dma0;
                sb.moved[w] = moved;
            };
            const StreamRun* runs = pl->runs.data() + sb.run0;
            put(1, sb.head_off, 0, sb.head);
            for (uint32_t k = 0; k < sb.nrun; ++k) {
                const StreamRun& u = runs[k];
                if (S.i8) {
                    put(0, S.a_ssize + size_t(u.s0) * 4, sb.o_ssize + size_t(u.sb0) * 4, size_t(u.ns) * 4);
                    put(0, S.a_sbox + size_t(u.s0) * 2 * a * 4, sb.o_sbox + size_t(u.sb0) * 2 * a * 4,
                        size_t(u.ns) * 2 * a * 4);
                    // rows of a run move by one amount: batch row - resident row (mod 2^32)
                    put(0, S.a_tmeta + size_t(u.t0) * MW * 4, sb.o_tmeta + size_t(u.tb0) * MW * 4, size_t(u.nt) * MW * 4,
                        1, 0, 0, u.r0 - u.g0, MW);
                }
                put(0, S.a_vec + size_t(u.g0) * rb, sb.o_vec + size_t(u.r0) * rb, size_t(u.rows) * rb);
                put(0, S.a_gidx + size_t(u.g0) * 4, sb.o_gidx + size_t(u.r0) * 4, size_t(u.rows) * 4);
            }
            level(0);
            for (uint32_t k = 0; k < sb.nrun; ++k) {
                const StreamRun& u = runs[k];
                put(0, S.a_attrs + size_t(u.g0) * a * 4, sb.o_attrs + size_t(u.r0) * a * 4, size_t(u.rows) * a * 4);
            }
            level(1);
            for (uint32_t k = 0; k < sb.nrun; ++k) {
                const StreamRun& u = runs[k];
                put(0, S.a_graph + size_t(u.g0) * R * 4, sb.o_graph + size_t(u.r0) * R * 4, size_t(u.rows) * R * 4);
                put(0, S.a_lrow + size_t(u.g0) * 4, sb.o_lrow + size_t(u.r0) * 4, size_t(u.rows) * 4);
                // cross edges of run u's rows into the cells of run v: image rows
                // (v.i0 + j) * rows + u.r0, arena rows (v.c0 + j) * N + u.g0
                for (uint32_t k2 = 0; k2 < sb.nrun; ++k2) {
                    const StreamRun& v = runs[k2];
                    put(0, S.a_cross + (size_t(v.c0) * S.rows + u.g0) * E * 4,
                        sb.o_cross + (size_t(v.i0) * sb.rows + u.r0) * E * 4, size_t(u.rows) * E * 4, v.n,
                        size_t(S.rows) * E * 4, size_t(sb.rows) * E * 4);
                }
            }
            level(2);
        }
        if (ds.empty()) ds.push_back(GatherDesc{});
        if (reuse && reuse->desc.n >= ds.size()) {
            std::swap(pl->desc.p, reuse->desc.p);
            std::swap(pl->desc.n, reuse->desc.n);
        } else {
            pl->desc.alloc(ds.size());
        }
        GF_HIP(hipMemcpy(pl->desc.p, ds.data(), ds.size() * sizeof(GatherDesc), hipMemcpyHostToDevice));
    }
    {
        // sized for any plan (P cells, P batches) so that a later plan reuses them
        std::vector<uint32_t> pc, po(1, 0);
        for (const auto& cl : cells) {
            pc.insert(pc.end(), cl.begin(), cl.end());
            po.push_back(uint32_t(pc.size()));
        }
        if (reuse && reuse->plan_cells.n == size_t(P) + 1 && reuse->plan_off.n == size_t(P) + 1) {
            std::swap(pl->plan_cells.p, reuse->plan_cells.p);
            std::swap(pl->plan_cells.n, reuse->plan_cells.n);
            std::swap(pl->plan_off.p, reuse->plan_off.p);
            std::swap(pl->plan_off.n, reuse->plan_off.n);
        } else {
            pl->plan_cells.alloc(size_t(P) + 1);
            pl->plan_off.alloc(size_t(P) + 1);
        }
        if (!pc.empty()) GF_HIP(hipMemcpy(pl->plan_cells.p, pc.data(), pc.size() * 4, hipMemcpyHostToDevice));
        GF_HIP(hipMemcpy(pl->plan_off.p, po.data(), po.size() * 4, hipMemcpyHostToDevice));
    }
    if (turn > S.turn[0].n)
        for (int t = 0; t < 2; ++t) S.turn[t].alloc(turn);
    if (S.i8 && tiles > S.trec_tiles) {
        S.trec.alloc(tiles * bf_rec_bytes(ix.D, S.AW));
        S.trec_tiles = tiles;
    }
    pl->cells = std::move(cells);
    return pl;
}

void build_streamed(const gf_index_host& h, const gf_open_opts* opts, const gf_stream_plan* plan, gf_index& ix) {
    GF_REQUIRE(plan, GF_E_ARG, "null stream plan");
    std::vector<uint32_t> size, gidx, lrow;
    map_cells(h, opts, ix, size, gidx, lrow);
    GF_REQUIRE(ix.vdtype != GF_VEC_F16 && ix.vdtype != GF_VEC_I8Q && ix.vdtype != GF_VEC_F16_REF, GF_E_UNSUPPORTED,
               "a streamed index holds GF_VEC_F32 or GF_VEC_U8 vectors");
    const uint32_t P = ix.P, R = ix.R, E = ix.E, a = ix.a, D = ix.D;
    const uint32_t N = ix.offset_h[P];

    // The build-time plan: explicit batches, or consecutive cells.
    std::vector<std::vector<uint32_t>> plan_cells;
    if (plan->nbatch == 0) {
        const uint32_t bc = plan->batch_cells ? plan->batch_cells : 16u;
        for (uint32_t c = 0; c < P; c += bc) {
            std::vector<uint32_t> v;
            for (uint32_t k = c; k < std::min(P, c + bc); ++k) v.push_back(k);
            plan_cells.push_back(v);
        }
    } else {
        GF_REQUIRE(plan->sizes && plan->cells, GF_E_ARG, "stream plan without sizes or cells");
        size_t k = 0;
        for (uint32_t i = 0; i < plan->nbatch; ++i) {
            GF_REQUIRE(plan->sizes[i] >= 1, GF_E_ARG, "empty batch in the stream plan");
            GF_REQUIRE(plan->sizes[i] <= P, GF_E_ARG, "stream plan batch larger than the grid");
            plan_cells.emplace_back(plan->cells + k, plan->cells + k + plan->sizes[i]);
            k += plan->sizes[i];
        }
    }

    std::unique_ptr<StreamIndex> sx(new StreamIndex());
    StreamIndex& S = *sx;
    S.budget = plan->device_budget;
    S.rows = N;
    S.size = size;
    // Sub-cells for the MFMA brute force (u8 vectors, D a multiple of 64 up to 256).
    S.i8 = ix.vdtype == GF_VEC_U8 && D % 64 == 0 && D <= 256 &&
           compute_subcells(h, gidx, size, ix.offset_h, a, P, S.sh);
    S.AW = S.sh.AW;
    const uint32_t MW = 16 * (1 + S.AW);
    S.min_cell = 0;
    for (uint32_t c = 0; c < P; ++c)
        if (size[c] && (S.min_cell == 0 || size[c] < S.min_cell)) S.min_cell = size[c];

    // The arena.
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = align_up(o + bytes);
        return at;
    };
    S.a_vec = take(size_t(N) * ix.rowbytes);
    S.a_gidx = take(size_t(N) * 4);
    S.a_attrs = take(size_t(N) * a * 4);
    S.a_graph = take(size_t(N) * R * 4);
    S.a_lrow = take(size_t(N) * 4);
    S.a_cross = take(size_t(P) * N * E * 4);
    if (S.i8) {
        S.a_ssize = take(size_t(S.sh.NS) * 4);
        S.a_sbox = take(size_t(S.sh.NS) * 2 * a * 4);
        S.a_tmeta = take(size_t(S.sh.ntile) * MW * 4);
    }

    S.arena_bytes = o;
    ix.sx = std::move(sx);
    // the build-time plan sizes the device buffers (and checks the plan and
    // the budget before any device call)
    S.plan = make_stream_plan(ix, std::move(plan_cells), nullptr);
    GF_HIP(hipSetDevice(ix.device));
    GF_HIP(hipStreamCreateWithFlags(&ix.stream, hipStreamNonBlocking));
    GF_HIP(hipStreamCreateWithFlags(&S.copy, hipStreamNonBlocking));
    for (int t = 0; t < 2; ++t) {
        GF_HIP(hipEventCreateWithFlags(&S.ready[t], hipEventDisableTiming));
        GF_HIP(hipEventCreateWithFlags(&S.freed[t], hipEventDisableTiming));
    }

    S.host.alloc(std::max<size_t>(S.arena_bytes, 1), hipHostMallocCoherent);
    char* A = S.host.p;
    parallel_for(N, 4096, [&](size_t lo, size_t hi) {
        for (size_t g = lo; g < hi; ++g) {
            const uint32_t pt = gidx[g];
            const float* x = h.vectors + size_t(pt) * D;
            if (ix.vdtype == GF_VEC_U8) {
                uint8_t* y = reinterpret_cast<uint8_t*>(A + S.a_vec) + g * ix.rowbytes;
                for (uint32_t j = 0; j < D; ++j) y[j] = uint8_t(x[j]);
            } else {
                std::memcpy(A + S.a_vec + g * ix.rowbytes, x, size_t(D) * 4);
            }
            float* at = reinterpret_cast<float*>(A + S.a_attrs) + g * a;
            for (uint32_t d = 0; d < a; ++d) at[d] = h.attrs[size_t(pt) * a + d];
        }
    });
    std::memcpy(A + S.a_gidx, gidx.data(), size_t(N) * 4);
    std::memcpy(A + S.a_graph, h.cell_graphs, size_t(N) * R * 4);
    std::memcpy(A + S.a_lrow, lrow.data(), size_t(N) * 4);
    // cross edges, point-major in the input, target-major in the arena;
    // blocks of rows so that a block's input rows stay in cache
    parallel_for((size_t(N) + 255) / 256, 4, [&](size_t lo, size_t hi) {
        uint32_t* X = reinterpret_cast<uint32_t*>(A + S.a_cross);
        for (size_t blk = lo; blk < hi; ++blk) {
            const size_t g0 = blk * 256, g1 = std::min<size_t>(N, g0 + 256);
            for (uint32_t c = 0; c < P; ++c)
                for (size_t g = g0; g < g1; ++g)
                    for (uint32_t e = 0; e < E; ++e)
                        X[(size_t(c) * N + g) * E + e] = h.cross[(size_t(gidx[g]) * P + c) * E + e];
        }
    });
    if (S.i8) {
        std::memcpy(A + S.a_ssize, S.sh.ssize.data(), S.sh.ssize.size() * 4);
        std::memcpy(A + S.a_sbox, S.sh.sbox.data(), S.sh.sbox.size() * 4);
        std::memcpy(A + S.a_tmeta, S.sh.tmeta.data(), S.sh.tmeta.size() * 4);
        // the plans need the offsets only
        std::vector<uint32_t>().swap(S.sh.ssize);
        std::vector<int32_t>().swap(S.sh.sbox);
        std::vector<uint32_t>().swap(S.sh.tmeta);
        std::vector<uint32_t>().swap(S.sh.sorder);
        std::vector<uint32_t>().swap(S.sh.scell);
        ix.i8 = true;   // gf_batch_create keeps int8 queries
    }
    GF_HIP(hipDeviceGetAttribute(&ix.ncu, hipDeviceAttributeMultiprocessorCount, ix.device));
    ix.offset.upload(ix.offset_h);
    ix.grid.upload(ix.grid_h);
}

// Batch plan from a query batch's cell lists: the out-of-core pipeline's
// cell scheduling (README.md:5: cells are grouped so that few queries are
// active in each batch; the shipped driver fixes its batches by hand,
// bigdataset_experiment.cu:271-277, 746-756).  A query is active in a batch
// when it selects one of the batch's cells; each active (query, batch) pair
// restarts the query's search on fresh entries and costs a pass of its
// schedule, so the plan minimises the sum over batches of active queries.
//
// A range query selects a box of the grid (the Cartesian product of one
// cell interval per attribute), so batches are boxes too: the plan is the
// best guillotine partition of the grid into boxes that fit a batch (at most
// max_cells non-empty cells and max_points points; 0 = no limit), found by
// dynamic programming over every box of the grid.  Cutting a box X in two
// between cells t-1 and t of axis d adds to the objective exactly the
// queries that select cells on both sides: those whose interval on d holds
// t-1 and t and whose box meets X on every other axis.  So
//   cost(X) = 0 when X fits a batch, else
//   min over (d, t) of cut(X, d, t) + cost(lower part) + cost(upper part),
// compared as (cost, batches) with ties to the first (d, t) in ascending
// order; a batch is a leaf box's non-empty cells in id order, leaves in
// recursion order (lower part first), empty leaves dropped.  A query's
// lists are read as their bounding box; the returned objective is recounted
// from the lists themselves.
uint64_t plan_cells(const uint32_t* cells, const uint32_t* counts, uint32_t Q, uint32_t a, const uint32_t* grid,
                    const uint32_t* cell_size, uint64_t max_points, uint32_t max_cells,
                    std::vector<std::vector<uint32_t>>& plan) {
    GF_REQUIRE(a >= 1 && a <= kMaxAttr, GF_E_ARG, "plan_cells: attribute count out of range");
    uint64_t P = 1, nbox = 1;
    uint32_t stride[kMaxAttr];
    for (uint32_t d = 0; d < a; ++d) {
        GF_REQUIRE(grid[d] >= 1, GF_E_ARG, "plan_cells: empty grid axis");
        P *= grid[d];
        nbox *= uint64_t(grid[d]) * grid[d];
        GF_REQUIRE(nbox <= (uint64_t(1) << 22), GF_E_UNSUPPORTED, "plan_cells: grid too large to plan (more than 2^22 box slots)");
    }
    for (int d = int(a) - 1, s = 1; d >= 0; --d) {
        stride[d] = uint32_t(s);
        s *= int(grid[d]);
    }
    // Each query's box (bounding box of its listed cells).
    std::vector<uint32_t> qlo, qhi;   // Qb x a
    const size_t W = (size_t(Q) + 63) / 64;
    std::vector<uint64_t> sel(size_t(P) * W, 0);
    for (uint32_t q = 0; q < Q; ++q) {
        GF_REQUIRE(counts[q] <= P, GF_E_ARG, "plan_cells: a query lists more cells than the grid holds");
        if (!counts[q]) continue;
        uint32_t lo[kMaxAttr], hi[kMaxAttr];
        for (uint32_t d = 0; d < a; ++d) { lo[d] = grid[d]; hi[d] = 0; }
        for (uint32_t i = 0; i < counts[q]; ++i) {
            const uint32_t c = cells[size_t(q) * P + i];
            GF_REQUIRE(c < P, GF_E_ARG, "plan_cells: cell id out of range");
            sel[size_t(c) * W + q / 64] |= uint64_t(1) << (q % 64);
            for (uint32_t d = 0; d < a; ++d) {
                const uint32_t x = c / stride[d] % grid[d];
                lo[d] = std::min(lo[d], x);
                hi[d] = std::max(hi[d], x);
            }
        }
        qlo.insert(qlo.end(), lo, lo + a);
        qhi.insert(qhi.end(), hi, hi + a);
    }
    plan_boxes(qlo, qhi, a, grid, cell_size, max_points, max_cells, plan);
    uint64_t total = 0;
    std::vector<uint64_t> act(W);
    for (const auto& bt : plan) {
        std::fill(act.begin(), act.end(), 0);
        for (uint32_t c : bt)
            for (size_t w = 0; w < W; ++w) act[w] |= sel[size_t(c) * W + w];
        for (size_t w = 0; w < W; ++w) total += uint64_t(__builtin_popcountll(act[w]));
    }
    return total;
}

namespace {

// Grid coordinates of box i: (x0, x1) per axis; false for an empty slot
// (x0 > x1).
inline bool box_coords(const PlanFrame& F, size_t i, uint32_t* x0, uint32_t* x1) {
    for (uint32_t d = 0; d < F.a; ++d) {
        const uint32_t g = F.grid[d], v = uint32_t((i / F.bstride[d]) % (size_t(g) * g));
        x0[d] = v / g;
        x1[d] = v % g;
        if (x0[d] > x1[d]) return false;
    }
    return true;
}

void build_frame(PlanFrame& F, uint32_t a, const uint32_t* grid, const uint32_t* cell_size, uint64_t max_points,
                 uint32_t max_cells) {
    F.a = a;
    F.grid.assign(grid, grid + a);
    F.max_points = max_points;
    F.max_cells = max_cells;
    F.nbox = 1;
    for (uint32_t d = 0; d < a; ++d) F.nbox *= size_t(grid[d]) * grid[d];
    for (int d = int(a) - 1, s = 1, bs = 1; d >= 0; --d) {
        F.stride[d] = uint32_t(s);
        F.bstride[d] = uint32_t(bs);
        s *= int(grid[d]);
        bs *= int(grid[d] * grid[d]);
    }
    // boxes by total extent (counting sort): both parts of a cut come first
    uint32_t emax = 0;
    for (uint32_t d = 0; d < a; ++d) emax += grid[d] - 1;
    std::vector<uint32_t> ext(F.nbox, UINT32_MAX), count(emax + 2, 0);
    uint32_t x0[kMaxAttr], x1[kMaxAttr];
    for (size_t i = 0; i < F.nbox; ++i) {
        if (!box_coords(F, i, x0, x1)) continue;
        uint32_t e = 0;
        for (uint32_t d = 0; d < a; ++d) e += x1[d] - x0[d];
        ext[i] = e;
        ++count[e + 1];
    }
    for (uint32_t e = 1; e <= emax + 1; ++e) count[e] += count[e - 1];
    std::vector<uint32_t> byext(count[emax + 1]);
    for (size_t i = 0; i < F.nbox; ++i)
        if (ext[i] != UINT32_MAX) byext[count[ext[i]]++] = uint32_t(i);
    std::vector<uint64_t> npts(F.nbox, 0);
    std::vector<uint32_t> ncell(F.nbox, 0);
    F.leaf.assign(F.nbox, 0);
    F.order.clear();
    for (uint32_t i : byext) {
        box_coords(F, i, x0, x1);
        uint32_t d0 = a;
        for (uint32_t d = 0; d < a; ++d)
            if (x1[d] > x0[d]) { d0 = d; break; }
        if (d0 == a) {   // one cell
            uint32_t c = 0;
            for (uint32_t d = 0; d < a; ++d) c += x0[d] * F.stride[d];
            npts[i] = cell_size[c];
            ncell[i] = cell_size[c] ? 1u : 0u;
            F.leaf[i] = uint8_t(ncell[i]);
            continue;
        }
        // the slab x0 of axis d0 and the rest
        const size_t ia = i - size_t(x1[d0] - x0[d0]) * F.bstride[d0];
        const size_t ib = i + size_t(grid[d0]) * F.bstride[d0];
        npts[i] = npts[ia] + npts[ib];
        ncell[i] = ncell[ia] + ncell[ib];
        if ((max_cells == 0 || ncell[i] <= max_cells) && (max_points == 0 || npts[i] <= max_points)) {
            F.leaf[i] = ncell[i] ? 1u : 0u;
        } else {
            F.leaf[i] = 2;
            F.order.push_back(i);
        }
    }
}

}  // namespace

void plan_boxes(const std::vector<uint32_t>& qlo, const std::vector<uint32_t>& qhi, uint32_t a, const uint32_t* grid,
                const uint32_t* cell_size, uint64_t max_points, uint32_t max_cells,
                std::vector<std::vector<uint32_t>>& plan, std::unique_ptr<PlanFrame>* cache) {
    GF_REQUIRE(a >= 1 && a <= kMaxAttr, GF_E_ARG, "plan_cells: attribute count out of range");
    GF_REQUIRE(qlo.size() == qhi.size() && qlo.size() % a == 0, GF_E_ARG, "plan_cells: malformed query boxes");
    uint64_t nbox = 1;
    for (uint32_t d = 0; d < a; ++d) {
        GF_REQUIRE(grid[d] >= 1, GF_E_ARG, "plan_cells: empty grid axis");
        nbox *= uint64_t(grid[d]) * grid[d];
        GF_REQUIRE(nbox <= (uint64_t(1) << 22), GF_E_UNSUPPORTED, "plan_cells: grid too large to plan (more than 2^22 box slots)");
    }
    for (size_t k = 0; k < qlo.size(); ++k)
        GF_REQUIRE(qlo[k] <= qhi[k] && qhi[k] < grid[k % a], GF_E_ARG, "plan_cells: query box outside the grid");
    std::unique_ptr<PlanFrame> local;
    std::unique_ptr<PlanFrame>& slot = cache ? *cache : local;
    if (!slot || slot->a != a || !std::equal(grid, grid + a, slot->grid.begin()) || slot->max_points != max_points ||
        slot->max_cells != max_cells) {
        slot.reset(new PlanFrame());
        build_frame(*slot, a, grid, cell_size, max_points, max_cells);
    }
    const PlanFrame& F = *slot;
    const size_t Qb = qlo.size() / a;
    // cut(X, d, t).  One attribute: the queries straddling t; two: per (d,
    // t) a table over the other axis' [x0, x1] of the straddling queries
    // whose interval meets it (suffix sums over hi, prefix sums over lo of a
    // (lo, hi) histogram); more: a scan of the straddling queries.
    std::vector<std::vector<std::vector<uint32_t>>> strad(a);   // [d][t] query indices (a > 2)
    std::vector<std::vector<uint64_t>> tab(a);                  // [d] (t * ge + x0) * ge + x1 (a <= 2)
    for (uint32_t d = 0; d < a; ++d) {
        const uint32_t e = a == 2 ? 1 - d : d, ge = a == 2 ? grid[e] : 1;
        if (a > 2) {
            strad[d].resize(grid[d]);
            for (size_t q = 0; q < Qb; ++q)
                for (uint32_t t = qlo[q * a + d] + 1; t <= qhi[q * a + d]; ++t) strad[d][t].push_back(uint32_t(q));
            continue;
        }
        std::vector<uint64_t>& T = tab[d];
        T.assign(size_t(grid[d]) * ge * ge, 0);
        // histogram of straddlers per t over (lo_e, hi_e)
        for (size_t q = 0; q < Qb; ++q) {
            const size_t key = a == 2 ? size_t(qlo[q * a + e]) * ge + qhi[q * a + e] : 0;
            for (uint32_t t = qlo[q * a + d] + 1; t <= qhi[q * a + d]; ++t) ++T[size_t(t) * ge * ge + key];
        }
        std::vector<uint64_t> h(size_t(ge) * ge);
        for (uint32_t t = 1; t < grid[d]; ++t) {
            uint64_t* Tt = &T[size_t(t) * ge * ge];
            std::copy(Tt, Tt + size_t(ge) * ge, h.begin());
            // T[x0 * ge + x1] = #{lo <= x1, hi >= x0}
            for (uint32_t lo = 0; lo < ge; ++lo)
                for (uint32_t hi = ge - 1; hi-- > 0;) h[size_t(lo) * ge + hi] += h[size_t(lo) * ge + hi + 1];
            for (uint32_t x0 = 0; x0 < ge; ++x0) {
                uint64_t n = 0;
                for (uint32_t x1 = 0; x1 < ge; ++x1) {
                    n += h[size_t(x1) * ge + x0];
                    Tt[size_t(x0) * ge + x1] = x1 >= x0 ? n : 0;
                }
            }
        }
    }
    // (cost, batches) of each box as one key, cost << 12 | batches (a box of
    // this size has fewer than 2^11 cells): adding two keys adds both parts,
    // and comparing keys compares (cost, batches) in that order
    constexpr uint32_t kLeafBits = 12;
    std::vector<uint64_t> key(F.nbox);
    std::vector<uint32_t> split(F.nbox, 0);   // 0 = leaf, else d * 65536 + t
    for (size_t i = 0; i < F.nbox; ++i) key[i] = F.leaf[i] == 2 ? 0u : F.leaf[i];
    uint32_t x0[kMaxAttr], x1[kMaxAttr];
    for (uint32_t i : F.order) {
        box_coords(F, i, x0, x1);
        uint64_t best = UINT64_MAX;
        uint32_t bs = 0;
        for (uint32_t d = 0; d < a; ++d) {
            const size_t bd = F.bstride[d], gbd = size_t(grid[d]) * bd;
            // cut at t: lower part i - (x1 - t + 1) bd, upper part i + (t - x0) g bd
            const uint64_t* ka = key.data() + (i - size_t(x1[d] - x0[d]) * bd);
            const uint64_t* kb = key.data() + (i + gbd);
            const uint32_t n = x1[d] - x0[d];
            if (a <= 2) {
                const uint32_t e = a == 2 ? 1 - d : 0, ge = a == 2 ? grid[e] : 1;
                const size_t row = a == 2 ? size_t(x0[e]) * ge + x1[e] : 0, tstep = size_t(ge) * ge;
                const uint64_t* T = tab[d].data() + size_t(x0[d] + 1) * tstep + row;
                for (uint32_t k = 0; k < n; ++k) {
                    const uint64_t c = (T[k * tstep] << kLeafBits) + ka[k * bd] + kb[k * gbd];
                    if (c < best) { best = c; bs = d * 65536u + x0[d] + 1 + k; }
                }
            } else {
                for (uint32_t k = 0; k < n; ++k) {
                    const uint32_t t = x0[d] + 1 + k;
                    uint64_t cut = 0;
                    for (uint32_t q : strad[d][t]) {
                        bool meets = true;
                        for (uint32_t e = 0; e < a && meets; ++e)
                            if (e != d) meets = qlo[q * a + e] <= x1[e] && qhi[q * a + e] >= x0[e];
                        cut += meets;
                    }
                    const uint64_t c = (cut << kLeafBits) + ka[k * bd] + kb[k * gbd];
                    if (c < best) { best = c; bs = d * 65536u + t; }
                }
            }
        }
        key[i] = best;
        split[i] = bs;
    }
    // the leaves, lower parts first; a leaf's non-empty cells in id order
    plan.clear();
    size_t all = 0;
    for (uint32_t d = 0; d < a; ++d) all += size_t(grid[d] - 1) * F.bstride[d];   // x0 = 0, x1 = g - 1
    std::vector<size_t> stack(1, all);
    while (!stack.empty()) {
        const size_t i = stack.back();
        stack.pop_back();
        box_coords(F, i, x0, x1);
        if (split[i]) {
            const uint32_t d = split[i] / 65536u, t = split[i] % 65536u;
            const size_t bd = F.bstride[d];
            stack.push_back(i + size_t(t - x0[d]) * grid[d] * bd);   // upper part
            stack.push_back(i - size_t(x1[d] - t + 1) * bd);          // lower part, popped first
            continue;
        }
        std::vector<uint32_t> batch;
        uint32_t x[kMaxAttr];
        for (uint32_t d = 0; d < a; ++d) x[d] = x0[d];
        for (;;) {
            uint32_t c = 0;
            for (uint32_t d = 0; d < a; ++d) c += x[d] * F.stride[d];
            if (cell_size[c]) batch.push_back(c);
            int d = int(a) - 1;
            while (d >= 0 && ++x[d] > x1[d]) { x[d] = x0[d]; --d; }
            if (d < 0) break;
        }
        if (!batch.empty()) plan.push_back(std::move(batch));
    }
}

namespace {

// A new plan for b in the buffers of its current one; a failure after the
// buffers moved (a device error) leaves b on the index's build-time plan.
std::unique_ptr<StreamPlan> plan_reusing(gf_batch& b, std::vector<std::vector<uint32_t>> cells) {
    try {
        return make_stream_plan(*b.ix, std::move(cells), b.splan.get());
    } catch (...) {
        if (b.splan && (!b.splan->head.p || !b.splan->plan_cells.p)) b.splan.reset();
        throw;
    }
}

}  // namespace

// The plan of a query batch from its own stage A cell lists: each query's
// bounding box on the device (k_cell_boxes), the boxes to the host, the
// planner's dynamic program (plan_boxes), the plan's headers; the batch's
// active (query, batch) pairs counted on the device from its cell flags.
uint64_t stream_plan_batch(gf_batch& b, uint64_t max_points, uint32_t max_cells) {
    gf_index& ix = *b.ix;
    StreamIndex& S = *ix.sx;
    const uint32_t Q = b.Q, P = ix.P, a = ix.a;
    hipStream_t st = ix.stream;
    if (b.qbox.n < size_t(Q) * 2 * a) b.qbox.alloc(size_t(Q) * 2 * a);
    GF_HIP(launch_cell_boxes(Q, P, a, ix.grid.p, b.cells.p, b.counts.p, b.qbox.p, st));
    std::vector<uint32_t> box(size_t(Q) * 2 * a);
    if (Q) GF_HIP(hipMemcpyAsync(box.data(), b.qbox.p, box.size() * 4, hipMemcpyDeviceToHost, st));
    GF_HIP(hipStreamSynchronize(st));
    std::vector<uint32_t> qlo, qhi;
    for (uint32_t q = 0; q < Q; ++q) {
        const uint32_t* x = &box[size_t(q) * 2 * a];
        if (x[0] > x[a]) continue;   // no cell
        qlo.insert(qlo.end(), x, x + a);
        qhi.insert(qhi.end(), x + a, x + 2 * a);
    }
    std::vector<std::vector<uint32_t>> cells;
    plan_boxes(qlo, qhi, a, ix.grid_h.data(), S.size.data(), max_points, max_cells, cells, &S.frame);
    std::unique_ptr<StreamPlan> pl = plan_reusing(b, std::move(cells));
    const size_t nb = pl->batches.size();
    if (!b.flags_ready) {
        if (b.flags.n < size_t(Q) * P) b.flags.alloc(size_t(Q) * P);
        GF_HIP(launch_cell_flags(Q, P, b.cells.p, b.counts.p, b.little.p, b.flags.p, st));
    }
    if (b.need.n < 2 * std::max<size_t>(nb, 1)) b.need.alloc(2 * std::max<size_t>(nb, 1));
    GF_HIP(launch_batch_need(Q, P, uint32_t(nb), pl->plan_cells.p, pl->plan_off.p, b.flags.p, b.need.p, st));
    std::vector<uint32_t> act(nb);
    if (nb) GF_HIP(hipMemcpyAsync(act.data(), b.need.p + nb, nb * 4, hipMemcpyDeviceToHost, st));
    GF_HIP(hipStreamSynchronize(st));
    b.splan = std::move(pl);
    uint64_t total = 0;
    for (uint32_t x : act) total += x;
    return total;
}

void stream_set_plan(gf_batch& b, std::vector<std::vector<uint32_t>> cells) {
    if (cells.empty()) {
        b.splan.reset();
        return;
    }
    b.splan = plan_reusing(b, std::move(cells));
}

void stream_search(gf_batch& b, const gf_search_opts& o, uint32_t* ids, float* dists, gf_search_stats* stats) {
    gf_index& ix = *b.ix;
    StreamIndex& S = *ix.sx;
    const StreamPlan& pl = b.splan ? *b.splan : *S.plan;
    GF_REQUIRE(pl.max_bytes <= S.turn[0].n && (!S.i8 || pl.tmax <= S.trec_tiles), GF_E_STATE,
               "the stream plan's largest batch does not fit the index's device buffers");
    const uint32_t Q = b.Q, K = o.K, L = o.L, R = ix.R, P = ix.P, Bm = std::max<uint32_t>(pl.Bmax, 1u);
    hipStream_t st = ix.stream;

    // Entry points: the caller's, or the out-of-core host's draw: 10 L
    // distinct values below the smallest cell, shuffled, the first R used
    // (big_dataset_adapterV3.cuh:3862-3875).
    std::vector<uint32_t> ent(R);
    if (o.entry_points) std::copy(o.entry_points, o.entry_points + R, ent.begin());
    else entry_points_draw(std::max(S.min_cell, 1u), 10 * L, R, ent.data());
    b.entry.upload(ent);
    b.entry_src = nullptr;

    if (!b.flags_ready) {
        if (b.flags.n < size_t(Q) * P) b.flags.alloc(size_t(Q) * P);
        GF_HIP(launch_cell_flags(Q, P, b.cells.p, b.counts.p, b.little.p, b.flags.p, st));
    }
    if (b.slist.n < size_t(Q) * Bm) b.slist.alloc(size_t(Q) * Bm);
    if (b.scount.n < Q) { b.scount.alloc(Q); b.slittle.alloc(Q); }
    if (b.sched.n < Q) b.sched.alloc(Q);
    if (b.s_ids.n < size_t(Q) * K) { b.s_ids.alloc(size_t(Q) * K); b.s_dist.alloc(size_t(Q) * K); }
    if (b.s_ctr.n < size_t(Q) * GF_NCOUNTERS) b.s_ctr.alloc(size_t(Q) * GF_NCOUNTERS);
    if (b.out_ids.n < size_t(Q) * K) { b.out_ids.alloc(size_t(Q) * K); b.out_dist.alloc(size_t(Q) * K); }
    if (b.counters.n < size_t(Q) * GF_NCOUNTERS) b.counters.alloc(size_t(Q) * GF_NCOUNTERS);

    const uint32_t hsize = visited_slots(L + kXSlots + 4 * R);
    const uint32_t Lpad = round_up(L, 2);
    const uint32_t lds = trav_lds_bytes(Lpad, hsize, Bm);
    GF_REQUIRE(lds <= 64 * 1024, GF_E_UNSUPPORTED, "L too large for the LDS budget");

    TravArgs base{};
    base.rowbytes = ix.rowbytes;
    base.nch = ix.rs.nch;
    base.queries = reinterpret_cast<const char*>(b.qf32.p);
    base.qbytes = ix.D * 4;
    base.lo = b.lo.p;
    base.hi = b.hi.p;
    base.cells = b.slist.p;
    base.counts = b.scount.p;
    base.little = b.slittle.p;
    base.sched = b.sched.p;
    base.entry = b.entry.p;
    base.out_ids = b.s_ids.p;
    base.out_dist = b.s_dist.p;
    base.counters = b.s_ctr.p;
    base.a = ix.a; base.R = R; base.E = ix.E; base.L = L; base.K = K; base.rl = o.rl;
    base.hsize = hsize;
    base.offl = trav_offsets_in_lds(Bm) ? 1u : 0u;   // lds holds Bm + 1 >= B + 1 offsets
    base.Lpad = Lpad;
    uint32_t* tot = b.tot.p;

    const size_t nb = pl.batches.size();
    // per batch: copy start/end (copy stream), traversal start, brute-force start/end (compute stream)
    std::vector<hipEvent_t> ce(5 * nb, nullptr);
    hipEvent_t t0 = nullptr, t1 = nullptr;
    struct Ev {
        std::vector<hipEvent_t>& v;
        hipEvent_t* a;
        hipEvent_t* b;
        ~Ev() {
            for (auto e : v) if (e) (void)hipEventDestroy(e);
            if (*a) (void)hipEventDestroy(*a);
            if (*b) (void)hipEventDestroy(*b);
        }
    } guard{ce, &t0, &t1};
    for (auto& e : ce) GF_HIP(hipEventCreate(&e));
    GF_HIP(hipEventCreate(&t0));
    GF_HIP(hipEventCreate(&t1));

    // MFMA brute force on the streamed batches: int8 queries, K within the
    // route's limit; schedule buffers sized like the resident path's.
    const bool gemm = S.i8 && b.i8 && K <= kBfKMax;
    if (gemm) {
        const uint32_t NS = std::max(pl.NSmax, 1u);
        if (b.bcnt.n < NS) { b.bcnt.alloc(NS); b.bin.alloc(NS); b.bstart.alloc(NS); b.icnt.alloc(NS); b.ioff.alloc(NS); }
        if (b.nsub.n < Q) { b.nsub.alloc(Q); b.part_off.alloc(Q); b.pcnt.alloc(Q); b.gbound.alloc(Q); }
        // items <= pairs x chunks / 64 + (sub-cell, chunk) slots (k_bfitems)
        // sized for this plan's largest batch (a batch's plan may change
        // between searches)
        const size_t slots = pl.tmax / kStreamTileChunk + NS;
        if (!b.pairs_fit(Q, NS, slots)) b.alloc_pairs(std::max<size_t>(b.pair_cap, size_t(Q) * 64), K, Q, NS, slots);
        if (b.part.n < b.pair_cap * K) b.part.alloc(b.pair_cap * K);
        if (b.bfmask.n < size_t(Q) * Bm) b.bfmask.alloc(size_t(Q) * Bm);
        if (b.note.n < 2 * std::max<size_t>(nb, 1)) b.note.alloc(2 * std::max<size_t>(nb, 1));
    }
    std::vector<hipEvent_t> ge(2 * nb, nullptr);   // around each batch's MFMA kernel
    struct EvG {
        std::vector<hipEvent_t>& v;
        ~EvG() { for (auto e : v) if (e) (void)hipEventDestroy(e); }
    } gguard{ge};
    if (gemm) for (auto& e : ge) GF_HIP(hipEventCreate(&e));

    // Filtered brute force of one batch on int8 MFMA: the resident path's
    // item schedule (k_bfsched / k_bfitems / k_bf_i8 / k_bf_final) on the
    // batch's sub-cells, restricted by bfmask to the cells the batch lists.
    auto mfma_bruteforce = [&](size_t bi, const StreamBatch& sb, char* dev) {
        SubArgs sa{};
        sa.sbase = reinterpret_cast<const uint32_t*>(dev + sb.o_sbase);
        sa.scell = reinterpret_cast<const uint32_t*>(dev + sb.o_scell);
        sa.ssize = reinterpret_cast<const uint32_t*>(dev + sb.o_ssize);
        sa.stile = reinterpret_cast<const uint32_t*>(dev + sb.o_stile);
        sa.sbox = reinterpret_cast<const int32_t*>(dev + sb.o_sbox);
        sa.tmeta = reinterpret_cast<const uint32_t*>(dev + sb.o_tmeta);
        sa.abase = reinterpret_cast<const int32_t*>(dev + sb.o_abase);
        sa.a = ix.a; sa.AW = S.AW; sa.P = sb.B; sa.NS = sb.NS;
        GF_HIP(launch_tile_rec(dev + sb.o_vec, true, ix.D, sa.tmeta, S.AW, sb.ntile, S.trec.p, st));
        GF_HIP(launch_cell_flags(Q, sb.B, b.slist.p, b.scount.p, b.slittle.p, b.bfmask.p, st));
        BfSchedArgs sc{};
        sc.sa = sa;
        sc.Q = Q; sc.postfilter = 0xFFFFFFFFu; sc.counts = b.scount.p; sc.little = b.slittle.p;
        sc.lo = b.lo.p; sc.hi = b.hi.p; sc.nsub = b.nsub.p; sc.bcnt = b.bcnt.p; sc.bin = b.bin.p; sc.bstart = b.bstart.p;
        sc.bq = b.bq.p; sc.qcap = b.qcap; sc.ok = tot + 3; sc.nbf = tot + 9; sc.bfm = b.bfmask.p; sc.bP = sb.B;
        sc.qlist = b.sched.p; sc.qrange = tot + 14;
        // a batch holds few, small sub-cells: items of kStreamTileChunk tiles
        // give the persistent kernel enough of them to fill the GPU
        sc.tch = kStreamTileChunk;
        GF_HIP(launch_bf_reset(Q, b.nsub.p, b.pcnt.p, b.gbound.p, st));
        if (sb.NS) {
            GF_HIP(launch_bfsched(sc, false, st));
            if (!b.qcap) GF_HIP(launch_scan_small(b.bcnt.p, sb.NS, b.bstart.p, st));
        }
        GF_HIP(launch_scan_small(b.nsub.p, Q, b.part_off.p, st));
        GF_HIP(launch_total(b.nsub.p, b.part_off.p, Q, uint32_t(std::min<size_t>(b.pair_cap, UINT32_MAX)), K, b.part.n,
                            tot + 2, st));
        GF_HIP(hipMemsetAsync(tot + 4, 0, sizeof(uint32_t), st));
        if (sb.NS) {
            if (!b.qcap) GF_HIP(launch_bfsched(sc, true, st));
            GF_HIP(launch_bfitems(b.bcnt.p, b.bin.p, b.bstart.p, b.qcap, sa.stile, kStreamTileChunk, sb.NS, b.icnt.p,
                                  b.ioff.p, b.items.p, tot + 4, tot + 3, false, st));
            GF_HIP(launch_scan_small(b.icnt.p, sb.NS, b.ioff.p, st));
            GF_HIP(launch_bfitems(b.bcnt.p, b.bin.p, b.bstart.p, b.qcap, sa.stile, kStreamTileChunk, sb.NS, b.icnt.p,
                                  b.ioff.p, b.items.p, tot + 4, tot + 3, true, st));
        }
        BfGemmArgs ga{};
        ga.sa = sa;
        ga.rec = S.trec.p; ga.q8 = b.q8.p; ga.nq = b.nq.p; ga.lo = b.lo.p; ga.hi = b.hi.p;
        ga.items = b.items.p; ga.nitems = tot + 4; ga.bq = b.bq.p; ga.pcnt = b.pcnt.p; ga.part_off = b.part_off.p;
        ga.part = b.part.p; ga.gbound = b.gbound.p; ga.ok = tot + 3; ga.K = K; ga.D = ix.D;
        GF_HIP(hipEventRecord(ge[2 * bi], st));
        GF_HIP(launch_bf_i8(ga, uint32_t(std::max(ix.ncu, 1)), st));
        GF_HIP(hipEventRecord(ge[2 * bi + 1], st));
        BfFinalArgs fa{};
        fa.gbound = b.gbound.p; fa.bfq = b.sched.p; fa.srange = tot + 14; fa.part_off = b.part_off.p; fa.pcnt = b.pcnt.p; fa.ok = tot + 3;
        fa.part = b.part.p; fa.counts = b.scount.p; fa.cells = b.slist.p;
        fa.offset = reinterpret_cast<const uint32_t*>(dev + sb.o_offset); fa.selcount = b.selcount.p;
        fa.gidx = reinterpret_cast<const uint32_t*>(dev + sb.o_gidx); fa.out_ids = b.s_ids.p;
        fa.out_dist = b.s_dist.p; fa.counters = b.s_ctr.p; fa.K = K; fa.P = sb.B;
        GF_HIP(launch_bf_final(fa, Q, st));
        GF_HIP(launch_note_bf(tot, b.note.p + 2 * bi, st));
    };

    // A batch's image from the arena and the plan's header block, on the
    // copy stream: DMA for the large pieces, then one k_stream_gather for the
    // rest; the pieces the MFMA brute force reads (kCopyCore), and the
    // attributes (kCopyAttrs, the gather brute force), and the graph and
    // cross edges (kCopyAll, the traversal).
    double bytes = 0.0;
    auto enqueue_copy = [&](size_t bi, int t, int what) {
        const StreamBatch& sb = pl.batches[bi];
        hipStream_t cs = S.copy;
        GF_HIP(hipStreamWaitEvent(cs, S.freed[t], 0));
        GF_HIP(hipEventRecord(ce[5 * bi], cs));
        for (uint32_t k = 0; k < sb.ndma[what]; ++k) {
            const StreamCopy& c = pl.dma[sb.dma0 + k];
            GF_HIP(hipMemcpyAsync(S.turn[t].p + c.dst, S.host.p + c.src, c.bytes, hipMemcpyHostToDevice, cs));
        }
        GF_HIP(launch_stream_gather(pl.desc.p + sb.desc0, sb.ndesc[what], S.host.p, pl.head.p, S.turn[t].p, cs));
        bytes += double(sb.moved[what]);
        GF_HIP(hipEventRecord(ce[5 * bi + 1], cs));
        GF_HIP(hipEventRecord(S.ready[t], cs));
    };
    // One batch on the compute stream: its cell lists and routes, the
    // traversal (unless skipped), the brute force, the merge.
    auto enqueue_compute = [&](size_t bi, int t, bool traverse, bool first) {
        const StreamBatch& sb = pl.batches[bi];
        char* dev = S.turn[t].p;
        GF_HIP(hipStreamWaitEvent(st, S.ready[t], 0));
        const uint32_t* bcell = reinterpret_cast<const uint32_t*>(dev + sb.o_bcell);
        GF_HIP(launch_stream_lists(Q, P, sb.B, bcell, b.flags.p, b.slist.p, b.scount.p, b.slittle.p, st));
        SchedArgs sa{};
        sa.Q = Q; sa.P = sb.B; sa.postfilter = 0xFFFFFFFFu; sa.counts = b.scount.p; sa.little = b.slittle.p;
        sa.sched = b.sched.p; sa.tot = tot + 8; sa.ranges = tot + 12;
        GF_HIP(launch_sched(sa, st));
        GF_HIP(launch_reset_results(Q, K, b.s_ids.p, b.s_dist.p, b.s_ctr.p, st));
        TravArgs at = base;
        at.vec = dev + sb.o_vec;
        at.graph = reinterpret_cast<const uint32_t*>(dev + sb.o_graph);
        at.attrs = reinterpret_cast<const float*>(dev + sb.o_attrs);
        at.gidx = reinterpret_cast<const uint32_t*>(dev + sb.o_gidx);
        at.lrow = reinterpret_cast<const uint32_t*>(dev + sb.o_lrow);
        at.cross = reinterpret_cast<const uint32_t*>(dev + sb.o_cross);
        at.xrow = ix.E;
        at.xcell = uint64_t(sb.rows) * ix.E;
        at.offset = reinterpret_cast<const uint32_t*>(dev + sb.o_offset);
        at.P = sb.B;
        at.srange = tot + 12;
        GF_HIP(hipEventRecord(ce[5 * bi + 2], st));
        if (traverse) GF_HIP(launch_traverse(ix.rs, at, lds, Q, st));
        GF_HIP(hipEventRecord(ce[5 * bi + 3], st));
        if (gemm) {
            mfma_bruteforce(bi, sb, dev);
        } else {
            TravArgs ab = at;
            ab.srange = tot + 14;
            GF_HIP(launch_bruteforce(ix.rs, ab, Q, st));
        }
        GF_HIP(hipEventRecord(ce[5 * bi + 4], st));
        GF_HIP(launch_merge_stream(Q, K, b.out_ids.p, b.out_dist.p, b.s_ids.p, b.s_dist.p, b.counters.p, b.s_ctr.p,
                                   first, st));
        GF_HIP(hipEventRecord(S.freed[t], st));
    };

    GF_HIP(hipEventRecord(t0, st));
    // Which batches this query batch needs, and which prefix of each image:
    // skipped batches cost nothing; a batch no query traverses moves only
    // its brute-force sections.
    if (b.need.n < 2 * std::max<size_t>(nb, 1)) b.need.alloc(2 * std::max<size_t>(nb, 1));
    GF_HIP(launch_batch_need(Q, P, uint32_t(nb), pl.plan_cells.p, pl.plan_off.p, b.flags.p, b.need.p, st));
    std::vector<uint32_t> need(2 * nb, 0);   // flags, then active queries per batch
    if (nb) {
        GF_HIP(hipMemcpyAsync(need.data(), b.need.p, 2 * nb * 4, hipMemcpyDeviceToHost, st));
        GF_HIP(hipStreamSynchronize(st));
    }
    if (gemm) {
        GF_HIP(hipMemsetAsync(b.note.p, 0xFF, 2 * nb * sizeof(uint32_t), st));
        // the MFMA route does not count passing points on a streamed batch:
        // its PASS counter stays 0
        GF_HIP(hipMemsetAsync(b.selcount.p, 0, size_t(Q) * sizeof(uint32_t), st));
    }
    // The copy stream starts after everything queued so far on the compute
    // stream (flags, entries): a turn buffer is never in use at this point.
    GF_HIP(hipEventRecord(S.freed[0], st));
    GF_HIP(hipEventRecord(S.freed[1], st));
    std::vector<size_t> ran;
    for (size_t bi = 0; bi < nb; ++bi) {
        if (!need[bi]) continue;
        const bool trav = (need[bi] & 2u) != 0;
        const int t = int(ran.size() & 1);
        enqueue_copy(bi, t, trav ? kCopyAll : (gemm ? kCopyCore : kCopyAttrs));
        enqueue_compute(bi, t, trav, ran.empty());
        ran.push_back(bi);
    }
    if (ran.empty()) {
        GF_HIP(launch_fill_results(b.out_ids.p, b.out_dist.p, Q * K, st));
        GF_HIP(hipMemsetAsync(b.counters.p, 0, size_t(Q) * GF_NCOUNTERS * sizeof(uint32_t), st));
    }
    if (gemm && !ran.empty()) {
        // A batch whose brute-force pairs outgrew the buffers skipped its
        // brute force (its routed queries merged no result): grow the
        // buffers and run the brute force of those batches again.
        GF_HIP(hipStreamSynchronize(st));
        std::vector<uint32_t> note(2 * nb);
        GF_HIP(hipMemcpy(note.data(), b.note.p, note.size() * 4, hipMemcpyDeviceToHost));
        size_t need = 0;
        for (size_t bi = 0; bi < nb; ++bi)
            if (!note[2 * bi]) need = std::max<size_t>(need, note[2 * bi + 1]);
        if (need) {
            const uint32_t NS = std::max(pl.NSmax, 1u);
            b.alloc_pairs(need + need / 4 + 1024, K, Q, NS, pl.tmax / kStreamTileChunk + NS);
            for (size_t bi = 0; bi < nb; ++bi)
                if (!note[2 * bi]) {
                    enqueue_copy(bi, 0, kCopyCore);
                    enqueue_compute(bi, 0, false, false);
                }
            GF_HIP(hipStreamSynchronize(st));
            GF_HIP(hipMemcpy(note.data(), b.note.p, note.size() * 4, hipMemcpyDeviceToHost));
            for (size_t bi = 0; bi < nb; ++bi)
                GF_REQUIRE(note[2 * bi], GF_E_STATE, "brute-force schedule does not fit after growing");
        }
    }
    GF_HIP(hipEventRecord(t1, st));
    GF_HIP(hipEventSynchronize(t1));
    GF_HIP(hipStreamSynchronize(S.copy));

    GF_HIP(hipMemcpy(ids, b.out_ids.p, size_t(Q) * K * sizeof(uint32_t), hipMemcpyDeviceToHost));
    if (dists) GF_HIP(hipMemcpy(dists, b.out_dist.p, size_t(Q) * K * sizeof(float), hipMemcpyDeviceToHost));
    if (stats) {
        float ms = 0.0f;
        GF_HIP(hipEventElapsedTime(&ms, t0, t1));
        double h2d = 0.0, tr = 0.0, bf = 0.0;
        for (size_t bi : ran) {
            float c = 0.0f, t = 0.0f, f = 0.0f;
            GF_HIP(hipEventElapsedTime(&c, ce[5 * bi], ce[5 * bi + 1]));
            GF_HIP(hipEventElapsedTime(&t, ce[5 * bi + 2], ce[5 * bi + 3]));
            GF_HIP(hipEventElapsedTime(&f, ce[5 * bi + 3], ce[5 * bi + 4]));
            h2d += c;
            tr += t;
            bf += f;
        }
        std::vector<uint32_t> ctr(size_t(Q) * GF_NCOUNTERS);
        GF_HIP(hipMemcpy(ctr.data(), b.counters.p, ctr.size() * 4, hipMemcpyDeviceToHost));
        std::memset(stats, 0, sizeof(*stats));
        double g = 0.0;
        if (gemm)
            for (size_t bi : ran) {
                float x = 0.0f;
                GF_HIP(hipEventElapsedTime(&x, ge[2 * bi], ge[2 * bi + 1]));
                g += x;
            }
        stats->ms_total = ms;
        stats->ms_traverse = tr;
        stats->ms_bruteforce = bf;
        stats->ms_bf_kernel = g;
        stats->bf_mfma = gemm ? 1u : 0u;
        stats->n_batches = uint32_t(ran.size());
        for (size_t bi : ran) stats->n_active += need[nb + bi];
        stats->bytes_h2d = bytes;
        stats->ms_h2d = h2d;
        uint64_t sum[GF_NCOUNTERS] = {0};
        double t_dist = 0.0, b_dist = 0.0;
        for (uint32_t q = 0; q < Q; ++q) {
            const uint32_t* c = &ctr[size_t(q) * GF_NCOUNTERS];
            for (uint32_t k = 0; k < 7; ++k) sum[k] += c[k];
            stats->q_traverse += (c[7] & 0xFFFFu) ? 1 : 0;
            stats->q_bruteforce += (c[7] >> 16) ? 1 : 0;
            stats->q_empty += c[7] ? 0 : 1;
            // the brute force's distances are its passing points (gather) or
            // its scanned points (MFMA); the rest are traversal's
            const double bd = gemm ? double(c[5]) : double(c[6]);
            t_dist += double(c[1]) - bd;
            b_dist += bd;
        }
        stats->n_expand = sum[0]; stats->n_dist = sum[1]; stats->n_attr = sum[2]; stats->n_cross = sum[3];
        stats->n_lrow = sum[4]; stats->n_scan = sum[5]; stats->n_pass = sum[6];
        stats->bytes_traverse = t_dist * ix.rowbytes + double(sum[0]) * R * 4.0 + double(sum[2]) * ix.a * 4.0 +
                                double(sum[3]) * ix.E * 4.0 + double(sum[4]) * (base.offl ? 0.0 : 4.0);
        stats->bytes_bruteforce = double(sum[5]) * ix.a * 4.0 + b_dist * ix.rowbytes;
        stats->ops_bruteforce = 3.0 * b_dist * ix.D;
    }
}

}  // namespace gf
