// Streamed (out-of-core) index and search: the reference's out-of-core
// scheduler batch_graph_search_gpu_with_prefilter_batch_process_compressed_graph_T_dataset_resident_u8
// (big_dataset_adapterV3.cuh:3719-4117), rebuilt around one packed pinned
// image per batch.
//
// The reference issues one cudaMemcpyAsync per cell graph and per (cell,
// cell') cross-edge slice of a batch (big_dataset_adapterV3.cuh:3925-3946),
// then serialises the pipeline with cudaDeviceSynchronize (:4010) and
// re-ranks L candidates per query on 9 host threads (:3741-3797).  Here the
// plan is fixed when the index is built, so each batch is packed once, at
// build time, into a contiguous image in pinned memory laid out as a small
// index of the batch's cells (gf_state.h, StreamBatch).  A search then moves
// each image with one hipMemcpyAsync on a side stream into one of two device
// buffers, while the compute stream searches the previous batch; events
// order buffer reuse, and no host synchronisation happens inside the loop.
// Distances are exact on the device (fp32 or u8 data), so the per-batch top
// K merges into a running top K on the device instead of a host re-rank.
#include <algorithm>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gf_state.h"

namespace gf {
namespace {

constexpr size_t kAlign = 256;
constexpr uint32_t kStreamTileChunk = 16;   // tiles per MFMA brute-force item on a streamed batch
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

uint32_t next_pow2(uint32_t x) {
    uint32_t p = 1;
    while (p < x) p <<= 1;
    return p;
}

}  // namespace

void build_streamed(const gf_index_host& h, const gf_open_opts* opts, const gf_stream_plan* plan, gf_index& ix) {
    GF_REQUIRE(plan, GF_E_ARG, "null stream plan");
    std::vector<uint32_t> size, gidx, lrow;
    map_cells(h, opts, ix, size, gidx, lrow);
    GF_REQUIRE(ix.vdtype != GF_VEC_F16 && ix.vdtype != GF_VEC_I8Q && ix.vdtype != GF_VEC_F16_REF, GF_E_UNSUPPORTED,
               "a streamed index holds GF_VEC_F32 or GF_VEC_U8 vectors");
    const uint32_t P = ix.P, R = ix.R, E = ix.E, a = ix.a, D = ix.D, N = ix.N;

    // The static plan: explicit batches, or consecutive cells.
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
        std::vector<char> seen(P, 0);
        size_t k = 0;
        for (uint32_t i = 0; i < plan->nbatch; ++i) {
            GF_REQUIRE(plan->sizes[i] >= 1, GF_E_ARG, "empty batch in the stream plan");
            std::vector<uint32_t> v;
            for (uint32_t j = 0; j < plan->sizes[i]; ++j, ++k) {
                const uint32_t c = plan->cells[k];
                GF_REQUIRE(c < P, GF_E_ARG, "stream plan cell id out of range");
                GF_REQUIRE(!seen[c], GF_E_ARG, "cell " + std::to_string(c) + " appears twice in the stream plan");
                seen[c] = 1;
                v.push_back(c);
            }
            plan_cells.push_back(v);
        }
    }

    std::unique_ptr<StreamIndex> sx(new StreamIndex());
    sx->budget = plan->device_budget;
    // Sub-cells for the MFMA brute force (u8 vectors, D a multiple of 64 up to 256).
    SubHost sh;
    sx->i8 = ix.vdtype == GF_VEC_U8 && D % 64 == 0 && D <= 256 &&
             compute_subcells(h, gidx, size, ix.offset_h, a, P, sh);
    sx->AW = sh.AW;
    const uint32_t MW = 16 * (1 + sh.AW);
    size_t total = 0;
    for (const auto& cl : plan_cells) {
        StreamBatch sb;
        sb.B = uint32_t(cl.size());
        uint64_t rows = 0;
        for (uint32_t c : cl) rows += size[c];
        sb.rows = uint32_t(rows);
        if (sx->i8)
            for (uint32_t c : cl) {
                sb.NS += sh.sbase[c + 1] - sh.sbase[c];
                sb.ntile += sh.stile[sh.sbase[c + 1]] - sh.stile[sh.sbase[c]];
            }
        sb.o_vec = 0;
        sb.o_gidx = align_up(sb.o_vec + rows * ix.rowbytes);
        sb.o_offset = align_up(sb.o_gidx + rows * 4);
        sb.o_bcell = align_up(sb.o_offset + (size_t(sb.B) + 1) * 4);
        size_t end = sb.o_bcell + size_t(sb.B) * 4;
        if (sx->i8) {
            sb.o_sbase = align_up(end);
            sb.o_scell = align_up(sb.o_sbase + (size_t(sb.B) + 1) * 4);
            sb.o_ssize = align_up(sb.o_scell + size_t(sb.NS) * 4);
            sb.o_stile = align_up(sb.o_ssize + size_t(sb.NS) * 4);
            sb.o_sbox = align_up(sb.o_stile + (size_t(sb.NS) + 1) * 4);
            sb.o_abase = align_up(sb.o_sbox + size_t(sb.NS) * 2 * a * 4);
            sb.o_tmeta = align_up(sb.o_abase + size_t(sb.B) * a * 4);
            end = sb.o_tmeta + size_t(sb.ntile) * MW * 4;
        }
        sb.bytes_mfma = align_up(end);
        sb.o_attrs = sb.bytes_mfma;
        sb.bytes_bf = align_up(sb.o_attrs + rows * a * 4);
        sb.o_graph = sb.bytes_bf;
        sb.o_lrow = align_up(sb.o_graph + rows * R * 4);
        sb.o_cross = align_up(sb.o_lrow + rows * 4);
        sb.bytes = align_up(sb.o_cross + size_t(sb.B) * rows * E * 4);
        sb.host_off = total;
        total += sb.bytes;
        sx->max_bytes = std::max(sx->max_bytes, sb.bytes);
        sx->Bmax = std::max(sx->Bmax, sb.B);
        sx->NSmax = std::max(sx->NSmax, sb.NS);
        sx->tmax = std::max(sx->tmax, sb.ntile);
        sx->batches.push_back(sb);
    }
    const size_t tile_bytes = size_t(D / 64) * 1024 + 32 * 4;
    const uint64_t need = 2 * uint64_t(sx->max_bytes) + (sx->i8 ? uint64_t(sx->tmax) * tile_bytes : 0);
    GF_REQUIRE(sx->budget == 0 || need <= sx->budget, GF_E_UNSUPPORTED,
               "the largest batch needs " + std::to_string(need) + " device bytes (two images" +
                   (sx->i8 ? std::string(" and its int8 tiles") : std::string()) + "), over the device budget of " +
                   std::to_string(sx->budget));
    sx->min_cell = 0;
    for (uint32_t c = 0; c < P; ++c)
        if (size[c] && (sx->min_cell == 0 || size[c] < sx->min_cell)) sx->min_cell = size[c];

    GF_HIP(hipSetDevice(ix.device));
    sx->host.alloc(total);
    // Pack the images.
    for (size_t bi = 0; bi < plan_cells.size(); ++bi) {
        const auto& cl = plan_cells[bi];
        const StreamBatch& sb = sx->batches[bi];
        char* img = sx->host.p + sb.host_off;
        std::memset(img, 0, sb.bytes);
        std::vector<uint32_t> boff(sb.B + 1, 0);
        for (uint32_t i = 0; i < sb.B; ++i) boff[i + 1] = boff[i] + size[cl[i]];
        uint32_t* g_graph = reinterpret_cast<uint32_t*>(img + sb.o_graph);
        float* g_attrs = reinterpret_cast<float*>(img + sb.o_attrs);
        uint32_t* g_gidx = reinterpret_cast<uint32_t*>(img + sb.o_gidx);
        uint32_t* g_lrow = reinterpret_cast<uint32_t*>(img + sb.o_lrow);
        uint32_t* g_cross = reinterpret_cast<uint32_t*>(img + sb.o_cross);
        for (uint32_t i = 0; i < sb.B; ++i) {
            const uint32_t c = cl[i], n = size[c], r0 = ix.offset_h[c];
            std::memcpy(g_graph + size_t(boff[i]) * R, h.cell_graphs + size_t(r0) * R, size_t(n) * R * 4);
            for (uint32_t l = 0; l < n; ++l) {
                const uint32_t r = boff[i] + l, pt = gidx[r0 + l];
                const float* x = h.vectors + size_t(pt) * D;
                if (ix.vdtype == GF_VEC_U8) {
                    uint8_t* y = reinterpret_cast<uint8_t*>(img + sb.o_vec) + size_t(r) * ix.rowbytes;
                    for (uint32_t j = 0; j < D; ++j) y[j] = uint8_t(x[j]);
                } else {
                    std::memcpy(img + sb.o_vec + size_t(r) * ix.rowbytes, x, size_t(D) * 4);
                }
                for (uint32_t d = 0; d < a; ++d) g_attrs[size_t(r) * a + d] = h.attrs[size_t(pt) * a + d];
                g_gidx[r] = pt;
                g_lrow[r] = l;
                for (uint32_t t = 0; t < sb.B; ++t)
                    for (uint32_t e = 0; e < E; ++e)
                        g_cross[(size_t(t) * sb.rows + r) * E + e] = h.cross[(size_t(pt) * P + cl[t]) * E + e];
            }
        }
        std::memcpy(img + sb.o_offset, boff.data(), boff.size() * 4);
        std::memcpy(img + sb.o_bcell, cl.data(), cl.size() * 4);
        if (sx->i8) {
            uint32_t* g_sbase = reinterpret_cast<uint32_t*>(img + sb.o_sbase);
            uint32_t* g_scell = reinterpret_cast<uint32_t*>(img + sb.o_scell);
            uint32_t* g_ssize = reinterpret_cast<uint32_t*>(img + sb.o_ssize);
            uint32_t* g_stile = reinterpret_cast<uint32_t*>(img + sb.o_stile);
            int32_t* g_sbox = reinterpret_cast<int32_t*>(img + sb.o_sbox);
            int32_t* g_abase = reinterpret_cast<int32_t*>(img + sb.o_abase);
            uint32_t* g_tmeta = reinterpret_cast<uint32_t*>(img + sb.o_tmeta);
            uint32_t ns = 0, nt = 0;
            for (uint32_t i = 0; i < sb.B; ++i) {
                const uint32_t c = cl[i];
                g_sbase[i] = ns;
                for (uint32_t d = 0; d < a; ++d) g_abase[size_t(i) * a + d] = sh.abase[size_t(c) * a + d];
                for (uint32_t s0 = sh.sbase[c]; s0 < sh.sbase[c + 1]; ++s0, ++ns) {
                    g_scell[ns] = i;
                    g_ssize[ns] = sh.ssize[s0];
                    g_stile[ns] = nt;
                    for (uint32_t k = 0; k < 2 * a; ++k) g_sbox[size_t(ns) * 2 * a + k] = sh.sbox[size_t(s0) * 2 * a + k];
                    for (uint32_t t = sh.stile[s0]; t < sh.stile[s0 + 1]; ++t, ++nt) {
                        const uint32_t* src = &sh.tmeta[size_t(t) * MW];
                        uint32_t* dst = g_tmeta + size_t(nt) * MW;
                        std::memcpy(dst, src, MW * 4);
                        for (uint32_t j = 0; j < 16; ++j)   // rows become batch rows
                            if (src[j] != 0xFFFFFFFFu) dst[j] = src[j] - ix.offset_h[c] + boff[i];
                    }
                }
            }
            g_sbase[sb.B] = ns;
            g_stile[ns] = nt;
        }
    }

    GF_HIP(hipStreamCreateWithFlags(&ix.stream, hipStreamNonBlocking));
    GF_HIP(hipStreamCreateWithFlags(&sx->copy, hipStreamNonBlocking));
    for (int t = 0; t < 2; ++t) {
        GF_HIP(hipEventCreateWithFlags(&sx->ready[t], hipEventDisableTiming));
        GF_HIP(hipEventCreateWithFlags(&sx->freed[t], hipEventDisableTiming));
        sx->turn[t].alloc(sx->max_bytes);
    }
    {
        std::vector<uint32_t> pc, po(1, 0);
        for (const auto& cl : plan_cells) {
            pc.insert(pc.end(), cl.begin(), cl.end());
            po.push_back(uint32_t(pc.size()));
        }
        if (pc.empty()) pc.push_back(0);
        sx->plan_cells.upload(pc);
        sx->plan_off.upload(po);
    }
    if (sx->i8) {
        sx->trec.alloc(size_t(std::max(sx->tmax, 1u)) * bf_rec_bytes(D, sx->AW));
        ix.i8 = true;   // gf_batch_create keeps int8 queries
    }
    GF_HIP(hipDeviceGetAttribute(&ix.ncu, hipDeviceAttributeMultiprocessorCount, ix.device));
    ix.offset.upload(ix.offset_h);
    ix.grid.upload(ix.grid_h);
    ix.sx = std::move(sx);
    (void)N;
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
namespace {

struct PlanBox {
    uint32_t x0[kMaxAttr], x1[kMaxAttr];
};

}  // namespace

uint64_t plan_cells(const uint32_t* cells, const uint32_t* counts, uint32_t Q, uint32_t a, const uint32_t* grid,
                    const uint32_t* cell_size, uint64_t max_points, uint32_t max_cells,
                    std::vector<std::vector<uint32_t>>& plan) {
    GF_REQUIRE(a >= 1 && a <= kMaxAttr, GF_E_ARG, "plan_cells: attribute count out of range");
    uint64_t P = 1, nbox = 1;
    uint32_t stride[kMaxAttr], bstride[kMaxAttr];
    for (uint32_t d = 0; d < a; ++d) {
        GF_REQUIRE(grid[d] >= 1, GF_E_ARG, "plan_cells: empty grid axis");
        P *= grid[d];
        nbox *= uint64_t(grid[d]) * grid[d];
        GF_REQUIRE(nbox <= (uint64_t(1) << 22), GF_E_UNSUPPORTED, "plan_cells: grid too large to plan (more than 2^22 box slots)");
    }
    for (int d = int(a) - 1, s = 1, bs = 1; d >= 0; --d) {
        stride[d] = uint32_t(s);
        bstride[d] = uint32_t(bs);
        s *= int(grid[d]);
        bs *= int(grid[d] * grid[d]);
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
    const size_t Qb = qlo.size() / a;
    // cut(X, d, t).  Two attributes: per (d, t) a table over the other
    // axis' [x0, x1] of the straddling queries whose interval meets it
    // (prefix sums of a (lo, hi) histogram); one attribute: the straddle
    // count; more: a scan of the straddling queries.
    std::vector<std::vector<std::vector<uint32_t>>> strad(a);   // [d][t] query indices
    std::vector<std::vector<std::vector<uint64_t>>> tab(a);     // [d][t] table (a <= 2)
    for (uint32_t d = 0; d < a; ++d) {
        strad[d].resize(grid[d]);
        tab[d].resize(grid[d]);
        for (size_t q = 0; q < Qb; ++q)
            for (uint32_t t = qlo[q * a + d] + 1; t <= qhi[q * a + d]; ++t) strad[d][t].push_back(uint32_t(q));
        if (a > 2) continue;
        const uint32_t e = 1 - d, ge = a == 2 ? grid[e] : 1;
        for (uint32_t t = 1; t < grid[d]; ++t) {
            std::vector<uint64_t> h(size_t(ge) * ge, 0), T(size_t(ge) * ge, 0);
            for (uint32_t q : strad[d][t]) {
                if (a == 2) ++h[size_t(qlo[q * a + e]) * ge + qhi[q * a + e]];
                else ++h[0];
            }
            // T[x0 * ge + x1] = #{lo <= x1, hi >= x0}
            for (uint32_t x0 = 0; x0 < ge; ++x0)
                for (uint32_t x1 = x0; x1 < ge; ++x1) {
                    uint64_t n = 0;
                    for (uint32_t lo = 0; lo <= x1; ++lo)
                        for (uint32_t hi = std::max(lo, x0); hi < ge; ++hi) n += h[size_t(lo) * ge + hi];
                    T[size_t(x0) * ge + x1] = n;
                }
            tab[d][t] = std::move(T);
        }
    }
    auto cut = [&](const PlanBox& X, uint32_t d, uint32_t t) -> uint64_t {
        if (a == 1) return tab[d][t][0];
        if (a == 2) {
            const uint32_t e = 1 - d;
            return tab[d][t][size_t(X.x0[e]) * grid[e] + X.x1[e]];
        }
        uint64_t n = 0;
        for (uint32_t q : strad[d][t]) {
            bool meets = true;
            for (uint32_t e = 0; e < a && meets; ++e)
                if (e != d) meets = qlo[q * a + e] <= X.x1[e] && qhi[q * a + e] >= X.x0[e];
            n += meets;
        }
        return n;
    };
    auto index = [&](const PlanBox& X) {
        size_t i = 0;
        for (uint32_t d = 0; d < a; ++d) i += size_t(X.x0[d] * grid[d] + X.x1[d]) * bstride[d];
        return i;
    };
    // Every box, smaller extents first (both parts of a cut come before it).
    std::vector<PlanBox> boxes;
    {
        PlanBox X{};
        std::vector<uint32_t> pos(a, 0);   // enumerate (x0, x1) pairs per axis
        std::vector<std::vector<std::pair<uint32_t, uint32_t>>> iv(a);
        for (uint32_t d = 0; d < a; ++d)
            for (uint32_t x0 = 0; x0 < grid[d]; ++x0)
                for (uint32_t x1 = x0; x1 < grid[d]; ++x1) iv[d].push_back({x0, x1});
        for (;;) {
            for (uint32_t d = 0; d < a; ++d) { X.x0[d] = iv[d][pos[d]].first; X.x1[d] = iv[d][pos[d]].second; }
            boxes.push_back(X);
            uint32_t d = 0;
            while (d < a && ++pos[d] == iv[d].size()) pos[d++] = 0;
            if (d == a) break;
        }
        auto ext = [&](const PlanBox& B) {
            uint32_t s = 0;
            for (uint32_t d = 0; d < a; ++d) s += B.x1[d] - B.x0[d];
            return s;
        };
        std::stable_sort(boxes.begin(), boxes.end(), [&](const PlanBox& u, const PlanBox& v) { return ext(u) < ext(v); });
    }
    std::vector<uint64_t> cost(nbox, 0), npts(nbox, 0);
    std::vector<uint32_t> nleaf(nbox, 0), ncell(nbox, 0), split(nbox, 0);   // split: 0 = leaf, else d * 65536 + t
    auto halves = [&](const PlanBox& X, uint32_t d, uint32_t t, PlanBox& A, PlanBox& B) {
        A = X;
        B = X;
        A.x1[d] = t - 1;
        B.x0[d] = t;
    };
    for (const PlanBox& X : boxes) {
        const size_t i = index(X);
        uint32_t d0 = a;
        for (uint32_t d = 0; d < a; ++d)
            if (X.x1[d] > X.x0[d]) { d0 = d; break; }
        if (d0 == a) {   // one cell
            uint32_t c = 0;
            for (uint32_t d = 0; d < a; ++d) c += X.x0[d] * stride[d];
            npts[i] = cell_size[c];
            ncell[i] = cell_size[c] ? 1u : 0u;
            nleaf[i] = ncell[i];
            continue;
        }
        PlanBox A, B;
        halves(X, d0, X.x0[d0] + 1, A, B);
        npts[i] = npts[index(A)] + npts[index(B)];
        ncell[i] = ncell[index(A)] + ncell[index(B)];
        if ((max_cells == 0 || ncell[i] <= max_cells) && (max_points == 0 || npts[i] <= max_points)) {
            nleaf[i] = ncell[i] ? 1u : 0u;
            continue;
        }
        bool have = false;
        for (uint32_t d = 0; d < a; ++d)
            for (uint32_t t = X.x0[d] + 1; t <= X.x1[d]; ++t) {
                halves(X, d, t, A, B);
                const size_t ia = index(A), ib = index(B);
                const uint64_t c = cut(X, d, t) + cost[ia] + cost[ib];
                const uint32_t l = nleaf[ia] + nleaf[ib];
                if (!have || c < cost[i] || (c == cost[i] && l < nleaf[i])) {
                    have = true;
                    cost[i] = c;
                    nleaf[i] = l;
                    split[i] = d * 65536u + t;
                }
            }
    }
    plan.clear();
    std::vector<PlanBox> stack;
    PlanBox all{};
    for (uint32_t d = 0; d < a; ++d) { all.x0[d] = 0; all.x1[d] = grid[d] - 1; }
    stack.push_back(all);
    while (!stack.empty()) {
        const PlanBox X = stack.back();
        stack.pop_back();
        const size_t i = index(X);
        if (split[i]) {
            PlanBox A, B;
            halves(X, split[i] / 65536u, split[i] % 65536u, A, B);
            stack.push_back(B);   // lower part first
            stack.push_back(A);
            continue;
        }
        std::vector<uint32_t> batch;
        for (uint32_t c = 0; c < P; ++c) {
            bool in = cell_size[c] > 0;
            for (uint32_t d = 0; d < a && in; ++d) {
                const uint32_t x = c / stride[d] % grid[d];
                in = x >= X.x0[d] && x <= X.x1[d];
            }
            if (in) batch.push_back(c);
        }
        if (!batch.empty()) plan.push_back(std::move(batch));
    }
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

void stream_search(gf_batch& b, const gf_search_opts& o, uint32_t* ids, float* dists, gf_search_stats* stats) {
    gf_index& ix = *b.ix;
    StreamIndex& S = *ix.sx;
    const uint32_t Q = b.Q, K = o.K, L = o.L, R = ix.R, P = ix.P, Bm = std::max<uint32_t>(S.Bmax, 1u);
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

    const uint32_t hsize = std::max<uint32_t>(256, next_pow2(2 * (L + kXSlots + 4 * R)));
    uint32_t hbits = 0;
    while ((1u << hbits) < hsize) ++hbits;
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
    base.hbits = hbits;
    base.offl = trav_offsets_in_lds(Bm) ? 1u : 0u;   // lds holds Bm + 1 >= B + 1 offsets
    base.Lpad = Lpad;
    uint32_t* tot = b.tot.p;

    const size_t nb = S.batches.size();
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
        const uint32_t NS = std::max(S.NSmax, 1u);
        if (b.bcnt.n < NS) { b.bcnt.alloc(NS); b.bin.alloc(NS); b.bstart.alloc(NS); b.icnt.alloc(NS); b.ioff.alloc(NS); }
        if (b.nsub.n < Q) { b.nsub.alloc(Q); b.part_off.alloc(Q); b.pcnt.alloc(Q); b.gbound.alloc(Q); }
        // items <= pairs x chunks / 64 + (sub-cell, chunk) slots (k_bfitems)
        if (!b.part.n) b.alloc_pairs(size_t(Q) * 64, K, Q, NS, S.tmax / kStreamTileChunk + NS);
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

    double bytes = 0.0;
    auto enqueue_copy = [&](size_t bi, int t, size_t nbytes) {
        const StreamBatch& sb = S.batches[bi];
        GF_HIP(hipStreamWaitEvent(S.copy, S.freed[t], 0));
        GF_HIP(hipEventRecord(ce[5 * bi], S.copy));
        GF_HIP(hipMemcpyAsync(S.turn[t].p, S.host.p + sb.host_off, nbytes, hipMemcpyHostToDevice, S.copy));
        GF_HIP(hipEventRecord(ce[5 * bi + 1], S.copy));
        GF_HIP(hipEventRecord(S.ready[t], S.copy));
        bytes += double(nbytes);
    };
    // One batch on the compute stream: its cell lists and routes, the
    // traversal (unless skipped), the brute force, the merge.
    auto enqueue_compute = [&](size_t bi, int t, bool traverse, bool first) {
        const StreamBatch& sb = S.batches[bi];
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
    GF_HIP(launch_batch_need(Q, P, uint32_t(nb), S.plan_cells.p, S.plan_off.p, b.flags.p, b.need.p, st));
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
        const StreamBatch& sb = S.batches[bi];
        const bool trav = (need[bi] & 2u) != 0;
        const int t = int(ran.size() & 1);
        enqueue_copy(bi, t, trav ? sb.bytes : (gemm ? sb.bytes_mfma : sb.bytes_bf));
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
            const uint32_t NS = std::max(S.NSmax, 1u);
            b.alloc_pairs(need + need / 4 + 1024, K, Q, NS, S.tmax / kStreamTileChunk + NS);
            for (size_t bi = 0; bi < nb; ++bi)
                if (!note[2 * bi]) {
                    enqueue_copy(bi, 0, S.batches[bi].bytes_mfma);
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
