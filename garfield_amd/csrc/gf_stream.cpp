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
    GF_REQUIRE(ix.vdtype != GF_VEC_F16, GF_E_UNSUPPORTED, "a streamed index holds GF_VEC_F32 or GF_VEC_U8 vectors");
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
    size_t total = 0;
    for (const auto& cl : plan_cells) {
        StreamBatch sb;
        sb.B = uint32_t(cl.size());
        uint64_t rows = 0;
        for (uint32_t c : cl) rows += size[c];
        sb.rows = uint32_t(rows);
        sb.o_vec = 0;
        sb.o_graph = align_up(sb.o_vec + rows * ix.rowbytes);
        sb.o_attrs = align_up(sb.o_graph + rows * R * 4);
        sb.o_gidx = align_up(sb.o_attrs + rows * a * 4);
        sb.o_lrow = align_up(sb.o_gidx + rows * 4);
        sb.o_cross = align_up(sb.o_lrow + rows * 4);
        sb.o_offset = align_up(sb.o_cross + size_t(sb.B) * rows * E * 4);
        sb.o_bcell = align_up(sb.o_offset + (size_t(sb.B) + 1) * 4);
        sb.bytes = align_up(sb.o_bcell + size_t(sb.B) * 4);
        sb.host_off = total;
        total += sb.bytes;
        sx->max_bytes = std::max(sx->max_bytes, sb.bytes);
        sx->Bmax = std::max(sx->Bmax, sb.B);
        sx->batches.push_back(sb);
    }
    GF_REQUIRE(sx->budget == 0 || 2 * sx->max_bytes <= sx->budget, GF_E_UNSUPPORTED,
               "the largest batch needs 2 x " + std::to_string(sx->max_bytes) +
                   " device bytes, over the device budget of " + std::to_string(sx->budget));
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
    }

    GF_HIP(hipStreamCreateWithFlags(&ix.stream, hipStreamNonBlocking));
    GF_HIP(hipStreamCreateWithFlags(&sx->copy, hipStreamNonBlocking));
    for (int t = 0; t < 2; ++t) {
        GF_HIP(hipEventCreateWithFlags(&sx->ready[t], hipEventDisableTiming));
        GF_HIP(hipEventCreateWithFlags(&sx->freed[t], hipEventDisableTiming));
        sx->turn[t].alloc(sx->max_bytes);
    }
    GF_HIP(hipDeviceGetAttribute(&ix.ncu, hipDeviceAttributeMultiprocessorCount, ix.device));
    ix.offset.upload(ix.offset_h);
    ix.grid.upload(ix.grid_h);
    ix.sx = std::move(sx);
    (void)N;
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
    const uint32_t lds = Lpad * 8 + kXSlots * 8 + 128 * 4 + hsize * 4;
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
    base.Lpad = Lpad;
    uint32_t* tot = b.tot.p;

    const size_t nb = S.batches.size();
    std::vector<hipEvent_t> ce(2 * nb, nullptr);
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

    GF_HIP(hipEventRecord(t0, st));
    // The copy stream starts after everything queued so far on the compute
    // stream (flags, entries): a turn buffer is never in use at this point.
    GF_HIP(hipEventRecord(S.freed[0], st));
    GF_HIP(hipEventRecord(S.freed[1], st));
    double bytes = 0.0;
    for (size_t bi = 0; bi < nb; ++bi) {
        const StreamBatch& sb = S.batches[bi];
        const int t = int(bi & 1);
        char* dev = S.turn[t].p;
        GF_HIP(hipStreamWaitEvent(S.copy, S.freed[t], 0));
        GF_HIP(hipEventRecord(ce[2 * bi], S.copy));
        GF_HIP(hipMemcpyAsync(dev, S.host.p + sb.host_off, sb.bytes, hipMemcpyHostToDevice, S.copy));
        GF_HIP(hipEventRecord(ce[2 * bi + 1], S.copy));
        GF_HIP(hipEventRecord(S.ready[t], S.copy));
        bytes += double(sb.bytes);

        GF_HIP(hipStreamWaitEvent(st, S.ready[t], 0));
        const uint32_t* bcell = reinterpret_cast<const uint32_t*>(dev + sb.o_bcell);
        GF_HIP(launch_stream_lists(Q, P, sb.B, bcell, b.flags.p, b.slist.p, b.scount.p, b.slittle.p, st));
        SchedArgs sa{};
        sa.Q = Q; sa.P = sb.B; sa.postfilter = 0xFFFFFFFFu; sa.counts = b.scount.p; sa.little = b.slittle.p;
        sa.sched = b.sched.p; sa.tot = tot + 8; sa.ranges = tot + 12;
        GF_HIP(launch_sched(sa, st));
        GF_HIP(launch_fill_results(b.s_ids.p, b.s_dist.p, Q * K, st));
        GF_HIP(hipMemsetAsync(b.s_ctr.p, 0, size_t(Q) * GF_NCOUNTERS * sizeof(uint32_t), st));
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
        GF_HIP(launch_traverse(ix.rs, at, lds, Q, st));
        TravArgs ab = at;
        ab.srange = tot + 14;
        GF_HIP(launch_bruteforce(ix.rs, ab, Q, st));
        GF_HIP(launch_merge_stream(Q, K, b.out_ids.p, b.out_dist.p, b.s_ids.p, b.s_dist.p, b.counters.p, b.s_ctr.p,
                                   bi == 0, st));
        GF_HIP(hipEventRecord(S.freed[t], st));
    }
    if (nb == 0) {
        GF_HIP(launch_fill_results(b.out_ids.p, b.out_dist.p, Q * K, st));
        GF_HIP(hipMemsetAsync(b.counters.p, 0, size_t(Q) * GF_NCOUNTERS * sizeof(uint32_t), st));
    }
    GF_HIP(hipEventRecord(t1, st));
    GF_HIP(hipEventSynchronize(t1));
    GF_HIP(hipStreamSynchronize(S.copy));

    GF_HIP(hipMemcpy(ids, b.out_ids.p, size_t(Q) * K * sizeof(uint32_t), hipMemcpyDeviceToHost));
    if (dists) GF_HIP(hipMemcpy(dists, b.out_dist.p, size_t(Q) * K * sizeof(float), hipMemcpyDeviceToHost));
    if (stats) {
        float ms = 0.0f;
        GF_HIP(hipEventElapsedTime(&ms, t0, t1));
        double h2d = 0.0;
        for (size_t bi = 0; bi < nb; ++bi) {
            float c = 0.0f;
            GF_HIP(hipEventElapsedTime(&c, ce[2 * bi], ce[2 * bi + 1]));
            h2d += c;
        }
        std::vector<uint32_t> ctr(size_t(Q) * GF_NCOUNTERS);
        GF_HIP(hipMemcpy(ctr.data(), b.counters.p, ctr.size() * 4, hipMemcpyDeviceToHost));
        std::memset(stats, 0, sizeof(*stats));
        stats->ms_total = ms;
        stats->n_batches = uint32_t(nb);
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
            // brute-force distances equal the passing points; the rest are traversal's
            t_dist += double(c[1]) - double(c[6]);
            b_dist += double(c[6]);
        }
        stats->n_expand = sum[0]; stats->n_dist = sum[1]; stats->n_attr = sum[2]; stats->n_cross = sum[3];
        stats->n_lrow = sum[4]; stats->n_scan = sum[5]; stats->n_pass = sum[6];
        stats->bytes_traverse = t_dist * ix.rowbytes + double(sum[0]) * R * 4.0 + double(sum[2]) * ix.a * 4.0 +
                                double(sum[3]) * ix.E * 4.0 + double(sum[4]) * 4.0;
        stats->bytes_bruteforce = double(sum[5]) * ix.a * 4.0 + b_dist * ix.rowbytes;
        stats->ops_bruteforce = 3.0 * b_dist * ix.D;
    }
}

}  // namespace gf
