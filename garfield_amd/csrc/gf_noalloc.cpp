// gf_search_noalloc: one query batch through stages A, B and C without any
// allocation.  It runs the kernels of gf_batch_create + gf_mark_cells +
// gf_order_cells + gf_search (traversal, and the gather brute force for the
// routed queries), with every buffer those calls allocate per batch taken
// from `scratch`, a file-scope device array of kScratchBytes that each GPU
// holds from the library's load until the process ends.
//
// Host code never uses the array's name as a device address (in host code it
// names a host-side stand-in): the address of each device's copy comes from
// hipGetSymbolAddress, once per device, on the first call there.
//
// Calls on one device share its array and keep the last call's contents:
// everything a call reads before writing is cleared by a fill kernel, and two
// calls that overlap on one device race (the caller serialises them, as every
// call on one gf_index).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>

#include "gf_state.h"

namespace {

constexpr size_t kScratchBytes = size_t(GF_NOALLOC_SCRATCH_MB) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on `device` (made current by the caller).
void* scratch_ptr(int device) {
    GF_REQUIRE(device >= 0 && device < kMaxDevices, GF_E_ARG, "device ordinal out of range");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            throw gf::Error{GF_E_DEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e)};
        g_scratch[device] = p;
    }
    return g_scratch[device];
}

// Bump carving of the scratch array: 256-byte aligned sections.
struct Carve {
    char* base;
    size_t used = 0;
    template <typename T>
    T* take(size_t count) {
        T* p = reinterpret_cast<T*>(base + used);
        used += (count * sizeof(T) + 255) / 256 * 256;
        return p;
    }
};


}  // namespace

extern "C" gf_status gf_search_noalloc(gf_index* ix, const float* queries, uint32_t Q, const float* lo,
                                       const float* hi, const gf_noalloc_opts* o, uint32_t* ids, float* dists) {
    try {
        GF_REQUIRE(ix && queries && lo && hi && o && ids, GF_E_ARG, "null argument");
        GF_REQUIRE(Q > 0, GF_E_ARG, "empty batch");
        GF_REQUIRE(!ix->sx, GF_E_UNSUPPORTED, "gf_search_noalloc needs a resident index");
        GF_REQUIRE(ix->vdtype != GF_VEC_I8Q, GF_E_UNSUPPORTED, "gf_search_noalloc does not take GF_VEC_I8Q indexes");
        const gf_search_opts& so = o->search;
        const uint32_t L = so.L, K = so.K, rl = so.rl, R = ix->R, P = ix->P, a = ix->a, D = ix->D;
        GF_REQUIRE(L >= 1 && L < (1u << 16), GF_E_ARG, "L must be in [1, 65535]");
        GF_REQUIRE(K >= 1 && K <= 64, GF_E_ARG, "K must be in [1, 64]");
        GF_REQUIRE(rl >= 1 && rl <= 16, GF_E_ARG, "rl must be in [1, 16]");
        GF_REQUIRE(!ix->C || (o->topc >= 1 && o->topc <= 4), GF_E_ARG, "topc must be in [1, 4]");
        GF_REQUIRE(so.entry_points || ix->entry_ref.n == R, GF_E_ARG,
                   "the index has no room for the reference's entry-point draw: pass entry_points");
        const uint32_t hsize = gf::visited_slots(L + gf::kXSlots + 4 * R);
        const uint32_t Lpad = gf::round_up(L, 2);
        const uint32_t lds = gf::trav_lds_bytes(Lpad, hsize, ix->P);
        GF_REQUIRE(lds <= 64 * 1024, GF_E_UNSUPPORTED, "L too large for the LDS budget");

        // Sections, in the order gf_batch_create and the stage calls make them.
        const uint32_t Qp = gf::round_up(Q, 16);
        Carve cv{nullptr};
        auto layout = [&](Carve& c) {
            struct {
                float *qf32, *lo, *hi, *qnorm, *out_dist;
                uint16_t *q16v, *q16;
                uint32_t *cells, *counts, *little, *selcount, *cellq, *ccount, *cstart, *cfill, *topk, *sched,
                    *tot, *entry, *out_ids, *counters;
            } s{};
            s.qf32 = c.take<float>(size_t(Q) * D);
            s.lo = c.take<float>(size_t(Q) * a);
            s.hi = c.take<float>(size_t(Q) * a);
            if (gf::half_rows(ix->vdtype)) s.q16v = c.take<uint16_t>(size_t(Q) * D);
            if (ix->C) {
                s.q16 = c.take<uint16_t>(size_t(Qp) * ix->Dp);
                s.qnorm = c.take<float>(Qp);
                s.topk = c.take<uint32_t>(size_t(Q) * 4);
            }
            s.cells = c.take<uint32_t>(size_t(Q) * P);
            s.counts = c.take<uint32_t>(Q);
            s.little = c.take<uint32_t>(Q);
            s.selcount = c.take<uint32_t>(Q);
            if (!ix->sub) {
                s.cellq = c.take<uint32_t>(size_t(Q) * P);
                s.ccount = c.take<uint32_t>(P);
                s.cstart = c.take<uint32_t>(P);
                s.cfill = c.take<uint32_t>(P);
            }
            s.sched = c.take<uint32_t>(Q);
            s.tot = c.take<uint32_t>(24);
            s.entry = c.take<uint32_t>(R);
            s.out_ids = c.take<uint32_t>(size_t(Q) * K);
            s.out_dist = c.take<float>(size_t(Q) * K);
            s.counters = c.take<uint32_t>(size_t(Q) * GF_NCOUNTERS);
            return s;
        };
        {
            Carve probe{nullptr};
            (void)layout(probe);
            GF_REQUIRE(probe.used <= kScratchBytes, GF_E_UNSUPPORTED,
                       "batch needs " + std::to_string(probe.used) + " bytes of scratch, more than the " +
                           std::to_string(kScratchBytes) + " of gf_search_noalloc: use fewer queries");
        }
        GF_HIP(hipSetDevice(ix->device));
        cv.base = static_cast<char*>(scratch_ptr(ix->device));
        const auto s = layout(cv);
        hipStream_t st = ix->stream;

        // gf_batch_create: queries, ranges and their converted copies.
        GF_HIP(hipMemcpyAsync(s.qf32, queries, size_t(Q) * D * 4, hipMemcpyHostToDevice, st));
        GF_HIP(hipMemcpyAsync(s.lo, lo, size_t(Q) * a * 4, hipMemcpyHostToDevice, st));
        GF_HIP(hipMemcpyAsync(s.hi, hi, size_t(Q) * a * 4, hipMemcpyHostToDevice, st));
        if (s.q16v) GF_HIP(gf::launch_f2h(s.qf32, s.q16v, size_t(Q) * D, ix->alpha, st));
        if (ix->C) {
            GF_HIP(gf::launch_f2h_pad(s.qf32, Q, D, s.q16, Qp, ix->Dp, ix->alpha, st));
            GF_HIP(gf::launch_norms_f16(s.q16, Qp, ix->Dp, ix->Dp, s.qnorm, st));
        }

        // Stage A (gf_mark_cells).
        GF_HIP(gf::launch_cells(Q, a, s.lo, s.hi, ix->grid.p, ix->doff.p, ix->l_q.p, ix->r_q.p, P, ix->offset.p,
                                s.cells, s.counts, st));
        GF_HIP(gf::launch_zero_u32(s.selcount, Q, st));
        if (o->prefilter < 1.0f) {
            if (ix->sub) {
                gf::SubSelArgs sl{};
                sl.sa.sbase = ix->sbase.p; sl.sa.scell = ix->scell.p; sl.sa.ssize = ix->ssize.p;
                sl.sa.stile = ix->stile.p; sl.sa.sbox = ix->sbox.p; sl.sa.tmeta = ix->tmeta.p;
                sl.sa.abase = ix->abase.p; sl.sa.a = a; sl.sa.AW = ix->AW; sl.sa.P = P; sl.sa.NS = ix->NS;
                sl.Q = Q; sl.lo = s.lo; sl.hi = s.hi; sl.selcount = s.selcount;
                GF_HIP(gf::launch_subsel(sl, st));
            } else {
                GF_HIP(gf::launch_zero_u32(s.ccount, P, st));
                GF_HIP(gf::launch_zero_u32(s.cfill, P, st));
                GF_HIP(gf::launch_cellq_count(Q, P, s.cells, s.counts, s.ccount, st));
                GF_HIP(gf::launch_scan_small(s.ccount, P, s.cstart, st));
                GF_HIP(gf::launch_cellq_fill(Q, P, s.cells, s.counts, s.cstart, s.cfill, s.cellq, st));
                GF_HIP(gf::launch_selcount(ix->ntiles, ix->tile_cell.p, ix->tile_row0.p, ix->tile_n.p, ix->attrs.p,
                                           a, s.cstart, s.ccount, s.cellq, s.lo, s.hi, s.selcount, st));
            }
        }
        GF_HIP(gf::launch_route(Q, ix->N, o->prefilter, s.selcount, s.counts, s.little, st));

        // Stage B (gf_order_cells, nearest centres straight from the MFMA tiles).
        if (ix->C) {
            GF_HIP(gf::launch_centroid_top(s.q16, ix->centres.p, s.qnorm, ix->cnorm.p, Q, ix->C, Qp, ix->Cp, ix->Dp,
                                           o->topc, s.topk, st));
            GF_HIP(gf::launch_order(Q, ix->C, P, o->topc, nullptr, ix->hist.p, s.cells, s.counts, s.topk, st, true,
                                    ix->ref_ties));
        }

        // Stage C (gf_search): schedule, traversal, gather brute force.
        if (so.entry_points)
            GF_HIP(hipMemcpyAsync(s.entry, so.entry_points, size_t(R) * 4, hipMemcpyHostToDevice, st));
        else
            GF_HIP(hipMemcpyAsync(s.entry, ix->entry_ref.p, size_t(R) * 4, hipMemcpyDeviceToDevice, st));
        gf::TravArgs t{};
        t.vec = ix->vec.p;
        t.rowbytes = ix->rowbytes;
        t.nch = ix->rs.nch;
        t.attrs = ix->attrs.p;
        t.graph = ix->graph.p;
        t.cross = ix->cross.p;
        t.xrow = uint64_t(P) * ix->E;
        t.xcell = ix->E;
        t.offset = ix->offset.p;
        t.gidx = ix->gidx.p;
        t.lrow = ix->lrow.p;
        const bool hq = gf::half_rows(ix->vdtype);
        t.queries = hq ? reinterpret_cast<const char*>(s.q16v)
                                             : reinterpret_cast<const char*>(s.qf32);
        t.qbytes = hq ? D * 2 : D * 4;
        t.lo = s.lo;
        t.hi = s.hi;
        t.cells = s.cells;
        t.counts = s.counts;
        t.little = s.little;
        t.sched = s.sched;
        t.entry = s.entry;
        t.out_ids = s.out_ids;
        t.out_dist = s.out_dist;
        t.counters = s.counters;
        t.a = a; t.P = P; t.R = R; t.E = ix->E; t.L = L; t.K = K; t.rl = rl;
        t.hsize = hsize;
        t.offl = gf::trav_offsets_in_lds(ix->P) ? 1u : 0u;
        t.Lpad = Lpad;
        gf::SchedArgs sa{};
        sa.Q = Q; sa.P = P; sa.postfilter = so.postfilter; sa.counts = s.counts; sa.little = s.little;
        sa.sched = s.sched; sa.tot = s.tot + 8; sa.ranges = s.tot + 12;
        sa.full = ix->FD ? 1u : 0u;
        sa.franges = ix->FD ? s.tot + 16 : nullptr;
        GF_HIP(gf::launch_reset_results(Q, K, s.out_ids, s.out_dist, s.counters, st));
        GF_HIP(gf::launch_sched(sa, st));
        gf::TravArgs tt = t;
        tt.srange = s.tot + 12;
        GF_HIP(gf::launch_traverse(ix->rs, tt, lds, Q, st));
        if (ix->FD && so.postfilter <= P) {
            gf::TravArgs tf = t;
            const uint32_t hs = gf::visited_slots(L + 5 * ix->FD);
            tf.hsize = hs;
            const uint32_t lds_f = Lpad * 8 + gf::kXSlots * 8 + 128 * 4 + hs * 4;
            GF_REQUIRE(lds_f <= 64 * 1024, GF_E_UNSUPPORTED, "L too large for the LDS budget");
            tf.fgraph = ix->fgraph.p;
            tf.fentry = ix->fentry.p;
            tf.FD = ix->FD;
            tf.frange = s.tot + 16;
            GF_HIP(gf::launch_fullgraph(ix->rs, tf, lds_f, Q, st));
        }
        gf::TravArgs tb = t;
        tb.srange = s.tot + 14;
        GF_HIP(gf::launch_bruteforce(ix->rs, tb, Q, st));
        GF_HIP(hipMemcpyAsync(ids, s.out_ids, size_t(Q) * K * 4, hipMemcpyDeviceToHost, st));
        if (dists) GF_HIP(hipMemcpyAsync(dists, s.out_dist, size_t(Q) * K * 4, hipMemcpyDeviceToHost, st));
        GF_HIP(hipStreamSynchronize(st));
        return GF_OK;
    } catch (const gf::Error& e) {
        gf::set_last_error(e.msg);
        return e.code;
    } catch (const std::exception& e) {
        gf::set_last_error(e.what());
        return GF_E_ARG;
    }
}
