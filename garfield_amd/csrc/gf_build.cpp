// Index builder of libgarfield.so: the rank-quantile grid and the exact
// per-cell and cross-cell graphs of a GMG index, in the layouts
// gf_index_create (and the index files) take.
//
// The reference builds these with Python scripts over cuVS: grid_scatter_V2
// (indexbuild/tools.py:88-125) for the grid, a CAGRA graph per cell
// (indexbuild/cagra_build.py:94-127, cell-local ids) and, for the cross-cell
// graph, a CAGRA search of every point against every cell's index
// (indexbuild/global_graph_build.py:106-176, local ids, own cell included).
// Here both graphs are exact nearest neighbours ordered by (squared
// distance, cell-local id).  For integer data in [0, 255] the distances are
// integer dot products on the int8 MFMA units (k_knn_i8) over the brute
// force's tile layout.  Other float data runs the same kernels on a u8
// quantisation of it (one scale for every dimension), keeping kFloatMargin
// more candidates per list than it returns, and those candidates are
// re-ranked by their exact fp32 distances (k_rerank).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <numeric>
#include <vector>

#include "gf_state.h"

namespace gf {

namespace {

constexpr uint32_t kFloatMargin = 16;   // extra candidates per list for the re-rank of float data

// Float data that are not all integers in [0, 255].
bool float_data(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D) {
    if (vec_dtype != GF_VEC_F32) return false;
    const float* s = static_cast<const float*>(vectors);
    for (size_t i = 0; i < size_t(N) * D; ++i)
        if (!(s[i] >= 0.0f && s[i] <= 255.0f && s[i] == std::floor(s[i]))) return true;
    return false;
}

// The first N rows of v8 (Dp wide, padding left as it is) from the input:
// u8 and integer float data as they are; other float data quantised as
// rint((x - min) / s), s = (max - min) / 255 in double over all values (all
// 0 when they are equal).
void rows_u8(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D, uint32_t Dp, bool fmode,
             std::vector<uint8_t>& v8) {
    if (vec_dtype == GF_VEC_U8) {
        const uint8_t* s = static_cast<const uint8_t*>(vectors);
        for (uint32_t i = 0; i < N; ++i) std::memcpy(&v8[size_t(i) * Dp], s + size_t(i) * D, D);
        return;
    }
    const float* s = static_cast<const float*>(vectors);
    if (!fmode) {
        for (uint32_t i = 0; i < N; ++i)
            for (uint32_t k = 0; k < D; ++k) v8[size_t(i) * Dp + k] = uint8_t(s[size_t(i) * D + k]);
        return;
    }
    double lo = s[0], hi = s[0];
    for (size_t i = 0; i < size_t(N) * D; ++i) {
        lo = std::min(lo, double(s[i]));
        hi = std::max(hi, double(s[i]));
    }
    GF_REQUIRE(std::isfinite(lo) && std::isfinite(hi), GF_E_UNSUPPORTED, "non-finite vectors");
    const double sc = (hi - lo) / 255.0;
    for (uint32_t i = 0; i < N; ++i)
        for (uint32_t k = 0; k < D; ++k) {
            const double q = sc > 0.0 ? std::nearbyint((double(s[size_t(i) * D + k]) - lo) / sc) : 0.0;
            v8[size_t(i) * Dp + k] = uint8_t(std::min(255.0, std::max(0.0, q)));
        }
}

// Stable ascending argsort of floats: LSD radix sort (three 11-bit digits)
// of the order-preserving integer image of each value; -0 counts as +0, as
// in a comparison sort.
void stable_argsort(const std::vector<float>& v, std::vector<uint32_t>& order) {
    const size_t n = v.size();
    std::vector<uint32_t> key(n), k2(n), o2(n);
    for (size_t i = 0; i < n; ++i) {
        uint32_t u;
        const float x = v[i] == 0.0f ? 0.0f : v[i];
        std::memcpy(&u, &x, 4);
        key[i] = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
        order[i] = uint32_t(i);
    }
    for (int shift = 0; shift < 33; shift += 11) {
        std::vector<size_t> cnt(2049, 0);
        for (size_t i = 0; i < n; ++i) ++cnt[((key[i] >> shift) & 2047u) + 1];
        for (int b = 0; b < 2048; ++b) cnt[b + 1] += cnt[b];
        for (size_t i = 0; i < n; ++i) {
            const size_t d = cnt[(key[i] >> shift) & 2047u]++;
            k2[d] = key[i];
            o2[d] = order[i];
        }
        key.swap(k2);
        order.swap(o2);
    }
}

}  // namespace

void grid_scatter(const float* attrs, uint32_t N, uint32_t a, const uint32_t* grid, float* l_q, float* r_q,
                  uint32_t* pid_lists, uint32_t* global_pid) {
    GF_REQUIRE(attrs && grid && N > 0 && a > 0, GF_E_ARG, "grid_scatter: empty input");
    uint64_t P = 1;
    for (uint32_t d = 0; d < a; ++d) {
        GF_REQUIRE(grid[d] > 0, GF_E_ARG, "grid_scatter: a grid dimension is 0");
        const uint64_t avg = (uint64_t(N) + grid[d] - 1) / grid[d];
        // the last cell's first rank must exist (tools.py:101 indexes it)
        GF_REQUIRE((grid[d] - 1) * avg < N, GF_E_ARG, "grid_scatter: more cells than the points can fill");
        P *= grid[d];
        GF_REQUIRE(P <= 0x7FFFFFFFu, GF_E_ARG, "grid_scatter: too many cells");
    }
    std::vector<uint32_t> order(N), idx(size_t(a) * N);
    std::vector<float> col(N);
    uint32_t qoff = 0;
    for (uint32_t d = 0; d < a; ++d) {
        for (uint32_t i = 0; i < N; ++i) col[i] = attrs[size_t(i) * a + d];
        // stable argsort (tools.py:98): equal values keep point-id order
        stable_argsort(col, order);
        const uint32_t g = grid[d];
        const uint32_t avg = uint32_t((uint64_t(N) + g - 1) / g);
        for (uint32_t j = 0; j < g; ++j) {
            const uint32_t s = j * avg, e = j + 1 < g ? (j + 1) * avg : N;
            for (uint32_t r = s; r < e; ++r) idx[size_t(d) * N + order[r]] = j;
            if (l_q) l_q[qoff + j] = col[order[s]];
            if (r_q) r_q[qoff + j] = col[order[e - 1]];
        }
        qoff += g;
    }
    if (pid_lists) std::memcpy(pid_lists, idx.data(), idx.size() * sizeof(uint32_t));
    if (global_pid) {
        // row-major cell id, the last attribute fastest (tools.py:111-120)
        for (uint32_t i = 0; i < N; ++i) {
            uint64_t pid = 0;
            for (uint32_t d = 0; d < a; ++d) pid = pid * grid[d] + idx[size_t(d) * N + i];
            global_pid[i] = uint32_t(pid);
        }
    }
}

void build_graphs(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D, const uint32_t* global_pid,
                  uint32_t P, uint32_t R, uint32_t E, int32_t device, uint32_t* cell_graphs, uint32_t* cross,
                  gf_build_stats* stats) {
    GF_REQUIRE(vectors && global_pid && N > 0 && D > 0 && P > 0, GF_E_ARG, "build_graphs: empty input");
    GF_REQUIRE(vec_dtype == GF_VEC_F32 || vec_dtype == GF_VEC_U8, GF_E_ARG,
               "build_graphs: vectors must be GF_VEC_F32 or GF_VEC_U8");
    GF_REQUIRE(!cell_graphs || (R > 0 && R + 1 <= kKnnKMax), GF_E_UNSUPPORTED,
               "build_graphs: degree R must be in [1, " + std::to_string(kKnnKMax - 1) + "]");
    GF_REQUIRE(!cross || (E > 0 && E <= kKnnKMax), GF_E_UNSUPPORTED,
               "build_graphs: E must be in [1, " + std::to_string(kKnnKMax) + "]");
    GF_REQUIRE(uint64_t(N) * P * (cross ? E : 0) < (uint64_t(1) << 40), GF_E_UNSUPPORTED,
               "build_graphs: cross-cell graph too large");
    const uint32_t KS = knn_ks(D);
    GF_REQUIRE(KS > 0, GF_E_UNSUPPORTED, "build_graphs: dimension above 1024");
    const uint32_t Dp = KS * 64, QT = knn_qt(KS);
    // Float data that are not all integers in [0, 255]: candidates from a u8
    // quantisation, kFloatMargin more per list, then the exact re-rank.
    const bool fmode = float_data(vectors, vec_dtype, N, D);
    uint32_t Rk = R, Ek = E;   // list sizes the kNN kernel keeps
    if (fmode) {
        GF_REQUIRE(!cell_graphs || R + 1 <= 64, GF_E_UNSUPPORTED, "build_graphs: float data supports R up to 63");
        GF_REQUIRE(!cross || E <= 64, GF_E_UNSUPPORTED, "build_graphs: float data supports E up to 64");
        Rk = std::min(R + kFloatMargin, 63u);
        Ek = std::min(E + kFloatMargin, 64u);
    }

    using clock = std::chrono::steady_clock;
    const auto c0 = clock::now();
    auto ms_since = [](clock::time_point a) {
        return std::chrono::duration<double, std::milli>(clock::now() - a).count();
    };
    // Vectors as u8 rows of Dp (padding 128 is 0 after the -128 shift and
    // adds nothing to norms or dot products): integer data as it is; other
    // float data quantised as rint((x - min) / s), s = (max - min) / 255 in
    // double over all values (all 0 when they are equal).  u8 rows of a
    // multiple of 64 are uploaded as they are.
    const bool direct = vec_dtype == GF_VEC_U8 && D == Dp;
    std::vector<uint8_t> v8(direct ? 0 : size_t(N) * Dp, uint8_t(128));
    if (!direct) rows_u8(vectors, vec_dtype, N, D, Dp, fmode, v8);

    // Cells: members in ascending point id (the cell-local id order of the
    // index), each cell padded to whole 16-point tiles.
    std::vector<uint32_t> size(P, 0), coff(P + 1, 0), ctile(P + 1, 0);
    for (uint32_t i = 0; i < N; ++i) {
        GF_REQUIRE(global_pid[i] < P, GF_E_ARG, "build_graphs: global_pid out of range");
        ++size[global_pid[i]];
    }
    for (uint32_t c = 0; c < P; ++c) {
        coff[c + 1] = coff[c] + size[c];
        ctile[c + 1] = ctile[c] + (size[c] + 15) / 16;
    }
    const uint32_t ntile = ctile[P];
    std::vector<uint32_t> trow(size_t(ntile) * 16, 0xFFFFFFFFu), fill(P, 0);
    for (uint32_t i = 0; i < N; ++i) {
        const uint32_t c = global_pid[i];
        trow[size_t(ctile[c]) * 16 + fill[c]++] = i;
    }
    // Items: groups of four query tiles of a cell; the graph pass pairs each
    // with its own cell, the cross pass with every non-empty cell, target
    // cell outermost so that concurrent waves stream the same candidates.
    std::vector<KnnItem> gitems, citems;
    for (uint32_t c = 0; c < P; ++c)
        for (uint32_t t = ctile[c]; t < ctile[c + 1]; t += QT) gitems.push_back(KnnItem{t, c, c});
    if (cross) {
        citems.reserve(gitems.size() * P);
        for (uint32_t tc = 0; tc < P; ++tc) {
            if (!size[tc]) continue;
            for (const KnnItem& g : gitems) citems.push_back(KnnItem{g.qtile, g.qcell, tc});
        }
    }

    const double ms_prep = ms_since(c0);
    const auto c1 = clock::now();
    GF_HIP(hipSetDevice(device));
    int ncu = 0;
    GF_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device));
    hipStream_t st = nullptr, st2 = nullptr;
    hipEvent_t ev[4] = {};
    struct Guard {
        hipStream_t& st;
        hipStream_t& st2;
        hipEvent_t* ev;
        ~Guard() {
            for (int i = 0; i < 4; ++i)
                if (ev[i]) (void)hipEventDestroy(ev[i]);
            if (st2) (void)hipStreamDestroy(st2);
            if (st) (void)hipStreamDestroy(st);
        }
    } guard{st, st2, ev};
    GF_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    GF_HIP(hipStreamCreateWithFlags(&st2, hipStreamNonBlocking));
    for (auto& e : ev) GF_HIP(hipEventCreate(&e));

    DevBuf<uint8_t> dvec;
    DevBuf<uint32_t> dtrow, dctile, dcoff, dout_g, dout_c;
    DevBuf<int8_t> vt;
    DevBuf<int32_t> tnorm;
    DevBuf<KnnItem> dgi, dci;
    if (direct)
        dvec.upload(static_cast<const uint8_t*>(vectors), size_t(N) * D);
    else
        dvec.upload(v8);
    dtrow.upload(trow);
    dctile.upload(ctile);
    dcoff.upload(coff);
    dgi.upload(gitems);
    dci.upload(citems);
    vt.alloc(size_t(ntile) * KS * 1024);
    tnorm.alloc(size_t(ntile) * 32);
    if (cell_graphs) dout_g.alloc(size_t(N) * Rk);
    if (cross) {
        dout_c.alloc(size_t(N) * P * Ek);
        // rows into empty cells are never written by a kernel: zero them
        GF_HIP(hipMemsetAsync(dout_c.p, 0, dout_c.bytes(), st));
    }

    GF_HIP(hipStreamSynchronize(st));
    const double ms_upload = ms_since(c1);
    const auto c2 = clock::now();
    GF_HIP(hipEventRecord(ev[0], st));
    GF_HIP(launch_tile_i8(dvec.p, true, Dp, dtrow.p, 0, ntile, vt.p, tnorm.p, st));
    GF_HIP(hipEventRecord(ev[1], st));
    // Candidates stream in chunks of about 1 MiB of tiles per target cell, one
    // launch per chunk, so that an XCD's share of a launch (items of one or
    // two target cells) keeps its chunk in L2; the keys carry over between
    // launches in `state`.
    const uint32_t ctiles = 1024 / KS;
    uint32_t tmax = 0;
    for (uint32_t c = 0; c < P; ++c) tmax = std::max(tmax, ctile[c + 1] - ctile[c]);
    const uint32_t nchunk = (tmax + ctiles - 1) / ctiles;
    DevBuf<uint64_t> state;
    state.alloc(std::max(cell_graphs ? size_t(N) * (Rk + 1) : 0, cross ? size_t(N) * P * Ek : 0));
    KnnArgs ka{};
    ka.vt = vt.p;
    ka.tnorm = tnorm.p;
    ka.trow = dtrow.p;
    ka.ctile = dctile.p;
    ka.coff = dcoff.p;
    ka.P = P;
    ka.ctiles = ctiles;
    ka.state = state.p;
    if (cell_graphs) {
        ka.items = dgi.p;
        ka.nitems = uint32_t(gitems.size());
        ka.K = Rk + 1;
        ka.R = Rk;
        ka.out = dout_g.p;
        for (ka.chunk = 0; ka.chunk < nchunk; ++ka.chunk) GF_HIP(launch_knn_i8(ka, KS, uint32_t(ncu), st));
    }
    GF_HIP(hipEventRecord(ev[2], st));
    if (cross) {
        GF_REQUIRE(citems.size() < 0xFFFFFFFFull, GF_E_UNSUPPORTED, "build_graphs: too many cross items");
        ka.items = dci.p;
        ka.nitems = uint32_t(citems.size());
        ka.K = Ek;
        ka.R = 0;
        ka.out = dout_c.p;
        for (ka.chunk = 0; ka.chunk < nchunk; ++ka.chunk) GF_HIP(launch_knn_i8(ka, KS, uint32_t(ncu), st));
    }
    DevBuf<uint32_t> dfin_g, dfin_c;
    if (fmode) {
        // The candidates' exact fp32 distances: rows cell-major, zero padded
        // to whole 16-byte chunks (the layout of the row-distance helpers).
        const uint32_t nch = (D + 3) / 4, rw = nch * 4;
        std::vector<float> rows(size_t(N) * rw, 0.0f);
        std::vector<uint32_t> cmrow(N), rowcell(N);
        const float* s = static_cast<const float*>(vectors);
        std::vector<uint32_t> pos(coff.begin(), coff.end() - 1);
        for (uint32_t i = 0; i < N; ++i) {
            const uint32_t r = pos[global_pid[i]]++;
            cmrow[i] = r;
            rowcell[r] = global_pid[i];
            std::memcpy(&rows[size_t(r) * rw], s + size_t(i) * D, size_t(D) * 4);
        }
        DevBuf<float> drows;
        DevBuf<uint32_t> dcm, drc;
        drows.upload(rows);
        dcm.upload(cmrow);
        drc.upload(rowcell);
        RerankArgs ra{};
        ra.vec = drows.p;
        ra.rowbytes = rw * 4;
        ra.nch = nch;
        ra.coff = dcoff.p;
        ra.rowcell = drc.p;
        ra.cmrow = dcm.p;
        ra.P = P;
        if (cell_graphs) {
            dfin_g.alloc(size_t(N) * R);
            ra.cand = dout_g.p;
            ra.nc = Rk;
            ra.keep = R;
            ra.graph = 1;
            ra.out = dfin_g.p;
            GF_HIP(launch_rerank(ra, D, N, st));
        }
        if (cross) {
            dfin_c.alloc(size_t(N) * P * E);
            GF_HIP(hipMemsetAsync(dfin_c.p, 0, dfin_c.bytes(), st));
            ra.cand = dout_c.p;
            ra.nc = Ek;
            ra.keep = E;
            ra.graph = 0;
            ra.out = dfin_c.p;
            GF_REQUIRE(uint64_t(N) * P < 0x80000000ull, GF_E_UNSUPPORTED, "build_graphs: too many cross lists");
            GF_HIP(launch_rerank(ra, D, uint32_t(uint64_t(N) * P), st));
        }
        GF_HIP(hipStreamSynchronize(st));   // the row buffers go out of scope
    }
    const uint32_t* res_g = fmode ? dfin_g.p : dout_g.p;
    const uint32_t* res_c = fmode ? dfin_c.p : dout_c.p;
    GF_HIP(hipEventRecord(ev[3], st));
    // The graphs travel to the caller on a second stream while the cross
    // edges are computed.
    if (cell_graphs) {
        GF_HIP(hipStreamWaitEvent(st2, fmode ? ev[3] : ev[2], 0));
        GF_HIP(hipMemcpyAsync(cell_graphs, res_g, size_t(N) * R * 4, hipMemcpyDeviceToHost, st2));
        GF_HIP(hipStreamSynchronize(st2));
    }
    GF_HIP(hipStreamSynchronize(st));
    const double ms_run = ms_since(c2);
    const auto c3 = clock::now();
    if (cross) GF_HIP(hipMemcpy(cross, res_c, size_t(N) * P * E * 4, hipMemcpyDeviceToHost));
    if (stats) {
        stats->ms_prep = ms_prep;
        stats->ms_upload = ms_upload;
        stats->ms_run = ms_run;
        stats->ms_download = ms_since(c3);
        stats->ms_total = ms_since(c0);
        float ms = 0;
        GF_HIP(hipEventElapsedTime(&ms, ev[0], ev[1]));
        stats->ms_tiles = ms;
        GF_HIP(hipEventElapsedTime(&ms, ev[1], ev[2]));
        stats->ms_graph = ms;
        GF_HIP(hipEventElapsedTime(&ms, ev[2], ev[3]));
        stats->ms_cross = ms;
        uint64_t gp = 0, cp = 0;
        for (uint32_t c = 0; c < P; ++c) gp += uint64_t(size[c]) * size[c];
        for (uint32_t c = 0; c < P; ++c) cp += uint64_t(N) * size[c];
        stats->pairs_graph = cell_graphs ? gp : 0;
        stats->pairs_cross = cross ? cp : 0;
        stats->dim = Dp;
    }
}

void optimize_graphs(const uint32_t* knn, uint32_t N, uint32_t I, const uint32_t* cell_size, uint32_t P,
                     uint32_t R, int32_t device, uint32_t* graphs, double* ms) {
    const auto t0 = std::chrono::steady_clock::now();
    GF_REQUIRE(knn && cell_size && graphs, GF_E_ARG, "null argument");
    GF_REQUIRE(N > 0 && P > 0, GF_E_ARG, "empty graph");
    GF_REQUIRE(I >= 1 && I <= 64, GF_E_UNSUPPORTED, "input degree must be in [1, 64]");
    GF_REQUIRE(R >= 1 && R <= I, GF_E_ARG, "output degree must be in [1, input degree]");
    std::vector<uint32_t> offset(P + 1, 0);
    for (uint32_t c = 0; c < P; ++c) offset[c + 1] = offset[c] + cell_size[c];
    GF_REQUIRE(offset[P] == N, GF_E_ARG, "cell sizes do not add up to N");
    for (uint32_t c = 0; c < P; ++c)
        for (size_t k = size_t(offset[c]) * I; k < size_t(offset[c + 1]) * I; ++k)
            GF_REQUIRE(knn[k] < cell_size[c], GF_E_FORMAT, "kNN graph holds an id beyond its cell");
    std::vector<uint32_t> ord(size_t(N) * I);
    {
        GF_HIP(hipSetDevice(device));
        hipStream_t st = nullptr;
        GF_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
        struct StreamGuard {
            hipStream_t s;
            ~StreamGuard() { (void)hipStreamDestroy(s); }
        } guard{st};
        DevBuf<uint32_t> dk, doff, dout;
        dk.upload(knn, size_t(N) * I);
        doff.upload(offset);
        dout.alloc(size_t(N) * I);
        GF_HIP(launch_prune(dk.p, N, I, doff.p, P, dout.p, st));
        GF_HIP(hipMemcpyAsync(ord.data(), dout.p, ord.size() * 4, hipMemcpyDeviceToHost, st));
        GF_HIP(hipStreamSynchronize(st));
    }
    // Reverse edges: for every rank k of the pruned lists (their first R
    // entries), in node order, the edge A -> B adds A to B's reverse list
    // (at most R, a node never lists itself).  Each row then keeps the first
    // R / 2 pruned edges, appends reverse edges, then the rest of its
    // reordered list, each id once; a row still short (a cell of fewer than
    // R + 1 points) repeats its first entry.
    const uint32_t keep = R / 2;
    std::vector<uint32_t> mark;
    for (uint32_t c = 0; c < P; ++c) {
        const uint32_t off = offset[c], n = cell_size[c];
        std::vector<uint32_t> rev(size_t(n) * R), rcnt(n, 0);
        for (uint32_t k = 0; k < R; ++k)
            for (uint32_t a = 0; a < n; ++a) {
                const uint32_t b = ord[(size_t(off) + a) * I + k];
                if (b != a && rcnt[b] < R) rev[size_t(b) * R + rcnt[b]++] = a;
            }
        mark.assign(n, 0);
        for (uint32_t a = 0; a < n; ++a) {
            const uint32_t* o = &ord[(size_t(off) + a) * I];
            uint32_t* g = graphs + (size_t(off) + a) * R;
            const uint32_t stamp = a + 1;
            uint32_t m = 0;
            auto put = [&](uint32_t x) {
                if (m < R && mark[x] != stamp) { mark[x] = stamp; g[m++] = x; }
            };
            for (uint32_t k = 0; k < keep; ++k) put(o[k]);
            for (uint32_t t = 0; t < rcnt[a]; ++t) put(rev[size_t(a) * R + t]);
            for (uint32_t k = keep; k < I; ++k) put(o[k]);
            for (; m < R; ++m) g[m] = g[0];
        }
    }
    if (ms) *ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

void kmeans_labels(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D, uint32_t C, uint32_t iters,
                   const uint32_t* init_ids, int32_t device, int32_t* labels, uint8_t* centres, double* ms) {
    GF_REQUIRE(vectors && init_ids && labels && N > 0 && D > 0, GF_E_ARG, "kmeans: empty input");
    GF_REQUIRE(vec_dtype == GF_VEC_F32 || vec_dtype == GF_VEC_U8, GF_E_ARG,
               "kmeans: vectors must be GF_VEC_F32 or GF_VEC_U8");
    GF_REQUIRE(C > 0 && C <= N, GF_E_ARG, "kmeans: need 0 < C <= N");
    GF_REQUIRE(uint64_t(N) + C < 0xFFFFFFF0ull, GF_E_UNSUPPORTED, "kmeans: too many points");
    const uint32_t KS = knn_ks(D);
    GF_REQUIRE(KS > 0, GF_E_UNSUPPORTED, "kmeans: dimension above 1024");
    const uint32_t Dp = KS * 64, QT = knn_qt(KS);
    for (uint32_t c = 0; c < C; ++c) GF_REQUIRE(init_ids[c] < N, GF_E_ARG, "kmeans: init id out of range");
    const auto c0 = std::chrono::steady_clock::now();

    // Rows: the N points, then the C centres (u8, Dp wide, padding 128).
    // Float data that are not integers in [0, 255] are clustered in the u8
    // quantisation the graph builder uses.
    std::vector<uint8_t> v8(size_t(N + C) * Dp, uint8_t(128));
    rows_u8(vectors, vec_dtype, N, D, Dp, float_data(vectors, vec_dtype, N, D), v8);
    for (uint32_t c = 0; c < C; ++c)
        std::memcpy(&v8[size_t(N + c) * Dp], &v8[size_t(init_ids[c]) * Dp], Dp);
    // Two "cells": the points (queries) and the centres (candidates); an
    // assignment is the cross-edge pass with E = 1 (nearest centre, ties to
    // the smaller centre index).
    const uint32_t Tp = (N + 15) / 16, Tc = (C + 15) / 16, ntile = Tp + Tc;
    std::vector<uint32_t> trow(size_t(ntile) * 16, 0xFFFFFFFFu);
    for (uint32_t i = 0; i < N; ++i) trow[i] = i;
    for (uint32_t c = 0; c < C; ++c) trow[size_t(Tp) * 16 + c] = N + c;
    const std::vector<uint32_t> ctile{0, Tp, ntile}, coff{0, N, N + C};
    std::vector<KnnItem> items;
    for (uint32_t t = 0; t < Tp; t += QT) items.push_back(KnnItem{t, 0, 1});

    GF_HIP(hipSetDevice(device));
    int ncu = 0;
    GF_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device));
    hipStream_t st = nullptr;
    struct Guard {
        hipStream_t& st;
        ~Guard() {
            if (st) (void)hipStreamDestroy(st);
        }
    } guard{st};
    GF_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    DevBuf<uint8_t> dvec;
    DevBuf<uint32_t> dtrow, dctile, dcoff, out2, cnt, cstart, cfill, cmem;
    DevBuf<int32_t> tnorm;
    DevBuf<int8_t> vt;
    DevBuf<KnnItem> ditems;
    DevBuf<uint64_t> state;
    dvec.upload(v8);
    dtrow.upload(trow);
    dctile.upload(ctile);
    dcoff.upload(coff);
    ditems.upload(items);
    vt.alloc(size_t(ntile) * KS * 1024);
    tnorm.alloc(size_t(ntile) * 32);
    out2.alloc(size_t(N) * 2);
    state.alloc(size_t(N) * 2);
    cnt.alloc(C);
    cstart.alloc(C);
    cfill.alloc(C);
    cmem.alloc(N);
    const uint32_t ctiles = 1024 / KS, nchunk = (Tc + ctiles - 1) / ctiles;
    KnnArgs ka{};
    ka.vt = vt.p;
    ka.tnorm = tnorm.p;
    ka.trow = dtrow.p;
    ka.ctile = dctile.p;
    ka.coff = dcoff.p;
    ka.items = ditems.p;
    ka.nitems = uint32_t(items.size());
    ka.K = 1;
    ka.R = 0;
    ka.P = 2;
    ka.out = out2.p;
    ka.ctiles = ctiles;
    ka.state = state.p;
    GF_HIP(launch_tile_i8(dvec.p, true, Dp, dtrow.p, 0, ntile, vt.p, tnorm.p, st));
    for (uint32_t it = 0;; ++it) {
        for (ka.chunk = 0; ka.chunk < nchunk; ++ka.chunk) GF_HIP(launch_knn_i8(ka, KS, uint32_t(ncu), st));
        if (it == iters) break;
        GF_HIP(hipMemsetAsync(cnt.p, 0, cnt.bytes(), st));
        GF_HIP(hipMemsetAsync(cfill.p, 0, cfill.bytes(), st));
        GF_HIP(launch_kmeans_update(dvec.p, Dp, out2.p, N, C, cnt.p, cstart.p, cfill.p, cmem.p,
                                    dvec.p + size_t(N) * Dp, st));
        GF_HIP(launch_tile_i8(dvec.p, true, Dp, dtrow.p + size_t(Tp) * 16, 0, Tc, vt.p + size_t(Tp) * KS * 1024,
                              tnorm.p + size_t(Tp) * 32, st));
    }
    GF_HIP(hipStreamSynchronize(st));
    std::vector<uint32_t> h2(size_t(N) * 2);
    GF_HIP(hipMemcpy(h2.data(), out2.p, out2.bytes(), hipMemcpyDeviceToHost));
    for (uint32_t i = 0; i < N; ++i) labels[i] = int32_t(h2[size_t(i) * 2 + 1]);
    if (centres) {
        std::vector<uint8_t> hc(size_t(C) * Dp);
        GF_HIP(hipMemcpy(hc.data(), dvec.p + size_t(N) * Dp, hc.size(), hipMemcpyDeviceToHost));
        for (uint32_t c = 0; c < C; ++c) std::memcpy(centres + size_t(c) * D, &hc[size_t(c) * Dp], D);
    }
    if (ms) *ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - c0).count();
}

}  // namespace gf
