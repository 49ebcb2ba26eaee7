// CPU oracle for the Garfield query path -- TEST INFRASTRUCTURE ONLY.
// Restates the reference (ZJU-DAILY/Garfield indexsearch/*.cu) in plain C++;
// see garfield_oracle.h for the rules that replace the reference's races and
// out-of-bounds reads.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg load this library; the product (libgarfield.so) never does.
#include "garfield_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <random>
#include <unordered_set>
#include <vector>
#include <omp.h>

namespace {

const uint32_t SENT = 0xFFFFFFFFu;   // reference's empty candidate id
const uint32_t EXPL = 0x80000000u;   // reference's "explored" bit
const uint32_t IDM = 0x7FFFFFFFu;
const uint32_t ID30 = 0x3FFFFFFFu;   // point id under the dual-channel traversal's two explored bits
const float INF = std::numeric_limits<float>::infinity();
const uint32_t MAX_ITER = 10000;     // gpu_graph.cu:39
const uint32_t HASH_RESET = 4;       // gpu_graph.cu:34
const uint32_t XSLOTS = 128;         // gpu_graph.cu:42 EXTEND_POINTS_NUM
const uint32_t XSTEP = 64;           // 128 / base_number(2), gpu_graph.cu:3267

uint32_t f32_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

// Lanes per row of the HIP distance kernels: a row is split in 16-byte chunks
// (4 fp32, 8 fp16 or 16 u8 elements), LPR = next power of two >= chunk
// count, clamped to [8, 64].
uint32_t chunk_elems(int vdtype) { return vdtype == 0 ? 4u : (vdtype == 1 ? 8u : 16u); }

uint32_t lanes_per_row(uint32_t D, int vdtype) {
    const uint32_t elems = chunk_elems(vdtype);
    uint32_t nch = (D + elems - 1) / elems;
    uint32_t lpr = 8;
    while (lpr < nch && lpr < 64) lpr <<= 1;
    return lpr;
}

// Canonical distance: lane l of LPR accumulates chunks l, l+LPR, ... with fp32
// fma in element order; the lane sums are combined by an xor butterfly.
// Elements past D (row padding) are zero in both operands.  vdtype 3: q holds
// c_k = fma(s_k, z_k, query_k) and the element term is fma(-s_k, x_k, c_k),
// the query less the dequantised s_k (x_k - z_k).
float canon_dist(const float* q, const float* x, uint32_t D, int vdtype, const float* s3 = nullptr) {
    const uint32_t ce = chunk_elems(vdtype);
    const uint32_t nch = (D + ce - 1) / ce;
    const uint32_t lpr = lanes_per_row(D, vdtype);
    float s[64];
    for (uint32_t l = 0; l < lpr; ++l) {
        float acc = 0.0f;
        for (uint32_t c = l; c < nch; c += lpr)
            for (uint32_t e = 0; e < ce; ++e) {
                const uint32_t k = c * ce + e;
                float d = k >= D ? 0.0f : (vdtype == 3 ? std::fmaf(-s3[k], x[k], q[k]) : q[k] - x[k]);
                acc = std::fmaf(d, d, acc);
            }
        s[l] = acc;
    }
    for (uint32_t m = lpr / 2; m >= 1; m >>= 1) {
        float t[64];
        for (uint32_t l = 0; l < lpr; ++l) t[l] = s[l] + s[l ^ m];
        std::memcpy(s, t, sizeof(float) * lpr);
    }
    return s[0];
}

// ---------------------------------------------------------------- REF_HFMA2
// The reference's fp16 distance (gpu_graph.cu:3394-3403, 3508-3530; half4
// loads tools.cuh:40-53): lane j of a 32-lane warp takes the 4-element chunks
// j, j + 32, ... of the row; per chunk acc = hfma2(q.xy - x.xy, q.xy - x.xy,
// acc) then the same for .zw, so acc.x sums elements 4c and 4c + 2 and acc.y
// elements 4c + 1 and 4c + 3, in chunk order; then five hadd2 steps with
// shfl_down 16, 8, 4, 2, 1 (a lane whose source is beyond the warp keeps its
// own value); lane 0 returns float(acc.x) + float(acc.y) in fp32.  Every
// half operation is its exact result rounded once to binary16 (nearest,
// ties to even); hsub and hadd of two halves and the fma of two halves plus
// a non-negative half are exact in double, or off by far less than a half
// ulp where they are not (a tiny product next to a large accumulator).
uint16_t half_rne(double v) {
    if (v != v) return 0x7E00u;
    const uint16_t sign = std::signbit(v) ? 0x8000u : 0u;
    double a = std::fabs(v);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u);   // beyond the largest half plus half an ulp
    if (a < std::ldexp(1.0, -14)) {                          // subnormal: quantum 2^-24
        const double m = std::nearbyint(a * std::ldexp(1.0, 24));
        return (uint16_t)(sign | (uint16_t)m);               // m = 1024 is the smallest normal's encoding
    }
    int e;
    (void)std::frexp(a, &e);                                 // a in [2^(e-1), 2^e)
    const double q = std::ldexp(1.0, e - 11);
    double m = std::nearbyint(a / q);                        // 1024 .. 2048
    if (m >= 2048.0) { m /= 2.0; ++e; }
    if (e - 1 + 15 >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (uint16_t)((e - 1 + 15) << 10) | (uint16_t)((uint32_t)m - 1024u));
}
double h2d(uint16_t h) { return (double)orc_h2f(h); }

float hfma2_dist(const uint16_t* q, const uint16_t* x, uint32_t D) {
    uint16_t ax[32], ay[32];
    for (uint32_t l = 0; l < 32; ++l) { ax[l] = 0; ay[l] = 0; }
    const uint32_t nc = D / 4;
    for (uint32_t l = 0; l < 32; ++l)
        for (uint32_t c = l; c < nc; c += 32) {
            for (uint32_t p = 0; p < 2; ++p) {                // .xy then .zw
                const uint32_t k = 4 * c + 2 * p;
                const uint16_t dx = half_rne(h2d(q[k]) - h2d(x[k]));
                const uint16_t dy = half_rne(h2d(q[k + 1]) - h2d(x[k + 1]));
                ax[l] = half_rne(std::fma(h2d(dx), h2d(dx), h2d(ax[l])));
                ay[l] = half_rne(std::fma(h2d(dy), h2d(dy), h2d(ay[l])));
            }
        }
    for (uint32_t m = 16; m >= 1; m >>= 1) {
        uint16_t nx[32], ny[32];
        for (uint32_t l = 0; l < 32; ++l) {
            const uint32_t s = l + m < 32 ? l + m : l;
            nx[l] = half_rne(h2d(ax[l]) + h2d(ax[s]));
            ny[l] = half_rne(h2d(ay[l]) + h2d(ay[s]));
        }
        std::memcpy(ax, nx, sizeof(ax));
        std::memcpy(ay, ny, sizeof(ay));
    }
    return orc_h2f(ax[0]) + orc_h2f(ay[0]);
}

// Distance arithmetic of the fp16 path (orc_set_dist_mode): 0 binary16 values
// accumulated in fp32 in the kernels' canonical order; 1 the reference's
// REF_HFMA2 arithmetic above.
int g_dist_mode = 0;

struct Cand { float d; uint32_t id; };

// Order of equal distances (orc_set_tie_mode):
//   0  (distance, cell-major position), a total order, the HIP kernels' rule:
//      every sort and merge then has one result;
//   1  the reference's: distance alone, with its own sorting networks
//      deciding between equal distances -- warpSort (gpu_graph.cu:144-159)
//      for the R neighbours, bitonic_sort_id_by_dis_no_explore (:77-101) for
//      the 128 cross slots and the final list -- and merge_top's ranks.
int g_tie_mode = 0;
// Planted mistakes (orc_set_mutation), for tests that show that the pinning
// checks catch them; 0 in every other use.
int g_mutation = 0;

struct Ctx {
    const orc_index* ix;
    const uint32_t* cmpos;   // point id -> cell-major position (tie key)
    const uint32_t* cellof;  // point id -> cell
    int tie;
};

inline uint32_t tiekey(const Ctx& c, uint32_t id) {
    return id == SENT ? 0xFFFFFFFFu : c.cmpos[id & ID30];
}
inline bool cless(const Ctx& c, const Cand& x, const Cand& y) {
    if (x.d != y.d) return x.d < y.d;
    if (c.tie == 1) return false;
    return tiekey(c, x.id) < tiekey(c, y.id);
}

void sort_stable(const Ctx& c, Cand* v, size_t n) {
    std::stable_sort(v, v + n, [&](const Cand& x, const Cand& y) { return cless(c, x, y); });
}

// bitonic_sort_id_by_dis_no_explore (gpu_graph.cu:77-101): ascending by
// distance; pairs (u, d) of one (stride, step) pass are disjoint, so the
// sequential replay equals the block's.
void bitonic_no_explore(float* dis, uint32_t* ids, uint32_t len) {
    for (uint32_t stride = 1; stride < len; stride <<= 1)
        for (uint32_t step = stride; step > 0; step >>= 1)
            for (uint32_t k = 0; k < len / 2; ++k) {
                const uint32_t a = 2 * step * (k / step), b = k % step;
                const uint32_t u = step == stride ? a + step - 1 - b : a + b;
                const uint32_t d = a + b + step;
                if (d < len && dis[u] > dis[d]) { std::swap(dis[u], dis[d]); std::swap(ids[u], ids[d]); }
            }
}

// warpSort (gpu_graph.cu:144-159) over len lanes: every lane reads its xor
// partner's pair, then all lanes write; a lane takes its partner's pair only
// when the keys differ.  A partner beyond len (not active) is never taken.
void warp_sort(float* key, uint32_t* val, uint32_t len) {
    std::vector<float> k1(len);
    std::vector<uint32_t> v1(len);
    for (uint32_t b = 1; b <= len; b <<= 1)
        for (uint32_t cc = b / 2; cc >= 1; cc >>= 1) {
            for (uint32_t l = 0; l < len; ++l) {
                const uint32_t o = l ^ cc;
                k1[l] = o < len ? key[o] : key[l];
                v1[l] = o < len ? val[o] : val[l];
            }
            for (uint32_t l = 0; l < len; ++l) {
                const bool p = ((l & b) != 0) == ((l & cc) != 0);
                if (key[l] != k1[l] && ((key[l] < k1[l]) != p)) { key[l] = k1[l]; val[l] = v1[l]; }
            }
        }
}

// Sorts of the neighbour list (net = 0) and of the slots / final list (net = 1).
void sort_cands(const Ctx& c, Cand* v, size_t n, int net) {
    if (c.tie != 1) { sort_stable(c, v, n); return; }
    std::vector<float> d(n);
    std::vector<uint32_t> id(n);
    for (size_t i = 0; i < n; ++i) { d[i] = v[i].d; id[i] = v[i].id; }
    if (net == 0) warp_sort(d.data(), id.data(), (uint32_t)n);
    else bitonic_no_explore(d.data(), id.data(), (uint32_t)n);
    for (size_t i = 0; i < n; ++i) v[i] = {d[i], id[i]};
}

enum {
    MUT_MERGE_A_FIRST = 1,        // merge ties put the list entry before the incoming one
    MUT_RESET_EVERY_3 = 2,        // visited set rebuilt every 3 iterations, not 4
    MUT_SLOT_HALF = 3,            // cross slot i follows candidate i / 2, not i % 64
    MUT_RECYCLE_UNFILTERED = 4,   // evicted entries kept whether or not they pass the filter
    MUT_NO_END_EXPLORE = 5,       // the end of a cell leaves the list's explored bits as they are
    MUT_CROSS_LAST_FIRST = 6,     // cross edges tried from the last to the first
    MUT_ENTRY_LOCAL_KEY = 7,      // first-cell entries enter the visited set by local id
    MUT_DROP_SEEN = 8,            // neighbours seen before are dropped instead of entering at +inf
    MUT_NO_POSTFILTER = 9,        // the final list is not filtered
    MUT_ENTRIES_AFTER = 10,       // the next cell's entries are slots R..2R-1, not 0..R-1
    MUT_RECYCLE_ENTRY_FIRST = 11, // recycle merge ties put the recycle entry before the evictee
    MUT_SLOT_32 = 12,             // cross slot i follows candidate i % 32 (only the first 32 feed the slots)
    MUT_CROSS_OWN_CELL = 13,      // cross edges read for the current cell instead of the next
    MUT_FULL_NO_B_REHASH = 14,    // full graph: the reset re-inserts the list only, not the B region
    MUT_FULL_ENTRY_UNSEEN = 15,   // full graph: entry points are not put in the visited set
    MUT_FULL_OWN_AS_CROSS = 16,   // full graph assembly: own-cell edges read from the cross edges
};
// Per-cell iteration cap (gpu_graph.cu:39 MAX_ITER); tests lower it to reach
// the end-of-cell step with unexplored entries left.  The dual-channel
// traversal caps its epochs over all cells with the same value.
uint32_t g_max_iter = MAX_ITER;
// Traversal of the traversal-routed queries (orc_set_channels): 1 the
// cell-by-cell search of the fused kernel, 2 the dual-channel search.
int g_channels = 1;
// Planted mistakes of the dual-channel search (orc_set_dual_mutation).
int g_dual_mutation = 0;
enum {
    DMUT_NO_PARTNER = 1,          // the other channel gets no partner expansion
    DMUT_PARTNER_LAST_EDGE = 2,   // the partner is sought from the last cross edge to the first
    DMUT_NO_TURN = 3,             // the turn never passes to the other channel
    DMUT_SWITCH_EDGE0 = 4,        // the cell switch reads cross edge 0 for all 128 slots
    DMUT_ENTRY_SPLIT_HALF = 5,    // entries split at floor(L / 2) instead of ceil(L / 2)
    DMUT_PEEK_ROW = 6,            // the partner test looks up the point id, not the local id's value
};

// Merged position of every element of sorted X (n) and sorted Y (m):
// X_i -> i + #{Y <= X_i}, Y_j -> j + #{X < Y_j}  (gpu_graph.cu:162-222): an
// incoming Y entry goes before an equal X entry.
void merge_positions(const Ctx& c, const Cand* X, size_t n, const Cand* Y, size_t m,
                     std::vector<size_t>& px, std::vector<size_t>& py, bool x_first = false) {
    px.resize(n); py.resize(m);
    auto lt = [&](const Cand& a, const Cand& b) { return cless(c, a, b); };
    for (size_t i = 0; i < n; ++i)
        px[i] = i + (x_first ? std::lower_bound(Y, Y + m, X[i], lt) : std::upper_bound(Y, Y + m, X[i], lt)) - Y;
    for (size_t j = 0; j < m; ++j)
        py[j] = j + (x_first ? std::upper_bound(X, X + n, Y[j], lt) : std::lower_bound(X, X + n, Y[j], lt)) - X;
}

// merge_top (gpu_graph.cu:162-222): X keeps the n smallest, Y the next m.
void merge_plain(const Ctx& c, Cand* X, size_t n, Cand* Y, size_t m, bool x_first = false) {
    std::vector<size_t> px, py;
    merge_positions(c, X, n, Y, m, px, py, x_first || g_mutation == MUT_MERGE_A_FIRST);
    std::vector<Cand> out(n + m);
    for (size_t i = 0; i < n; ++i) out[px[i]] = X[i];
    for (size_t j = 0; j < m; ++j) out[py[j]] = Y[j];
    std::copy(out.begin(), out.begin() + n, X);
    std::copy(out.begin() + n, out.end(), Y);
}

struct QueryState {
    const Ctx* c;
    const float* q;          // query as fp32 values (fp16 path: converted)
    const uint16_t* qh;      // fp16 path: the query's binary16 values
    const float* lo;
    const float* hi;
    std::vector<float> xbuf;
    uint32_t ctr[ORC_NCNT];
};

bool passes(const QueryState& s, uint32_t gid) {
    const orc_index* ix = s.c->ix;
    for (uint32_t d = 0; d < ix->a; ++d) {
        float v = ix->attrs[(size_t)gid * ix->a + d];
        if (!(v >= s.lo[d] && v <= s.hi[d])) return false;
    }
    return true;
}

float point_dist(QueryState& s, uint32_t gid) {
    const orc_index* ix = s.c->ix;
    const uint32_t D = ix->D;
    if (ix->vdtype != 1)
        return canon_dist(s.q, ix->vec_f32 + (size_t)gid * D, D, ix->vdtype, ix->qscale);
    if (g_dist_mode == 1) return hfma2_dist(s.qh, ix->vec_f16 + (size_t)gid * D, D);
    s.xbuf.resize(D);
    for (uint32_t i = 0; i < D; ++i) s.xbuf[i] = orc_h2f(ix->vec_f16[(size_t)gid * D + i]);
    return canon_dist(s.q, s.xbuf.data(), D, 1);
}

// merge_top_with_recycle_list (gpu_graph.cu:224-315) followed by the
// evictee sort and merge into the recycle list (gpu_graph.cu:3412-3425,
// 3536-3546).  B holds the leftovers afterwards (the reference's B region).
void merge_with_recycle(QueryState& s, Cand* A, size_t L, Cand* B, size_t R,
                        Cand* Rc, size_t rl) {
    const Ctx& c = *s.c;
    std::vector<size_t> px, py;
    merge_positions(c, A, L, B, R, px, py, g_mutation == MUT_MERGE_A_FIRST);
    std::vector<Cand> nA(L), nB(R);
    for (size_t i = 0; i < L; ++i) {
        if (px[i] < L) { nA[px[i]] = A[i]; continue; }
        Cand x = A[i];
        if (x.id != SENT && g_mutation != MUT_RECYCLE_UNFILTERED && !passes(s, x.id & 0x3FFFFFFFu))
            x = {INF, SENT};
        nB[px[i] - L] = x;
    }
    for (size_t j = 0; j < R; ++j) {
        if (py[j] < L) nA[py[j]] = B[j];
        else nB[py[j] - L] = {INF, SENT};
    }
    std::copy(nA.begin(), nA.end(), A);
    std::copy(nB.begin(), nB.end(), B);
    sort_cands(c, B, R, 0);
    if (B[0].id != SENT) merge_plain(c, Rc, rl, B, R, g_mutation == MUT_RECYCLE_ENTRY_FIRST);
}

bool in_cell(const Ctx& c, uint32_t gid, uint32_t cell) { return c.cellof[gid] == cell; }

// Optional record of one query's traversal: the point ids it expands, in
// order, the cell each expansion ran in, and the final recycle list.
struct Trace {
    std::vector<uint32_t> expanded, expanded_cell;
    std::vector<Cand> recycle;
};

void search_one(const Ctx& c, const void* queries, uint32_t qi, const float* lo_all,
                const float* hi_all, const uint32_t* cells, const uint32_t* counts,
                const uint32_t* little, const uint32_t* entry, uint32_t L, uint32_t K,
                uint32_t rl, uint32_t postfilter, uint32_t* out_ids, float* out_dist,
                uint32_t* counters, Trace* tr = nullptr) {
    const orc_index* ix = c.ix;
    const uint32_t D = ix->D, R = ix->R, E = ix->E, P = ix->P, a = ix->a;
    std::vector<float> qv(D);
    const uint16_t* qh = nullptr;
    if (ix->vdtype != 1) {
        std::memcpy(qv.data(), (const float*)queries + (size_t)qi * D, sizeof(float) * D);
        if (ix->vdtype == 3)
            for (uint32_t k = 0; k < D; ++k) qv[k] = std::fmaf(ix->qscale[k], float(ix->qzero[k]), qv[k]);
    } else {
        qh = (const uint16_t*)queries + (size_t)qi * D;
        for (uint32_t i = 0; i < D; ++i) qv[i] = orc_h2f(qh[i]);
    }
    QueryState s;
    s.c = &c; s.q = qv.data(); s.qh = qh; s.lo = lo_all + (size_t)qi * a; s.hi = hi_all + (size_t)qi * a;
    std::memset(s.ctr, 0, sizeof(s.ctr));

    const uint32_t* cl = cells + (size_t)qi * P;
    const uint32_t cnt = counts[qi], lit = little[qi];
    const bool traverse = (cnt < postfilter && cnt != lit);   // gpu_graph.cu:3377
    const bool full = !traverse && ix->FD && cnt != lit;      // gpu_graph.cu:3644
    std::vector<Cand> out;

    auto cell_size = [&](uint32_t cc) { return ix->offset[cc + 1] - ix->offset[cc]; };
    const uint32_t reset_every = g_mutation == MUT_RESET_EVERY_3 ? 3u : HASH_RESET;

    if (traverse && g_channels == 2) {
        // Dual-channel traversal: the traversal of
        // select_path_contain_attr_filter_V2_without_output_dual_channel_in_turn_with_prefilter
        // (gpu_graph.cu:6249-6640; launched like batch_graph_search_gpu,
        // gpu_graph.cu:12223-12300).  Two channels walk two cells of the
        // query's list at once over one candidate list; an entry carries the
        // reference's two explored bits (bit 31: channel 0, bit 30: channel
        // 1), and a channel's own points enter with the other channel's bit
        // set, so that each channel expands only its own.  Per epoch the
        // channel `turn` expands its first unexplored entry and the other
        // channel a partner: the first of that entry's cross edges into the
        // other channel's cell whose local id is not in the visited set
        // (which holds point ids: the reference tests the local id's value),
        // expanded through R - 1 neighbours plus itself.  A channel with
        // nothing left moves to the next cell of the list through 128
        // cross-edge slots; with no cell left it joins the other channel.
        s.ctr[ORC_C_ROUTE] = 4;
        const uint32_t NONE = 0xFFFFFFFFu;
        std::vector<Cand> A(L, Cand{INF, SENT}), T(2 * R, Cand{INF, SENT}), Rc(rl, Cand{INF, SENT});
        std::unordered_set<uint32_t> H;
        H.reserve(4 * (L + XSLOTS + 10 * R));
        uint32_t pid[2] = {cl[0], cnt >= 2 ? cl[1] : cl[0]};
        auto gid_of = [&](uint32_t cc, uint32_t lid) { return ix->global_idx[ix->offset[cc] + lid]; };
        auto dist_of = [&](Cand& x) {
            x.d = point_dist(s, x.id & ID30);
            s.ctr[ORC_C_DIST]++; s.ctr[ORC_C_ATTR]++;
        };
        // Entries (gpu_graph.cu:6318-6329): entry i < ceil(L / 2) in channel
        // 0's cell, the rest in channel 1's; entry[i] reduced modulo the cell
        // size (the reference draws from [0, 62500)).  All L are evaluated
        // and sorted (gpu_graph.cu:6338-6362).
        const uint32_t L2 = g_dual_mutation == DMUT_ENTRY_SPLIT_HALF ? std::max(1u, L / 2) : (L + 1) / 2;
        for (uint32_t i = 0; i < L; ++i) {
            const uint32_t ch = std::min(1u, i / L2);
            const uint32_t mask = pid[0] == pid[1] ? 0u : (1u << (30 + ch));
            const uint32_t g = gid_of(pid[ch], entry[i] % cell_size(pid[ch]));
            A[i] = {INF, g | mask};
            H.insert(g);
            dist_of(A[i]);
        }
        sort_cands(c, A.data(), L, 1);
        uint32_t cur = cnt >= 2 ? 2 : 1, main_ch = 0, turn = 0;
        for (uint32_t ep = 0; ep < g_max_iter; ++ep) {
            if ((ep + 1) % reset_every == 0) {               // gpu_graph.cu:6364-6378
                H.clear();
                for (const auto* arr : {&A, &T})
                    for (const Cand& x : *arr)
                        if (x.id != SENT) H.insert(x.id & ID30);
            }
            // Selection (gpu_graph.cu:6380-6420).
            uint32_t te[2] = {NONE, NONE};
            {
                const uint32_t mask = 1u << (pid[0] == pid[1] ? 31 - main_ch : 31 - turn);
                for (uint32_t j = 0; j < L; ++j)
                    if ((A[j].id & mask) == 0) {
                        te[turn] = ix->local_idx[A[j].id & ID30];
                        A[j].id |= mask;
                        break;
                    }
                if (te[turn] != NONE && g_dual_mutation != DMUT_NO_PARTNER) {
                    const uint32_t g = gid_of(pid[turn], te[turn]);
                    const uint32_t ne = std::min(2u, E);
                    for (uint32_t jj = 0; jj < ne; ++jj) {
                        const uint32_t j = g_dual_mutation == DMUT_PARTNER_LAST_EDGE ? ne - 1 - jj : jj;
                        const uint32_t v = ix->cross[(size_t)g * P * E + (size_t)pid[turn ^ 1] * E + j];
                        const uint32_t key = g_dual_mutation == DMUT_PEEK_ROW ? gid_of(pid[turn ^ 1], v) : v;
                        if (!H.count(key)) { te[turn ^ 1] = v; break; }
                    }
                }
            }
            if (te[turn] == NONE) {                          // gpu_graph.cu:6422-6547
                if (cur == cnt && pid[0] == pid[1]) break;
                if (cur == cnt) {                            // join the other channel's cell
                    pid[turn] = pid[turn ^ 1];
                    main_ch = turn ^ 1;
                    continue;
                }
                // Move channel `turn` to the next cell: slot i follows entry
                // i % 64 through its cross edge i / 64 (an edge index beyond E
                // is skipped: the reference reads the next cell's edges there).
                const uint32_t nxt = cl[cur];
                const uint32_t mask = 1u << (30 + turn);
                std::vector<Cand> W(XSLOTS, Cand{INF, SENT});
                for (uint32_t i = 0; i < XSLOTS; ++i) {
                    const uint32_t si = i % XSTEP;
                    const uint32_t e = g_dual_mutation == DMUT_SWITCH_EDGE0 ? 0 : i / XSTEP;
                    if (si >= L || A[si].id == SENT || e >= E) continue;
                    const uint32_t nl = ix->cross[(size_t)(A[si].id & ID30) * P * E + (size_t)nxt * E + e];
                    const uint32_t g = gid_of(nxt, nl);
                    if (H.insert(g).second) { W[i] = {0.0f, g | mask}; s.ctr[ORC_C_CROSS]++; }
                }
                for (Cand& x : W)
                    if (x.id != SENT) dist_of(x);
                sort_cands(c, W.data(), XSLOTS, 1);
                merge_with_recycle(s, A.data(), L, W.data(), XSLOTS, Rc.data(), rl);
                pid[turn] = nxt;
                ++cur;
                continue;
            }
            // Expansion (gpu_graph.cu:6549-6581): R slots per channel, filled
            // in slot order (the reference's two warps race on the visited
            // set; here a lower slot takes a point first).
            for (uint32_t ch = 0; ch < 2; ++ch) {
                Cand* tc = T.data() + ch * R;
                for (uint32_t j = 0; j < R; ++j) tc[j] = {INF, SENT};
                if (te[ch] == NONE) continue;
                if (te[ch] >= cell_size(pid[ch])) {
                    // a channel's unexplored entries lie in its own cell (it
                    // leaves a cell only when none is left there)
                    std::fprintf(stderr, "orc dual: expansion outside the channel's cell\n");
                    std::abort();
                }
                s.ctr[ORC_C_EXPAND]++;
                const uint32_t mask = pid[0] == pid[1] ? 0u : (1u << (30 + ch));
                const uint32_t base = ix->offset[pid[ch]];
                const bool partner = ch != turn;
                for (uint32_t j = 0, k = 0; j < R; ++j) {
                    uint32_t g;
                    if (partner && j == R - 1) g = gid_of(pid[ch], te[ch]);
                    else g = gid_of(pid[ch], ix->graph[(size_t)(base + te[ch]) * R + k++]);
                    if (H.insert(g).second) tc[j] = {0.0f, g | mask};
                }
            }
            if (g_dual_mutation != DMUT_NO_TURN) turn ^= 1;
            for (Cand& x : T)                                // gpu_graph.cu:6582-6602
                if (x.id != SENT) dist_of(x);
            // One sort of the 2R slots (the reference's warpSort over 2R
            // lanes spans two 32-lane warps, whose halves it sorts apart).
            sort_cands(c, T.data(), 2 * R, 0);
            if (T[0].id != SENT)                             // gpu_graph.cu:6603-6616
                merge_with_recycle(s, A.data(), L, T.data(), 2 * R, Rc.data(), rl);
        }
        // Post-filter + recycle merge (gpu_graph.cu:6618-6639).
        for (Cand& x : A)
            if (x.id != SENT && !passes(s, x.id & ID30)) x = {INF, SENT};
        sort_cands(c, A.data(), L, 1);
        if (Rc[0].id != SENT) merge_plain(c, A.data(), L, Rc.data(), rl);
        out = A;
    } else if (traverse) {
        s.ctr[ORC_C_ROUTE] = 1;
        std::vector<Cand> A(L, Cand{INF, SENT}), B(R, Cand{INF, SENT}), Rc(rl, Cand{INF, SENT});
        std::vector<Cand> W(XSLOTS);
        std::unordered_set<uint32_t> H;
        H.reserve(4 * (L + XSLOTS + 4 * R));
        // Entry points of the first cell (gpu_graph.cu:3347-3351).  The
        // reference inserts their *point ids* into the visited set, which is
        // otherwise keyed by cell-local ids; kept as is.  entry[j] is reduced
        // modulo the cell size (the reference draws them from
        // [0, N-(P-1)*ceil(N/P)) and reads past a smaller first cell).
        {
            const uint32_t c0 = cl[0], sz0 = cell_size(c0);
            for (uint32_t j = 0; j < R; ++j) {
                const uint32_t lid = entry[j] % sz0;
                uint32_t gid = ix->global_idx[ix->offset[c0] + lid];
                B[j] = {INF, gid};
                H.insert(g_mutation == MUT_ENTRY_LOCAL_KEY ? lid : gid);
            }
        }
        for (uint32_t p_i = 0; p_i < cnt; ++p_i) {
            const uint32_t cur = cl[p_i];
            const uint32_t base = ix->offset[cur];
            // Distances of the cell's entries (gpu_graph.cu:3384-3405).  For
            // later cells the entries come from the sorted cross-edge slots,
            // whose distances were just computed; the reference recomputes the
            // same values, here they are reused.
            for (uint32_t j = 0; j < R; ++j) {
                if (B[j].id == SENT) { B[j].d = INF; continue; }
                if (p_i > 0) continue;
                B[j].d = point_dist(s, B[j].id);
                s.ctr[ORC_C_DIST]++; s.ctr[ORC_C_ATTR]++;
            }
            sort_cands(c, B.data(), R, 0);
            merge_with_recycle(s, A.data(), L, B.data(), R, Rc.data(), rl);

            for (uint32_t it = 0; it < g_max_iter; ++it) {
                if ((it + 1) % reset_every == 0) {            // gpu_graph.cu:3441-3454
                    H.clear();
                    for (const auto* arr : {&A, &B})
                        for (const Cand& x : *arr) {
                            if (x.id == SENT) continue;
                            uint32_t g = x.id & IDM;
                            H.insert(ix->local_idx[g]);
                            if (!in_cell(c, g, cur)) s.ctr[ORC_C_LROW]++;
                        }
                }
                uint32_t sel = L;                            // gpu_graph.cu:3457-3485
                for (uint32_t j = 0; j < L; ++j)
                    if ((A[j].id & EXPL) == 0) { sel = j; break; }
                if (sel == L) break;
                A[sel].id |= EXPL;
                s.ctr[ORC_C_EXPAND]++;
                if (tr) { tr->expanded.push_back(A[sel].id & IDM); tr->expanded_cell.push_back(cur); }
                const uint32_t tl = ix->local_idx[A[sel].id & IDM];
                for (uint32_t j = 0; j < R; ++j) {           // gpu_graph.cu:3500-3530
                    uint32_t nl = ix->graph[(size_t)(base + tl) * R + j];
                    uint32_t gid = ix->global_idx[base + nl];
                    bool isnew = H.insert(nl).second;
                    B[j] = {INF, gid};
                    s.ctr[ORC_C_ATTR]++;
                    if (isnew) { B[j].d = point_dist(s, gid); s.ctr[ORC_C_DIST]++; }
                    else if (g_mutation == MUT_DROP_SEEN) B[j].id = SENT;
                }
                sort_cands(c, B.data(), R, 0);
                if (B[0].id != SENT)
                    merge_with_recycle(s, A.data(), L, B.data(), R, Rc.data(), rl);
            }
            // End of cell (gpu_graph.cu:3555-3560).
            if (g_mutation != MUT_NO_END_EXPLORE)
                for (Cand& x : A) x.id |= EXPL;
            H.clear();
            if (p_i + 1 < cnt) {                             // gpu_graph.cu:3564-3642
                const uint32_t nxt = cl[p_i + 1];
                const uint32_t nbase = ix->offset[nxt], nsz = cell_size(nxt);
                for (uint32_t i = 0; i < XSLOTS; ++i) W[i] = {INF, SENT};
                for (uint32_t i = 0; i < std::min(XSTEP, L); ++i)
                    if (A[i].id != SENT) s.ctr[ORC_C_CROSS]++;
                for (uint32_t i = 0; i < XSLOTS; ++i) {
                    const uint32_t ci = g_mutation == MUT_SLOT_HALF ? i / 2 : (g_mutation == MUT_SLOT_32 ? i % 32 : i % XSTEP);
                    if (ci >= L || A[ci].id == SENT) continue;  // in-bounds guard (the reference tests ci > L)
                    const uint32_t g = A[ci].id & IDM;
                    bool got = false;
                    for (uint32_t jj = 0; jj < E && !got; ++jj) {
                        const uint32_t j = g_mutation == MUT_CROSS_LAST_FIRST ? E - 1 - jj : jj;
                        const uint32_t xc = g_mutation == MUT_CROSS_OWN_CELL ? cur : nxt;
                        uint32_t nl = ix->cross[(size_t)g * P * E + (size_t)xc * E + j] % nsz;
                        if (H.insert(nl).second) { W[i].id = ix->global_idx[nbase + nl]; got = true; }
                    }
                    if (!got)                                // fallback: scan [0, |cell|), not [0, 62500)
                        for (uint32_t rp = 0; rp < nsz; ++rp)
                            if (H.insert(rp).second) { W[i].id = ix->global_idx[nbase + rp]; break; }
                }
                for (uint32_t i = 0; i < XSLOTS; ++i) {
                    if (W[i].id == SENT) continue;
                    W[i].d = point_dist(s, W[i].id);
                    s.ctr[ORC_C_DIST]++; s.ctr[ORC_C_ATTR]++;
                }
                sort_cands(c, W.data(), XSLOTS, 1);
                H.clear();
                const uint32_t e0 = g_mutation == MUT_ENTRIES_AFTER ? R : 0;
                for (uint32_t j = 0; j < R; ++j) B[j] = W[e0 + j];
                if (e0) for (uint32_t j = 0; j < R; ++j) W[R + j] = W[j];
                for (uint32_t i = 0; i < XSLOTS; ++i)
                    if (W[i].id != SENT) H.insert(ix->local_idx[W[i].id]);
                merge_plain(c, A.data(), L, W.data() + R, XSTEP);
                for (const Cand& x : A) {
                    if (x.id == SENT) continue;
                    uint32_t g = x.id & IDM;
                    H.insert(ix->local_idx[g]);
                    if (!in_cell(c, g, nxt)) s.ctr[ORC_C_LROW]++;
                }
            }
        }
        // Post-filter + recycle merge (gpu_graph.cu:4025-4047).
        if (g_mutation != MUT_NO_POSTFILTER)
            for (Cand& x : A)
                if (x.id != SENT && !passes(s, x.id & IDM)) x = {INF, SENT};
        sort_cands(c, A.data(), L, 1);
        if (tr) tr->recycle = Rc;
        if (Rc[0].id != SENT) merge_plain(c, A.data(), L, Rc.data(), rl);
        out = A;
    } else if (full) {
        // The full-graph branch (gpu_graph.cu:3644-3787, disabled in the
        // reference by `&& false`): a graph search over the full graph from
        // its FD entry points, visited set keyed by point id, neighbours seen
        // before dropped, plain merge_top; every fourth iteration the visited
        // set is rebuilt from the list and the B region.  Then the common
        // post-filter (gpu_graph.cu:4025-4041); the recycle list is empty.
        s.ctr[ORC_C_ROUTE] = 3;
        const uint32_t FD = ix->FD;
        std::vector<Cand> A(L, Cand{INF, SENT}), B(FD, Cand{INF, SENT});
        std::unordered_set<uint32_t> H;
        for (uint32_t j = 0; j < FD; ++j) {                  // gpu_graph.cu:3646-3683
            const uint32_t g = ix->fentry[j];
            if (g_mutation != MUT_FULL_ENTRY_UNSEEN) H.insert(g);
            B[j] = {point_dist(s, g), g};
            s.ctr[ORC_C_DIST]++; s.ctr[ORC_C_ATTR]++;
        }
        sort_cands(c, B.data(), FD, 1);
        merge_plain(c, A.data(), L, B.data(), FD);
        for (uint32_t it = 0; it < g_max_iter; ++it) {
            if ((it + 1) % reset_every == 0) {            // gpu_graph.cu:3688-3702
                H.clear();
                for (const auto* arr : {&A, &B}) {
                    if (arr == &B && g_mutation == MUT_FULL_NO_B_REHASH) continue;
                    for (const Cand& x : *arr)
                        if (x.id != SENT) H.insert(x.id & IDM);
                }
            }
            uint32_t sel = L;                            // gpu_graph.cu:3704-3732
            for (uint32_t j = 0; j < L; ++j)
                if ((A[j].id & EXPL) == 0) { sel = j; break; }
            if (sel == L) break;
            A[sel].id |= EXPL;
            s.ctr[ORC_C_EXPAND]++;
            if (tr) { tr->expanded.push_back(A[sel].id & IDM); tr->expanded_cell.push_back(P); }
            const uint32_t g = A[sel].id & IDM;
            for (uint32_t j = 0; j < FD; ++j) {           // gpu_graph.cu:3741-3775
                const uint32_t nb = ix->fgraph[(size_t)g * FD + j];
                B[j] = {INF, SENT};
                if (nb == SENT || !H.insert(nb).second) continue;
                B[j] = {point_dist(s, nb), nb};
                s.ctr[ORC_C_DIST]++; s.ctr[ORC_C_ATTR]++;
            }
            sort_cands(c, B.data(), FD, 1);
            merge_plain(c, A.data(), L, B.data(), FD);
        }
        if (g_mutation != MUT_NO_POSTFILTER)
            for (Cand& x : A)
                if (x.id != SENT && !passes(s, x.id & IDM)) x = {INF, SENT};
        sort_cands(c, A.data(), L, 1);
        out = A;
    } else {
        // Filtered brute force over the first `little` cells (gpu_graph.cu:3788-4022).
        s.ctr[ORC_C_ROUTE] = lit ? 2 : 0;
        std::vector<Cand> found;
        for (uint32_t g = 0; g < lit; ++g) {
            const uint32_t cc = cl[g];
            const uint32_t b = ix->offset[cc], sz = cell_size(cc);
            s.ctr[ORC_C_SCAN] += sz;
            for (uint32_t l = 0; l < sz; ++l) {
                uint32_t gid = ix->global_idx[b + l];
                if (!passes(s, gid)) continue;
                s.ctr[ORC_C_PASS]++;
                s.ctr[ORC_C_DIST]++;
                found.push_back({point_dist(s, gid), gid});
            }
        }
        size_t kk = std::min<size_t>(K, found.size());
        Ctx ct = c;
        ct.tie = 0;   // the brute force keeps (distance, cell-major position) order in both tie modes
        std::partial_sort(found.begin(), found.begin() + kk, found.end(),
                          [&](const Cand& x, const Cand& y) { return cless(ct, x, y); });
        found.resize(kk);
        out = found;
    }
    // Output: the first K distinct ids (the reference merges top and recycle
    // without deduplication and may repeat an id, gpu_graph.cu:4044-4047).
    // In tie mode 0 the copies of one id are adjacent (equal keys) and every
    // empty entry follows the valid ones; in mode 1 equal distances of other
    // points, empty entries included, may sit between them.
    uint32_t n = 0;
    for (const Cand& x : out) {
        if (n >= K) break;
        if (x.id == SENT) continue;
        uint32_t id = x.id & ID30;
        bool dup = false;
        for (uint32_t t = 0; t < n && !dup; ++t) dup = out_ids[(size_t)qi * K + t] == id;
        if (dup) continue;
        out_ids[(size_t)qi * K + n] = id;
        out_dist[(size_t)qi * K + n] = x.d;
        ++n;
    }
    for (; n < K; ++n) {
        out_ids[(size_t)qi * K + n] = ORC_SENTINEL_ID;
        out_dist[(size_t)qi * K + n] = INF;
    }
    if (counters) std::memcpy(counters + (size_t)qi * ORC_NCNT, s.ctr, sizeof(s.ctr));
}

}  // namespace

extern "C" {

void orc_idx_mapper(uint32_t N, uint32_t P, const uint32_t* global_pid,
                    uint32_t* global_idx, uint32_t* local_idx, uint32_t* offset) {
    std::vector<uint32_t> sz(P, 0), fill(P, 0);
    for (uint32_t i = 0; i < N; ++i) sz[global_pid[i]]++;
    offset[0] = 0;
    for (uint32_t c = 0; c < P; ++c) offset[c + 1] = offset[c] + sz[c];
    for (uint32_t i = 0; i < N; ++i) {
        uint32_t c = global_pid[i];
        global_idx[offset[c] + fill[c]] = i;
        local_idx[i] = fill[c]++;
    }
}

uint16_t orc_f2h_one(float x, float alpha) {
    float f = x * alpha;
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t ex = (u >> 23) & 0xFFu, man = u & 0x7FFFFFu;
    if (ex == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0u));
    if (ex == 0 && man == 0) return sign;
    int e = (int)ex - 127 + 15;
    if (e <= 0) {                       // binary16 subnormal (or zero)
        uint32_t m = man | (ex ? 0x800000u : 0u);
        int shift = 14 - e;
        if (shift > 24) return sign;
        uint32_t hm = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13, rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) {
        hm++;
        if (hm == 0x400u) { hm = 0; e++; }
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | hm);
}

void orc_f2h(const float* x, size_t n, float alpha, uint16_t* out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f2h_one(x[i], alpha);
}

float orc_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    uint32_t u;
    if (ex == 0) {
        if (man == 0) u = sign;
        else {                           // subnormal: normalise
            int e = -1;
            do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (ex == 0x1Fu) {
        u = sign | 0x7F800000u | (man << 13);
    } else {
        u = sign | ((ex - 15 + 127) << 23) | (man << 13);
    }
    float f; std::memcpy(&f, &u, 4); return f;
}

void orc_row_norms_f16(const uint16_t* x, uint32_t n, uint32_t D, float* out) {
    for (uint32_t r = 0; r < n; ++r) {
        float s[64];
        for (uint32_t l = 0; l < 64; ++l) {
            float acc = 0.0f;
            for (uint32_t j = l; j < D; j += 64) {
                float v = orc_h2f(x[(size_t)r * D + j]);
                acc = std::fmaf(v, v, acc);
            }
            s[l] = acc;
        }
        for (uint32_t m = 32; m >= 1; m >>= 1) {
            float t[64];
            for (uint32_t l = 0; l < 64; ++l) t[l] = s[l] + s[l ^ m];
            std::memcpy(s, t, sizeof(s));
        }
        out[r] = s[0];
    }
}

void orc_centres_hist(uint32_t N, uint32_t D, uint32_t C, uint32_t P,
                      const float* data, const int32_t* labels,
                      const uint32_t* global_pid, int32_t contiguous,
                      float* centres, uint32_t* hist) {
    std::vector<uint32_t> num(C, 0);
    std::fill(centres, centres + (size_t)C * D, 0.0f);
    std::fill(hist, hist + (size_t)P * C, 0u);
    const uint32_t avg = (N + P - 1) / P;
    for (uint32_t i = 0; i < N; ++i) {
        uint32_t pid = contiguous ? std::min(i / avg, P - 1) : global_pid[i];
        uint32_t cid = (uint32_t)labels[i];
        num[cid]++; hist[(size_t)pid * C + cid]++;
        for (uint32_t j = 0; j < D; ++j) centres[(size_t)cid * D + j] += data[(size_t)i * D + j];
    }
    for (uint32_t c = 0; c < C; ++c)
        for (uint32_t j = 0; j < D; ++j) centres[(size_t)c * D + j] /= (float)num[c];
}

void orc_cells(uint32_t Q, uint32_t a, const float* lo, const float* hi,
               const uint32_t* grid, const float* l_q, const float* r_q,
               const uint32_t* cell_size, uint32_t* cells, uint32_t* counts) {
    uint32_t P = 1;
    for (uint32_t d = 0; d < a; ++d) P *= grid[d];
    std::vector<uint32_t> doff(a, 0);
    for (uint32_t d = 1; d < a; ++d) doff[d] = doff[d - 1] + grid[d - 1];
    for (uint32_t q = 0; q < Q; ++q) {
        std::vector<int64_t> cl(a), ch(a);
        bool empty = false;
        for (uint32_t d = 0; d < a; ++d) {
            const uint32_t g = grid[d];
            const float* rq = r_q + doff[d];
            const float* lq = l_q + doff[d];
            int64_t i = 0;                           // to_lower_bound_linear_scan
            while (i < g && rq[i] < lo[(size_t)q * a + d]) ++i;
            int64_t j = 0;                           // to_upper_bound_linear_scan
            while (j < g && lq[j] <= hi[(size_t)q * a + d]) ++j;
            cl[d] = i; ch[d] = j - 1;
            if (cl[d] >= g || ch[d] < 0) empty = true;   // range outside every cell
            ch[d] = std::max(ch[d], cl[d]);
        }
        std::vector<char> sel(P, 0);
        if (!empty) {
            std::vector<int64_t> idx(cl);
            while (true) {
                uint32_t pid = 0, f = 1;
                for (int d = (int)a - 1; d >= 0; --d) { pid += (uint32_t)idx[d] * f; f *= grid[d]; }
                sel[pid] = 1;
                uint32_t pos = 0;
                while (pos < a) {
                    idx[pos]++;
                    if (idx[pos] <= ch[pos]) break;
                    idx[pos] = cl[pos];
                    ++pos;
                }
                if (pos >= a) break;
            }
        }
        uint32_t n = 0;
        for (uint32_t p = 0; p < P; ++p)
            if (sel[p] && (!cell_size || cell_size[p] > 0)) cells[(size_t)q * P + n++] = p;
        counts[q] = n;
    }
}

void orc_cells_grid(uint32_t Q, uint32_t a, const float* lo, const float* hi, const uint32_t* grid,
                    const float* amin, const float* width, double thr, const uint32_t* cell_size,
                    uint32_t* cells, uint32_t* counts, uint32_t* little, uint8_t* flags) {
    uint32_t P = 1;
    for (uint32_t d = 0; d < a; ++d) P *= grid[d];
    for (uint32_t q = 0; q < Q; ++q) {
        uint8_t* fl = flags + (size_t)q * P;
        std::memset(fl, 0, P);
        std::vector<int64_t> cl(a), ch(a);
        bool empty = false;
        for (uint32_t d = 0; d < a; ++d) {
            const float vl = lo[(size_t)q * a + d], vh = hi[(size_t)q * a + d];
            const int64_t g = grid[d];
            if (!(vl <= vh)) empty = true;
            // (unsigned)((l - min) / width) in fp32, both ends clamped to [0, g - 1]
            auto index = [&](float v) -> int64_t {
                const float x = (v - amin[d]) / width[d];
                if (!(x > 0.0f)) return 0;
                if (x >= (float)g) return g - 1;
                return (int64_t)x;
            };
            cl[d] = index(vl);
            ch[d] = index(vh);
        }
        uint32_t n = 0, nl = 0;
        if (!empty) {
            std::vector<int64_t> idx(cl);
            while (true) {
                uint32_t pid = 0, f = 1;
                for (int d = (int)a - 1; d >= 0; --d) { pid += (uint32_t)idx[d] * f; f *= grid[d]; }
                if (!cell_size || cell_size[pid] > 0) {
                    double area = 1.0;                      // gpu_graph.cu:11158-11168
                    for (uint32_t d = 0; d < a; ++d) {
                        const double step = (double)idx[d], w = (double)width[d], m = (double)amin[d];
                        const double lb = std::max(m + step * w, (double)lo[(size_t)q * a + d]);
                        const double rb = std::min(m + (step + 1.0) * w, (double)hi[(size_t)q * a + d]);
                        area *= (rb - lb) / w;
                    }
                    const bool lit = area <= thr;
                    cells[(size_t)q * P + n++] = pid;
                    nl += lit;
                    fl[pid] = (uint8_t)(1u | (lit ? 2u : 0u));
                }
                int d = (int)a - 1;                           // last attribute fastest: ascending ids
                for (; d >= 0; --d) {
                    if (++idx[d] <= ch[d]) break;
                    idx[d] = cl[d];
                }
                if (d < 0) break;
            }
        }
        counts[q] = n;
        little[q] = nl;
    }
}

void orc_selectivity(uint32_t Q, uint32_t N, uint32_t a, const float* attrs,
                     const float* lo, const float* hi, float threshold,
                     const uint32_t* counts, uint32_t* selcount, uint32_t* little,
                     int nthreads) {
#pragma omp parallel for schedule(dynamic, 4) num_threads(nthreads > 0 ? nthreads : omp_get_max_threads())
    for (int64_t q = 0; q < (int64_t)Q; ++q) {
        uint32_t cnt = 0;
        for (uint32_t i = 0; i < N; ++i) {
            bool ok = true;
            for (uint32_t d = 0; d < a && ok; ++d) {
                float v = attrs[(size_t)i * a + d];
                ok = v >= lo[q * a + d] && v <= hi[q * a + d];
            }
            cnt += ok;
        }
        selcount[q] = cnt;
        float proportion = (float)((1.0 * cnt) / (1.0 * N));   // real_dataset_adapter.cuh:378
        little[q] = proportion <= threshold ? counts[q] : 0u;
    }
}

void orc_centroid_dist_f64(uint32_t Q, uint32_t C, uint32_t D,
                           const uint16_t* qh, const uint16_t* ch, double* out) {
    for (uint32_t q = 0; q < Q; ++q)
        for (uint32_t c = 0; c < C; ++c) {
            double qq = 0, cc = 0, qc = 0;
            for (uint32_t j = 0; j < D; ++j) {
                double x = orc_h2f(qh[(size_t)q * D + j]), y = orc_h2f(ch[(size_t)c * D + j]);
                qq += x * x; cc += y * y; qc += x * y;
            }
            out[(size_t)q * C + c] = qq + cc - 2.0 * qc;
        }
}

void orc_topk_clusters(uint32_t Q, uint32_t C, uint32_t k, const float* dist, uint32_t* out) {
    std::vector<uint32_t> idx(C);
    for (uint32_t q = 0; q < Q; ++q) {
        const float* d = dist + (size_t)q * C;
        for (uint32_t c = 0; c < C; ++c) idx[c] = c;
        auto key = [&](uint32_t c) { float v = d[c]; return std::isnan(v) ? INF : v; };
        uint32_t kk = std::min(k, C);
        std::partial_sort(idx.begin(), idx.begin() + kk, idx.end(), [&](uint32_t x, uint32_t y) {
            float a = key(x), b = key(y);
            return a != b ? a < b : x < y;
        });
        for (uint32_t t = 0; t < k; ++t) out[(size_t)q * k + t] = t < kk ? idx[t] : 0u;
    }
}

void orc_sort_cells(uint32_t Q, uint32_t P, uint32_t C, uint32_t k, uint32_t* cells,
                    const uint32_t* counts, const uint32_t* topk, const uint32_t* hist) {
    for (uint32_t q = 0; q < Q; ++q) {
        uint32_t* cl = cells + (size_t)q * P;
        const uint32_t n = counts[q];
        std::vector<std::pair<int64_t, uint32_t>> v(n);
        for (uint32_t i = 0; i < n; ++i) {
            int64_t sc = 0;
            for (uint32_t t = 0; t < k; ++t) sc += hist[(size_t)cl[i] * C + topk[(size_t)q * k + t]];
            v[i] = {sc, cl[i]};
        }
        if (g_tie_mode == 1) {
            // bitonic_sort_id_by_num_int (gpu_graph.cu:123-141): descending,
            // a swap when the upper score is smaller, over the stage A order
            for (uint32_t stride = 1; stride < n; stride <<= 1)
                for (uint32_t step = stride; step > 0; step >>= 1)
                    for (uint32_t kk = 0; kk < n / 2; ++kk) {
                        const uint32_t a0 = 2 * step * (kk / step), b0 = kk % step;
                        const uint32_t u = step == stride ? a0 + step - 1 - b0 : a0 + b0;
                        const uint32_t d = a0 + b0 + step;
                        if (d < n && (int32_t)v[u].first < (int32_t)v[d].first) std::swap(v[u], v[d]);
                    }
        } else {
            std::sort(v.begin(), v.end(), [](const std::pair<int64_t, uint32_t>& x,
                                             const std::pair<int64_t, uint32_t>& y) {
                return x.first != y.first ? x.first > y.first : x.second < y.second;
            });
        }
        for (uint32_t i = 0; i < n; ++i) cl[i] = v[i].second;
    }
}

void orc_entry_draw(uint32_t range, uint32_t ndraw, uint32_t R, uint32_t* out) {
    std::mt19937 rng;
    std::uniform_int_distribution<> intd(0, (int)range - 1);
    const uint32_t want = std::min<uint32_t>(ndraw, range);
    std::vector<unsigned> v(want);
    std::unordered_set<unsigned> seen;
    uint32_t k = 0;
    while (k < want) {
        unsigned t = (unsigned)intd(rng);
        if (!seen.count(t)) { seen.insert(t); v[k++] = t; }
    }
    std::srand(1);
    std::random_shuffle(v.begin(), v.begin() + want);
    for (uint32_t j = 0; j < R; ++j) out[j] = j < want ? v[j] : j;
}

void orc_entry_points(uint32_t N, uint32_t P, uint32_t R, uint32_t* out) {
    const uint32_t avg = (N + P - 1) / P;
    orc_entry_draw(N - (P - 1) * avg, R * 10, R, out);
}

void orc_entry_points_pair(uint32_t N, uint32_t P, uint32_t R, uint32_t FD, uint32_t* out, uint32_t* outf) {
    // One mt19937 for both draws; random_shuffle's std::rand seeded once
    // (gpu_graph.cu:12506-12537).
    const uint32_t avg = (N + P - 1) / P;
    std::mt19937 rng;
    auto draw = [&](uint32_t range, uint32_t want, std::vector<unsigned>& v) {
        std::uniform_int_distribution<> intd(0, (int)range - 1);
        want = std::min(want, range);
        v.assign(want, 0);
        std::unordered_set<unsigned> seen;
        for (uint32_t k = 0; k < want;) {
            const unsigned t = (unsigned)intd(rng);
            if (seen.insert(t).second) v[k++] = t;
        }
    };
    std::vector<unsigned> v;
    draw(N - (P - 1) * avg, 10 * R, v);
    std::srand(1);
    std::random_shuffle(v.begin(), v.end());
    for (uint32_t j = 0; j < R; ++j) out[j] = j < v.size() ? v[j] : j;
    if (!FD) return;
    draw(N, 10 * FD, v);
    std::random_shuffle(v.begin(), v.end());
    for (uint32_t j = 0; j < FD; ++j) outf[j] = j < v.size() ? v[j] : j;
}

void orc_full_graph(const orc_index* ix, uint32_t FE, uint32_t* out) {
    const uint32_t N = ix->N, P = ix->P, R = ix->R, E = ix->E, FD = FE * P;
    std::vector<uint32_t> cellof(N);
    for (uint32_t c = 0; c < P; ++c)
        for (uint32_t r = ix->offset[c]; r < ix->offset[c + 1]; ++r) cellof[ix->global_idx[r]] = c;
    for (uint32_t g = 0; g < N; ++g)
        for (uint32_t c = 0; c < P; ++c) {
            const uint32_t sz = ix->offset[c + 1] - ix->offset[c];
            for (uint32_t e = 0; e < FE; ++e) {
                uint32_t v = SENT;
                if (sz) {
                    const uint32_t l = c == cellof[g] && g_mutation != MUT_FULL_OWN_AS_CROSS
                        ? ix->graph[(size_t)(ix->offset[c] + ix->local_idx[g]) * R + e]
                        : ix->cross[(size_t)g * P * E + (size_t)c * E + e];
                    v = ix->global_idx[ix->offset[c] + l % sz];
                }
                out[(size_t)g * FD + (size_t)c * FE + e] = v;
            }
        }
}

void orc_canon_dists(const float* q, const float* X, uint32_t n, uint32_t D, float* out) {
    for (uint32_t i = 0; i < n; ++i) out[i] = canon_dist(q, X + (size_t)i * D, D, 0);
}

float orc_distance(const orc_index* ix, const void* q, uint32_t gid) {
    std::vector<float> qv(ix->D), xv(ix->D);
    if (ix->vdtype == 3) {
        for (uint32_t k = 0; k < ix->D; ++k)
            qv[k] = std::fmaf(ix->qscale[k], float(ix->qzero[k]), ((const float*)q)[k]);
        return canon_dist(qv.data(), ix->vec_f32 + (size_t)gid * ix->D, ix->D, 3, ix->qscale);
    }
    if (ix->vdtype != 1)
        return canon_dist((const float*)q, ix->vec_f32 + (size_t)gid * ix->D, ix->D, ix->vdtype);
    if (g_dist_mode == 1) return hfma2_dist((const uint16_t*)q, ix->vec_f16 + (size_t)gid * ix->D, ix->D);
    for (uint32_t i = 0; i < ix->D; ++i) {
        qv[i] = orc_h2f(((const uint16_t*)q)[i]);
        xv[i] = orc_h2f(ix->vec_f16[(size_t)gid * ix->D + i]);
    }
    return canon_dist(qv.data(), xv.data(), ix->D, 1);
}

void orc_search(const orc_index* ix, const void* queries, uint32_t Q,
                const float* lo, const float* hi,
                const uint32_t* cells, const uint32_t* counts, const uint32_t* little,
                const uint32_t* entry, uint32_t L, uint32_t K, uint32_t rl,
                uint32_t postfilter, uint32_t* out_ids, float* out_dist,
                uint32_t* counters, int nthreads) {
    std::vector<uint32_t> cmpos(ix->N), cellof(ix->N);
    for (uint32_t c = 0; c < ix->P; ++c)
        for (uint32_t r = ix->offset[c]; r < ix->offset[c + 1]; ++r) {
            cmpos[ix->global_idx[r]] = r;
            cellof[ix->global_idx[r]] = c;
        }
    Ctx c{ix, cmpos.data(), cellof.data(), g_tie_mode};
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : omp_get_max_threads())
    for (int64_t q = 0; q < (int64_t)Q; ++q)
        search_one(c, queries, (uint32_t)q, lo, hi, cells, counts, little, entry, L, K, rl,
                   postfilter, out_ids, out_dist, counters);
}

void orc_set_tie_mode(int mode) { g_tie_mode = mode; }
void orc_set_dist_mode(int mode) { g_dist_mode = mode; }
uint16_t orc_half_rne(double v) { return half_rne(v); }
float orc_hfma2_dist(const uint16_t* q, const uint16_t* x, uint32_t D) { return hfma2_dist(q, x, D); }
void orc_set_mutation(int m) { g_mutation = m; }
void orc_set_max_iter(uint32_t n) { g_max_iter = n ? n : MAX_ITER; }
void orc_set_channels(int n) { g_channels = n == 2 ? 2 : 1; }
void orc_set_dual_mutation(int m) { g_dual_mutation = m; }

uint32_t orc_search_trace(const orc_index* ix, const void* queries, uint32_t qi, const float* lo, const float* hi,
                          const uint32_t* cells, const uint32_t* counts, const uint32_t* entry, uint32_t L,
                          uint32_t K, uint32_t rl, uint32_t* out_ids, float* out_dist, uint32_t* counters,
                          uint32_t* expanded, uint32_t* expanded_cell, uint32_t cap, uint32_t* rec_ids,
                          float* rec_dist, uint32_t postfilter) {
    std::vector<uint32_t> cmpos(ix->N), cellof(ix->N);
    for (uint32_t c = 0; c < ix->P; ++c)
        for (uint32_t r = ix->offset[c]; r < ix->offset[c + 1]; ++r) {
            cmpos[ix->global_idx[r]] = r;
            cellof[ix->global_idx[r]] = c;
        }
    Ctx c{ix, cmpos.data(), cellof.data(), g_tie_mode};
    Trace tr;
    std::vector<uint32_t> little(qi + 1, 0);
    std::vector<uint32_t> ids((size_t)(qi + 1) * K), ctr((size_t)(qi + 1) * ORC_NCNT);
    std::vector<float> dist((size_t)(qi + 1) * K);
    search_one(c, queries, qi, lo, hi, cells, counts, little.data(), entry, L, K, rl, postfilter, ids.data(),
               dist.data(), ctr.data(), &tr);
    std::memcpy(out_ids, &ids[(size_t)qi * K], K * sizeof(uint32_t));
    std::memcpy(out_dist, &dist[(size_t)qi * K], K * sizeof(float));
    std::memcpy(counters, &ctr[(size_t)qi * ORC_NCNT], ORC_NCNT * sizeof(uint32_t));
    for (size_t i = 0; i < tr.expanded.size() && i < cap; ++i) {
        expanded[i] = tr.expanded[i];
        expanded_cell[i] = tr.expanded_cell[i];
    }
    for (uint32_t t = 0; t < rl; ++t) {
        rec_ids[t] = tr.recycle.empty() || tr.recycle[t].id == SENT ? ORC_SENTINEL_ID : (tr.recycle[t].id & IDM);
        rec_dist[t] = tr.recycle.empty() ? INF : tr.recycle[t].d;
    }
    return (uint32_t)tr.expanded.size();
}

void orc_bitonic_sort_dis(float* dis, uint32_t* ids, uint32_t len) { bitonic_no_explore(dis, ids, len); }
void orc_warp_sort(float* key, uint32_t* val, uint32_t len) { warp_sort(key, val, len); }

void orc_merge_top(float* d1, uint32_t* i1, uint32_t n, float* d2, uint32_t* i2, uint32_t m, int tie) {
    std::vector<uint32_t> ident;
    uint32_t mx = 0;
    for (uint32_t i = 0; i < n; ++i) if (i1[i] != SENT) mx = std::max(mx, i1[i] & IDM);
    for (uint32_t j = 0; j < m; ++j) if (i2[j] != SENT) mx = std::max(mx, i2[j] & IDM);
    ident.resize((size_t)mx + 1);
    for (uint32_t i = 0; i <= mx; ++i) ident[i] = i;
    Ctx c{nullptr, ident.data(), nullptr, tie};
    std::vector<Cand> X(n), Y(m);
    for (uint32_t i = 0; i < n; ++i) X[i] = {d1[i], i1[i]};
    for (uint32_t j = 0; j < m; ++j) Y[j] = {d2[j], i2[j]};
    merge_plain(c, X.data(), n, Y.data(), m);
    for (uint32_t i = 0; i < n; ++i) { d1[i] = X[i].d; i1[i] = X[i].id; }
    for (uint32_t j = 0; j < m; ++j) { d2[j] = Y[j].d; i2[j] = Y[j].id; }
}

void orc_merge_recycle(const float* attrs, uint32_t a, const float* lo, const float* hi, float* dA, uint32_t* iA,
                       uint32_t L, float* dB, uint32_t* iB, uint32_t R, float* dR, uint32_t* iR, uint32_t rl,
                       int tie) {
    std::vector<uint32_t> ident;
    uint32_t mx = 0;
    for (uint32_t i = 0; i < L; ++i) if (iA[i] != SENT) mx = std::max(mx, iA[i] & IDM);
    for (uint32_t j = 0; j < R; ++j) if (iB[j] != SENT) mx = std::max(mx, iB[j] & IDM);
    for (uint32_t j = 0; j < rl; ++j) if (iR[j] != SENT) mx = std::max(mx, iR[j] & IDM);
    ident.resize((size_t)mx + 1);
    for (uint32_t i = 0; i <= mx; ++i) ident[i] = i;
    orc_index ix{};
    ix.a = a;
    ix.attrs = attrs;
    Ctx c{&ix, ident.data(), nullptr, tie};
    QueryState s;
    s.c = &c; s.q = nullptr; s.lo = lo; s.hi = hi;
    std::vector<Cand> A(L), B(R), Rc(rl);
    for (uint32_t i = 0; i < L; ++i) A[i] = {dA[i], iA[i]};
    for (uint32_t j = 0; j < R; ++j) B[j] = {dB[j], iB[j]};
    for (uint32_t j = 0; j < rl; ++j) Rc[j] = {dR[j], iR[j]};
    merge_with_recycle(s, A.data(), L, B.data(), R, Rc.data(), rl);
    for (uint32_t i = 0; i < L; ++i) { dA[i] = A[i].d; iA[i] = A[i].id; }
    for (uint32_t j = 0; j < R; ++j) { dB[j] = B[j].d; iB[j] = B[j].id; }
    for (uint32_t j = 0; j < rl; ++j) { dR[j] = Rc[j].d; iR[j] = Rc[j].id; }
}

void orc_ground_truth(uint32_t N, uint32_t D, uint32_t a, const float* data,
                      const float* attrs, uint32_t Q, const float* queries,
                      const float* lo, const float* hi, uint32_t K,
                      uint32_t* gt_ids, double* gt_dist, int nthreads) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : omp_get_max_threads())
    for (int64_t q = 0; q < (int64_t)Q; ++q) {
        std::vector<std::pair<double, uint32_t>> best;   // max-heap of size K
        auto cmp = [](const std::pair<double, uint32_t>& x, const std::pair<double, uint32_t>& y) {
            return x.first != y.first ? x.first < y.first : x.second < y.second;
        };
        const float* qv = queries + (size_t)q * D;
        for (uint32_t i = 0; i < N; ++i) {
            bool ok = true;
            for (uint32_t d = 0; d < a && ok; ++d) {
                float v = attrs[(size_t)i * a + d];
                ok = v >= lo[q * a + d] && v <= hi[q * a + d];
            }
            if (!ok) continue;
            double s = 0;
            const float* x = data + (size_t)i * D;
            for (uint32_t j = 0; j < D; ++j) { double t = (double)qv[j] - (double)x[j]; s += t * t; }
            std::pair<double, uint32_t> e{s, i};
            if (best.size() < K) { best.push_back(e); std::push_heap(best.begin(), best.end(), cmp); }
            else if (cmp(e, best.front())) {
                std::pop_heap(best.begin(), best.end(), cmp);
                best.back() = e;
                std::push_heap(best.begin(), best.end(), cmp);
            }
        }
        std::sort(best.begin(), best.end(), cmp);
        for (uint32_t k = 0; k < K; ++k) {
            gt_ids[(size_t)q * K + k] = k < best.size() ? best[k].second : ORC_SENTINEL_ID;
            gt_dist[(size_t)q * K + k] = k < best.size() ? best[k].first : (double)INF;
        }
    }
}

double orc_recall(uint32_t Q, uint32_t K, const uint32_t* res, const uint32_t* gt,
                  const double* gt_dist, const double* res_dist_exact, int tie_aware) {
    double total = 0;
    for (uint32_t q = 0; q < Q; ++q) {
        std::vector<uint32_t> g, r;
        double kth = -1;
        for (uint32_t k = 0; k < K; ++k) {
            if (gt[(size_t)q * K + k] != ORC_SENTINEL_ID) {
                g.push_back(gt[(size_t)q * K + k]);
                kth = gt_dist[(size_t)q * K + k];
            }
        }
        if (g.empty()) { total += 1.0; continue; }
        uint32_t hit = 0;
        if (!tie_aware) {
            for (uint32_t k = 0; k < K; ++k) r.push_back(res[(size_t)q * K + k]);
            std::sort(r.begin(), r.end());
            std::sort(g.begin(), g.end());
            std::vector<uint32_t> inter;
            std::set_intersection(r.begin(), r.end(), g.begin(), g.end(), std::back_inserter(inter));
            hit = (uint32_t)inter.size();
        } else {
            std::unordered_set<uint32_t> seen;
            for (uint32_t k = 0; k < K; ++k) {
                uint32_t id = res[(size_t)q * K + k];
                if (id == ORC_SENTINEL_ID || seen.count(id)) continue;
                seen.insert(id);
                if (res_dist_exact[(size_t)q * K + k] <= kth) hit++;
            }
            hit = std::min<uint32_t>(hit, (uint32_t)g.size());
        }
        total += (double)hit / (double)g.size();
    }
    return total / Q;
}

}  // extern "C"
