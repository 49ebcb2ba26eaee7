// Host side of libgarfield.so: the C ABI declared in include/garfield.h.
//
// gf_index_create lays every per-point array out cell-major on the device
// (row offset[c] + l is the l-th point of cell c in ascending point id order,
// the reference's get_idx_mapper order, tools.cuh:862-915), validates every
// id the kernels will dereference, and precomputes the cluster centres and
// the cell x cluster histogram (tools.cuh:569-602).  The three stage calls
// mirror the reference's host functions; see the header for the citations.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <functional>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <new>
#include <numeric>
#include <random>
#include <string>
#include <unordered_set>
#include <vector>

#include "gf_state.h"

using gf::Error;

namespace {

thread_local std::string g_last_error;

gf_status run_guarded(const std::function<void()>& fn);

}  // namespace

using gf::DevBuf;
using gf::round_up;
using gf::set_device;

namespace {

gf_status run_guarded(const std::function<void()>& fn) {
    try {
        fn();
        return GF_OK;
    } catch (const Error& e) {
        g_last_error = e.msg;
        return e.code;
    } catch (const std::bad_alloc&) {
        g_last_error = "host allocation failed";
        return GF_E_NOMEM;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return GF_E_ARG;
    }
}


// Sub-cells of every cell, built when all attributes are integers whose
// spread inside each cell is below 65534 and a <= 4 (otherwise ix.sub stays
// false and stage A / the brute force use the per-cell kernels).  A cell of n
// points gets S = round((n / 1024)^(1/a)) bins per attribute (S^a <= 4096):
// bin of a point = rank of its value among the cell's (ties by row) * S / n,
// sub-cell = row-major bin tuple.  Tiles list each sub-cell's points in
// ascending row order, padded to 16 (row 0xFFFFFFFF, low attribute half
// 65535, which no range accepts).
void build_subcells(const gf_index_host& h, const std::vector<uint32_t>& gidx, const std::vector<uint32_t>& size,
                    gf_index& ix) {
    gf::SubHost sh;
    if (!gf::compute_subcells(h, gidx, size, ix.offset_h, ix.a, ix.P, sh)) return;
    ix.AW = sh.AW;
    ix.NS = sh.NS;
    ix.ntile = sh.ntile;
    ix.ssize_h = sh.ssize;
    ix.stile_h = sh.stile;
    ix.abase.upload(sh.abase);
    ix.sbase.upload(sh.sbase);
    ix.scell.upload(sh.scell);
    ix.ssize.upload(sh.ssize);
    ix.stile.upload(sh.stile);
    ix.sbox.upload(sh.sbox);
    ix.tmeta.upload(sh.tmeta);
    ix.sorder.upload(sh.sorder);
    ix.ns1 = sh.ns1;
    ix.shash_h = std::move(sh.shash);
    ix.sub = true;
}

}  // namespace

namespace gf {

void set_last_error(const std::string& msg) { g_last_error = msg; }

// Per-dimension int8 quantisation with the reference loader's host rules
// (indexsearch/production_adapter.cuh:113-165), in fp32: x *= alpha; per
// dimension min and max starting from 100000 and -100000; scale = (max - min)
// / 255; zero point = round(-128 - min / scale) clamped to [-128, 127]; q =
// round(x / scale) + zero point clamped to [-128, 127]; round() half away from
// zero.  A dimension with max == min, where the reference divides by zero,
// takes scale 1.
void quantise_i8(const float* x, uint64_t n, uint32_t D, float alpha, std::vector<float>& scale,
                 std::vector<int32_t>& zero, int8_t* out) {
    scale.assign(D, 1.0f);
    zero.assign(D, 0);
    for (uint32_t d = 0; d < D; ++d) {
        float mn = 100000.0f, mx = -100000.0f;
        for (uint64_t i = 0; i < n; ++i) {
            const float v = x[i * D + d] * alpha;
            mn = std::min(mn, v);
            mx = std::max(mx, v);
        }
        float s = (mx - mn) / 255.0f;
        if (!(s > 0.0f)) s = 1.0f;
        // clamped in double: the reference's int conversions overflow first
        const double zr = std::round(float(-128) - mn / s);
        const int z = int(std::max(-128.0, std::min(127.0, zr)));
        for (uint64_t i = 0; i < n; ++i) {
            const double q = double(std::round(x[i * D + d] * alpha / s)) + z;
            out[i * D + d] = int8_t(std::max(-128.0, std::min(127.0, q)));
        }
        scale[d] = s;
        zero[d] = z;
    }
}

void first_pass_order(const std::vector<uint32_t>& shash, uint32_t m, std::vector<uint32_t>& order, uint32_t& ns1) {
    const uint32_t NS = uint32_t(shash.size());
    order.clear();
    for (uint32_t s = 0; s < NS; ++s)
        if (shash[s] % m == 0u) order.push_back(s);
    ns1 = uint32_t(order.size());
    for (uint32_t s = 0; s < NS; ++s)
        if (shash[s] % m != 0u) order.push_back(s);
}

bool compute_subcells(const gf_index_host& h, const std::vector<uint32_t>& gidx, const std::vector<uint32_t>& size,
                      const std::vector<uint32_t>& offset_h, uint32_t a, uint32_t P, SubHost& out) {
    if (a > 4) return false;
    std::vector<int32_t> abase(size_t(P) * a, 0);
    for (uint32_t c = 0; c < P; ++c)
        for (uint32_t d = 0; d < a; ++d) {
            double mn = 0.0, mx = 0.0;
            for (uint32_t r = offset_h[c]; r < offset_h[c + 1]; ++r) {
                const double x = h.attrs[size_t(gidx[r]) * a + d];
                if (!(x == std::floor(x) && x >= -2147483648.0 && x < 2147483648.0)) return false;
                mn = r == offset_h[c] ? x : std::min(mn, x);
                mx = r == offset_h[c] ? x : std::max(mx, x);
            }
            if (mx - mn > 65533.0) return false;
            abase[size_t(c) * a + d] = int32_t(mn);
        }
    const uint32_t AW = (a + 1) / 2, MW = 16 * (1 + AW);
    std::vector<uint32_t> sbase(P + 1, 0), scell, ssize, stile, tmeta;
    out.shash.clear();
    std::vector<int32_t> sbox;
    auto attr = [&](uint32_t r, uint32_t d) { return int32_t(h.attrs[size_t(gidx[r]) * a + d]); };
    for (uint32_t c = 0; c < P; ++c) {
        const uint32_t off = offset_h[c], n = size[c];
        uint32_t S = n ? std::max<uint32_t>(1u, uint32_t(std::lround(std::pow(n / 1024.0, 1.0 / a)))) : 1u;
        while (S > 1 && std::pow(double(S), double(a)) > 4096.0) --S;
        uint32_t nsc = 1;
        for (uint32_t d = 0; d < a; ++d) nsc *= S;
        std::vector<uint32_t> sid(n, 0), ord(n);
        for (uint32_t d = 0; d < a; ++d) {
            for (uint32_t i = 0; i < n; ++i) ord[i] = i;
            std::stable_sort(ord.begin(), ord.end(),
                             [&](uint32_t x, uint32_t y) { return attr(off + x, d) < attr(off + y, d); });
            for (uint32_t k = 0; k < n; ++k) sid[ord[k]] = sid[ord[k]] * S + uint32_t(uint64_t(k) * S / n);
        }
        std::vector<std::vector<uint32_t>> members(nsc);
        for (uint32_t i = 0; i < n; ++i) members[sid[i]].push_back(off + i);
        for (uint32_t k = 0; k < nsc; ++k) {
            const auto& m = members[k];
            // First-pass sub-cells: grid coordinates (s_0, ..., s_{a-1}) with
            // h = s_0 + 3 s_1 + 5 s_2 + 7 s_3 = 0 (mod 8), one in eight of the
            // grid and spread over every row and column of it (the float
            // route takes h = 0 mod 4: first_pass_order).
            uint32_t h = 0;
            for (uint32_t d = 0, kk = k; d < a; ++d, kk /= S) h += (2u * (a - 1u - d) + 1u) * (kk % S);
            out.shash.push_back(h);
            scell.push_back(c);
            ssize.push_back(uint32_t(m.size()));
            stile.push_back(uint32_t(tmeta.size() / MW));
            for (uint32_t d = 0; d < a; ++d) {
                int32_t mn = INT32_MAX, mx = INT32_MIN;
                for (uint32_t r : m) { mn = std::min(mn, attr(r, d)); mx = std::max(mx, attr(r, d)); }
                sbox.push_back(mn);
                sbox.push_back(mx);
            }
            for (size_t t0 = 0; t0 < m.size(); t0 += 16) {
                const size_t base = tmeta.size();
                tmeta.resize(base + MW, 0);
                for (uint32_t j = 0; j < 16; ++j) {
                    const bool valid = t0 + j < m.size();
                    const uint32_t r = valid ? m[t0 + j] : 0xFFFFFFFFu;
                    tmeta[base + j] = r;
                    for (uint32_t w = 0; w < AW; ++w) {
                        uint32_t word = 65535u;
                        if (valid) {
                            word = uint32_t(attr(r, 2 * w) - abase[size_t(c) * a + 2 * w]);
                            if (2 * w + 1 < a) word |= uint32_t(attr(r, 2 * w + 1) - abase[size_t(c) * a + 2 * w + 1]) << 16;
                        }
                        tmeta[base + 16 * (1 + w) + j] = word;
                    }
                }
            }
        }
        sbase[c + 1] = sbase[c] + nsc;
    }
    stile.push_back(uint32_t(tmeta.size() / MW));
    out.AW = AW;
    out.NS = sbase[P];
    first_pass_order(out.shash, 8, out.sorder, out.ns1);
    out.ntile = stile.back();
    out.sbase = std::move(sbase);
    out.scell = std::move(scell);
    out.ssize = std::move(ssize);
    out.stile = std::move(stile);
    out.sbox = std::move(sbox);
    out.tmeta = std::move(tmeta);
    out.abase = std::move(abase);
    return true;
}

void map_cells(const gf_index_host& h, const gf_open_opts* opts, gf_index& ix, std::vector<uint32_t>& size,
               std::vector<uint32_t>& gidx, std::vector<uint32_t>& lrow) {
    GF_REQUIRE(h.N > 0 && h.D > 0, GF_E_ARG, "N and D must be positive");
    GF_REQUIRE(h.a >= 1 && h.a <= gf::kMaxAttr, GF_E_UNSUPPORTED, "attribute count must be in [1, 8]");
    GF_REQUIRE(h.R >= 1 && h.R <= 64, GF_E_UNSUPPORTED, "graph degree must be in [1, 64]");
    GF_REQUIRE(h.E >= 1 && h.E <= gf::kMaxE, GF_E_UNSUPPORTED, "cross edges per cell must be in [1, 4]");
    GF_REQUIRE(h.N < (1u << 30), GF_E_UNSUPPORTED, "at most 2^30 points");
    GF_REQUIRE(h.vectors && h.attrs && h.grid_shape && h.l_q && h.r_q && h.global_pid && h.cell_graphs && h.cross,
               GF_E_ARG, "missing index array");
    ix.device = opts ? opts->device : 0;
    ix.vdtype = opts ? opts->vec_dtype : GF_VEC_F32;
    ix.alpha = (opts && opts->f2h_factor != 0.0f) ? opts->f2h_factor : 1.0f;
    ix.ref_ties = opts && opts->ref_ties;
    GF_REQUIRE(ix.vdtype == GF_VEC_F32 || ix.vdtype == GF_VEC_F16 || ix.vdtype == GF_VEC_U8 ||
                   ix.vdtype == GF_VEC_I8Q || ix.vdtype == GF_VEC_F16_REF, GF_E_ARG,
               "vec_dtype must be GF_VEC_F32, GF_VEC_F16, GF_VEC_U8, GF_VEC_I8Q or GF_VEC_F16_REF");
    const bool half_rows = gf::half_rows(ix.vdtype);
    GF_REQUIRE(!(opts && opts->degree) || opts->degree == h.R, GF_E_FORMAT, "--degree does not match the graph files");
    const uint32_t elems = ix.vdtype == GF_VEC_F32 ? 4u : (half_rows ? 8u : 16u);
    GF_REQUIRE(h.D % elems == 0, GF_E_UNSUPPORTED, "D must be a multiple of 4 (fp32), 8 (fp16) or 16 (u8, int8)");
    ix.rs = gf::row_shape(h.D, ix.vdtype);
    GF_REQUIRE(ix.rs.cpl <= gf::row_shape_max_cpl(ix.vdtype), GF_E_UNSUPPORTED, "D too large for this build");
    ix.rowbytes = h.D * (ix.vdtype == GF_VEC_F32 ? 4u : (half_rows ? 2u : 1u));   // u8, int8: 1

    const uint32_t N = h.N, D = h.D, a = h.a, R = h.R, E = h.E;
    uint64_t P64 = 1;
    for (uint32_t d = 0; d < a; ++d) {
        GF_REQUIRE(h.grid_shape[d] >= 1, GF_E_FORMAT, "empty grid dimension");
        P64 *= h.grid_shape[d];
    }
    GF_REQUIRE(P64 == h.P, GF_E_FORMAT, "grid shape product differs from P");
    GF_REQUIRE(P64 <= 4096, GF_E_UNSUPPORTED, "at most 4096 cells");
    const uint32_t P = uint32_t(P64);
    ix.N = N; ix.D = D; ix.a = a; ix.P = P; ix.R = R; ix.E = E;
    ix.grid_h.assign(h.grid_shape, h.grid_shape + a);

    // idx mapper (tools.cuh:862-915)
    size.assign(P, 0);
    gidx.assign(N, 0);
    lrow.assign(N, 0);
    std::vector<uint32_t> fill(P, 0);
    for (uint32_t i = 0; i < N; ++i) {
        GF_REQUIRE(h.global_pid[i] < P, GF_E_FORMAT, "global_pid out of range");
        size[h.global_pid[i]]++;
    }
    ix.offset_h.assign(P + 1, 0);
    for (uint32_t c = 0; c < P; ++c) ix.offset_h[c + 1] = ix.offset_h[c] + size[c];
    for (uint32_t i = 0; i < N; ++i) {
        const uint32_t c = h.global_pid[i];
        const uint32_t r = ix.offset_h[c] + fill[c];
        gidx[r] = i;
        lrow[r] = fill[c]++;
    }
    // Every id the kernels dereference is checked here once.
    for (uint32_t c = 0; c < P; ++c)
        for (size_t k = size_t(ix.offset_h[c]) * R; k < size_t(ix.offset_h[c + 1]) * R; ++k)
            GF_REQUIRE(h.cell_graphs[k] < size[c], GF_E_FORMAT,
                       "per-cell graph " + std::to_string(c) + " holds an id beyond the cell");
    for (uint32_t i = 0; i < N; ++i) {
        const uint32_t* src = h.cross + size_t(i) * P * E;
        for (uint32_t c = 0; c < P; ++c)
            for (uint32_t e = 0; e < E; ++e)
                // edges into an empty cell are never followed (no query selects it)
                GF_REQUIRE(src[c * E + e] < size[c] || size[c] == 0, GF_E_FORMAT,
                           "cross-cell graph holds an id beyond its cell");
    }
    if (ix.vdtype == GF_VEC_U8) {
        const size_t n = size_t(N) * D;
        for (size_t i = 0; i < n; ++i) {
            const float x = h.vectors[i];
            GF_REQUIRE(x >= 0.0f && x <= 255.0f && x == std::floor(x), GF_E_ARG,
                       "GF_VEC_U8 needs vectors of integers in [0, 255]");
        }
    }
}

void entry_points_draw(uint32_t range, uint32_t ndraw, uint32_t R, uint32_t* out) {
    GF_REQUIRE(range >= 1, GF_E_ARG, "no room for entry points");
    std::mt19937 rng;
    std::uniform_int_distribution<> intd(0, int(range) - 1);
    const uint32_t want = std::min<uint32_t>(ndraw, range);
    std::vector<unsigned> v(want);
    std::unordered_set<unsigned> seen;
    uint32_t k = 0;
    while (k < want) {
        const unsigned t = unsigned(intd(rng));
        if (!seen.count(t)) { seen.insert(t); v[k++] = t; }
    }
    std::srand(1);
    std::random_shuffle(v.begin(), v.begin() + want);
    for (uint32_t j = 0; j < R; ++j) out[j] = j < want ? v[j] : j;
}

void entry_points_pair(uint32_t range1, uint32_t R, uint32_t range2, uint32_t BD, uint32_t* out1, uint32_t* out2) {
    GF_REQUIRE(range1 >= 1 && range2 >= 1, GF_E_ARG, "no room for entry points");
    std::mt19937 rng;
    auto draw = [&](uint32_t range, uint32_t ndraw, std::vector<unsigned>& v) {
        std::uniform_int_distribution<> intd(0, int(range) - 1);
        const uint32_t want = std::min<uint32_t>(ndraw, range);
        v.assign(want, 0);
        std::unordered_set<unsigned> seen;
        uint32_t k = 0;
        while (k < want) {
            const unsigned t = unsigned(intd(rng));
            if (!seen.count(t)) { seen.insert(t); v[k++] = t; }
        }
    };
    std::vector<unsigned> v;
    draw(range1, 10 * R, v);
    std::srand(1);
    std::random_shuffle(v.begin(), v.end());
    for (uint32_t j = 0; j < R; ++j) out1[j] = j < v.size() ? v[j] : j;
    if (!BD) return;
    draw(range2, 10 * BD, v);
    std::random_shuffle(v.begin(), v.end());
    for (uint32_t j = 0; j < BD; ++j) out2[j] = j < v.size() ? v[j] : j;
}

}  // namespace gf

namespace {

void build_index(const gf_index_host& h, const gf_open_opts* opts, gf_index& ix) {
    std::vector<uint32_t> size, gidx, lrow;
    gf::map_cells(h, opts, ix, size, gidx, lrow);
    const uint32_t N = ix.N, D = ix.D, a = ix.a, P = ix.P, R = ix.R, E = ix.E;
    std::vector<uint32_t> cross_cm(size_t(N) * P * E);
    for (uint32_t r = 0; r < N; ++r)
        std::memcpy(&cross_cm[size_t(r) * P * E], h.cross + size_t(gidx[r]) * P * E, sizeof(uint32_t) * P * E);
    // All ids are validated; from here on the device is used.
    GF_HIP(hipSetDevice(ix.device));
    GF_HIP(hipStreamCreateWithFlags(&ix.stream, hipStreamNonBlocking));
    GF_HIP(hipDeviceGetAttribute(&ix.ncu, hipDeviceAttributeMultiprocessorCount, ix.device));
    GF_HIP(hipDeviceGetAttribute(&ix.wclk_khz, hipDeviceAttributeWallClockRate, ix.device));
    ix.wclk_khz = std::max(ix.wclk_khz, 1);
    ix.ncu = std::max(ix.ncu, 1);
    ix.cross.upload(cross_cm);
    std::vector<uint32_t>().swap(cross_cm);
    ix.graph.upload(h.cell_graphs, size_t(N) * R);
    ix.offset.upload(ix.offset_h);
    ix.gidx.upload(gidx);
    ix.lrow.upload(lrow);
    {
        std::vector<float> at(size_t(N) * a);
        for (uint32_t r = 0; r < N; ++r)
            for (uint32_t d = 0; d < a; ++d) at[size_t(r) * a + d] = h.attrs[size_t(gidx[r]) * a + d];
        ix.attrs.upload(at);
    }
    {
        std::vector<float> v(size_t(N) * D);
        for (uint32_t r = 0; r < N; ++r)
            std::memcpy(&v[size_t(r) * D], h.vectors + size_t(gidx[r]) * D, sizeof(float) * D);
        DevBuf<float> tmp;
        const float* vec_f32_dev = nullptr;
        if (ix.vdtype == GF_VEC_F32) {
            ix.vec.upload(reinterpret_cast<const char*>(v.data()), v.size() * sizeof(float));
            vec_f32_dev = reinterpret_cast<const float*>(ix.vec.p);
        } else if (gf::half_rows(ix.vdtype)) {
            tmp.upload(v);
            ix.vec.alloc(v.size() * sizeof(uint16_t));
            GF_HIP(gf::launch_f2h(tmp.p, reinterpret_cast<uint16_t*>(ix.vec.p), v.size(), ix.alpha, ix.stream));
            vec_f32_dev = tmp.p;
        } else if (ix.vdtype == GF_VEC_I8Q) {
            std::vector<char> u(v.size());
            gf::quantise_i8(v.data(), N, D, ix.alpha, ix.qscale, ix.qzero, reinterpret_cast<int8_t*>(u.data()));
            ix.vec.upload(u);
            tmp.upload(v);
            vec_f32_dev = tmp.p;
        } else {
            std::vector<char> u(v.size());
            for (size_t i = 0; i < v.size(); ++i) u[i] = char(uint8_t(v[i]));
            ix.vec.upload(u);
            tmp.upload(v);
            vec_f32_dev = tmp.p;
        }
        build_subcells(h, gidx, size, ix);
        // Integer-valued data in [0, 255]: int8 tiles of the MFMA brute force.
        bool ints = ix.sub && !gf::half_rows(ix.vdtype) && ix.vdtype != GF_VEC_I8Q && D % 64 == 0 && D <= 256;
        for (size_t i = 0; ints && i < v.size(); ++i) ints = v[i] >= 0.0f && v[i] <= 255.0f && v[i] == std::floor(v[i]);
        if (ints) {
            ix.trec.alloc(size_t(ix.ntile) * gf::bf_rec_bytes(D, ix.AW));
            GF_HIP(gf::launch_tile_rec(vec_f32_dev, false, D, ix.tmeta.p, ix.AW, ix.ntile, ix.trec.p,
                                      ix.stream));
            ix.i8 = true;
        }
        // Float rows with sub-cells and no int8 route: |x|^2 per row (fp32:
        // binary16 rows as k_norms_f16 sums their values, fp32 rows from a
        // float64 sum) and the largest |x| for the MFMA brute force's error
        // bound (a binary16 value is within 2^-11 of x * alpha, or 2^-25 for
        // subnormals).
        const int fvt = ix.vdtype == GF_VEC_F16 ? 1 : (ix.vdtype == GF_VEC_F32 ? 0 : -1);
        if (ix.sub && !ix.i8 && fvt >= 0 && gf::bf_float_supported(fvt, D, ix.AW, 1)) {
            std::vector<float> xn(fvt == 0 ? N : 0);
            double xm = 0.0;
            for (uint32_t r = 0; r < N; ++r) {
                double s = 0.0;
                for (uint32_t d = 0; d < D; ++d) {
                    const double x = double(v[size_t(r) * D + d]) * (fvt == 1 ? ix.alpha : 1.0f);
                    s += x * x;
                }
                xm = std::max(xm, s);
                if (fvt == 0) xn[r] = float(s);
            }
            if (fvt == 1) {
                ix.xnormf.alloc(N);
                GF_HIP(gf::launch_norms_f16(reinterpret_cast<const uint16_t*>(ix.vec.p), N, D, D, ix.xnormf.p,
                                            ix.stream));
                ix.xmaxf = std::sqrt(xm) * (1.0 + 1.0 / 1024.0) + std::sqrt(double(D)) * std::ldexp(1.0, -24);
            } else {
                ix.xnormf.upload(xn);
                ix.xmaxf = std::sqrt(xm) * (1.0 + 1e-6);
            }
            // the brute force's tile records: its tiles' rows in MFMA operand
            // order, contiguous per tile, with their meta records and norms
            const uint32_t KS = fvt == 1 ? D / 32 : D / 16;
            ix.frec.alloc(size_t(ix.ntile) * gf::bf_frec_bytes(KS, ix.AW));
            GF_HIP(gf::launch_tile_frec(ix.vec.p, fvt, D, ix.tmeta.p, ix.xnormf.p, ix.AW, ix.ntile, ix.frec.p,
                                        ix.stream));
            ix.hf = true;
            // Binary16 rows' first pass (a launch of its own): one in four
            // sub-cells (C4: 4.1-4.2 ms per search against 5.5-5.7 ms at one
            // in eight; one in two as fast as one in four, one in sixteen
            // 6.5 ms).  fp32 rows run one launch and keep one in eight (C3:
            // 5.9 ms against 6.05 ms at one in four).
            if (fvt == 1) {
                std::vector<uint32_t> order;
                uint32_t ns1 = 0;
                gf::first_pass_order(ix.shash_h, gf::kBfHFirstPass, order, ns1);
                ix.sorder.upload(order);
                ix.ns1 = ns1;
            }
        }
        GF_HIP(hipStreamSynchronize(ix.stream));
    }
    // Grid (real_dataset_adapter.cuh:563-619).
    uint32_t gsum = 0;
    std::vector<uint32_t> doff(a);
    for (uint32_t d = 0; d < a; ++d) { doff[d] = gsum; gsum += h.grid_shape[d]; }
    ix.l_q.upload(h.l_q, gsum);
    // The full graph (P <= 64: FE = min(E, R, 64 / P) edges into each cell,
    // at most 64 per row) and the reference's entry-point draws
    // (gpu_graph.cu:12503-12539), made once per index: R entries for the
    // traversal and FD distinct point ids below N, mapped to rows, for the
    // full graph.  An index with no room for the first draw
    // (N <= (P - 1) * ceil(N / P)) searches with the caller's entry points
    // only; one with fewer than FD points has no full graph.
    if (P <= 64 && E > 0 && N >= std::min(std::min(E, R), 64u / P) * P) {
        ix.FE = std::min(std::min(E, R), 64u / P);
        ix.FD = ix.FE * P;
        std::vector<uint32_t> rowcell(N);
        for (uint32_t c = 0; c < P; ++c)
            for (uint32_t r = ix.offset_h[c]; r < ix.offset_h[c + 1]; ++r) rowcell[r] = c;
        DevBuf<uint32_t> drc;
        drc.upload(rowcell);
        ix.fgraph.alloc(size_t(N) * ix.FD);
        GF_HIP(gf::launch_assemble_full(ix.graph.p, ix.cross.p, ix.offset.p, drc.p, N, P, R, E, ix.FE, ix.fgraph.p,
                                        ix.stream));
        GF_HIP(hipStreamSynchronize(ix.stream));
    }
    {
        const uint32_t avg = (N + P - 1) / P;
        if (N > (P - 1) * avg) {
            std::vector<uint32_t> ent(R), entf(std::max<uint32_t>(ix.FD, 1));
            gf::entry_points_pair(N - (P - 1) * avg, R, N, ix.FD, ent.data(), entf.data());
            ix.entry_ref.upload(ent);
            ++ix.entry_gen;
            if (ix.FD) {
                std::vector<uint32_t> rowof(N);
                for (uint32_t r = 0; r < N; ++r) rowof[gidx[r]] = r;
                for (auto& e : entf) e = rowof[e];
                ix.fentry.upload(entf.data(), ix.FD);
            }
        } else {
            ix.fgraph.release();
            ix.FE = ix.FD = 0;
        }
    }
    ix.r_q.upload(h.r_q, gsum);
    ix.grid.upload(ix.grid_h);
    ix.doff.upload(doff);
    // Selectivity tiles: kSelTile rows of one cell each.
    {
        std::vector<uint32_t> tc, tr, tn;
        for (uint32_t c = 0; c < P; ++c)
            for (uint32_t r = ix.offset_h[c]; r < ix.offset_h[c + 1]; r += gf::kSelTile) {
                tc.push_back(c);
                tr.push_back(r);
                tn.push_back(std::min(gf::kSelTile, ix.offset_h[c + 1] - r));
            }
        ix.ntiles = uint32_t(tc.size());
        ix.tile_cell.upload(tc);
        ix.tile_row0.upload(tr);
        ix.tile_n.upload(tn);
    }
    // Cluster centres + cell x cluster histogram (tools.cuh:569-602).
    if (h.labels) {
        int32_t cmax = -1;
        for (uint32_t i = 0; i < N; ++i) {
            GF_REQUIRE(h.labels[i] >= 0, GF_E_FORMAT, "negative cluster label");
            cmax = std::max(cmax, h.labels[i]);
        }
        const uint32_t C = uint32_t(cmax) + 1;
        GF_REQUIRE(C <= (1u << 20), GF_E_UNSUPPORTED, "too many clusters");
        const bool contiguous = opts && opts->hist_contiguous;
        const uint32_t avg = (N + P - 1) / P;
        std::vector<float> cen(size_t(C) * D, 0.0f);
        std::vector<uint32_t> num(C, 0), hist(size_t(P) * C, 0);
        for (uint32_t i = 0; i < N; ++i) {
            const uint32_t cid = uint32_t(h.labels[i]);
            const uint32_t pid = contiguous ? std::min(i / avg, P - 1) : h.global_pid[i];
            num[cid]++;
            hist[size_t(pid) * C + cid]++;
            const float* x = h.vectors + size_t(i) * D;
            float* y = &cen[size_t(cid) * D];
            for (uint32_t j = 0; j < D; ++j) y[j] += x[j];
        }
        for (uint32_t c = 0; c < C; ++c)
            for (uint32_t j = 0; j < D; ++j) cen[size_t(c) * D + j] /= float(num[c]);
        ix.C = C;
        ix.Dp = round_up(D, 32);
        ix.Cp = round_up(C, 64);
        DevBuf<float> tmp;
        tmp.upload(cen);
        ix.centres.alloc(size_t(ix.Cp) * ix.Dp);
        GF_HIP(gf::launch_f2h_pad(tmp.p, C, D, ix.centres.p, ix.Cp, ix.Dp, ix.alpha, ix.stream));
        ix.cnorm.alloc(ix.Cp);
        GF_HIP(gf::launch_norms_f16(ix.centres.p, ix.Cp, ix.Dp, ix.Dp, ix.cnorm.p, ix.stream));
        GF_HIP(hipStreamSynchronize(ix.stream));
        ix.hist.upload(hist);
    }
}

void ensure_out(gf_batch& b, uint32_t K) {
    const size_t n = size_t(b.Q) * K;
    if (b.out_ids.n < n) { b.out_ids.alloc(n); b.out_dist.alloc(n); }
    if (b.counters.n < size_t(b.Q) * GF_NCOUNTERS) b.counters.alloc(size_t(b.Q) * GF_NCOUNTERS);
}

gf::SubArgs sub_args(const gf_index& ix) {
    gf::SubArgs sa{};
    sa.sbase = ix.sbase.p; sa.scell = ix.scell.p; sa.ssize = ix.ssize.p; sa.stile = ix.stile.p;
    sa.sbox = ix.sbox.p; sa.tmeta = ix.tmeta.p; sa.abase = ix.abase.p;
    sa.a = ix.a; sa.AW = ix.AW; sa.P = ix.P; sa.NS = ix.NS;
    return sa;
}


void entry_points_ref(uint32_t N, uint32_t P, uint32_t R, uint32_t* out) {
    const uint32_t avg = (N + P - 1) / P;
    const uint32_t rand_max = N - (P - 1) * avg;
    GF_REQUIRE(rand_max >= 1, GF_E_ARG, "no room for entry points");
    gf::entry_points_draw(rand_max, R * 10, R, out);
}

// Exact selectivity counts of the batch's ranges (prefiltering_tag_elements,
// real_dataset_adapter.cuh:346-383): sub-cells inside a range count whole,
// partially covered ones are scanned; without sub-cells, per-cell tiles.
void count_selectivity(gf_batch& b, hipStream_t st) {
    gf_index* ix = b.ix;
    GF_HIP(gf::launch_zero_u32(b.selcount.p, b.Q, st));
    if (ix->sub) {
        gf::SubSelArgs sl{};
        sl.sa = sub_args(*ix);
        sl.Q = b.Q; sl.lo = b.lo.p; sl.hi = b.hi.p; sl.selcount = b.selcount.p;
        GF_HIP(gf::launch_subsel(sl, st));
    } else {
        GF_HIP(gf::launch_zero_u32(b.ccount.p, ix->P, st));
        GF_HIP(gf::launch_zero_u32(b.cfill.p, ix->P, st));
        GF_HIP(gf::launch_cellq_count(b.Q, ix->P, b.cells.p, b.counts.p, b.ccount.p, st));
        GF_HIP(gf::launch_scan_small(b.ccount.p, ix->P, b.cstart.p, st));
        GF_HIP(gf::launch_cellq_fill(b.Q, ix->P, b.cells.p, b.counts.p, b.cstart.p, b.cfill.p, b.cellq.p, st));
        GF_HIP(gf::launch_selcount(ix->ntiles, ix->tile_cell.p, ix->tile_row0.p, ix->tile_n.p, ix->attrs.p, ix->a,
                                   b.cstart.p, b.ccount.p, b.cellq.p, b.lo.p, b.hi.p, b.selcount.p, st));
    }
}

// The exact counts, when gf_mark_cells skipped them.
void ensure_selcount(gf_batch& b) {
    if (b.sel_exact) return;
    count_selectivity(b, b.ix->stream);
    GF_HIP(hipStreamSynchronize(b.ix->stream));
    b.sel_exact = true;
}

// Stage A's kernels (gf_mark_cells) on st.  The stage's kernels take its
// timestamps: the cell kernel when it starts, the last kernel (ticket) when
// it ends.
void stage_a_enqueue(gf_batch* b, float prefilter, hipStream_t st) {
    gf_index* ix = b->ix;
    const bool count = prefilter < 1.0f;
    gf::CellsTail tl;
    tl.st_entry = b->stamps.p + gf_batch::kStampA;
    uint32_t* const ticket = b->ticket(gf_batch::kTicketA);
    uint64_t* const st_end = b->stamps.p + gf_batch::kStampA + 1;
    if (!count) {
        // prefilter >= 1: count / N <= prefilter holds for every count, so
        // every query is routed to the brute force without counting (the
        // routing is the reference's), in the cell kernel itself; the exact
        // counts are made when asked for.
        tl.selcount = b->selcount.p;
        tl.little = b->little.p;
        tl.ticket = ticket;
        tl.st_exit = st_end;
    }
    GF_HIP(gf::launch_cells(b->Q, ix->a, b->lo.p, b->hi.p, ix->grid.p, ix->doff.p, ix->l_q.p, ix->r_q.p, ix->P,
                            ix->offset.p, b->cells.p, b->counts.p, st, tl));
    if (count) {
        count_selectivity(*b, st);
        GF_HIP(gf::launch_route(b->Q, ix->N, prefilter, b->selcount.p, b->counts.p, b->little.p, st, ticket,
                                st_end));
    }
}
std::vector<uint64_t> stage_a_key(const gf_batch* b, float prefilter) {
    uint32_t pf = 0;
    std::memcpy(&pf, &prefilter, sizeof(pf));
    return {uint64_t(uintptr_t(b->ix)), pf, b->Q, uint64_t(uintptr_t(b->lo.p)), uint64_t(uintptr_t(b->hi.p)),
            uint64_t(uintptr_t(b->cells.p)), uint64_t(uintptr_t(b->counts.p)), uint64_t(uintptr_t(b->selcount.p)),
            uint64_t(uintptr_t(b->little.p)), uint64_t(uintptr_t(b->ccount.p)), uint64_t(uintptr_t(b->cfill.p)),
            uint64_t(uintptr_t(b->cstart.p)), uint64_t(uintptr_t(b->cellq.p)), uint64_t(uintptr_t(b->stamps.p))};
}
// Stage B's kernels (gf_order_cells, b->topc centres) on st.  Timestamps:
// the centre kernel when it starts, a stamp kernel at the end (k_order runs
// one workgroup per query: a ticket over that many workgroups costs more
// than a kernel).
void stage_b_enqueue(gf_batch* b, hipStream_t st) {
    gf_index* ix = b->ix;
    const uint32_t topc = b->topc;
    uint64_t* const st0 = b->stamps.p + gf_batch::kStampB;
    if (topc <= 4) {
        // nearest centres straight from the MFMA tiles; the distance matrix
        // is made only if gf_batch_get_centroid asks for it
        GF_HIP(gf::launch_centroid_top(b->q16.p, ix->centres.p, b->qnorm.p, ix->cnorm.p, b->Q, ix->C, b->Qp, ix->Cp,
                                       ix->Dp, topc, b->topk.p, st, st0));
        GF_HIP(gf::launch_order(b->Q, ix->C, ix->P, topc, nullptr, ix->hist.p, b->cells.p, b->counts.p, b->topk.p,
                                st, true, ix->ref_ties));
    } else {
        GF_HIP(gf::launch_centroid(b->q16.p, ix->centres.p, b->qnorm.p, ix->cnorm.p, b->Q, ix->C, b->Qp, ix->Cp,
                                   ix->Dp, b->cdist.p, st, st0));
        GF_HIP(gf::launch_order(b->Q, ix->C, ix->P, topc, b->cdist.p, ix->hist.p, b->cells.p, b->counts.p,
                                b->topk.p, st, false, ix->ref_ties));
    }
    GF_HIP(gf::launch_stamp(st0 + 1, st));
}
std::vector<uint64_t> stage_b_key(const gf_batch* b) {
    return {uint64_t(uintptr_t(b->ix)), b->topc, b->Q, uint64_t(uintptr_t(b->topk.p)), uint64_t(uintptr_t(b->cdist.p)),
            uint64_t(uintptr_t(b->q16.p)), uint64_t(uintptr_t(b->qnorm.p)), uint64_t(uintptr_t(b->cells.p)),
            uint64_t(uintptr_t(b->counts.p)), uint64_t(uintptr_t(b->stamps.p))};
}
// Enqueues the stage calls recorded without ms (gf_mark_cells, then
// gf_order_cells), each as its own graph.  Every call that reads or writes
// the stage buffers, other than the search (which takes them into its own
// graph), flushes first.
void flush_stages(gf_batch* b) {
    hipStream_t st = b->ix->stream;
    if (b->pend_a) {
        b->pend_a = false;
        const float pf = b->pend_pf;
        b->sg[gf_batch::kGraphA].run(stage_a_key(b, pf), st, [&]() { stage_a_enqueue(b, pf, st); });
    }
    if (b->pend_b) {
        b->pend_b = false;
        b->sg[gf_batch::kGraphB].run(stage_b_key(b), st, [&]() { stage_b_enqueue(b, st); });
    }
}

}  // namespace

extern "C" {

const char* gf_status_str(gf_status s) {
    switch (s) {
        case GF_OK: return "ok";
        case GF_E_ARG: return "invalid argument";
        case GF_E_IO: return "i/o error";
        case GF_E_FORMAT: return "bad index format";
        case GF_E_DEVICE: return "device error";
        case GF_E_NOMEM: return "out of memory";
        case GF_E_UNSUPPORTED: return "unsupported";
        case GF_E_STATE: return "call out of order";
        default: return "unknown status";
    }
}

const char* gf_last_error(void) { return g_last_error.c_str(); }

gf_status gf_index_create(const gf_index_host* host, const gf_open_opts* opts, gf_index** out) {
    return run_guarded([&] {
        GF_REQUIRE(host && out, GF_E_ARG, "null argument");
        *out = nullptr;
        std::unique_ptr<gf_index> ix(new gf_index());
        build_index(*host, opts, *ix);
        *out = ix.release();
    });
}

gf_status gf_index_open(const gf_index_paths* paths, const gf_open_opts* opts, gf_index** out) {
    return run_guarded([&] {
        GF_REQUIRE(paths && out, GF_E_ARG, "null argument");
        *out = nullptr;
        gf::HostIndex hi;
        gf::read_index_files(*paths, opts ? opts->degree : 0, hi);
        gf_index_host h{};
        h.N = hi.N; h.D = hi.D; h.a = hi.a; h.P = hi.P; h.R = hi.R; h.E = hi.E;
        h.vectors = hi.vectors.data();
        h.attrs = hi.attrs.data();
        h.grid_shape = hi.grid.data();
        h.l_q = hi.l_q.data();
        h.r_q = hi.r_q.data();
        h.global_pid = hi.global_pid.data();
        h.cell_graphs = hi.cell_graphs.data();
        h.cross = hi.cross.data();
        h.labels = hi.has_labels ? hi.labels.data() : nullptr;
        std::unique_ptr<gf_index> ix(new gf_index());
        build_index(h, opts, *ix);
        *out = ix.release();
    });
}

gf_status gf_index_create_streamed(const gf_index_host* host, const gf_open_opts* opts, const gf_stream_plan* plan,
                                   gf_index** out) {
    return run_guarded([&] {
        GF_REQUIRE(host && plan && out, GF_E_ARG, "null argument");
        *out = nullptr;
        std::unique_ptr<gf_index> ix(new gf_index());
        gf::build_streamed(*host, opts, plan, *ix);
        *out = ix.release();
    });
}

gf_status gf_index_open_streamed(const gf_index_paths* paths, const gf_open_opts* opts, const gf_stream_plan* plan,
                                 gf_index** out) {
    return run_guarded([&] {
        GF_REQUIRE(paths && plan && out, GF_E_ARG, "null argument");
        *out = nullptr;
        gf::HostIndex hi;
        gf::read_index_files(*paths, opts ? opts->degree : 0, hi);
        gf_index_host h{};
        h.N = hi.N; h.D = hi.D; h.a = hi.a; h.P = hi.P; h.R = hi.R; h.E = hi.E;
        h.vectors = hi.vectors.data();
        h.attrs = hi.attrs.data();
        h.grid_shape = hi.grid.data();
        h.l_q = hi.l_q.data();
        h.r_q = hi.r_q.data();
        h.global_pid = hi.global_pid.data();
        h.cell_graphs = hi.cell_graphs.data();
        h.cross = hi.cross.data();
        h.labels = nullptr;
        std::unique_ptr<gf_index> ix(new gf_index());
        gf::build_streamed(h, opts, plan, *ix);
        *out = ix.release();
    });
}

gf_status gf_index_close(gf_index* ix) {
    return run_guarded([&] {
        if (!ix) return;
        (void)hipSetDevice(ix->device);
        delete ix;
    });
}

gf_status gf_index_get_info(const gf_index* ix, gf_index_info* out) {
    return run_guarded([&] {
        GF_REQUIRE(ix && out, GF_E_ARG, "null argument");
        out->N = ix->N; out->D = ix->D; out->a = ix->a; out->P = ix->P;
        out->R = ix->R; out->E = ix->E; out->C = ix->C;
        out->vec_dtype = uint32_t(ix->vdtype);
        out->f2h_factor = ix->alpha;
        out->device_bytes = ix->device_bytes();
        out->streamed = ix->sx ? 1u : 0u;
        out->nbatch = ix->sx ? uint32_t(ix->sx->plan->batches.size()) : 0u;
    });
}

gf_status gf_batch_create(gf_index* ix, const float* queries, uint32_t Q, const float* lo, const float* hi,
                          gf_batch** out) {
    return run_guarded([&] {
        GF_REQUIRE(ix && queries && lo && hi && out, GF_E_ARG, "null argument");
        GF_REQUIRE(Q > 0, GF_E_ARG, "empty batch");
        *out = nullptr;
        set_device(ix);
        std::unique_ptr<gf_batch> b(new gf_batch());
        b->ix = ix;
        b->Q = Q;
        b->Qp = round_up(Q, 16);
        b->qf32.upload(queries, size_t(Q) * ix->D);
        b->lo.upload(lo, size_t(Q) * ix->a);
        b->hi.upload(hi, size_t(Q) * ix->a);
        if (gf::half_rows(ix->vdtype)) {
            b->q16v.alloc(size_t(Q) * ix->D);
            GF_HIP(gf::launch_f2h(b->qf32.p, b->q16v.p, size_t(Q) * ix->D, ix->alpha, ix->stream));
        }
        if (ix->hf) {
            // |q|^2 of the query as the rows hold it (binary16 or fp32), and
            // the bound eps_q of |d' - d| for the MFMA brute force of float
            // rows: d' = |q|^2 + |x|^2 - 2 q.x and the canonical d each hold
            // fp32 sums of D terms, within gamma_{D+2} (|q| + |x|)^2 of the
            // exact distance of the rows' vectors (plus two roundings of the
            // combination); doubled for margin, with a floor for subnormal
            // products.
            const uint32_t D = ix->D;
            const bool h = ix->vdtype == GF_VEC_F16;
            const double u = std::ldexp(1.0, -24), gam = (D + 2) * u / (1.0 - (D + 2) * u);
            std::vector<float> eps(Q), qn(h ? 0 : Q);
            for (uint32_t q = 0; q < Q; ++q) {
                double s = 0.0;
                for (uint32_t d = 0; d < D; ++d) {
                    const double x = double(queries[size_t(q) * D + d]) * (h ? ix->alpha : 1.0f);
                    s += x * x;
                }
                if (!h) qn[q] = float(s);
                const double nq = h ? std::sqrt(s) * (1.0 + 1.0 / 1024.0) + std::sqrt(double(D)) * std::ldexp(1.0, -24)
                                    : std::sqrt(s) * (1.0 + 1e-6);
                const double e = 2.0 * (3.0 * gam + 2.0 * u) * (nq + ix->xmaxf) * (nq + ix->xmaxf) +
                                 D * std::ldexp(1.0, -40);
                eps[q] = float(e * (1.0 + 1e-6));
            }
            if (h) {
                b->qnf.alloc(Q);
                GF_HIP(gf::launch_norms_f16(b->q16v.p, Q, D, D, b->qnf.p, ix->stream));
            } else {
                b->qnf.upload(qn);
            }
            b->heps.upload(eps);
        }
        if (ix->vdtype == GF_VEC_I8Q) {
            // rows [c | s]: c_d = fma(s_d, z_d, alpha q_d), the query less
            // the dequantised offset, then the scales
            const uint32_t D = ix->D;
            std::vector<float> rows(size_t(Q) * 2 * D);
            for (uint32_t q = 0; q < Q; ++q)
                for (uint32_t d = 0; d < D; ++d) {
                    const float x = queries[size_t(q) * D + d] * ix->alpha;
                    rows[size_t(q) * 2 * D + d] = std::fmaf(ix->qscale[d], float(ix->qzero[d]), x);
                    rows[size_t(q) * 2 * D + D + d] = ix->qscale[d];
                }
            b->qi8q.upload(rows);
        }
        if (ix->C) {
            b->q16.alloc(size_t(b->Qp) * ix->Dp);
            GF_HIP(gf::launch_f2h_pad(b->qf32.p, Q, ix->D, b->q16.p, b->Qp, ix->Dp, ix->alpha, ix->stream));
            b->qnorm.alloc(b->Qp);
            GF_HIP(gf::launch_norms_f16(b->q16.p, b->Qp, ix->Dp, ix->Dp, b->qnorm.p, ix->stream));
        }
        if (ix->i8) {
            bool ints = true;
            const size_t nq = size_t(Q) * ix->D;
            for (size_t i = 0; ints && i < nq; ++i)
                ints = queries[i] >= 0.0f && queries[i] <= 255.0f && queries[i] == std::floor(queries[i]);
            if (ints) {
                b->q8.alloc(nq);
                b->nq.alloc(Q);
                GF_HIP(gf::launch_q_i8(b->qf32.p, Q, ix->D, b->q8.p, b->nq.p, ix->stream));
                b->i8 = true;
            }
        }
        b->cells.alloc(size_t(Q) * ix->P);
        b->counts.alloc(Q);
        b->little.alloc(Q);
        b->selcount.alloc(Q);
        b->tot.alloc(24);
        if (!ix->sub) {
            b->cellq.alloc(size_t(Q) * ix->P);
            b->ccount.alloc(ix->P);
            b->cstart.alloc(ix->P);
            b->cfill.alloc(ix->P);
        }
        GF_HIP(hipStreamSynchronize(ix->stream));
        *out = b.release();
    });
}

gf_status gf_batch_free(gf_batch* b) {
    return run_guarded([&] {
        if (!b) return;
        (void)hipSetDevice(b->ix->device);
        delete b;
    });
}

gf_status gf_mark_cells(gf_batch* b, float prefilter, double* ms) {
    return run_guarded([&] {
        GF_REQUIRE(b, GF_E_ARG, "null batch");
        gf_index* ix = b->ix;
        GF_REQUIRE(!ix->sx, GF_E_UNSUPPORTED,
                   "a streamed index has no resident attributes: use gf_mark_cells_grid or gf_batch_set_cells");
        set_device(ix);
        hipStream_t st = ix->stream;
        b->ensure_stamps();
        // a stage B recorded before this call runs first
        if (b->pend_b) flush_stages(b);
        const bool count = prefilter < 1.0f;
        b->flags_ready = false;
        b->bf_all = true;
        b->sel_exact = count;
        b->route_bf = !count;
        b->time_a = gf_batch::kTimeStamps;
        b->marked = true;
        if (!ms) {
            // recorded: the next search enqueues it in its own graph (another
            // call that needs the stage's outputs enqueues it first)
            b->pend_a = true;
            b->pend_pf = prefilter;
            return;
        }
        b->pend_a = false;
        b->sg[gf_batch::kGraphA].run(stage_a_key(b, prefilter), st, [&]() { stage_a_enqueue(b, prefilter, st); });
        b->fetch_stamps(gf_batch::kStampA, 2, st);
        *ms = b->stamp_ms(gf_batch::kStampA);
    });
}

gf_status gf_mark_cells_grid(gf_batch* b, const float* attr_min, const float* attr_width, double threshold,
                             double* ms) {
    return run_guarded([&] {
        GF_REQUIRE(b && attr_min && attr_width, GF_E_ARG, "null argument");
        gf_index* ix = b->ix;
        for (uint32_t d = 0; d < ix->a; ++d)
            GF_REQUIRE(attr_width[d] > 0.0f && std::isfinite(attr_width[d]) && std::isfinite(attr_min[d]), GF_E_ARG,
                       "attr_width must be positive and finite, attr_min finite");
        set_device(ix);
        hipStream_t st = ix->stream;
        flush_stages(b);
        if (b->flags.n < size_t(b->Q) * ix->P) b->flags.alloc(size_t(b->Q) * ix->P);
        DevBuf<float> amin, width;
        amin.upload(attr_min, ix->a);
        width.upload(attr_width, ix->a);
        b->stage_event(0, st);
        GF_HIP(gf::launch_cells_grid(b->Q, ix->a, b->lo.p, b->hi.p, amin.p, width.p, ix->grid.p, ix->P, ix->offset.p,
                                     threshold, b->cells.p, b->counts.p, b->little.p, b->flags.p, st));
        GF_HIP(hipMemsetAsync(b->selcount.p, 0, b->Q * sizeof(uint32_t), st));
        b->stage_event(1, st);
        b->time_a = gf_batch::kTimeEvents;
        // amin and width are freed on return: their reads must be done first
        const double el = b->event_ms();
        if (ms) *ms = el;
        b->marked = true;
        b->flags_ready = true;
        b->bf_all = false;
        b->route_bf = false;
        b->sel_exact = true;   // the arithmetic-grid stage A counts nothing: selcount stays 0
    });
}

gf_status gf_order_cells(gf_batch* b, uint32_t topc, double* ms) {
    return run_guarded([&] {
        GF_REQUIRE(b, GF_E_ARG, "null batch");
        GF_REQUIRE(b->marked, GF_E_STATE, "gf_order_cells before gf_mark_cells");
        GF_REQUIRE(topc >= 1 && topc <= 16, GF_E_ARG, "topc must be in [1, 16]");
        gf_index* ix = b->ix;
        set_device(ix);
        if (!ix->C) { if (ms) *ms = 0.0; b->time_b = gf_batch::kTimeNone; return; }
        hipStream_t st = ix->stream;
        // a stage B recorded before runs first, so that the calls run in the
        // order they were made (the stage reorders the cell lists in place)
        if (b->pend_b) flush_stages(b);
        if (b->topk.n < size_t(b->Q) * topc) b->topk.alloc(size_t(b->Q) * topc);
        const bool top = topc <= 4;
        if (!top && !b->cdist.p) b->cdist.alloc(size_t(b->Q) * ix->C);
        b->topc = topc;
        b->ensure_stamps();
        b->cdist_ready = !top;
        b->ordered = true;
        b->time_b = gf_batch::kTimeStamps;
        if (!ms) {
            b->pend_b = true;   // recorded, as gf_mark_cells without ms
            return;
        }
        flush_stages(b);   // a recorded stage A
        b->sg[gf_batch::kGraphB].run(stage_b_key(b), st, [&]() { stage_b_enqueue(b, st); });
        b->fetch_stamps(gf_batch::kStampB, 2, st);
        *ms = b->stamp_ms(gf_batch::kStampB);
    });
}

// gf_search and gf_search_dual: channels 1 runs the traversal-routed
// queries through k_traverse, 2 through k_traverse_dual.
static void search_resident(gf_batch* b, const gf_search_opts* opts, uint32_t* ids, float* dists,
                            gf_search_stats* stats, uint32_t channels) {
    GF_REQUIRE(b && opts && ids, GF_E_ARG, "null argument");
    GF_REQUIRE(b->marked, GF_E_STATE, "gf_search before gf_mark_cells");
    gf_index* ix = b->ix;
    const uint32_t L = opts->L, K = opts->K, rl = opts->rl;
    GF_REQUIRE(L >= 1 && L < (1u << 16), GF_E_ARG, "L must be in [1, 65535]");
    GF_REQUIRE(K >= 1 && K <= 64, GF_E_ARG, "K must be in [1, 64]");
    GF_REQUIRE(rl >= 1 && rl <= 16, GF_E_ARG, "rl must be in [1, 16]");
    set_device(ix);
    // Device times of the latest stage calls (their events and timestamps
    // precede the search on the stream, which the search has waited for;
    // gathered: the resident search copied the timestamps with its results).
    auto stage_times = [&](bool gathered) {
        if (!stats) return;
        if (!gathered && (b->time_a == gf_batch::kTimeStamps || b->time_b == gf_batch::kTimeStamps))
            b->fetch_stamps(gf_batch::kStampA, 4, ix->stream);
        stats->ms_stage_a = b->time_a == gf_batch::kTimeEvents   ? b->event_ms()
                            : b->time_a == gf_batch::kTimeStamps ? b->stamp_ms(gf_batch::kStampA)
                                                                 : 0.0;
        stats->ms_stage_b = b->time_b == gf_batch::kTimeStamps ? b->stamp_ms(gf_batch::kStampB) : 0.0;
    };
    if (ix->sx) {
        flush_stages(b);
        gf::stream_search(*b, *opts, ids, dists, stats);
        stage_times(false);
        return;
    }
    // stage calls recorded without ms run at the start of this stage's graph
    const bool pend_a = b->pend_a, pend_b = b->pend_b;
    const float pend_pf = b->pend_pf;
    hipStream_t st = ix->stream;
    const uint32_t Q = b->Q, R = ix->R;

    // Entry points: the caller's, or the reference's draw (computed once per
    // index and count): R of them, L for the dual-channel traversal.
    const uint32_t nent = channels == 2 ? L : R;
    if (opts->entry_points) {
        b->entry.upload(opts->entry_points, nent);
        b->entry_src = nullptr;
    } else {
        DevBuf<uint32_t>& ref = channels == 2 ? ix->entry_dual : ix->entry_ref;
        if (ref.n != nent) {
            std::vector<uint32_t> ent(nent);
            entry_points_ref(ix->N, ix->P, nent, ent.data());
            ref.upload(ent);
            ++ix->entry_gen;
        }
        if (b->entry.n < nent) {
            b->entry.alloc(nent);
            b->entry_src = nullptr;
        }
        if (b->entry_src != ref.p || b->entry_src_n != nent || b->entry_src_gen != ix->entry_gen) {
            GF_HIP(hipMemcpyAsync(b->entry.p, ref.p, nent * sizeof(uint32_t), hipMemcpyDeviceToDevice, st));
            b->entry_src = ref.p;
            b->entry_src_n = nent;
            b->entry_src_gen = ix->entry_gen;
        }
    }
    if (channels == 2 && ix->prow.n != ix->N) {
        ix->prow.alloc(ix->N);
        GF_HIP(gf::launch_invert_rows(ix->gidx.p, ix->N, ix->prow.p, st));
    }
    ensure_out(*b, K);
    if (b->sched.n < Q) b->sched.alloc(Q);

    // Visited-set size for the keys live between two resets (the list, the
    // slots of four expansions and a cell's cross slots; the dual channel's
    // expansions fill 2R slots).
    const uint32_t hsize = gf::visited_slots(L + gf::kXSlots + (channels == 2 ? 10 * R : 4 * R));
    const uint32_t Lpad = round_up(L, 2);
    const uint32_t lds = channels == 2 ? gf::trav_dual_lds_bytes(Lpad, hsize) : gf::trav_lds_bytes(Lpad, hsize, ix->P);
    GF_REQUIRE(lds <= 64 * 1024, GF_E_UNSUPPORTED, "L too large for the LDS budget");

    // device scalars: tot[2] pairs, [3] fits, [4] items, [8..11] traversal /
    // brute-force / empty / full-graph counts, [12..13] traversal range,
    // [14..15] brute-force range, [16..17] full-graph range
    uint32_t* tot = b->tot.p;
    gf::TravArgs a{};
    a.vec = ix->vec.p;
    a.rowbytes = ix->rowbytes;
    a.nch = ix->rs.nch;
    a.attrs = ix->attrs.p;
    a.graph = ix->graph.p;
    a.cross = ix->cross.p;
    a.xrow = uint64_t(ix->P) * ix->E;
    a.xcell = ix->E;
    a.offset = ix->offset.p;
    a.gidx = ix->gidx.p;
    a.lrow = ix->lrow.p;
    a.prow = ix->prow.p;
    if (gf::half_rows(ix->vdtype)) {
        a.queries = reinterpret_cast<const char*>(b->q16v.p);
        a.qbytes = ix->D * 2;
    } else if (ix->vdtype == GF_VEC_I8Q) {
        a.queries = reinterpret_cast<const char*>(b->qi8q.p);
        a.qbytes = ix->D * 8;
    } else {
        a.queries = reinterpret_cast<const char*>(b->qf32.p);
        a.qbytes = ix->D * 4;
    }
    a.lo = b->lo.p;
    a.hi = b->hi.p;
    a.cells = b->cells.p;
    a.counts = b->counts.p;
    a.little = b->little.p;
    a.sched = b->sched.p;
    a.entry = b->entry.p;
    a.out_ids = b->out_ids.p;
    a.out_dist = b->out_dist.p;
    a.counters = b->counters.p;
    a.a = ix->a; a.P = ix->P; a.R = R; a.E = ix->E; a.L = L; a.K = K; a.rl = rl;
    a.hsize = hsize;
    a.offl = gf::trav_offsets_in_lds(ix->P) ? 1u : 0u;
    a.Lpad = Lpad;
    // The full-graph route: its own visited-set size (L + FD list and B
    // region entries plus four expansions' FD between resets).
    gf::TravArgs af = a;
    uint32_t lds_f = 0;
    if (ix->FD) {
        const uint32_t hs = gf::visited_slots(L + 5 * ix->FD);
        af.hsize = hs;
        lds_f = Lpad * 8 + gf::kXSlots * 8 + 128 * 4 + hs * 4;
        GF_REQUIRE(lds_f <= 64 * 1024, GF_E_UNSUPPORTED, "L too large for the LDS budget");
        af.fgraph = ix->fgraph.p;
        af.fentry = ix->fentry.p;
        af.FD = ix->FD;
        af.frange = tot + 16;
    }

    // Brute-force route on MFMA when vectors and queries are int8-exact:
    // work items of (sub-cell, <= 64 queries whose range reaches it),
    // scheduled on the device.
    const bool gemm = ix->i8 && b->i8 && K <= gf::kBfKMax;
    // Binary16 rows: the same items on fp16 MFMA, candidates within the
    // distances' error bound re-ranked exactly (k_bf_f16, k_bf_f16_final).
    const int fvt = ix->vdtype == GF_VEC_F16 ? 1 : 0;
    const bool gemm_h = !gemm && ix->hf && b->qnf.n == Q && gf::bf_float_supported(fvt, ix->D, ix->AW, K);
    const bool sched_bf = gemm || gemm_h;
    const uint32_t KP = gemm_h ? gf::kBfHKT : K;   // keys per (query, item) in the partial area
    const uint32_t seed_tiles = gemm_h ? gf::kBfHSeedTiles : gf::kBfSeedTiles;
    const uint32_t NS = ix->NS;
    b->pass_pending = sched_bf && !b->sel_exact;
    if (sched_bf) {
        if (!b->bcnt.n) {
            b->bcnt.alloc(NS); b->bin.alloc(NS); b->bstart.alloc(NS); b->icnt.alloc(NS); b->ioff.alloc(NS);
            b->nsub.alloc(Q); b->part_off.alloc(Q); b->pcnt.alloc(Q);
        }
        // item slots: a sub-cell adds up to two partial query blocks per
        // tile chunk beyond pairs / 64
        const size_t islots = size_t(NS) + ix->ntile / gf::kBfMaxItemTiles + 1;
        if (!b->part.n) b->alloc_pairs(size_t(Q) * 64, KP, Q, NS, islots);
        if (b->rq.n < Q) {
            b->rq.alloc(Q); b->rseed.alloc(Q);
            b->rlo.alloc(size_t(Q) * ix->a); b->rhi.alloc(size_t(Q) * ix->a);
        }
        if (b->scnt.n < NS) {
            b->scnt.alloc(NS);
            // a seed sub-cell s with ns queries makes ceil(ns / 64) items per
            // chunk of seed tiles (sized for the smaller chunk of the two
            // routes); every query seeds one sub-cell
            uint32_t tmax = 0;
            for (uint32_t s = 0; s < NS; ++s) tmax = std::max(tmax, ix->stile_h[s + 1] - ix->stile_h[s]);
            const uint32_t sch = std::min(gf::kBfSeedTiles, gf::kBfHSeedTiles);
            const size_t chunks = (tmax + sch - 1) / sch;
            b->sitems.alloc((size_t(Q) / gf::kBfQB + NS + 1) * std::max<size_t>(chunks, 1));
        }
        if (b->part.n < b->pair_cap * KP) b->part.alloc(b->pair_cap * KP);
        if (b->gbound.n < Q) b->gbound.alloc(Q);
        if (gemm_h && b->hover.n < Q) b->hover.alloc(Q);
        if (!b->bf_all && b->bfmask.n < size_t(Q) * ix->P) b->bfmask.alloc(size_t(Q) * ix->P);
    }
    // events: [0] search start, [1] after traversal, [2] end, [3..4] around the MFMA kernel alone
    // Device timestamps (wall clock, kernels on the stream, so that they
    // time a replayed graph too): [0] search start, [1] after traversal,
    // [2] end, [3..4] around the MFMA brute-force launches.
    b->ensure_stamps();
    uint64_t* stamp = b->stamps.p;
    // reset_done: k_reset_results already did k_bf_reset's work
    auto launch_gemm = [&](bool reset_done) {
        gf::BfSchedArgs sc{};
        sc.sa = sub_args(*ix);
        sc.Q = Q; sc.postfilter = opts->postfilter; sc.counts = b->counts.p;
        sc.little = b->little.p; sc.lo = b->lo.p; sc.hi = b->hi.p; sc.nsub = b->nsub.p; sc.bcnt = b->bcnt.p; sc.bin = b->bin.p;
        sc.bstart = b->bstart.p; sc.bq = b->bq.p; sc.qcap = b->qcap;
        sc.ok = tot + 3; sc.nbf = tot + 9;
        sc.qlist = b->sched.p; sc.qrange = tot + 14;   // the brute-force queries of the schedule
        sc.tch = gf::kBfMaxItemTiles;
        if (!b->bf_all) {
            GF_HIP(gf::launch_cell_flags(Q, ix->P, b->cells.p, b->counts.p, b->little.p, b->bfmask.p, st));
            sc.bfm = b->bfmask.p;
            sc.bP = ix->P;
        }
        // Seeds (one-pass lists): each query's best-filled sub-cell runs first.
        const bool seeds = b->qcap != 0;
        if (!reset_done)
            GF_HIP(gf::launch_bf_reset(Q, b->nsub.p, b->pcnt.p, b->gbound.p, st, seeds ? NS : 0,
                                       seeds ? b->scnt.p : nullptr, seeds ? tot + 5 : nullptr));
        if (seeds) {
            gf::BfSeedArgs sd{};
            sd.sa = sc.sa; sd.Q = Q; sd.postfilter = sc.postfilter; sd.counts = sc.counts; sd.little = sc.little;
            sd.cells = b->cells.p; sd.lo = sc.lo; sd.hi = sc.hi; sd.bfm = sc.bfm; sd.bP = sc.bP;
            sd.qlist = sc.qlist; sd.qrange = sc.qrange; sd.qcap = b->qcap; sd.tch = seed_tiles;
            sd.itch = gf::kBfMaxItemTiles;
            sd.scnt = b->scnt.p; sd.bq = b->bq.p; sd.nsub = b->nsub.p;
            sd.rq = b->rq.p; sd.rseed = b->rseed.p; sd.rlo = b->rlo.p; sd.rhi = b->rhi.p;
            GF_HIP(gf::launch_bfseed(sd, Q, st));
            sc.scnt = b->scnt.p;
            sc.rq = b->rq.p; sc.rseed = b->rseed.p; sc.rlo = b->rlo.p; sc.rhi = b->rhi.p;
        }
        if (seeds) GF_HIP(gf::launch_bfsched_direct(sc, st));
        else GF_HIP(gf::launch_bfsched(sc, false, st));
        if (!b->qcap) GF_HIP(gf::launch_scan_small(b->bcnt.p, NS, b->bstart.p, st));
        GF_HIP(gf::launch_scan_total(b->nsub.p, Q, b->part_off.p, uint32_t(std::min<size_t>(b->pair_cap, UINT32_MAX)),
                                     KP, b->part.n, tot + 2, st));
        if (!b->qcap) GF_HIP(gf::launch_bfsched(sc, true, st));
        // Two passes (resident index): the seeds and the items of the
        // first-pass sub-cells, then a merge that lowers each query's
        // bound to the K-th smallest distance found so far, then the rest
        // of the items under those bounds.  Both k_bfitems launches take
        // the sub-cells in the same order (counts, scan, fill).
        const bool two = ix->sorder.n == NS && ix->ns1 > 0 && ix->ns1 < NS;
        GF_HIP(gf::launch_bfitems(b->bcnt.p, b->bin.p, b->bstart.p, b->qcap, ix->stile.p, gf::kBfMaxItemTiles, NS, b->icnt.p, b->ioff.p,
                                  b->items.p, tot + 4, tot + 3, false, st, nullptr, nullptr, nullptr, 0,
                                  two ? ix->sorder.p : nullptr, two ? ix->ns1 : 0u, nullptr));
        GF_HIP(gf::launch_scan_small(b->icnt.p, NS, b->ioff.p, st));
        const uint32_t scap = uint32_t(b->sitems.n);
        GF_HIP(gf::launch_bfitems(b->bcnt.p, b->bin.p, b->bstart.p, b->qcap, ix->stile.p, gf::kBfMaxItemTiles, NS, b->icnt.p, b->ioff.p,
                                  b->items.p, tot + 4, tot + 3, true, st, seeds ? b->scnt.p : nullptr,
                                  b->sitems.p, tot + 5, scap, two ? ix->sorder.p : nullptr, two ? ix->ns1 : 0u,
                                  two ? tot + 6 : nullptr, seed_tiles));
        if (gemm_h) {
            GF_HIP(gf::launch_zero_u32(b->hover.p, Q, st));
            gf::BfHArgs ha{};
            ha.sa = sub_args(*ix);
            ha.rec = ix->frec.p;
            ha.q16 = fvt == 1 ? static_cast<const void*>(b->q16v.p) : static_cast<const void*>(b->qf32.p);
            ha.qnorm = b->qnf.p; ha.eps = b->heps.p; ha.lo = b->lo.p; ha.hi = b->hi.p;
            ha.items = b->items.p; ha.nitems = tot + 4; ha.bq = b->bq.p; ha.part_off = b->part_off.p;
            ha.pcnt = b->pcnt.p; ha.part = b->part.p; ha.gbound = b->gbound.p; ha.over = b->hover.p;
            ha.ok = tot + 3;
            if (seeds) { ha.sitems = b->sitems.p; ha.nseed = tot + 5; ha.nseed_cap = scap; ha.seeds_on = 1; }
            ha.K = K; ha.D = ix->D;
            GF_HIP(gf::launch_stamp(stamp + 3, st));
            // Binary16 rows: the seeds alone, then (two passes) the
            // first-pass sub-cells' items, then the rest, each launch
            // starting from the bounds the earlier ones left in gbound
            // (C4, 768-d, one in eight sub-cells in the first pass: 5.5 ms
            // against 7.6 ms in one launch).  fp32 rows:
            // one launch, seeds first in each workgroup (C3, 96-d: 5.9 ms
            // against 7.3 ms in three).
            const bool split = fvt == 1;
            if (seeds && split) {
                ha.irange = 3;
                GF_HIP(gf::launch_bf_float(ha, fvt, ix->AW, uint32_t(ix->ncu), st));
                ha.seeds_on = 0;
            }
            if (two && split) {
                ha.nitems_a = tot + 6;
                ha.irange = 1;
                GF_HIP(gf::launch_bf_float(ha, fvt, ix->AW, uint32_t(ix->ncu), st));
                ha.irange = 2;
            } else {
                ha.irange = 0;
            }
            GF_HIP(gf::launch_bf_float(ha, fvt, ix->AW, uint32_t(ix->ncu), st));
            GF_HIP(gf::launch_stamp(stamp + 4, st));
            gf::TravArgs ab = a;
            ab.srange = tot + 14;
            const gf::BfHFinal hf{tot + 3, b->hover.p, b->pcnt.p, b->part_off.p, b->part.p, b->heps.p, b->selcount.p};
            GF_HIP(gf::launch_bf_f16_final(ix->rs, ab, hf, Q, st));
            return;
        }
        gf::BfGemmArgs ga{};
        ga.sa = sub_args(*ix);
        ga.rec = ix->trec.p; ga.q8 = b->q8.p; ga.nq = b->nq.p; ga.lo = b->lo.p;
        ga.hi = b->hi.p; ga.items = b->items.p; ga.nitems = tot + 4; ga.bq = b->bq.p; ga.pcnt = b->pcnt.p;
        ga.part_off = b->part_off.p; ga.part = b->part.p; ga.gbound = b->gbound.p;
        ga.ok = tot + 3;
        if (seeds) { ga.sitems = b->sitems.p; ga.nseed = tot + 5; ga.nseed_cap = scap; ga.seeds_on = 1; }
        ga.K = K; ga.D = ix->D;
        gf::BfFinalArgs fa{};
        fa.gbound = b->gbound.p; fa.bfq = b->sched.p; fa.srange = tot + 14; fa.part_off = b->part_off.p; fa.pcnt = b->pcnt.p;
        fa.ok = tot + 3; fa.part = b->part.p; fa.counts = b->counts.p; fa.cells = b->cells.p;
        fa.offset = ix->offset.p; fa.selcount = b->selcount.p; fa.gidx = ix->gidx.p; fa.out_ids = b->out_ids.p;
        fa.out_dist = b->out_dist.p; fa.counters = b->counters.p; fa.K = K; fa.P = ix->P;
        // timestamps [3] and [4]: the first MFMA launch when it starts, the
        // final merge when it starts
        ga.stamp = stamp + 3;
        if (two) {
            // the seeds alone, then a merge (each query's bound becomes the
            // K-th of its seed sub-cell), the first pass under those
            // bounds, a merge, the rest
            ga.nitems_a = tot + 6;
            if (seeds) {
                ga.irange = 3;
                GF_HIP(gf::launch_bf_i8(ga, uint32_t(ix->ncu), st));
                ga.stamp = nullptr;
                fa.bound_only = 1;
                GF_HIP(gf::launch_bf_final(fa, Q, st));
                ga.seeds_on = 0;
            }
            ga.irange = 1;
            GF_HIP(gf::launch_bf_i8(ga, uint32_t(ix->ncu), st));
            ga.stamp = nullptr;
            fa.bound_only = 1;
            GF_HIP(gf::launch_bf_final(fa, Q, st));
            fa.bound_only = 0;
            ga.irange = 2;
        }
        GF_HIP(gf::launch_bf_i8(ga, uint32_t(ix->ncu), st));
        fa.stamp = stamp + 4;
        GF_HIP(gf::launch_bf_final(fa, Q, st));
    };

    // Results, statistics and the schedule's totals come back through
    // pinned staging with one synchronisation.
    const size_t nr = size_t(Q) * K;
    if (b->h_ids.n < nr) { b->h_ids.alloc(nr); b->h_dist.alloc(nr); }
    if (!b->h_tot.n) { b->h_tot.alloc(24); b->h_stats.alloc(16); }
    if (stats && b->stats.n < 16) b->stats.alloc(16);
    // Results go straight into the caller's arrays when HIP knows them as
    // page-locked host memory; otherwise through the batch's pinned
    // buffers and a host copy after the wait.
    auto page_locked = [](const void* ptr) {
        if (!ptr) return false;
        hipPointerAttribute_t at{};
        if (hipPointerGetAttributes(&at, ptr) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        return at.type == hipMemoryTypeHost;
    };
    const bool ids_direct = page_locked(ids), dist_direct = page_locked(dists);
    uint32_t* ids_dst = ids_direct ? ids : b->h_ids.p;
    float* dist_dst = dist_direct ? dists : b->h_dist.p;
    // zero_stats: the sums start from zero here (in the whole stage,
    // k_reset_results has zeroed them)
    auto enqueue_copies = [&](bool zero_stats) {
        if (stats) {
            if (zero_stats) GF_HIP(gf::launch_zero_u32(reinterpret_cast<uint32_t*>(b->stats.p), 32, st));
            gf::StatsArgs sa2{};
            sa2.Q = Q; sa2.NS = sched_bf ? NS : 0; sa2.counters = b->counters.p;
            sa2.bcnt = sched_bf ? b->bcnt.p : nullptr;
            sa2.bin = b->bin.p; sa2.split = b->qcap != 0; sa2.sseed = b->qcap ? b->scnt.p : nullptr;
            sa2.ssize = ix->ssize.p; sa2.stile = ix->stile.p; sa2.out = b->stats.p;
            GF_HIP(gf::launch_stats(sa2, st));
        }
        GF_HIP(gf::launch_gather_meta(stats ? b->stats.p : nullptr, tot, b->stamps.p, b->h_stats.p, b->h_tot.p,
                                      b->h_stamps.p, st));
        GF_HIP(hipMemcpyAsync(ids_dst, b->out_ids.p, nr * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
        if (dists) GF_HIP(hipMemcpyAsync(dist_dst, b->out_dist.p, nr * sizeof(float), hipMemcpyDeviceToHost, st));
    };
    auto enqueue_tail = [&]() {
        enqueue_copies(true);
        GF_HIP(hipStreamSynchronize(st));
    };
    // prefilter >= 1 in the latest stage A: k_sched routes no query to the
    // traversal or the full graph, so neither is launched
    const bool route_bf = b->route_bf;
    // The whole stage, schedule to copies: no allocation, no host wait.
    auto enqueue = [&]() {
        if (pend_a) stage_a_enqueue(b, pend_pf, st);
        if (pend_b) stage_b_enqueue(b, st);
        // Schedule (gpu_graph.cu:12485-12493) on the device.
        gf::SchedArgs sa{};
        sa.Q = Q; sa.P = ix->P; sa.postfilter = opts->postfilter; sa.counts = b->counts.p; sa.little = b->little.p;
        sa.sched = b->sched.p; sa.tot = tot + 8; sa.ranges = tot + 12;
        sa.full = ix->FD ? 1u : 0u;
        sa.franges = ix->FD ? tot + 16 : nullptr;
        // timestamps: [0] (and [1] with no traversal) when the reset starts,
        // [2] when the gather of the results starts (k_gather_meta)
        // with the brute-force schedule, the reset also does k_bf_reset's work
        gf::BfReset br;
        if (sched_bf) {
            br.nsub = b->nsub.p;
            br.pcnt = b->pcnt.p;
            br.gbound = b->gbound.p;
            if (b->qcap) {
                br.NS = NS;
                br.scnt = b->scnt.p;
                br.nseed = tot + 5;
            }
        }
        GF_HIP(gf::launch_reset_results(Q, K, b->out_ids.p, b->out_dist.p, b->counters.p, st,
                                        stats ? reinterpret_cast<uint32_t*>(b->stats.p) : nullptr, stats ? 32u : 0u,
                                        stamp + 0, route_bf ? 2u : 1u, br));
        GF_HIP(gf::launch_sched(sa, st));
        if (!route_bf) {
            // (with route_bf every query takes the brute force or has no
            // cell: no traversal is launched)
            gf::TravArgs at = a;
            at.srange = tot + 12;
            if (channels == 2) GF_HIP(gf::launch_traverse_dual(ix->rs, at, lds, Q, st));
            else GF_HIP(gf::launch_traverse(ix->rs, at, lds, Q, st));
            // queries with postfilter or more cells: the full graph
            if (ix->FD && opts->postfilter <= ix->P) GF_HIP(gf::launch_fullgraph(ix->rs, af, lds_f, Q, st));
            GF_HIP(gf::launch_stamp(stamp + 1, st));
        }
        if (sched_bf) {
            launch_gemm(true);
        } else {
            gf::TravArgs ab = a;
            ab.srange = tot + 14;
            GF_HIP(gf::launch_bruteforce(ix->rs, ab, Q, st));
        }
        enqueue_copies(false);
    };
    // From a batch's second search on, the stage runs as a HIP graph,
    // captured once per layout (buffers, options, route) and replayed:
    // one launch instead of some twenty, no gaps between the kernels.
    const uint64_t key[] = {uint64_t(L), K, rl, opts->postfilter,
                            uint64_t(gemm) | uint64_t(gemm_h) << 1 | uint64_t(route_bf) << 2,
                            uint64_t(b->bf_all), channels, uint64_t(uintptr_t(b->hover.p)),
                            uint64_t(b->qcap), uint64_t(stats != nullptr), uint64_t(dists != nullptr),
                            uint64_t(uintptr_t(b->part.p)), uint64_t(uintptr_t(b->items.p)),
                            uint64_t(uintptr_t(b->bq.p)), b->pair_cap, uint64_t(uintptr_t(b->out_ids.p)),
                            uint64_t(uintptr_t(b->counters.p)), uint64_t(uintptr_t(b->sched.p)),
                            uint64_t(uintptr_t(ids_dst)), uint64_t(uintptr_t(dist_dst)),
                            uint64_t(uintptr_t(b->stats.p)), uint64_t(uintptr_t(b->bfmask.p)),
                            uint64_t(uintptr_t(b->entry.p)), uint64_t(uintptr_t(b->sitems.p)),
                            uint64_t(uintptr_t(b->out_dist.p)), uint64_t(uintptr_t(b->selcount.p)),
                            uint64_t(uintptr_t(b->cells.p)), uint64_t(uintptr_t(b->gbound.p)),
                            uint64_t(uintptr_t(b->scnt.p)), uint64_t(uintptr_t(b->rq.p)),
                            uint64_t(uintptr_t(b->bcnt.p)), uint64_t(uintptr_t(b->h_tot.p)),
                            uint64_t(uintptr_t(b->stamps.p)), uint64_t(uintptr_t(b->h_stamps.p))};
    std::vector<uint64_t> gkey(std::begin(key), std::end(key));
    uint32_t ppf = 0;
    std::memcpy(&ppf, &pend_pf, sizeof(ppf));
    gkey.push_back(uint64_t(pend_a) | uint64_t(pend_b) << 1 | uint64_t(pend_a ? ppf : 0u) << 2);
    if (pend_a) {
        const auto ka = stage_a_key(b, pend_pf);
        gkey.insert(gkey.end(), ka.begin(), ka.end());
    }
    if (pend_b) {
        const auto kb = stage_b_key(b);
        gkey.insert(gkey.end(), kb.begin(), kb.end());
    }
    b->pend_a = b->pend_b = false;
    b->run_stage(gkey, st, enqueue);
    GF_HIP(hipStreamSynchronize(st));
    const uint32_t* dt = b->h_tot.p;
    if (sched_bf && !dt[3]) {
        // the pair lists outgrew their buffers: grow them and run the brute force again
        b->alloc_pairs(size_t(dt[2]) + dt[2] / 4 + 1024, KP, Q, NS, size_t(NS) + ix->ntile / gf::kBfMaxItemTiles + 1);
        GF_HIP(gf::launch_stamp(stamp + 1, st));
        launch_gemm(false);
        enqueue_tail();
        GF_REQUIRE(dt[3], GF_E_STATE, "brute-force schedule does not fit after growing");
    }
    if (!ids_direct) std::memcpy(ids, b->h_ids.p, nr * sizeof(uint32_t));
    if (dists && !dist_direct) std::memcpy(dists, b->h_dist.p, nr * sizeof(float));
    if (stats) {
        float t_tr = 0, t_bf = 0, t_g = 0;
        const uint64_t* ts = b->h_stamps.p;
        const double tick_ms = 1.0 / double(ix->wclk_khz);
        t_tr = float(double(ts[1] - ts[0]) * tick_ms);
        t_bf = float(double(ts[2] - ts[1]) * tick_ms);
        if (sched_bf) t_g = float(double(ts[4] - ts[3]) * tick_ms);
        const unsigned long long* sm = b->h_stats.p;
        std::memset(stats, 0, sizeof(*stats));
        stats->ms_traverse = t_tr;
        stats->ms_bruteforce = t_bf;
        stats->ms_total = double(t_tr) + double(t_bf);
        stats->ms_bf_kernel = t_g;
        // a recorded stage ran in the search's graph
        const bool ra = pend_a ? b->graph_replayed() : b->sg[gf_batch::kGraphA].replayed;
        const bool rb = pend_b ? b->graph_replayed() : b->sg[gf_batch::kGraphB].replayed;
        stats->graph = (b->graph_replayed() ? 1u : 0u) | (ra ? 2u : 0u) | (rb ? 4u : 0u);
        stats->q_traverse = dt[8];
        stats->q_bruteforce = dt[9];
        stats->q_empty = dt[10];
        stats->q_fullgraph = ix->FD ? dt[11] : 0u;
        stats->n_expand = sm[0]; stats->n_dist = sm[1]; stats->n_attr = sm[2]; stats->n_cross = sm[3];
        stats->n_lrow = sm[4]; stats->n_scan = sm[5]; stats->n_pass = sm[6];
        // Algorithmic bytes: what each kernel must read from HBM given
        // its counters (rows gathered, graph rows, attributes, cross-edge
        // slices, local-id lookups unless the offsets sit in LDS) plus
        // its result writes.
        const double t_dist = double(sm[7]), b_dist = double(sm[8]);
        const double lrow_bytes = gf::trav_offsets_in_lds(ix->P) ? 0.0 : 4.0;
        stats->bytes_traverse = t_dist * ix->rowbytes + double(stats->n_expand) * R * 4.0 +
                                double(stats->n_attr) * ix->a * 4.0 + double(stats->n_cross) * ix->E * 4.0 +
                                double(stats->n_lrow) * lrow_bytes + double(dt[8]) * (K * 8.0 + ix->P * 4.0);
        if (gemm && dt[9]) {
            // Item schedule: every (query, sub-cell) pair costs 2 D ops per
            // point; every item streams its sub-cell's tiles once; the final
            // merge reads the appended keys.
            const double tile_bytes = (ix->D / 64) * 1024.0 + 32 * 4.0 + 16.0 * (1 + ix->AW) * 4.0;
            stats->ops_bruteforce = 2.0 * ix->D * double(sm[9]);
            stats->bytes_bruteforce = double(sm[10]) * tile_bytes + double(dt[9]) * K * 16.0;
            stats->bf_mfma = 1;
        } else if (gemm_h && dt[9]) {
            // fp16 items: every (query, sub-cell) pair costs 2 D flops per
            // point; every item streams its sub-cell's rows and meta; the
            // final re-rank gathers the candidates' rows
            const double tile_bytes = 16.0 * ix->D * 2.0 + 16.0 * (2 + ix->AW) * 4.0;
            stats->ops_bruteforce = 2.0 * ix->D * double(sm[9]);
            stats->bytes_bruteforce = double(sm[10]) * tile_bytes + b_dist * ix->rowbytes + double(dt[9]) * K * 16.0;
            stats->bf_mfma = 2;
        } else {
            stats->bytes_bruteforce = double(stats->n_scan) * ix->a * 4.0 + b_dist * ix->rowbytes +
                                      double(dt[9]) * (K * 8.0 + ix->P * 4.0);
            stats->ops_bruteforce = 3.0 * b_dist * ix->D;
            stats->bf_mfma = 0;
        }
        stage_times(true);
    }
}

gf_status gf_search(gf_batch* b, const gf_search_opts* opts, uint32_t* ids, float* dists,
                    gf_search_stats* stats) {
    return run_guarded([&] { search_resident(b, opts, ids, dists, stats, 1); });
}

gf_status gf_search_dual(gf_batch* b, const gf_search_opts* opts, uint32_t* ids, float* dists,
                         gf_search_stats* stats) {
    return run_guarded([&] {
        GF_REQUIRE(b && !b->ix->sx, GF_E_UNSUPPORTED, "gf_search_dual needs a resident index");
        GF_REQUIRE(b->ix->R <= 32, GF_E_UNSUPPORTED, "gf_search_dual supports R <= 32");
        search_resident(b, opts, ids, dists, stats, 2);
    });
}

gf_status gf_batch_get_cells(const gf_batch* b, uint32_t* cells, uint32_t* counts, uint32_t* little,
                             uint32_t* selcount) {
    return run_guarded([&] {
        GF_REQUIRE(b, GF_E_ARG, "null batch");
        GF_REQUIRE(b->marked, GF_E_STATE, "cells not marked");
        set_device(b->ix);
        // the stage calls return once recorded or enqueued: run and wait for them
        flush_stages(const_cast<gf_batch*>(b));
        GF_HIP(hipStreamSynchronize(b->ix->stream));
        if (selcount) ensure_selcount(*const_cast<gf_batch*>(b));
        const size_t Q = b->Q;
        if (cells) GF_HIP(hipMemcpy(cells, b->cells.p, Q * b->ix->P * 4, hipMemcpyDeviceToHost));
        if (counts) GF_HIP(hipMemcpy(counts, b->counts.p, Q * 4, hipMemcpyDeviceToHost));
        if (little) GF_HIP(hipMemcpy(little, b->little.p, Q * 4, hipMemcpyDeviceToHost));
        if (selcount) GF_HIP(hipMemcpy(selcount, b->selcount.p, Q * 4, hipMemcpyDeviceToHost));
    });
}

gf_status gf_batch_set_cells(gf_batch* b, const uint32_t* cells, const uint32_t* counts, const uint32_t* little) {
    return run_guarded([&] {
        GF_REQUIRE(b && cells && counts && little, GF_E_ARG, "null argument");
        set_device(b->ix);
        const uint32_t P = b->ix->P;
        for (uint32_t q = 0; q < b->Q; ++q) {
            GF_REQUIRE(counts[q] <= P && little[q] <= counts[q], GF_E_ARG, "cell count out of range");
            for (uint32_t i = 0; i < counts[q]; ++i) {
                const uint32_t c = cells[size_t(q) * P + i];
                GF_REQUIRE(c < P, GF_E_ARG, "cell id out of range");
                // the kernels draw entry points inside the first cell and read every listed cell
                GF_REQUIRE(b->ix->offset_h[c + 1] > b->ix->offset_h[c], GF_E_ARG, "cell list names a cell with no point");
            }
        }
        const size_t Q = b->Q;
        // an earlier stage call may still be writing these buffers
        flush_stages(b);
        GF_HIP(hipStreamSynchronize(b->ix->stream));
        GF_HIP(hipMemcpy(b->cells.p, cells, Q * P * 4, hipMemcpyHostToDevice));
        GF_HIP(hipMemcpy(b->counts.p, counts, Q * 4, hipMemcpyHostToDevice));
        GF_HIP(hipMemcpy(b->little.p, little, Q * 4, hipMemcpyHostToDevice));
        b->marked = true;
        b->flags_ready = false;
        b->bf_all = false;
        b->route_bf = false;
    });
}

gf_status gf_batch_get_centroid(const gf_batch* b, float* dist, uint32_t* topc) {
    return run_guarded([&] {
        GF_REQUIRE(b, GF_E_ARG, "null batch");
        GF_REQUIRE(b->ordered, GF_E_STATE, "gf_order_cells has not run");
        set_device(b->ix);
        const gf_index* ix = b->ix;
        flush_stages(const_cast<gf_batch*>(b));
        GF_HIP(hipStreamSynchronize(ix->stream));
        if (dist && !b->cdist_ready) {
            // the matrix the nearest centres were chosen from (same tiles, same rounding)
            gf_batch* mb = const_cast<gf_batch*>(b);
            if (!mb->cdist.p) mb->cdist.alloc(size_t(b->Q) * ix->C);
            GF_HIP(gf::launch_centroid(b->q16.p, ix->centres.p, b->qnorm.p, ix->cnorm.p, b->Q, ix->C, b->Qp, ix->Cp,
                                       ix->Dp, mb->cdist.p, ix->stream));
            GF_HIP(hipStreamSynchronize(ix->stream));
            mb->cdist_ready = true;
        }
        if (dist) GF_HIP(hipMemcpy(dist, b->cdist.p, size_t(b->Q) * ix->C * 4, hipMemcpyDeviceToHost));
        if (topc) GF_HIP(hipMemcpy(topc, b->topk.p, size_t(b->Q) * b->topc * 4, hipMemcpyDeviceToHost));
    });
}

gf_status gf_batch_get_cell_flags(const gf_batch* b, uint8_t* flags) {
    return run_guarded([&] {
        GF_REQUIRE(b && flags, GF_E_ARG, "null argument");
        GF_REQUIRE(b->marked, GF_E_STATE, "cells not marked");
        gf_batch* mb = const_cast<gf_batch*>(b);
        set_device(b->ix);
        flush_stages(mb);
        GF_HIP(hipStreamSynchronize(b->ix->stream));
        const size_t n = size_t(b->Q) * b->ix->P;
        if (!b->flags_ready) {
            if (mb->flags.n < n) mb->flags.alloc(n);
            GF_HIP(gf::launch_cell_flags(b->Q, b->ix->P, b->cells.p, b->counts.p, b->little.p, mb->flags.p,
                                         b->ix->stream));
            GF_HIP(hipStreamSynchronize(b->ix->stream));
        }
        GF_HIP(hipMemcpy(flags, b->flags.p, n, hipMemcpyDeviceToHost));
    });
}

gf_status gf_batch_get_counters(const gf_batch* b, uint32_t* counters) {
    return run_guarded([&] {
        GF_REQUIRE(b && counters, GF_E_ARG, "null argument");
        GF_REQUIRE(b->counters.p, GF_E_STATE, "gf_search has not run");
        set_device(b->ix);
        flush_stages(const_cast<gf_batch*>(b));
        GF_HIP(hipStreamSynchronize(b->ix->stream));
        GF_HIP(hipMemcpy(counters, b->counters.p, size_t(b->Q) * GF_NCOUNTERS * 4, hipMemcpyDeviceToHost));
        if (b->pass_pending) {
            // the MFMA brute force reports the exact count as PASS; it was
            // not made by gf_mark_cells: make it now
            gf_batch* mb = const_cast<gf_batch*>(b);
            ensure_selcount(*mb);
            std::vector<uint32_t> sel(b->Q);
            GF_HIP(hipMemcpy(sel.data(), b->selcount.p, size_t(b->Q) * 4, hipMemcpyDeviceToHost));
            for (uint32_t q = 0; q < b->Q; ++q)
                if (counters[size_t(q) * GF_NCOUNTERS + 7] == 2u) counters[size_t(q) * GF_NCOUNTERS + 6] = sel[q];
        }
    });
}

gf_status gf_f2h(const float* x, size_t n, float alpha, uint16_t* out) {
    return run_guarded([&] {
        GF_REQUIRE(x && out, GF_E_ARG, "null argument");
        if (!n) return;
        DevBuf<float> dx;
        DevBuf<uint16_t> dy;
        dx.upload(x, n);
        dy.alloc(n);
        GF_HIP(gf::launch_f2h(dx.p, dy.p, n, alpha, nullptr));
        GF_HIP(hipMemcpy(out, dy.p, n * 2, hipMemcpyDeviceToHost));
    });
}

gf_status gf_row_norms_f16(const uint16_t* x, uint32_t n, uint32_t D, float* out) {
    return run_guarded([&] {
        GF_REQUIRE(x && out, GF_E_ARG, "null argument");
        if (!n) return;
        DevBuf<uint16_t> dx;
        DevBuf<float> dy;
        dx.upload(x, size_t(n) * D);
        dy.alloc(n);
        GF_HIP(gf::launch_norms_f16(dx.p, n, D, D, dy.p, nullptr));
        GF_HIP(hipMemcpy(out, dy.p, size_t(n) * 4, hipMemcpyDeviceToHost));
    });
}

gf_status gf_grid_scatter(const float* attrs, uint32_t N, uint32_t a, const uint32_t* grid_shape, float* l_q,
                          float* r_q, uint32_t* pid_lists, uint32_t* global_pid) {
    return run_guarded([&] { gf::grid_scatter(attrs, N, a, grid_shape, l_q, r_q, pid_lists, global_pid); });
}

gf_status gf_build_graphs(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D,
                          const uint32_t* global_pid, uint32_t P, uint32_t R, uint32_t E, int32_t device,
                          uint32_t* cell_graphs, uint32_t* cross, gf_build_stats* stats) {
    return run_guarded([&] {
        gf::build_graphs(vectors, vec_dtype, N, D, global_pid, P, R, E, device, cell_graphs, cross, stats);
    });
}

gf_status gf_optimize_graphs(const uint32_t* knn_graphs, uint32_t N, uint32_t I, const uint32_t* cell_size,
                             uint32_t P, uint32_t R, int32_t device, uint32_t* graphs, double* ms) {
    return run_guarded([&] { gf::optimize_graphs(knn_graphs, N, I, cell_size, P, R, device, graphs, ms); });
}

gf_status gf_kmeans(const void* vectors, int32_t vec_dtype, uint32_t N, uint32_t D, uint32_t C, uint32_t iters,
                    const uint32_t* init_ids, int32_t device, int32_t* labels, uint8_t* centres, double* ms) {
    return run_guarded([&] {
        gf::kmeans_labels(vectors, vec_dtype, N, D, C, iters, init_ids, device, labels, centres, ms);
    });
}

gf_status gf_quantise_i8(const float* x, uint64_t n, uint32_t D, float alpha, float* scale, int32_t* zero,
                         int8_t* out) {
    return run_guarded([&] {
        GF_REQUIRE(D >= 1 && scale && zero && (n == 0 || (x && out)), GF_E_ARG, "gf_quantise_i8: bad argument");
        std::vector<float> s;
        std::vector<int32_t> z;
        gf::quantise_i8(x, n, D, alpha, s, z, out);
        std::memcpy(scale, s.data(), sizeof(float) * D);
        std::memcpy(zero, z.data(), sizeof(int32_t) * D);
    });
}

gf_status gf_host_alloc(size_t bytes, void** out) {
    return run_guarded([&] {
        GF_REQUIRE(out && bytes > 0, GF_E_ARG, "gf_host_alloc: null output or zero size");
        *out = nullptr;
        GF_HIP(hipHostMalloc(out, bytes, hipHostMallocDefault));
    });
}

gf_status gf_host_free(void* ptr) {
    return run_guarded([&] {
        if (ptr) GF_HIP(hipHostFree(ptr));
    });
}

gf_status gf_stream_plan_cells(const uint32_t* cells, const uint32_t* counts, uint32_t Q, uint32_t a,
                               const uint32_t* grid_shape, const uint32_t* cell_size, uint64_t max_points,
                               uint32_t max_cells, uint32_t* sizes, uint32_t* plan_cells, uint32_t* nbatch,
                               uint64_t* active) {
    return run_guarded([&] {
        GF_REQUIRE(grid_shape && cell_size && sizes && plan_cells && nbatch, GF_E_ARG,
                   "gf_stream_plan_cells: null argument");
        GF_REQUIRE(Q == 0 || (cells && counts), GF_E_ARG, "gf_stream_plan_cells: null cell lists");
        std::vector<std::vector<uint32_t>> plan;
        const uint64_t act = gf::plan_cells(cells, counts, Q, a, grid_shape, cell_size, max_points, max_cells, plan);
        size_t k = 0;
        for (size_t i = 0; i < plan.size(); ++i) {
            sizes[i] = uint32_t(plan[i].size());
            for (uint32_t c : plan[i]) plan_cells[k++] = c;
        }
        *nbatch = uint32_t(plan.size());
        if (active) *active = act;
    });
}

gf_status gf_batch_plan_stream(gf_batch* b, uint64_t max_points, uint32_t max_cells, uint32_t* nbatch,
                               uint64_t* active, double* ms) {
    return run_guarded([&] {
        const auto t0 = std::chrono::steady_clock::now();
        GF_REQUIRE(b, GF_E_ARG, "null batch");
        GF_REQUIRE(b->ix->sx, GF_E_UNSUPPORTED, "gf_batch_plan_stream: not a streamed index");
        GF_REQUIRE(b->marked, GF_E_STATE, "cells not marked");
        set_device(b->ix);
        flush_stages(b);
        const uint64_t act = gf::stream_plan_batch(*b, max_points, max_cells);
        if (nbatch) *nbatch = uint32_t(b->splan->batches.size());
        if (active) *active = act;
        if (ms) *ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    });
}

gf_status gf_batch_set_stream_plan(gf_batch* b, uint32_t nbatch, const uint32_t* sizes, const uint32_t* cells) {
    return run_guarded([&] {
        GF_REQUIRE(b, GF_E_ARG, "null batch");
        GF_REQUIRE(b->ix->sx, GF_E_UNSUPPORTED, "gf_batch_set_stream_plan: not a streamed index");
        GF_REQUIRE(nbatch == 0 || (sizes && cells), GF_E_ARG, "null plan");
        const uint32_t P = b->ix->P;
        std::vector<std::vector<uint32_t>> plan;
        size_t k = 0;
        for (uint32_t i = 0; i < nbatch; ++i) {
            GF_REQUIRE(sizes[i] >= 1 && sizes[i] <= P, GF_E_ARG, "stream plan batch size out of range");
            GF_REQUIRE(k + sizes[i] <= P, GF_E_ARG, "stream plan holds more cells than the grid");
            plan.emplace_back(cells + k, cells + k + sizes[i]);
            k += sizes[i];
        }
        set_device(b->ix);
        gf::stream_set_plan(*b, std::move(plan));
    });
}

gf_status gf_batch_get_stream_plan(const gf_batch* b, uint32_t* nbatch, uint32_t* sizes, uint32_t* cells) {
    return run_guarded([&] {
        GF_REQUIRE(b && nbatch, GF_E_ARG, "null argument");
        GF_REQUIRE(b->ix->sx, GF_E_UNSUPPORTED, "gf_batch_get_stream_plan: not a streamed index");
        const gf::StreamPlan& pl = b->splan ? *b->splan : *b->ix->sx->plan;
        *nbatch = uint32_t(pl.cells.size());
        size_t k = 0;
        for (size_t i = 0; i < pl.cells.size(); ++i) {
            if (sizes) sizes[i] = uint32_t(pl.cells[i].size());
            for (uint32_t c : pl.cells[i]) {
                if (cells) cells[k] = c;
                ++k;
            }
        }
    });
}

gf_status gf_entry_points(uint32_t N, uint32_t P, uint32_t R, uint32_t* out) {
    return run_guarded([&] {
        GF_REQUIRE(out && P >= 1 && N >= P, GF_E_ARG, "invalid arguments");
        entry_points_ref(N, P, R, out);
    });
}

}  // extern "C"
