// Readers for the GMG index files (formats written by the reference's
// indexbuild/*.py and read by indexsearch/tools.cuh, check.cu and
// real_dataset_adapter.cuh).  All fields are little-endian 32-bit.  Unlike the
// reference loaders (which exit(-1) on a missing file and never check sizes),
// every read is bounds-checked and a failure is reported as gf::Error.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "gf_internal.h"

namespace gf {
namespace {

struct File {
    FILE* f = nullptr;
    std::string path;
    explicit File(const std::string& p) : path(p) {
        f = std::fopen(p.c_str(), "rb");
        if (!f) throw Error{GF_E_IO, "cannot open " + p};
    }
    ~File() {
        if (f) std::fclose(f);
    }
    // File size in bytes; the read position is left where it was.
    size_t size() {
        const long pos = std::ftell(f);
        std::fseek(f, 0, SEEK_END);
        const long s = std::ftell(f);
        std::fseek(f, pos, SEEK_SET);
        return s < 0 ? 0 : size_t(s);
    }
    void read(void* dst, size_t bytes) {
        if (bytes && std::fread(dst, 1, bytes, f) != bytes) throw Error{GF_E_IO, "truncated file " + path};
    }
    int32_t i32() {
        int32_t v;
        read(&v, 4);
        return v;
    }
};

// .fvecs: per row i32 dim, dim x f32 (tools.cuh:85-106).
void read_fvecs(const std::string& p, std::vector<float>& out, uint32_t& n, uint32_t& dim) {
    File f(p);
    const size_t sz = f.size();
    if (sz < 4) throw Error{GF_E_FORMAT, "empty fvecs " + p};
    const int32_t d = f.i32();
    if (d <= 0) throw Error{GF_E_FORMAT, "bad dimension in " + p};
    const size_t row = 4 * (size_t(d) + 1);
    if (sz % row != 0) throw Error{GF_E_FORMAT, "fvecs size is not a multiple of the row size: " + p};
    n = uint32_t(sz / row);
    dim = uint32_t(d);
    out.resize(size_t(n) * dim);
    std::fseek(f.f, 0, SEEK_SET);
    for (uint32_t i = 0; i < n; ++i) {
        if (f.i32() != d) throw Error{GF_E_FORMAT, "inconsistent row dimension in " + p};
        f.read(&out[size_t(i) * dim], size_t(dim) * 4);
    }
}

// Graph file: i32 n, i32 k, n*k u32 (tools.cuh:205-223).
void read_graph(const std::string& p, std::vector<uint32_t>& out, uint32_t& n, uint32_t& k) {
    File f(p);
    const int32_t nn = f.i32(), kk = f.i32();
    if (nn < 0 || kk <= 0) throw Error{GF_E_FORMAT, "bad graph header in " + p};
    n = uint32_t(nn);
    k = uint32_t(kk);
    if (f.size() != 8 + size_t(n) * k * 4) throw Error{GF_E_FORMAT, "graph size mismatch in " + p};
    std::fseek(f.f, 8, SEEK_SET);
    out.resize(size_t(n) * k);
    f.read(out.data(), out.size() * 4);
}

}  // namespace

void read_index_files(const gf_index_paths& p, uint32_t degree, HostIndex& out) {
    if (!p.data_path || !p.cagra_prefix || !p.cagra_suffix || !p.global_graph || !p.grid || !p.attrs)
        throw Error{GF_E_ARG, "missing index path"};
    read_fvecs(p.data_path, out.vectors, out.N, out.D);

    // Grid: i32 N, i32 a, i32 g[a]; per attribute l_q[g], r_q[g], pid[N];
    // then global_pid[N] (indexbuild/tools.py:127-141).
    {
        File f(p.grid);
        const int32_t n = f.i32(), a = f.i32();
        if (n <= 0 || uint32_t(n) != out.N) throw Error{GF_E_FORMAT, "grid point count differs from the data"};
        if (a <= 0 || a > int32_t(kMaxAttr)) throw Error{GF_E_UNSUPPORTED, "grid attribute count out of range"};
        out.a = uint32_t(a);
        std::vector<int32_t> g(a);
        f.read(g.data(), size_t(a) * 4);
        uint64_t P = 1;
        for (int32_t v : g) {
            if (v <= 0) throw Error{GF_E_FORMAT, "bad grid shape"};
            out.grid.push_back(uint32_t(v));
            P *= uint64_t(v);
        }
        if (P > 4096) throw Error{GF_E_UNSUPPORTED, "more than 4096 cells"};
        out.P = uint32_t(P);
        std::vector<int32_t> tmp(out.N);
        for (int32_t d = 0; d < a; ++d) {
            std::vector<int32_t> lq(g[d]), rq(g[d]);
            f.read(lq.data(), lq.size() * 4);
            f.read(rq.data(), rq.size() * 4);
            for (int32_t v : lq) out.l_q.push_back(float(v));
            for (int32_t v : rq) out.r_q.push_back(float(v));
            f.read(tmp.data(), tmp.size() * 4);  // per-attribute cell index (unused)
        }
        f.read(tmp.data(), tmp.size() * 4);
        if (std::ftell(f.f) != long(f.size())) throw Error{GF_E_FORMAT, "grid file has trailing bytes: " + f.path};
        out.global_pid.resize(out.N);
        for (uint32_t i = 0; i < out.N; ++i) {
            if (tmp[i] < 0 || uint32_t(tmp[i]) >= out.P) throw Error{GF_E_FORMAT, "global_pid out of range"};
            out.global_pid[i] = uint32_t(tmp[i]);
        }
    }
    // Attributes: u32 N, u32 a, N*a i32, converted to float as the driver
    // does (tools.cuh:746-765, realdataset_search.cu:2182-2190).
    {
        File f(p.attrs);
        uint32_t n, a;
        f.read(&n, 4);
        f.read(&a, 4);
        if (n != out.N || a != out.a) throw Error{GF_E_FORMAT, "attribute file shape differs from the grid"};
        if (f.size() != 8 + size_t(n) * a * 4) throw Error{GF_E_FORMAT, "attribute file size mismatch"};
        std::vector<int32_t> v(size_t(n) * a);
        f.read(v.data(), v.size() * 4);
        out.attrs.resize(v.size());
        for (size_t i = 0; i < v.size(); ++i) out.attrs[i] = float(v[i]);
    }
    // Per-cell graphs prefix + i + suffix, concatenated in cell order
    // (check.cu:406-484).
    {
        std::vector<uint32_t> csize(out.P, 0);
        for (uint32_t i = 0; i < out.N; ++i) csize[out.global_pid[i]]++;
        out.cell_graphs.reserve(size_t(out.N) * (degree ? degree : 32));
        for (uint32_t c = 0; c < out.P; ++c) {
            std::vector<uint32_t> g;
            uint32_t n, k;
            read_graph(std::string(p.cagra_prefix) + std::to_string(c) + p.cagra_suffix, g, n, k);
            if (n != csize[c]) throw Error{GF_E_FORMAT, "graph " + std::to_string(c) + " size differs from its cell"};
            if (c == 0) out.R = k;
            if (k != out.R) throw Error{GF_E_FORMAT, "per-cell graphs have different degrees"};
            if (degree && k != degree) throw Error{GF_E_FORMAT, "--degree does not match the graph files"};
            out.cell_graphs.insert(out.cell_graphs.end(), g.begin(), g.end());
        }
    }
    // Cross-cell graph: i32 N, i32 P*E, N*(P*E) u32 (global_graph_build.py).
    {
        uint32_t n, k;
        read_graph(p.global_graph, out.cross, n, k);
        if (n != out.N || k % out.P != 0) throw Error{GF_E_FORMAT, "cross-cell graph shape mismatch"};
        out.E = k / out.P;
    }
    // Labels: i32 N, N*i32 (clustering.py:84-87).
    if (p.cluster && p.cluster[0]) {
        File f(p.cluster);
        const int32_t n = f.i32();
        if (n < 0 || uint32_t(n) != out.N) throw Error{GF_E_FORMAT, "cluster label count differs from the data"};
        out.labels.resize(out.N);
        f.read(out.labels.data(), size_t(out.N) * 4);
        out.has_labels = true;
    }
}

}  // namespace gf
