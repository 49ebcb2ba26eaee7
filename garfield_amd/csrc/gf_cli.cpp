// garfield_search: command-line driver with the flags of the reference's
// realdataset_search (realdataset_search.cu:2712-2751) on top of the C ABI.
//
// For every L of the sweep it runs the search on the whole query batch and
// writes one CSV row "ef,recall,qps,total_cost,cost1,cost2,cost3,kernal_cost"
// (realdataset_search.cu:271, 302): costs in seconds, cost1 = cell marking +
// selectivity (stage A), cost2 = cluster-guided cell order (stage B), cost3 =
// search device time for that L, kernal_cost = the search kernels' device time,
// qps = Q / (cost1 + cost2 + cost3) (realdataset_search.cu:2506-2508).  Recall
// is the mean over queries of |result ∩ ground truth| / |ground truth|, 1 for
// an empty ground truth (tools.cuh:384-453).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "garfield.h"

namespace {

[[noreturn]] void die(const std::string& msg) {
    std::fprintf(stderr, "garfield_search: %s\n", msg.c_str());
    std::exit(1);
}

void check(gf_status s, const char* what) {
    if (s != GF_OK) die(std::string(what) + ": " + gf_status_str(s) + ": " + gf_last_error());
}

std::vector<char> read_file(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) die("cannot open " + path);
    return std::vector<char>((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
}

// .fvecs: per vector an int32 dimension followed by that many floats.
std::vector<float> read_fvecs(const std::string& path, uint32_t& n, uint32_t& d) {
    const std::vector<char> raw = read_file(path);
    if (raw.size() < 4) die(path + ": empty fvecs file");
    int32_t dim;
    std::memcpy(&dim, raw.data(), 4);
    if (dim <= 0) die(path + ": bad dimension");
    const size_t row = 4 + size_t(dim) * 4;
    if (raw.size() % row) die(path + ": size is not a multiple of the row size");
    n = uint32_t(raw.size() / row);
    d = uint32_t(dim);
    std::vector<float> out(size_t(n) * d);
    for (uint32_t i = 0; i < n; ++i) std::memcpy(&out[size_t(i) * d], raw.data() + i * row + 4, size_t(d) * 4);
    return out;
}

void usage() {
    std::printf(
        "usage: garfield_search --data_path F --query_path F --range F --cagra_prefix P --cagra_suffix S\n"
        "                       --global_graph F --grid F --attrs F [--cluster F] [--gt F] [--result F]\n"
        "                       [--prefilter x] [--postfilter n] [--f2h_factor x] [--degree n]\n"
        "                       [--L l1,l2,...] [--vec_dtype f16|f32|i8q] [--channels 1|2] [--device n]\n");
}

}  // namespace

int main(int argc, char** argv) {
    std::string data_path, query_path, range_path, gt_path, cagra_prefix, cagra_suffix, global_graph, grid, attrs,
        cluster, result;
    float prefilter = 0.0f, f2h_factor = 1.0f;
    uint32_t postfilter = 0xFFFFFFFFu, degree = 0;
    int32_t vec_dtype = GF_VEC_F16, device = 0, channels = 1;
    // the reference's sweep (realdataset_search.cu:2757), ascending
    std::vector<uint32_t> Ls = {10,  15,  20,  25,  30,  35,  40,  45,  50,  55,  60,  70,   80,   90,   100,  120,
                                140, 160, 180, 200, 250, 300, 400, 500, 600, 700, 800, 900, 1000, 1100, 1400, 1700};
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--help" || a == "-h") { usage(); return 0; }
        if (i + 1 >= argc) die("missing value for " + a);
        const std::string v = argv[++i];
        if (a == "--data_path") data_path = v;
        else if (a == "--query_path") query_path = v;
        else if (a == "--range") range_path = v;
        else if (a == "--gt") gt_path = v;
        else if (a == "--cagra_prefix") cagra_prefix = v;
        else if (a == "--cagra_suffix") cagra_suffix = v;
        else if (a == "--global_graph") global_graph = v;
        else if (a == "--grid") grid = v;
        else if (a == "--attrs") attrs = v;
        else if (a == "--cluster") cluster = v;
        else if (a == "--result") result = v;
        else if (a == "--prefilter") prefilter = std::stof(v);
        else if (a == "--postfilter") postfilter = uint32_t(std::stoul(v));
        else if (a == "--f2h_factor") f2h_factor = std::stof(v);
        else if (a == "--degree") degree = uint32_t(std::stoul(v));
        else if (a == "--device") device = std::stoi(v);
        else if (a == "--channels") {
            channels = std::stoi(v);
            if (channels != 1 && channels != 2) die("--channels must be 1 or 2");
        }
        else if (a == "--vec_dtype") {
            if (v == "f16") vec_dtype = GF_VEC_F16;
            else if (v == "f32") vec_dtype = GF_VEC_F32;
            else if (v == "i8q") vec_dtype = GF_VEC_I8Q;
            else if (v == "f16ref") vec_dtype = GF_VEC_F16_REF;
            else die("--vec_dtype must be f16, f16ref, f32 or i8q");
        } else if (a == "--L") {
            Ls.clear();
            std::stringstream ss(v);
            std::string t;
            while (std::getline(ss, t, ',')) Ls.push_back(uint32_t(std::stoul(t)));
            if (Ls.empty()) die("--L needs at least one value");
        } else {
            usage();
            die("unknown flag " + a);
        }
    }
    if (data_path.empty() || query_path.empty() || range_path.empty() || cagra_prefix.empty() ||
        global_graph.empty() || grid.empty() || attrs.empty())
        die("--data_path, --query_path, --range, --cagra_prefix, --global_graph, --grid and --attrs are required");

    gf_index_paths paths{data_path.c_str(), cagra_prefix.c_str(), cagra_suffix.c_str(), global_graph.c_str(),
                         grid.c_str(),      attrs.c_str(),        cluster.empty() ? nullptr : cluster.c_str()};
    gf_open_opts oo{degree, f2h_factor, vec_dtype, 0, device, 0};
    gf_index* ix = nullptr;
    check(gf_index_open(&paths, &oo, &ix), "gf_index_open");
    gf_index_info info{};
    check(gf_index_get_info(ix, &info), "gf_index_get_info");

    uint32_t Q = 0, qd = 0;
    const std::vector<float> queries = read_fvecs(query_path, Q, qd);
    if (qd != info.D) die("query dimension differs from the data");
    // ranges: int32 (lo, hi) per attribute per query (load_range, tools.cuh:274-291)
    const std::vector<char> rr = read_file(range_path);
    if (rr.size() < size_t(Q) * info.a * 8) die(range_path + ": fewer ranges than queries");
    std::vector<float> lo(size_t(Q) * info.a), hi(size_t(Q) * info.a);
    for (size_t i = 0; i < size_t(Q) * info.a; ++i) {
        int32_t l, h;
        std::memcpy(&l, rr.data() + 8 * i, 4);
        std::memcpy(&h, rr.data() + 8 * i + 4, 4);
        lo[i] = float(l);
        hi[i] = float(h);
    }
    // ground truth: uint32 qnum, k, then qnum * k ids (load_ground_truth, tools.cuh:819-834)
    std::vector<std::vector<uint32_t>> gt;
    if (!gt_path.empty()) {
        const std::vector<char> g = read_file(gt_path);
        uint32_t gq = 0, gk = 0;
        if (g.size() < 8) die(gt_path + ": truncated");
        std::memcpy(&gq, g.data(), 4);
        std::memcpy(&gk, g.data() + 4, 4);
        if (g.size() < 8 + size_t(gq) * gk * 4 || gq < Q) die(gt_path + ": truncated or too few queries");
        gt.assign(Q, {});
        for (uint32_t q = 0; q < Q; ++q)
            for (uint32_t j = 0; j < gk; ++j) {
                uint32_t id;
                std::memcpy(&id, g.data() + 8 + (size_t(q) * gk + j) * 4, 4);
                if (id < info.N) gt[q].push_back(id);
            }
    }

    gf_batch* b = nullptr;
    check(gf_batch_create(ix, queries.data(), Q, lo.data(), hi.data(), &b), "gf_batch_create");
    double cost1 = 0, cost2 = 0;
    check(gf_mark_cells(b, prefilter, &cost1), "gf_mark_cells");
    if (info.C) check(gf_order_cells(b, 4, &cost2), "gf_order_cells");

    FILE* out = result.empty() ? nullptr : std::fopen(result.c_str(), "w");
    if (!result.empty() && !out) die("cannot write " + result);
    const char* header = "ef,recall,qps,total_cost,cost1,cost2,cost3,kernal_cost\n";
    std::fputs(header, stdout);
    if (out) std::fputs(header, out);
    const uint32_t K = 10;
    std::vector<uint32_t> ids(size_t(Q) * K);
    for (uint32_t L : Ls) {
        gf_search_opts so{L, K, 10, postfilter, nullptr};
        gf_search_stats st{};
        if (channels == 2) check(gf_search_dual(b, &so, ids.data(), nullptr, &st), "gf_search_dual");
        else check(gf_search(b, &so, ids.data(), nullptr, &st), "gf_search");
        double recall = -1.0;
        if (!gt.empty()) {
            double sum = 0;
            for (uint32_t q = 0; q < Q; ++q) {
                if (gt[q].empty()) { sum += 1.0; continue; }
                const std::set<uint32_t> g(gt[q].begin(), gt[q].end());
                std::set<uint32_t> hit;
                for (uint32_t j = 0; j < K; ++j)
                    if (g.count(ids[size_t(q) * K + j])) hit.insert(ids[size_t(q) * K + j]);
                sum += double(hit.size()) / double(g.size());
            }
            recall = sum / Q;
        }
        const double c1 = cost1 / 1e3, c2 = cost2 / 1e3, c3 = st.ms_total / 1e3;
        const double total = c1 + c2 + c3;
        char line[256];
        std::snprintf(line, sizeof(line), "%u,%.6f,%.1f,%.6f,%.6f,%.6f,%.6f,%.6f\n", L, recall, Q / total, total, c1,
                      c2, c3, c3);
        std::fputs(line, stdout);
        if (out) std::fputs(line, out);
    }
    if (out) std::fclose(out);
    gf_batch_free(b);
    gf_index_close(ix);
    return 0;
}
