// Test harness: runs the library's index-file reader (gf_io.cpp) on the CPU
// and writes every array it produced as raw little-endian files into an
// output directory, so a test can compare them with the arrays it wrote.
// usage: io_dump <prefix> <outdir>   (files <prefix>.fvecs, _cell<i>.graph,
// .cross, .grid, .attrs, .cluster)
#include <cstdio>
#include <string>
#include <vector>

#include "../../garfield_amd/csrc/gf_internal.h"

template <class T>
static bool dump(const std::string& path, const std::vector<T>& v) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = std::fwrite(v.data(), sizeof(T), v.size(), f) == v.size();
    std::fclose(f);
    return ok;
}

int main(int argc, char** argv) {
    if (argc != 3) return 2;
    const std::string p = argv[1], o = std::string(argv[2]) + "/";
    const std::string data = p + ".fvecs", cell = p + "_cell", sfx = ".graph", cross = p + ".cross",
                      grid = p + ".grid", attrs = p + ".attrs", cluster = p + ".cluster";
    gf_index_paths paths{data.c_str(), cell.c_str(), sfx.c_str(), cross.c_str(),
                         grid.c_str(), attrs.c_str(), cluster.c_str()};
    gf::HostIndex h;
    try {
        gf::read_index_files(paths, 0, h);
    } catch (const gf::Error& e) {
        std::fprintf(stderr, "%s\n", e.msg.c_str());
        return 1;
    }
    std::printf("%u %u %u %u %u %u\n", h.N, h.D, h.a, h.P, h.R, h.E);
    const bool ok = dump(o + "vectors", h.vectors) && dump(o + "attrs", h.attrs) && dump(o + "l_q", h.l_q) &&
                    dump(o + "r_q", h.r_q) && dump(o + "global_pid", h.global_pid) &&
                    dump(o + "cell_graphs", h.cell_graphs) && dump(o + "cross", h.cross) &&
                    dump(o + "labels", h.labels);
    return ok ? 0 : 3;
}
