// fmt_io.cpp - saving a built VCSR format to a file and loading it back,
// so that a matrix's format is built once (the reference rebuilds it on
// every run, src/main.cpp:128-149).  The file holds the host arrays
// bit-identically plus the row-tile view settings; the device copy and the
// views derived at upload are rebuilt by vcsr_fmt_upload.
//
// File layout (little-endian, every field 4 or 8 bytes):
//   "VCSRFMT1"                                       8 bytes
//   int32 M, N, segw, bundle, layout, num_segments,
//         tile_rows, tile_fixed                      8 x 4 bytes
//   int64 G (groups), P (slots)                      2 x 8 bytes
//   int32 group_ptr[G+1], group_depth[G], group_seg_base[G],
//         group_rows[G*bundle], lcol[P]; float val[P];
//   int32 segment_group_start[num_segments+1]
// A loaded file is checked against every invariant the kernels rely on
// (validate_vcsr) before it is accepted.
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>

#include "fmt_io.hpp"

namespace vcsr {
namespace {

constexpr int kEinval = 1;  // VCSR_EINVAL
constexpr int kEio = 2;     // VCSR_EIO
constexpr char kMagic[8] = {'V', 'C', 'S', 'R', 'F', 'M', 'T', '1'};

struct FileCloser {
    void operator()(FILE* f) const {
        if (f) std::fclose(f);
    }
};
using File = std::unique_ptr<FILE, FileCloser>;

void bad(const std::string& what) { throw Error(kEinval, "invalid VCSR format: " + what); }

template <class T>
void put(FILE* f, const T* p, size_t n, const std::string& path) {
    if (n && std::fwrite(p, sizeof(T), n, f) != n) throw Error(kEio, "write failed: " + path);
}

template <class T>
void get(FILE* f, T* p, size_t n, const std::string& path) {
    if (n && std::fread(p, sizeof(T), n, f) != n)
        throw Error(kEio, "truncated VCSR format file: " + path);
}

}  // namespace

void validate_vcsr(const Vcsr& v) {
    if (v.M < 0 || v.N < 0) bad("negative shape");
    if (v.segw <= 0 || v.bundle <= 0) bad("segw and bundle must be positive");
    if (v.layout != kLayoutH && v.layout != kLayoutS && v.layout != kLayoutTC) bad("layout");
    const int64_t S = ((int64_t)v.N + v.segw - 1) / v.segw;
    if (v.num_segments != S) bad("segment count does not match N and segw");
    const int64_t G = (int64_t)v.group_depth.size();
    const int64_t b = v.bundle;
    if ((int64_t)v.group_ptr.size() != G + 1 || (int64_t)v.group_seg_base.size() != G ||
        (int64_t)v.group_rows.size() != G * b)
        bad("group array sizes");
    if (v.lcol.size() != v.val.size()) bad("lcol and val sizes differ");
    if (v.group_ptr[0] != 0) bad("group_ptr[0] != 0");
    for (int64_t g = 0; g < G; ++g) {
        const int64_t d = v.group_depth[(size_t)g];
        // Every builder emits groups of depth >= 1 (layout H skips all-empty
        // bundles, layouts S and TC group active rows only), and the upload
        // reads each group's depth-0 slots.
        if (d < 1) bad("group depth below 1");
        if ((int64_t)v.group_ptr[(size_t)g + 1] - v.group_ptr[(size_t)g] != d * b)
            bad("group_ptr does not advance by depth * bundle");
    }
    if ((int64_t)v.group_ptr[(size_t)G] != (int64_t)v.lcol.size()) bad("slot count");
    if ((int64_t)v.segment_group_start.size() != S + 1) bad("segment_group_start size");
    if (v.segment_group_start[0] != 0 || v.segment_group_start[(size_t)S] != G)
        bad("segment_group_start ends");
    for (int64_t s = 0; s < S; ++s) {
        const int32_t a = v.segment_group_start[(size_t)s], e = v.segment_group_start[(size_t)s + 1];
        if (a > e) bad("segment_group_start not ascending");
        for (int32_t g = a; g < e; ++g)
            if ((int64_t)v.group_seg_base[(size_t)g] != s * v.segw) bad("group segment base");
    }
    for (int64_t g = 0; g < G; ++g) {
        const int64_t base = v.group_seg_base[(size_t)g];
        const int64_t p0 = v.group_ptr[(size_t)g], d = v.group_depth[(size_t)g];
        bool active = true;  // lanes with entries come first
        for (int64_t l = 0; l < b; ++l) {
            const int32_t row = v.group_rows[(size_t)(g * b + l)];
            if (row < -1 || row >= v.M) bad("group row out of range");
            // A lane's entries are packed from depth 0.
            int64_t cnt = 0;
            while (cnt < d && v.lcol[(size_t)(p0 + l + cnt * b)] >= 0) ++cnt;
            for (int64_t k = 0; k < d; ++k) {
                const int32_t c = v.lcol[(size_t)(p0 + l + k * b)];
                if (k < cnt) {
                    if (c >= v.segw || base + c >= v.N) bad("local column out of range");
                } else if (c != -1) {
                    bad("lane entries not packed from depth 0");
                }
            }
            if (cnt > 0 && (row < 0 || !active)) bad("active lanes are not a prefix with rows");
            if (cnt == 0) active = false;
        }
    }
}

void save_vcsr(const Vcsr& v, int32_t tile_rows, bool tile_fixed, const std::string& path) {
    File f(std::fopen(path.c_str(), "wb"));
    if (!f) throw Error(kEio, "cannot create " + path);
    put(f.get(), kMagic, sizeof kMagic, path);
    const int32_t hdr[8] = {v.M,      v.N,         v.segw,    v.bundle, v.layout,
                            v.num_segments, tile_rows, tile_fixed ? 1 : 0};
    put(f.get(), hdr, 8, path);
    const int64_t counts[2] = {(int64_t)v.group_depth.size(), (int64_t)v.lcol.size()};
    put(f.get(), counts, 2, path);
    put(f.get(), v.group_ptr.data(), v.group_ptr.size(), path);
    put(f.get(), v.group_depth.data(), v.group_depth.size(), path);
    put(f.get(), v.group_seg_base.data(), v.group_seg_base.size(), path);
    put(f.get(), v.group_rows.data(), v.group_rows.size(), path);
    put(f.get(), v.lcol.data(), v.lcol.size(), path);
    put(f.get(), v.val.data(), v.val.size(), path);
    put(f.get(), v.segment_group_start.data(), v.segment_group_start.size(), path);
    if (std::fflush(f.get()) != 0) throw Error(kEio, "write failed: " + path);
}

Vcsr load_vcsr(const std::string& path, int32_t* tile_rows, bool* tile_fixed) {
    File f(std::fopen(path.c_str(), "rb"));
    if (!f) throw Error(kEio, "cannot open " + path);
    std::fseek(f.get(), 0, SEEK_END);
    const long fsize = std::ftell(f.get());
    std::fseek(f.get(), 0, SEEK_SET);
    char magic[8];
    get(f.get(), magic, 8, path);
    if (std::memcmp(magic, kMagic, 8) != 0) bad("not a VCSR format file (magic)");
    int32_t hdr[8];
    get(f.get(), hdr, 8, path);
    int64_t counts[2];
    get(f.get(), counts, 2, path);
    Vcsr v;
    v.M = hdr[0];
    v.N = hdr[1];
    v.segw = hdr[2];
    v.bundle = hdr[3];
    v.layout = hdr[4];
    v.num_segments = hdr[5];
    const int64_t G = counts[0], P = counts[1];
    if (G < 0 || P < 0 || v.bundle <= 0 || v.num_segments < 0 || v.segw <= 0)
        bad("header counts");
    // The arrays must fit the file before anything is allocated for them.
    const double need = 8.0 + 32 + 16 + 4.0 * ((double)G + 1 + 2.0 * G + (double)G * v.bundle +
                                                2.0 * P + (double)v.num_segments + 1);
    if (need != (double)fsize) bad("file size does not match its header");
    v.group_ptr.resize((size_t)G + 1);
    v.group_depth.resize((size_t)G);
    v.group_seg_base.resize((size_t)G);
    v.group_rows.resize((size_t)(G * v.bundle));
    v.lcol.resize((size_t)P);
    v.val.resize((size_t)P);
    v.segment_group_start.resize((size_t)v.num_segments + 1);
    get(f.get(), v.group_ptr.data(), v.group_ptr.size(), path);
    get(f.get(), v.group_depth.data(), v.group_depth.size(), path);
    get(f.get(), v.group_seg_base.data(), v.group_seg_base.size(), path);
    get(f.get(), v.group_rows.data(), v.group_rows.size(), path);
    get(f.get(), v.lcol.data(), v.lcol.size(), path);
    get(f.get(), v.val.data(), v.val.size(), path);
    get(f.get(), v.segment_group_start.data(), v.segment_group_start.size(), path);
    validate_vcsr(v);
    const int32_t tr = hdr[6];
    if (tr != 0 && tr != 1 && tr != 2 && tr != 3 && tr != 4 && tr != 8 && tr != 16)
        bad("tile height");
    if (hdr[7] != 0 && hdr[7] != 1) bad("tile window flag");
    if (hdr[7] == 1 && tr == 0) bad("fixed windows without a tile height");
    if (tile_rows) *tile_rows = tr;
    if (tile_fixed) *tile_fixed = hdr[7] == 1;
    return v;
}

}  // namespace vcsr
