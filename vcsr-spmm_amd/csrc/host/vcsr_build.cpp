// vcsr_build.cpp - VCSR format builders (layouts H, S and TC).
//
// The arrays produced are bit-identical to the reference builders:
//   layout H  : csr_to_vcsr_spmm      include/vcsr.hpp:25-109
//   layout S  : csr_to_vcsr_seg/_opt  src/vcsr_seg.cu:24-113, src/vcsr_opt.cu:23-101
//   layout TC : csr_to_vcsr_tc        src/vcsr_tc.cu:26-106 (segw=16, bundle=16)
// Algorithm (the same steps as the reference, kept alike because the row
// permutation is part of the format):
//   1. every nnz goes to segment sid = col / segw with local column col % segw;
//   2. the entries of one (segment, row) are ordered by local column with
//      std::sort (vcsr.hpp:43-48, vcsr_seg.cu:45-50);
//   3. the rows of a segment are ordered by their entry count, descending,
//      with std::sort.  Layout H sorts all M row ids starting from 0..M-1
//      (vcsr.hpp:56-59); layouts S/TC sort the active rows starting from the
//      iteration order of a std::unordered_map<int,...> filled in ascending
//      row order (vcsr_seg.cu:32,40,57-65);
//   4. the sorted rows are cut into bundles of `bundle` lanes; a bundle's depth
//      is its largest count; layout H skips depth-0 bundles (vcsr.hpp:70);
//   5. group_rows holds the row of each lane: layout H keeps the ids of empty
//      rows and uses -1 only past M (vcsr.hpp:76-80), layouts S/TC use -1 past
//      the active rows (vcsr_seg.cu:83-86);
//   6. slots are packed depth-major, lane-minor; a lane with fewer entries
//      than the depth gets (lcol=-1, val=0) (vcsr.hpp:82-96, vcsr_seg.cu:89-107).
// Because std::sort is not stable, ties are ordered by libstdc++'s introsort;
// reproducing them requires the same std::sort over sequences with the same
// comparison outcomes, and the same unordered_map insertion sequence (its
// iteration order depends only on the keys inserted, their order and the
// rehash policy, not on the mapped type).  That is what is done here, with
// flat arrays instead of per-row vectors.
//
// Work is split by segment: each segment's groups depend only on that
// segment's entries, so segments are built in parallel into per-block
// buffers and concatenated in segment order, giving the sequential result.
#include <algorithm>
#include <cstring>
#include <numeric>
#include <string>
#include <unordered_map>

#include "core.hpp"
#include "parallel.hpp"

namespace vcsr {
namespace {

struct SegEntry {
    int32_t row;
    int32_t lcol;
    float v;
};

// A run of entries of one row inside one segment.
struct Run {
    int32_t row;
    int32_t begin;  // index into the segment's entry list
    int32_t len;
};

// Output of a block of consecutive segments.
struct BlockOut {
    std::vector<int32_t> depth, rows, lcol;
    std::vector<float> val;
    std::vector<int32_t> groups_per_seg;
};

// Buckets all nnz by segment, keeping (row ascending, p ascending) order
// inside a segment, the order in which the reference pushes them.
void bucket_by_segment(const Csr& csr, int segw, int S, std::vector<int64_t>& seg_off,
                       std::vector<SegEntry>& ent) {
    seg_off.assign((size_t)S + 1, 0);
    for (int32_t p = 0; p < csr.nnz; ++p) seg_off[(size_t)(csr.col[p] / segw) + 1]++;
    for (int s = 0; s < S; ++s) seg_off[s + 1] += seg_off[s];
    ent.resize((size_t)csr.nnz);
    std::vector<int64_t> cur(seg_off.begin(), seg_off.end() - 1);
    for (int32_t r = 0; r < csr.M; ++r) {
        for (int32_t p = csr.row_ptr[r]; p < csr.row_ptr[r + 1]; ++p) {
            const int32_t c = csr.col[p];
            const int32_t sid = c / segw;
            ent[(size_t)cur[sid]++] = SegEntry{r, c % segw, csr.val[p]};
        }
    }
}

// Splits a segment's entries into per-row runs and orders each run by local
// column with std::sort (the reference sorts a vector<Entry{lcol,v}> with the
// comparator lcol-less; comparing the same lcol values gives the same order).
void make_runs(SegEntry* e, int32_t n, std::vector<Run>& runs) {
    runs.clear();
    int32_t i = 0;
    while (i < n) {
        int32_t j = i + 1;
        while (j < n && e[j].row == e[i].row) ++j;
        runs.push_back(Run{e[i].row, i, j - i});
        if (j - i > 1)
            std::sort(e + i, e + j,
                      [](const SegEntry& a, const SegEntry& b) { return a.lcol < b.lcol; });
        i = j;
    }
}

// Appends one group (rows of `lane_run`, -1 for missing lanes) to `out`.
// lane_row[l] is the row id of lane l (or -1), lane_run[l] the run index
// holding that row's entries (or -1 for a row with no entries here).
void emit_group(BlockOut& out, int bundle, int depth, const int32_t* lane_row,
                const int32_t* lane_run, const std::vector<Run>& runs, const SegEntry* e) {
    out.depth.push_back(depth);
    for (int l = 0; l < bundle; ++l) out.rows.push_back(lane_row[l]);
    for (int d = 0; d < depth; ++d) {
        for (int l = 0; l < bundle; ++l) {
            const int32_t ri = lane_run[l];
            if (ri >= 0 && d < runs[ri].len) {
                const SegEntry& x = e[runs[ri].begin + d];
                out.lcol.push_back(x.lcol);
                out.val.push_back(x.v);
            } else {
                out.lcol.push_back(-1);
                out.val.push_back(0.f);
            }
        }
    }
}

// Layout S / TC groups of one segment.
void build_segment_S(SegEntry* e, int32_t n, int bundle, BlockOut& out,
                     std::vector<Run>& runs, std::vector<int32_t>& order,
                     std::vector<int32_t>& lane_row, std::vector<int32_t>& lane_run) {
    make_runs(e, n, runs);
    // Same insertion sequence as seg_entries[sid][r] over ascending r.
    std::unordered_map<int32_t, int32_t> m;
    for (int32_t i = 0; i < (int32_t)runs.size(); ++i) m[runs[i].row] = i;
    order.clear();
    for (const auto& kv : m) order.push_back(kv.second);
    // vcsr_seg.cu:63-65: entry count descending.
    std::sort(order.begin(), order.end(),
              [&runs](int32_t a, int32_t b) { return runs[a].len > runs[b].len; });
    const int32_t nact = (int32_t)order.size();
    int32_t ngroups = 0;
    for (int32_t start = 0; start < nact; start += bundle) {
        const int32_t end = std::min(start + bundle, nact);
        int depth = 0;
        for (int32_t i = start; i < end; ++i) depth = std::max(depth, runs[order[i]].len);
        if (depth == 0) continue;
        for (int l = 0; l < bundle; ++l) {
            const int32_t ridx = start + l;
            if (ridx < nact) {
                lane_run[l] = order[ridx];
                lane_row[l] = runs[order[ridx]].row;
            } else {
                lane_run[l] = -1;
                lane_row[l] = -1;
            }
        }
        emit_group(out, bundle, depth, lane_row.data(), lane_run.data(), runs, e);
        ++ngroups;
    }
    out.groups_per_seg.push_back(ngroups);
}

// Per-thread scratch of layout H (arrays of length M).
struct HScratch {
    std::vector<int32_t> cnt, run_of_row, rows;
};

// Layout H groups of one segment.
void build_segment_H(SegEntry* e, int32_t n, int32_t M, int bundle, BlockOut& out,
                     std::vector<Run>& runs, HScratch& hs, std::vector<int32_t>& lane_row,
                     std::vector<int32_t>& lane_run) {
    make_runs(e, n, runs);
    for (int32_t i = 0; i < (int32_t)runs.size(); ++i) {
        hs.cnt[runs[i].row] = runs[i].len;
        hs.run_of_row[runs[i].row] = i;
    }
    // vcsr.hpp:56-59: all rows 0..M-1, entry count descending.
    std::iota(hs.rows.begin(), hs.rows.end(), 0);
    const int32_t* cnt = hs.cnt.data();
    std::sort(hs.rows.begin(), hs.rows.end(),
              [cnt](int32_t a, int32_t b) { return cnt[a] > cnt[b]; });
    int32_t ngroups = 0;
    for (int64_t start = 0; start < M; start += bundle) {
        const int64_t end = std::min<int64_t>(start + bundle, M);
        int depth = 0;
        for (int64_t i = start; i < end; ++i) depth = std::max(depth, cnt[hs.rows[i]]);
        if (depth == 0) continue;
        for (int l = 0; l < bundle; ++l) {
            const int64_t ridx = start + l;
            if (ridx < M) {
                const int32_t row = hs.rows[ridx];
                lane_row[l] = row;
                lane_run[l] = cnt[row] > 0 ? hs.run_of_row[row] : -1;
            } else {
                lane_row[l] = -1;
                lane_run[l] = -1;
            }
        }
        emit_group(out, bundle, depth, lane_row.data(), lane_run.data(), runs, e);
        ++ngroups;
    }
    out.groups_per_seg.push_back(ngroups);
    for (const Run& r : runs) hs.cnt[r.row] = 0;
}

}  // namespace

Vcsr build_vcsr(const Csr& csr, int segw, int bundle, int layout, int nthreads) {
    validate_csr(csr);
    if (layout != kLayoutH && layout != kLayoutS && layout != kLayoutTC)
        throw Error(1, "unknown layout " + std::to_string(layout));
    if (layout == kLayoutTC) {  // src/vcsr_tc.cu:27-28
        segw = 16;
        bundle = 16;
    }
    if (segw <= 0) throw Error(1, "segw must be > 0");
    if (bundle <= 0) throw Error(1, "bundle must be > 0");
    if (nthreads <= 0) nthreads = default_threads();

    Vcsr V;
    V.M = csr.M;
    V.N = csr.N;
    V.segw = segw;
    V.bundle = bundle;
    V.layout = layout;
    const int64_t S64 = ((int64_t)csr.N + segw - 1) / segw;
    if (S64 > INT32_MAX) throw Error(5, "too many segments");
    const int32_t S = (int32_t)S64;
    V.num_segments = S;

    std::vector<int64_t> seg_off;
    std::vector<SegEntry> ent;
    bucket_by_segment(csr, segw, S, seg_off, ent);

    // Segments per task: layout H does O(M log M) work per segment.
    const int64_t grain = (layout == kLayoutH) ? 8 : 2048;
    const int64_t nblocks = (S + grain - 1) / grain;
    std::vector<BlockOut> blocks((size_t)nblocks);
    parallel_for(nblocks, 1, nthreads, [&](int64_t bb, int64_t be) {
        std::vector<Run> runs;
        std::vector<int32_t> order, lane_row(bundle), lane_run(bundle);
        HScratch hs;
        if (layout == kLayoutH) {
            hs.cnt.assign((size_t)csr.M, 0);
            hs.run_of_row.assign((size_t)csr.M, -1);
            hs.rows.resize((size_t)csr.M);
        }
        for (int64_t b = bb; b < be; ++b) {
            BlockOut& out = blocks[(size_t)b];
            const int64_t s0 = b * grain, s1 = std::min<int64_t>(S, s0 + grain);
            for (int64_t sid = s0; sid < s1; ++sid) {
                SegEntry* e = ent.data() + seg_off[sid];
                const int32_t n = (int32_t)(seg_off[sid + 1] - seg_off[sid]);
                if (layout == kLayoutH)
                    build_segment_H(e, n, csr.M, bundle, out, runs, hs, lane_row, lane_run);
                else
                    build_segment_S(e, n, bundle, out, runs, order, lane_row, lane_run);
            }
        }
    });

    // Concatenate in segment order.
    int64_t G = 0, P = 0;
    for (const BlockOut& b : blocks) {
        G += (int64_t)b.depth.size();
        P += (int64_t)b.lcol.size();
    }
    if (P > INT32_MAX) throw Error(5, "packed slot count exceeds int32");
    if (G * (int64_t)bundle > INT32_MAX) throw Error(5, "groups*bundle exceeds int32");
    V.group_ptr.reserve((size_t)G + 1);
    V.group_depth.reserve((size_t)G);
    V.group_seg_base.reserve((size_t)G);
    V.group_rows.reserve((size_t)(G * bundle));
    V.lcol.reserve((size_t)P);
    V.val.reserve((size_t)P);
    V.segment_group_start.reserve((size_t)S + 1);
    V.segment_group_start.push_back(0);
    int64_t slot = 0;
    for (int64_t b = 0; b < nblocks; ++b) {
        const BlockOut& out = blocks[(size_t)b];
        size_t gi = 0;
        for (size_t k = 0; k < out.groups_per_seg.size(); ++k) {
            const int32_t sid = (int32_t)(b * grain + (int64_t)k);
            for (int32_t q = 0; q < out.groups_per_seg[k]; ++q, ++gi) {
                V.group_ptr.push_back((int32_t)slot);
                V.group_depth.push_back(out.depth[gi]);
                V.group_seg_base.push_back(sid * segw);
                slot += (int64_t)out.depth[gi] * bundle;
            }
            V.segment_group_start.push_back((int32_t)V.group_depth.size());
        }
        V.group_rows.insert(V.group_rows.end(), out.rows.begin(), out.rows.end());
        V.lcol.insert(V.lcol.end(), out.lcol.begin(), out.lcol.end());
        V.val.insert(V.val.end(), out.val.begin(), out.val.end());
        blocks[(size_t)b] = BlockOut();  // release as we go
    }
    V.group_ptr.push_back((int32_t)slot);
    return V;
}

}  // namespace vcsr
