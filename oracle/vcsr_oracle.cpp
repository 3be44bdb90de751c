// vcsr_oracle.cpp - CPU restatement of the reference algorithms, used ONLY as
// test infrastructure: by tests/, by __graft_entry__.smoke() and by the
// cpu_baseline leg of bench.py, always as the checker, never as the thing
// measured or shipped.  The product (vcsr-spmm_amd/) never links or calls it.
//
// Each function restates one reference function step by step, in plain
// sequential C++ with the same standard containers where the result depends
// on them (std::sort on equal keys, std::unordered_map iteration order):
//   orc_read_mtx         include/mmio.hpp:22-46
//   orc_coo_to_csr       include/csr.hpp:16-37
//   orc_build_h          include/vcsr.hpp:25-109      (layout H)
//   orc_build_s          src/vcsr_seg.cu:24-113       (layout S; = vcsr_opt.cu:23-101)
//   orc_build_tc         src/vcsr_tc.cu:26-106        (layout S with segw=16, bundle=16)
//   orc_build_cst        src/fastspmm.cu:129-251      (FastSpMM condensed tiles)
//   orc_spmm_f32         src/kernels.cu:25-32 loop order (row; p ascending; k inner; FMA)
//   orc_spmm_f64         same sum in double (checker only)
//   orc_spmm_f{32,64}_mt the same two over row ranges on several threads
//                        (rows are independent: bit-identical results)
//   orc_vcsr_apply       src/vcsr_seg.cu:173-188 semantics (C += per-group partial
//                        sums) evaluated in double, to check that a format
//                        represents A
// How each is pinned (golden vectors, compiled reference, closed forms) is
// listed in tests/ (test_oracle_*.py).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <numeric>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

struct Coo {
    int M = 0, N = 0;
    std::vector<int> rows, cols;
    std::vector<float> vals;
};
struct Csr {
    int M = 0, N = 0, nnz = 0;
    std::vector<int> row_ptr, col;
    std::vector<float> val;
};
struct Fmt {
    int M = 0, N = 0, segw = 0, bundle = 0;
    std::vector<int> group_ptr, group_depth, group_seg_base, group_rows, lcol;
    std::vector<float> val;
    std::vector<int> segment_group_start;
};

// mmio.hpp:22-46: skip empty and '%' lines; "M N nnz"; nnz triples read with
// operator>> across lines; 1-based unless the first entry has a 0 index.
Coo read_mtx(const std::string& path) {
    std::ifstream in(path);
    if (!in) throw std::runtime_error("open");
    std::string line;
    while (std::getline(in, line)) {
        if (line.empty() || line[0] == '%') continue;
        std::istringstream iss(line);
        int M, N, nnz;
        if (!(iss >> M >> N >> nnz)) throw std::runtime_error("header");
        Coo coo;
        coo.M = M;
        coo.N = N;
        bool one_based = true;
        for (int i = 0; i < nnz; ++i) {
            int r, c;
            double v;
            if (!(in >> r >> c >> v)) throw std::runtime_error("data");
            if (i == 0 && (r == 0 || c == 0)) one_based = false;
            coo.rows.push_back(r - (one_based ? 1 : 0));
            coo.cols.push_back(c - (one_based ? 1 : 0));
            coo.vals.push_back((float)v);
        }
        return coo;
    }
    throw std::runtime_error("empty");
}

// csr.hpp:16-37.
Csr coo_to_csr(const Coo& coo) {
    Csr csr;
    csr.M = coo.M;
    csr.N = coo.N;
    csr.nnz = (int)coo.vals.size();
    csr.row_ptr.assign(csr.M + 1, 0);
    csr.col.resize(csr.nnz);
    csr.val.resize(csr.nnz);
    for (int r : coo.rows) {
        if (r < 0 || r >= csr.M) throw std::runtime_error("row range");
        csr.row_ptr[r + 1]++;
    }
    for (int i = 1; i <= csr.M; ++i) csr.row_ptr[i] += csr.row_ptr[i - 1];
    std::vector<int> ctr = csr.row_ptr;
    for (size_t i = 0; i < coo.vals.size(); ++i) {
        int dst = ctr[coo.rows[i]]++;
        csr.col[dst] = coo.cols[i];
        csr.val[dst] = coo.vals[i];
    }
    for (int r = 0; r < csr.M; ++r) {
        const int s = csr.row_ptr[r], e = csr.row_ptr[r + 1];
        std::vector<int> order(e - s);
        std::iota(order.begin(), order.end(), 0);
        std::sort(order.begin(), order.end(),
                  [&](int a, int b) { return csr.col[s + a] < csr.col[s + b]; });
        std::vector<int> c2(e - s);
        std::vector<float> v2(e - s);
        for (int i = 0; i < e - s; ++i) {
            c2[i] = csr.col[s + order[i]];
            v2[i] = csr.val[s + order[i]];
        }
        std::copy(c2.begin(), c2.end(), csr.col.begin() + s);
        std::copy(v2.begin(), v2.end(), csr.val.begin() + s);
    }
    return csr;
}

struct Ent {
    int lc;
    float v;
};

// Appends one bundle [start, end) of `order` (row ids; lanes past `order`
// are padding) to the format; `entries(row)` gives the row's sorted entries.
template <class Get>
void emit(Fmt& F, const std::vector<int>& order, size_t start, int depth, int sid, Get entries,
          bool tail_rows_are_ids) {
    F.group_ptr.push_back((int)F.val.size());
    F.group_depth.push_back(depth);
    F.group_seg_base.push_back(sid * F.segw);
    for (int lane = 0; lane < F.bundle; ++lane) {
        const size_t ridx = start + lane;
        F.group_rows.push_back(ridx < order.size() ? order[ridx] : -1);
    }
    (void)tail_rows_are_ids;
    for (int d = 0; d < depth; ++d) {
        for (int lane = 0; lane < F.bundle; ++lane) {
            const size_t ridx = start + lane;
            if (ridx >= order.size()) {
                F.lcol.push_back(-1);
                F.val.push_back(0.f);
                continue;
            }
            const std::vector<Ent>& e = entries(order[ridx]);
            if (d < (int)e.size()) {
                F.lcol.push_back(e[d].lc);
                F.val.push_back(e[d].v);
            } else {
                F.lcol.push_back(-1);
                F.val.push_back(0.f);
            }
        }
    }
}

// vcsr.hpp:25-109 (layout H): per (segment, row) entry lists over all S*M
// pairs; rows 0..M-1 sorted by count descending per segment; empty bundles
// skipped; lanes past M get row -1, other lanes keep their (maybe empty) row.
Fmt build_h(const Csr& csr, int segw, int bundle) {
    if (bundle <= 0 || segw <= 0) throw std::runtime_error("params");
    Fmt F;
    F.M = csr.M;
    F.N = csr.N;
    F.segw = segw;
    F.bundle = bundle;
    const int S = (csr.N + segw - 1) / segw;
    std::vector<std::vector<Ent>> cell((size_t)S * csr.M);
    for (int r = 0; r < csr.M; ++r)
        for (int p = csr.row_ptr[r]; p < csr.row_ptr[r + 1]; ++p)
            cell[(size_t)(csr.col[p] / segw) * csr.M + r].push_back({csr.col[p] % segw, csr.val[p]});
    for (auto& v : cell)
        std::sort(v.begin(), v.end(), [](const Ent& a, const Ent& b) { return a.lc < b.lc; });
    F.segment_group_start.push_back(0);
    for (int sid = 0; sid < S; ++sid) {
        auto entries = [&](int row) -> const std::vector<Ent>& {
            return cell[(size_t)sid * csr.M + row];
        };
        std::vector<int> rows(csr.M);
        std::iota(rows.begin(), rows.end(), 0);
        std::sort(rows.begin(), rows.end(),
                  [&](int a, int b) { return entries(a).size() > entries(b).size(); });
        for (size_t start = 0; start < rows.size(); start += bundle) {
            const size_t end = std::min(start + (size_t)bundle, rows.size());
            int depth = 0;
            for (size_t i = start; i < end; ++i) depth = std::max(depth, (int)entries(rows[i]).size());
            if (depth == 0) continue;
            emit(F, rows, start, depth, sid, entries, true);
        }
        F.segment_group_start.push_back((int)F.group_depth.size());
    }
    F.group_ptr.push_back((int)F.val.size());
    return F;
}

// vcsr_seg.cu:24-113 (layout S): per segment an unordered_map row -> entries
// filled in ascending row order; active rows taken in map iteration order,
// then sorted by count descending; lanes past the active rows get row -1.
Fmt build_s(const Csr& csr, int segw, int bundle) {
    if (bundle <= 0 || segw <= 0) throw std::runtime_error("params");
    Fmt F;
    F.M = csr.M;
    F.N = csr.N;
    F.segw = segw;
    F.bundle = bundle;
    const int S = (csr.N + segw - 1) / segw;
    std::vector<std::unordered_map<int, std::vector<Ent>>> seg(S);
    for (int r = 0; r < csr.M; ++r)
        for (int p = csr.row_ptr[r]; p < csr.row_ptr[r + 1]; ++p)
            seg[csr.col[p] / segw][r].push_back({csr.col[p] % segw, csr.val[p]});
    for (auto& m : seg)
        for (auto& kv : m)
            std::sort(kv.second.begin(), kv.second.end(),
                      [](const Ent& a, const Ent& b) { return a.lc < b.lc; });
    F.segment_group_start.push_back(0);
    for (int sid = 0; sid < S; ++sid) {
        std::vector<int> act;
        for (auto& kv : seg[sid])
            if (!kv.second.empty()) act.push_back(kv.first);
        std::sort(act.begin(), act.end(),
                  [&](int a, int b) { return seg[sid][a].size() > seg[sid][b].size(); });
        auto entries = [&](int row) -> const std::vector<Ent>& { return seg[sid][row]; };
        for (size_t start = 0; start < act.size(); start += bundle) {
            const size_t end = std::min(start + (size_t)bundle, act.size());
            int depth = 0;
            for (size_t i = start; i < end; ++i) depth = std::max(depth, (int)entries(act[i]).size());
            if (depth == 0) continue;
            emit(F, act, start, depth, sid, entries, false);
        }
        F.segment_group_start.push_back((int)F.group_depth.size());
    }
    F.group_ptr.push_back((int)F.val.size());
    return F;
}

// FastSpMM's condensed sparse tiles (src/fastspmm.cu:129-251; its header
// fastspmm.hpp is missing, and the window and block widths are 16 because
// the kernel's WMMA tiles are 16 x 16, fastspmm.cu:44-48,103).
struct Cst {
    int M = 0, N = 0, num_windows = 0, num_tcb = 0;
    std::vector<int> window_off;    // rowWindowOffset: first TCB of each window, + end
    std::vector<int> tcb_col_off;   // tcbColOffset: first entry of each TCB, + end
    std::vector<int> tcb_row_off;   // tcbRowOffset: 17 per TCB (uint16_t there, see below)
    std::vector<uint8_t> col_idx;   // tcbColIndex: column inside the TCB, 0..15
    std::vector<float> value;       // tcbValue (__half there, see below)
    std::vector<int> tcb2b;         // tcb2B: 16 per TCB, B row or -1
};

// Per window of 16 rows: the distinct columns of its rows in increasing
// order (:160-167; a window without any adds no TCB, :169-171); column i of
// that list belongs to TCB i / 16 at position i % 16 (:174-180, :194-196);
// each TCB lists, row by row, the row's nonzeros whose column it holds, in
// CSR order (:188-201, :215-224), with the running entry count before each
// row and after the last (:216, :225, :228), and its 16 columns (-1 past the
// window's last, :231-235).  The row offsets are absolute entry numbers; the
// reference stores them as uint16_t (:216, :225), which wraps once a matrix
// has more than 65535 entries, while its kernel subtracts the TCB's 32-bit
// first entry from them (fastspmm.cu:61-71): this restatement keeps them in
// int.  Values stay float: the reference rounds them to half (:221), its
// arithmetic precision, not part of the layout.
Cst build_cst(const Csr& csr) {
    constexpr int kWin = 16, kTcbW = 16;
    Cst s;
    s.M = csr.M;
    s.N = csr.N;
    s.num_windows = (csr.M + kWin - 1) / kWin;
    s.window_off.push_back(0);
    s.tcb_col_off.push_back(0);
    for (int w = 0; w < s.num_windows; ++w) {
        const int r0 = w * kWin, r1 = std::min(csr.M, r0 + kWin);
        std::vector<int> cols(csr.col.begin() + csr.row_ptr[r0], csr.col.begin() + csr.row_ptr[r1]);
        std::sort(cols.begin(), cols.end());
        cols.erase(std::unique(cols.begin(), cols.end()), cols.end());
        const int ntcb = ((int)cols.size() + kTcbW - 1) / kTcbW;
        for (int t = 0; t < ntcb; ++t) {
            for (int lr = 0; lr < kWin; ++lr) {
                s.tcb_row_off.push_back((int)s.col_idx.size());
                if (r0 + lr >= r1) continue;
                for (int p = csr.row_ptr[r0 + lr]; p < csr.row_ptr[r0 + lr + 1]; ++p) {
                    const int i = (int)(std::lower_bound(cols.begin(), cols.end(), csr.col[p]) -
                                        cols.begin());
                    if (i / kTcbW != t) continue;
                    s.col_idx.push_back((uint8_t)(i % kTcbW));
                    s.value.push_back(csr.val[p]);
                }
            }
            s.tcb_row_off.push_back((int)s.col_idx.size());
            s.tcb_col_off.push_back((int)s.col_idx.size());
            for (int j = 0; j < kTcbW; ++j) {
                const int i = t * kTcbW + j;
                s.tcb2b.push_back(i < (int)cols.size() ? cols[(size_t)i] : -1);
            }
        }
        s.num_tcb += ntcb;
        s.window_off.push_back(s.num_tcb);
    }
    return s;
}

thread_local std::string g_err;

template <class T>
T* dup(const std::vector<T>& v) {
    T* p = (T*)std::malloc(std::max<size_t>(1, v.size() * sizeof(T)));
    if (!v.empty()) std::memcpy(p, v.data(), v.size() * sizeof(T));
    return p;
}

}  // namespace

extern "C" {

// Arrays are malloc'ed; release with orc_free.
typedef struct {
    int M, N, segw, bundle, num_groups, num_segments;
    long long num_slots;
    int *group_ptr, *group_depth, *group_seg_base, *group_rows, *lcol;
    float* val;
    int* segment_group_start;
} orc_fmt;

typedef struct {
    int M, N, nnz;
    int *row_ptr, *col;
    float* val;
} orc_csr;

typedef struct {
    int M, N;
    long long nnz;
    int *rows, *cols;
    float* vals;
} orc_coo;

const char* orc_last_error(void) { return g_err.c_str(); }
void orc_free(void* p) { std::free(p); }

int orc_read_mtx(const char* path, orc_coo* out) {
    try {
        Coo c = read_mtx(path);
        out->M = c.M;
        out->N = c.N;
        out->nnz = (long long)c.vals.size();
        out->rows = dup(c.rows);
        out->cols = dup(c.cols);
        out->vals = dup(c.vals);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

int orc_coo_to_csr(int M, int N, long long nnz, const int* rows, const int* cols,
                   const float* vals, orc_csr* out) {
    try {
        Coo c;
        c.M = M;
        c.N = N;
        c.rows.assign(rows, rows + nnz);
        c.cols.assign(cols, cols + nnz);
        c.vals.assign(vals, vals + nnz);
        Csr s = coo_to_csr(c);
        out->M = s.M;
        out->N = s.N;
        out->nnz = s.nnz;
        out->row_ptr = dup(s.row_ptr);
        out->col = dup(s.col);
        out->val = dup(s.val);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

// layout: 0 = H, 1 = S, 2 = TC.
int orc_build(int M, int N, const int* row_ptr, const int* col, const float* val, int segw,
              int bundle, int layout, orc_fmt* out) {
    try {
        Csr c;
        c.M = M;
        c.N = N;
        c.nnz = row_ptr[M];
        c.row_ptr.assign(row_ptr, row_ptr + M + 1);
        c.col.assign(col, col + c.nnz);
        c.val.assign(val, val + c.nnz);
        Fmt F;
        if (layout == 0) F = build_h(c, segw, bundle);
        else if (layout == 1) F = build_s(c, segw, bundle);
        else F = build_s(c, 16, 16);  // vcsr_tc.cu:27-28 forces both
        out->M = F.M;
        out->N = F.N;
        out->segw = F.segw;
        out->bundle = F.bundle;
        out->num_groups = (int)F.group_depth.size();
        out->num_segments = (int)F.segment_group_start.size() - 1;
        out->num_slots = (long long)F.lcol.size();
        out->group_ptr = dup(F.group_ptr);
        out->group_depth = dup(F.group_depth);
        out->group_seg_base = dup(F.group_seg_base);
        out->group_rows = dup(F.group_rows);
        out->lcol = dup(F.lcol);
        out->val = dup(F.val);
        out->segment_group_start = dup(F.segment_group_start);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

typedef struct {
    int M, N, num_windows, num_tcb, num_entries;
    int *window_off, *tcb_col_off, *tcb_row_off;
    unsigned char* col_idx;
    float* value;
    int* tcb2b;
} orc_cst;

int orc_build_cst(int M, int N, const int* row_ptr, const int* col, const float* val,
                  orc_cst* out) {
    try {
        Csr c;
        c.M = M;
        c.N = N;
        c.nnz = row_ptr[M];
        c.row_ptr.assign(row_ptr, row_ptr + M + 1);
        c.col.assign(col, col + c.nnz);
        c.val.assign(val, val + c.nnz);
        Cst s = build_cst(c);
        out->M = s.M;
        out->N = s.N;
        out->num_windows = s.num_windows;
        out->num_tcb = s.num_tcb;
        out->num_entries = (int)s.col_idx.size();
        out->window_off = dup(s.window_off);
        out->tcb_col_off = dup(s.tcb_col_off);
        out->tcb_row_off = dup(s.tcb_row_off);
        out->col_idx = dup(s.col_idx);
        out->value = dup(s.value);
        out->tcb2b = dup(s.tcb2b);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

// kernels.cu:25-32: C[r,:] = 0; for p in row r: for k: C[r,k] += val[p]*B[col[p],k]
// (contracted to one FMA per term, as nvcc emits it).
void orc_spmm_f32(int M, const int* row_ptr, const int* col, const float* val, const float* B,
                  int O, float* C) {
    for (int r = 0; r < M; ++r) {
        float* c = C + (size_t)r * O;
        for (int k = 0; k < O; ++k) c[k] = 0.f;
        for (int p = row_ptr[r]; p < row_ptr[r + 1]; ++p) {
            const float a = val[p];
            const float* b = B + (size_t)col[p] * O;
            for (int k = 0; k < O; ++k) c[k] = std::fmaf(a, b[k], c[k]);
        }
    }
}

// The same sum accumulated in double (for error bounds).
void orc_spmm_f64(int M, const int* row_ptr, const int* col, const float* val, const float* B,
                  int O, double* C) {
    for (int r = 0; r < M; ++r) {
        double* c = C + (size_t)r * O;
        for (int k = 0; k < O; ++k) c[k] = 0.0;
        for (int p = row_ptr[r]; p < row_ptr[r + 1]; ++p) {
            const double a = val[p];
            const float* b = B + (size_t)col[p] * O;
            for (int k = 0; k < O; ++k) c[k] += a * (double)b[k];
        }
    }
}

// The two sums above over contiguous row ranges on `nthreads` threads (<= 0:
// every hardware thread).  Rows are independent, so each row's result is the
// single-thread one bit for bit; only the wall time changes (the all-cores
// CPU baseline, and whole-C checks of large products).
extern "C++" {
template <class T, class F>
static void rows_in_parallel(int M, const int* row_ptr, int O, T* C, int nthreads, F one) {
    int nt = nthreads > 0 ? nthreads : (int)std::thread::hardware_concurrency();
    nt = std::max(1, std::min(nt, std::max(M, 1)));
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t) {
        const int r0 = (int)((int64_t)M * t / nt), r1 = (int)((int64_t)M * (t + 1) / nt);
        th.emplace_back([=] { one(r1 - r0, row_ptr + r0, C + (size_t)r0 * O); });
    }
    for (auto& x : th) x.join();
}
}  // extern "C++"

void orc_spmm_f32_mt(int M, const int* row_ptr, const int* col, const float* val, const float* B,
                     int O, float* C, int nthreads) {
    rows_in_parallel(M, row_ptr, O, C, nthreads, [=](int m, const int* rp, float* c) {
        orc_spmm_f32(m, rp, col, val, B, O, c);
    });
}

void orc_spmm_f64_mt(int M, const int* row_ptr, const int* col, const float* val, const float* B,
                     int O, double* C, int nthreads) {
    rows_in_parallel(M, row_ptr, O, C, nthreads, [=](int m, const int* rp, double* c) {
        orc_spmm_f64(m, rp, col, val, B, O, c);
    });
}

// C += A_fmt * B in double, walking the packed format the way the reference
// VCSR kernels do (vcsr_seg.cu:173-188): per group, per lane with a row, sum
// val * B[seg_base + lcol, :] over the depth slots with lcol >= 0.
void orc_vcsr_apply(int M, int N, int segw, int bundle, int G, const int* group_ptr,
                    const int* group_depth, const int* group_seg_base, const int* group_rows,
                    const int* lcol, const float* val, const float* B, int O, double* C) {
    (void)M;
    (void)segw;
    std::vector<double> acc(O);
    for (int g = 0; g < G; ++g) {
        for (int lane = 0; lane < bundle; ++lane) {
            const int row = group_rows[(size_t)g * bundle + lane];
            if (row < 0) continue;
            std::fill(acc.begin(), acc.end(), 0.0);
            for (int d = 0; d < group_depth[g]; ++d) {
                const size_t idx = (size_t)group_ptr[g] + (size_t)d * bundle + lane;
                const int lc = lcol[idx];
                if (lc < 0) continue;
                const int brow = group_seg_base[g] + lc;
                if (brow >= N) continue;
                for (int k = 0; k < O; ++k) acc[k] += (double)val[idx] * (double)B[(size_t)brow * O + k];
            }
            for (int k = 0; k < O; ++k) C[(size_t)row * O + k] += acc[k];
        }
    }
}

}  // extern "C"
