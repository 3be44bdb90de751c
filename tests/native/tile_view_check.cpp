// tile_view_check.cpp - CPU checks of the row-tile view (host/tile_view.cpp)
// that the tile-stationary kernel walks.  Built and run by
// tests/test_tile_view.py against the library's host objects.
//
// For every matrix and tile height the view must
//  * hold exactly the CSR nonzeros: each (tile row, entry) slot that is not
//    -1 names a VCSR slot whose value and column (entry's B row) are one
//    nonzero of that row, and the multiset of those equals the CSR's;
//  * cover every row once: by a piece writing C, or as a split-tile row;
//  * chain its work items and pieces contiguously within the LDS limits the
//    kernel is compiled for (entries per item, pieces per item, rows per
//    piece);
//  * keep each tile's entries sorted by column (the B rows are walked in
//    the order of the row's nonzeros);
//  * for single-row views, put long rows' pieces in the run of work items
//    (one per XCD) whose eighth of B holds their columns.
// With fixed 16-row windows (the FastSpMM layout) the view must also be the
// oracle's restatement of FastSpMM's condensed sparse tiles
// (oracle/vcsr_oracle.cpp orc_build_cst, src/fastspmm.cu:129-251), linked in
// from the oracle's source: see check_cst.
// Exit status 0 and "ALL OK" when every case passes.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <cstdio>
#include <tuple>
#include <vector>

#include "../../vcsr-spmm_amd/csrc/host/core.hpp"
#include "../../vcsr-spmm_amd/csrc/host/tile_view.hpp"

using namespace vcsr;

// The oracle's C interface for the condensed tiles (oracle/vcsr_oracle.cpp).
extern "C" {
typedef struct {
    int M, N, num_windows, num_tcb, num_entries;
    int *window_off, *tcb_col_off, *tcb_row_off;
    unsigned char* col_idx;
    float* value;
    int* tcb2b;
} orc_cst;
int orc_build_cst(int M, int N, const int* row_ptr, const int* col, const float* val,
                  orc_cst* out);
void orc_free(void* p);
}

static int fail(const char* what, int M, int R) {
    std::printf("FAIL %s (M=%d R=%d)\n", what, M, R);
    return 1;
}

static bool same_bits(float a, float b) { return std::memcmp(&a, &b, sizeof a) == 0; }

// The fixed-window view at tile height 16 against FastSpMM's condensed
// sparse tiles.  Window w (rows 16w ..) is tile w of the view.  Where no row
// of the window holds a column twice:
//  * its entries are the window's TCBs, 16 per TCB: entry 16t + j reads the
//    B row tcb2B[16t + j], and TCB padding (-1) is a placeholder entry;
//  * row r of the window has a value in entry 16t + j exactly where TCB t
//    lists local column j for local row r, with the same value.
// A window without nonzeros has no TCB and one group of 16 placeholder
// entries in the view (a 16-row tile always has a whole entry group).  A row
// that holds a column twice has both entries in one TCB cell (the reference
// kernel keeps one of them, fastspmm.cu:74-79) and two entries in the view;
// there the view's (row, B row, value) multiset must equal the CST's, and
// its distinct B rows the window's column list.
static int check_cst(const Csr& csr, int segw, int bundle, int layout) {
    const int M = csr.M;
    const Vcsr v = build_vcsr(csr, segw, bundle, layout, 2);
    const TileView tv = make_tile_view(v, kTileMmaRows, 2, true);
    orc_cst c{};
    if (orc_build_cst(M, csr.N, csr.row_ptr.data(), csr.col.data(), csr.val.data(), &c) != 0)
        return fail("oracle build_cst", M, 16);
    int bad = 0;
    const int W = c.num_windows, np = (int)tv.pieces.size() / 4;
    const int64_t E = tv.n_entries();
    if (tv.n_tiles != W) bad = fail("tile count differs from window count", M, 16);
    // First entry of each window's tile: its first piece.
    std::vector<int64_t> first(W + 1, -1);
    first[W] = E;
    for (int p = 0; p < np && !bad; ++p) {
        const int w = tv.pieces[4 * p] / 16;
        if (first[w] < 0) first[w] = tv.pieces[4 * p + 2];
    }
    int dup_windows = 0, empty_windows = 0;
    for (int w = 0; w < W && !bad; ++w) {
        const int r0 = 16 * w, nr = std::min(16, M - r0);
        const int t0 = c.window_off[w], nt = c.window_off[w + 1] - t0;
        const int64_t e0 = first[w], e1 = first[w + 1];
        if (e0 < 0 || e1 < e0) { bad = fail("window's tile not found", M, 16); break; }
        bool dup = false;
        for (int r = r0; r < r0 + nr; ++r)
            for (int p = csr.row_ptr[r] + 1; p < csr.row_ptr[r + 1]; ++p)
                for (int q = csr.row_ptr[r]; q < p; ++q) dup |= csr.col[q] == csr.col[p];
        if (nt == 0) {
            ++empty_windows;
            if (e1 - e0 != 16) { bad = fail("empty window not one placeholder group", M, 16); break; }
            for (int64_t e = e0; e < e1; ++e)
                if (tv.mask[e] != 0 || tv.brow[e] != 0) bad = fail("empty window holds a value", M, 16);
            continue;
        }
        if (!dup) {
            if (e1 - e0 != 16LL * nt) { bad = fail("entries differ from 16 per TCB", M, 16); break; }
            for (int t = 0; t < nt && !bad; ++t) {
                const int T = t0 + t;
                for (int j = 0; j < 16; ++j) {
                    const int64_t e = e0 + 16 * t + j;
                    const int col = c.tcb2b[16 * T + j];
                    if (col < 0 ? (tv.mask[e] != 0 || tv.brow[e] != 0)
                                : (tv.mask[e] == 0 || tv.brow[e] != col))
                        bad = fail("entry differs from tcb2B", M, 16);
                }
                for (int lr = 0; lr < 16 && !bad; ++lr) {
                    // (local column, value) of the TCB row, against the view's.
                    std::vector<std::pair<int, float>> a, b;
                    for (int i = c.tcb_row_off[17 * T + lr]; i < c.tcb_row_off[17 * T + lr + 1]; ++i)
                        a.emplace_back(c.col_idx[i], c.value[i]);
                    for (int j = 0; j < 16; ++j) {
                        const int64_t e = e0 + 16 * t + j;
                        if ((tv.mask[e] >> lr) & 1)
                            b.emplace_back(j, tv.val[(size_t)tile_val_index(16, e, lr)]);
                    }
                    std::sort(a.begin(), a.end(), [](auto& x, auto& y) { return x.first < y.first; });
                    bool eq = a.size() == b.size() && (lr < nr || a.empty());
                    for (size_t i = 0; eq && i < a.size(); ++i)
                        eq = a[i].first == b[i].first && same_bits(a[i].second, b[i].second);
                    if (!eq) bad = fail("TCB row differs from the view's", M, 16);
                }
            }
            continue;
        }
        ++dup_windows;
        std::vector<std::tuple<int, int, uint32_t>> a, b;
        std::vector<int> cols, brows;
        for (int t = t0; t < t0 + nt; ++t) {
            for (int j = 0; j < 16; ++j)
                if (c.tcb2b[16 * t + j] >= 0) cols.push_back(c.tcb2b[16 * t + j]);
            for (int lr = 0; lr < 16; ++lr)
                for (int i = c.tcb_row_off[17 * t + lr]; i < c.tcb_row_off[17 * t + lr + 1]; ++i) {
                    uint32_t bits;
                    std::memcpy(&bits, &c.value[i], 4);
                    a.emplace_back(r0 + lr, c.tcb2b[16 * t + c.col_idx[i]], bits);
                }
        }
        for (int64_t e = e0; e < e1; ++e) {
            if (tv.mask[e] == 0) continue;
            brows.push_back(tv.brow[e]);
            for (int lr = 0; lr < nr; ++lr)
                if ((tv.mask[e] >> lr) & 1) {
                    uint32_t bits;
                    const float x = tv.val[(size_t)tile_val_index(16, e, lr)];
                    std::memcpy(&bits, &x, 4);
                    b.emplace_back(r0 + lr, tv.brow[e], bits);
                }
        }
        std::sort(a.begin(), a.end());
        std::sort(b.begin(), b.end());
        brows.erase(std::unique(brows.begin(), brows.end()), brows.end());
        if (a != b) bad = fail("window nonzeros differ from the CST's", M, 16);
        if (brows != cols) bad = fail("window columns differ from the CST's", M, 16);
    }
    if (!bad)
        std::printf("cst ok M=%d nnz=%d windows=%d tcbs=%d empty=%d with-duplicates=%d entries=%lld\n",
                    M, csr.nnz, W, c.num_tcb, empty_windows, dup_windows, (long long)E);
    orc_free(c.window_off);
    orc_free(c.tcb_col_off);
    orc_free(c.tcb_row_off);
    orc_free(c.col_idx);
    orc_free(c.value);
    orc_free(c.tcb2b);
    return bad;
}

static int check(const Csr& csr, int segw, int bundle, int layout, int R_req, int expect_R,
                 bool fixed = false) {
    const Vcsr v = build_vcsr(csr, segw, bundle, layout, 2);
    const TileView tv = make_tile_view(v, R_req, 2, fixed);
    const int R = tv.R, RS = tile_slot_stride(R), M = csr.M;
    if (expect_R > 0 && R != expect_R) return fail("tile height", M, R);
    const int64_t E = tv.n_entries();
    if ((int64_t)tv.slot.size() != E * RS) return fail("slot array size", M, R);
    if ((int64_t)tv.val.size() != E * RS) return fail("value array size", M, R);
    if ((int64_t)tv.mask.size() != E) return fail("mask array size", M, R);
    const int nc = (int)tv.chunks.size() / 4, np = (int)tv.pieces.size() / 4;
    const int cap = tile_piece_entries(R);
    int64_t prev_e = 0;
    int prev_p = 0;
    for (int c = 0; c < nc; ++c) {
        const int e0 = tv.chunks[4 * c], e1 = tv.chunks[4 * c + 1];
        const int p0 = tv.chunks[4 * c + 2], p1 = tv.chunks[4 * c + 3];
        if (e0 != prev_e || p0 != prev_p) return fail("items not contiguous", M, R);
        if (e1 - e0 < 1 || e1 - e0 > cap) return fail("item entry count", M, R);
        if (p1 - p0 < 1 || p1 - p0 > kTileChunkPieces) return fail("item piece count", M, R);
        if (tv.pieces[4 * p0 + 2] != e0) return fail("item's first piece", M, R);
        if (R == kTileMmaRows) {
            // Matrix-core tiles: one piece per item, whole 16-entry groups.
            if (p1 - p0 != 1) return fail("16-row item with several pieces", M, R);
            if (e0 % kTileMmaGroup != 0 || (e1 - e0) % kTileMmaGroup != 0)
                return fail("16-row item not in whole entry groups", M, R);
        }
        for (int p = p0; p < p1; ++p) {
            const int pe = p + 1 < p1 ? tv.pieces[4 * (p + 1) + 2] : e1;
            if (pe - tv.pieces[4 * p + 2] < 1) return fail("empty piece", M, R);
            if (tv.pieces[4 * p + 1] < 1 || tv.pieces[4 * p + 1] > R) return fail("piece rows", M, R);
        }
        prev_e = e1;
        prev_p = p1;
    }
    if (prev_e != E || prev_p != np) return fail("items do not cover the view", M, R);

    std::vector<std::tuple<int, int, float>> want, got;
    for (int r = 0; r < M; ++r)
        for (int p = csr.row_ptr[r]; p < csr.row_ptr[r + 1]; ++p)
            want.emplace_back(r, csr.col[p], csr.val[p]);
    std::vector<int> covered((size_t)M, 0);
    for (int p = 0; p < np; ++p) {
        const int row0 = tv.pieces[4 * p], nr = tv.pieces[4 * p + 1], b = tv.pieces[4 * p + 2];
        const int e = p + 1 < np ? tv.pieces[4 * (p + 1) + 2] : (int)E;
        int last = -1;  // B row of the piece's previous entry with a value
        for (int q = b; q < e; ++q) {
            if (tv.mask[q] == 0) {
                if (tv.brow[q] != 0) return fail("placeholder entry reads a B row", M, R);
            } else {
                if (tv.brow[q] < last) return fail("entries not in column order", M, R);
                last = tv.brow[q];
            }
            for (int r = 0; r < RS; ++r) {
                // The kernel reads the values and presence bits; the slots
                // say where those values come from.
                const int s = tv.slot[(size_t)q * RS + r];
                const float a = tv.val[(size_t)tile_val_index(R, q, r)];
                const bool present = (tv.mask[q] >> r) & 1;
                if (present != (s >= 0)) return fail("presence bit differs from slot", M, R);
                if (s < 0) {
                    if (a != 0.f || std::signbit(a)) return fail("absent value not +0", M, R);
                    continue;
                }
                if (r >= nr) return fail("slot beyond the tile's rows", M, R);
                if (s >= (int)v.lcol.size() || v.lcol[s] < 0) return fail("slot is padding", M, R);
                if (std::memcmp(&a, &v.val[s], sizeof a) != 0) return fail("value differs from slot's", M, R);
                got.emplace_back(row0 + r, tv.brow[q], a);
            }
        }
        if (fixed && (row0 % R != 0 || nr != std::min(R, M - row0)))
            return fail("fixed window not aligned or not full", M, R);
        if (tv.pieces[4 * p + 3] < 0)
            for (int r = 0; r < nr; ++r) covered[(size_t)(row0 + r)]++;
    }
    for (size_t i = 0; i < tv.split.size() / 4; ++i) {
        covered[(size_t)tv.split[4 * i]]++;
        const int q = tv.split[4 * i + 1], stride = tv.split[4 * i + 2], n = tv.split[4 * i + 3];
        if (n < 2 || q < 0 || (int64_t)q + (int64_t)(n - 1) * stride >= tv.n_partial_rows)
            return fail("split row partials out of range", M, R);
        if (i > 0 && n > tv.split[4 * i - 1])
            return fail("split rows not in decreasing piece count", M, R);
    }
    for (int r = 0; r < M; ++r)
        if (covered[(size_t)r] != 1) return fail("row not covered exactly once", M, R);
    std::sort(want.begin(), want.end());
    std::sort(got.begin(), got.end());
    if (want != got) return fail("nonzeros differ from the CSR", M, R);
    std::printf("ok M=%d nnz=%d layout=%d R=%d entries=%lld items=%d pieces=%d split_rows=%zu\n", M,
                csr.nnz, layout, R, (long long)E, nc, np, tv.split.size() / 4);
    return 0;
}

// Block rows of height bh with `blocks` random bh x bw blocks each; an entry
// is kept with probability keep_pct %.  Duplicate columns in a row appear
// when dup is set.
static Csr block_matrix(uint64_t seed, int nbr, int bh, int N, int blocks, int bw, int keep_pct,
                        bool dup) {
    Coo c;
    c.M = nbr * bh;
    c.N = N;
    uint64_t x = seed * 0x9E3779B97F4A7C15ULL + 1;
    auto next = [&]() {
        x ^= x >> 12;
        x ^= x << 25;
        x ^= x >> 27;
        return x * 0x2545F4914F6CDD1DULL;
    };
    const int nbc = std::max(1, N / bw);
    for (int br = 0; br < nbr; ++br)
        for (int k = 0; k < blocks; ++k) {
            const int bc = (int)(next() % (uint64_t)nbc);
            for (int i = 0; i < bh; ++i)
                for (int j = 0; j < bw; ++j) {
                    if ((int)(next() % 100) >= keep_pct) continue;
                    const int col = bc * bw + j;
                    if (col >= N) continue;
                    c.rows.push_back(br * bh + i);
                    c.cols.push_back(col);
                    c.vals.push_back((float)((int)(next() % 2001) - 1000) / 512.f);
                    if (dup && next() % 13 == 0) {
                        c.rows.push_back(br * bh + i);
                        c.cols.push_back(col);
                        c.vals.push_back(0.75f);
                    }
                }
        }
    return coo_to_csr(c);
}

// Single-row views move the pieces of rows cut into 8 or more pieces into
// the eighth of the work-item list whose eighth of B holds their middle
// column (one run per XCD).  A banded matrix with a few long random rows:
// the view stays valid, and nearly every moved piece sits in its run.
static int check_long_piece_runs() {
    Coo c;
    c.M = 8192;
    c.N = 8192;
    uint64_t x = 12345;
    auto next = [&]() {
        x ^= x >> 12;
        x ^= x << 25;
        x ^= x >> 27;
        return x * 0x2545F4914F6CDD1DULL;
    };
    for (int r = 0; r < c.M; ++r) {
        const bool long_row = r % 200 == 7;
        const int k = long_row ? 2000 : 6;
        for (int i = 0; i < k; ++i) {
            const int col = long_row ? (int)(next() % (uint64_t)c.N)
                                     : std::min(c.N - 1, std::max(0, r - 60 + (int)(next() % 121)));
            c.rows.push_back(r);
            c.cols.push_back(col);
            c.vals.push_back((float)((int)(next() % 201) - 100) / 64.f);
        }
    }
    const Csr csr = coo_to_csr(c);
    int bad = check(csr, 4, 64, kLayoutS, 1, 1);
    const Vcsr v = build_vcsr(csr, 4, 64, kLayoutS, 2);
    const TileView tv = make_tile_view(v, 1, 2, false);
    std::vector<int> npc((size_t)csr.M, 0);
    for (size_t i = 0; i < tv.split.size() / 4; ++i) npc[(size_t)tv.split[4 * i]] = tv.split[4 * i + 3];
    const int nc = (int)tv.chunks.size() / 4;
    int moved = 0, in_run = 0;
    for (int ch = 0; ch < nc; ++ch) {
        const int e0 = tv.chunks[4 * ch], e1 = tv.chunks[4 * ch + 1], p0 = tv.chunks[4 * ch + 2];
        if (tv.chunks[4 * ch + 3] - p0 != 1 || tv.pieces[4 * p0 + 3] < 0) continue;
        if (npc[(size_t)tv.pieces[4 * p0]] < 8) continue;
        ++moved;
        const int run = (int)((int64_t)ch * 8 / nc);
        const int want = (int)std::min<int64_t>(7, (int64_t)tv.brow[(size_t)(e0 + (e1 - e0) / 2)] * 8 / csr.N);
        in_run += run == want;
    }
    if (moved == 0 || in_run * 10 < moved * 9) bad |= fail("long pieces not in their column's run", csr.M, 1);
    std::printf("long pieces: %d of %d in their column's run\n", in_run, moved);
    return bad;
}

// The view never depends on the host thread count (rows are tiled in fixed
// blocks; the reordering of long rows' pieces is sequential): every array
// equal with 1 and 7 threads.
static int check_thread_independence(const Csr& csr, int R_req, bool fixed) {
    const Vcsr v = build_vcsr(csr, 4, 64, kLayoutS, 2);
    const TileView a = make_tile_view(v, R_req, 1, fixed), b = make_tile_view(v, R_req, 7, fixed);
    const bool same = a.R == b.R && a.n_tiles == b.n_tiles && a.chunks == b.chunks &&
                      a.pieces == b.pieces && a.brow == b.brow && a.slot == b.slot &&
                      a.mask == b.mask && a.split == b.split &&
                      a.n_partial_rows == b.n_partial_rows && a.val.size() == b.val.size() &&
                      std::memcmp(a.val.data(), b.val.data(), a.val.size() * sizeof(float)) == 0;
    if (!same) return fail("view depends on the thread count", csr.M, a.R);
    return 0;
}

int main() {
    int bad = 0;
    const Csr cfg1 = coo_to_csr(gen_coo(1, 0));
    bad |= check(cfg1, 4, 64, kLayoutS, 0, 1);  // random columns: no shared rows
    bad |= check(cfg1, 4, 64, kLayoutH, 2, 2);
    bad |= check(cfg1, 4, 64, kLayoutS, 8, 8);
    // Block rows: the automatic height follows the block height.
    bad |= check(block_matrix(1, 50, 3, 600, 9, 3, 100, false), 4, 64, kLayoutS, 0, 3);
    bad |= check(block_matrix(2, 40, 2, 500, 9, 3, 100, false), 4, 64, kLayoutS, 0, 2);
    bad |= check(block_matrix(3, 20, 8, 700, 9, 4, 100, false), 4, 64, kLayoutS, 0, 8);
    bad |= check(block_matrix(4, 30, 4, 400, 9, 3, 100, false), 8, 32, kLayoutH, 0, 4);
    // Partial blocks, duplicates, every forced height, every layout.
    for (int R : {1, 2, 3, 4, 8})
        for (int layout : {kLayoutH, kLayoutS, kLayoutTC}) {
            const Csr a = block_matrix(10 + R, 30, 3, 300, 7, 3, 75, true);
            bad |= check(a, 4, 64, layout, R, R);
        }
    // 16-row blocks: the automatic height is the matrix-core tile; 8-row
    // blocks stay at 8 (two neighbouring blocks share no columns).
    bad |= check(block_matrix(5, 12, 16, 900, 9, 16, 100, false), 4, 64, kLayoutS, 0, 16);
    bad |= check(block_matrix(6, 12, 16, 900, 9, 16, 100, false), 16, 16, kLayoutTC, 0, 16);
    for (int layout : {kLayoutH, kLayoutS, kLayoutTC}) {
        bad |= check(block_matrix(7, 10, 16, 500, 7, 16, 75, true), 4, 64, layout, 16, 16);
        bad |= check(block_matrix(8, 30, 3, 300, 7, 3, 75, true), 4, 64, layout, 16, 16);
    }
    bad |= check(cfg1, 4, 64, kLayoutS, 16, 16);
    // Fixed row windows (16 rows: FastSpMM's condensed tiles), any matrix.
    bad |= check(cfg1, 4, 64, kLayoutS, 16, 16, true);
    bad |= check(block_matrix(9, 30, 3, 300, 7, 3, 75, true), 4, 64, kLayoutS, 16, 16, true);
    bad |= check(block_matrix(9, 30, 3, 300, 7, 3, 75, true), 4, 64, kLayoutH, 4, 4, true);
    bad |= check(block_matrix(37, 4, 16, 8192, 700, 4, 90, false), 4, 64, kLayoutS, 16, 16, true);
    // The same windows against FastSpMM's condensed tiles: random rows
    // (cfg1), 3-row blocks with duplicates, windows over 1024 columns (cut
    // into pieces), and a partial last window after empty ones.
    bad |= check_cst(cfg1, 4, 64, kLayoutS);
    bad |= check_cst(block_matrix(9, 30, 3, 300, 7, 3, 75, true), 4, 64, kLayoutS);
    bad |= check_cst(block_matrix(9, 30, 3, 300, 7, 3, 75, true), 8, 32, kLayoutH);
    bad |= check_cst(block_matrix(38, 11, 16, 900, 9, 16, 100, false), 16, 16, kLayoutTC);
    bad |= check_cst(block_matrix(37, 4, 16, 8192, 700, 4, 90, false), 4, 64, kLayoutS);
    {
        Coo e;
        e.M = 16 * 5 + 7;
        e.N = 64;
        for (int r : {2, 3, 84, 86})
            for (int k = 0; k < 20; ++k) {
                e.rows.push_back(r);
                e.cols.push_back((r * 7 + k * 3) % 64);
                e.vals.push_back(0.25f * (float)(k - 9));
            }
        bad |= check_cst(coo_to_csr(e), 4, 64, kLayoutS);
        // Windows of about 3,000 distinct columns and no repeated one (cut
        // into pieces of up to 1024 entries).
        Coo g;
        g.M = 40;
        g.N = 8192;
        for (int r = 0; r < g.M; ++r)
            for (int k = 0; k < 400; ++k) {
                g.rows.push_back(r);
                g.cols.push_back((r * 37 + k * 5) % g.N);
                g.vals.push_back((float)((r + 3 * k) % 17 - 8) / 4.f);
            }
        bad |= check_cst(coo_to_csr(g), 4, 64, kLayoutS);
    }
    bad |= check_long_piece_runs();
    {
        const Csr cfg3 = coo_to_csr(gen_coo(3, 0));
        bad |= check_thread_independence(cfg3, 0, false);
        bad |= check_thread_independence(block_matrix(41, 300, 3, 2000, 9, 3, 90, true), 0, false);
        bad |= check_thread_independence(block_matrix(42, 40, 16, 900, 9, 16, 100, false), 16, true);
    }
    // Tiles wider than one work item (split into pieces with partial sums).
    for (int R : {1, 3, 8}) bad |= check(block_matrix(20 + R, 6, 8, 4096, 300, 4, 90, false), 4, 64, kLayoutS, R, R);
    bad |= check(block_matrix(36, 4, 16, 8192, 700, 4, 90, false), 4, 64, kLayoutS, 16, 16);
    // Empty rows and an empty matrix.
    {
        Coo c;
        c.M = 9;
        c.N = 5;
        c.rows = {2, 2, 6};
        c.cols = {0, 4, 4};
        c.vals = {1.f, 2.f, 3.f};
        for (int R : {0, 1, 2, 4, 16}) bad |= check(coo_to_csr(c), 4, 64, kLayoutS, R, R ? R : 0);
        Coo z;
        z.M = 7;
        z.N = 3;
        bad |= check(coo_to_csr(z), 4, 64, kLayoutS, 0, 0);
    }
    std::printf(bad ? "FAILED\n" : "ALL OK\n");
    return bad;
}
