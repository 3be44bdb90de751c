// tile_view.cpp - builds the row-tile view of a VCSR format (tile_view.hpp).
//
// Everything is recovered from the packed VCSR arrays (group_ptr,
// group_depth, group_seg_base, group_rows, lcol, val): the view's slot
// indices point into them and its values are copies of val[slot].
#include "tile_view.hpp"

#include <algorithm>
#include <numeric>
#include <string>
#include <unordered_map>

#include "parallel.hpp"

namespace vcsr {
namespace {

constexpr int kErange = 5;  // VCSR_ERANGE
constexpr int kEinval = 1;  // VCSR_EINVAL

// Entries of every row as (column, slot), row r at [ptr[r], ptr[r+1]), in
// column order.
struct RowLists {
    std::vector<int64_t> ptr;
    std::vector<int32_t> col, slot;
};

int32_t lane_entries(const Vcsr& v, int32_t g, int32_t l) {
    const int64_t s0 = (int64_t)v.group_ptr[g] + l;
    int32_t c = 0;
    while (c < v.group_depth[g] && v.lcol[(size_t)(s0 + (int64_t)c * v.bundle)] >= 0) ++c;
    return c;
}

RowLists row_lists(const Vcsr& v, int nthreads) {
    const int32_t G = v.num_groups(), M = v.M, b = v.bundle;
    RowLists rl;
    rl.ptr.assign((size_t)M + 1, 0);
    for (int32_t g = 0; g < G; ++g) {
        for (int32_t l = 0; l < b; ++l) {
            const int32_t c = lane_entries(v, g, l);
            if (c == 0) continue;
            const int32_t row = v.group_rows[(size_t)g * b + l];
            if (row < 0 || row >= M) throw Error(kEinval, "group row out of range");
            rl.ptr[(size_t)row + 1] += c;
        }
    }
    for (int32_t r = 0; r < M; ++r) rl.ptr[(size_t)r + 1] += rl.ptr[(size_t)r];
    const int64_t total = rl.ptr[(size_t)M];
    rl.col.resize((size_t)total);
    rl.slot.resize((size_t)total);
    std::vector<int64_t> cur(rl.ptr.begin(), rl.ptr.end() - 1);
    for (int32_t g = 0; g < G; ++g) {
        const int32_t base = v.group_seg_base[g];
        for (int32_t l = 0; l < b; ++l) {
            const int32_t c = lane_entries(v, g, l);
            if (c == 0) continue;
            int64_t& at = cur[(size_t)v.group_rows[(size_t)g * b + l]];
            for (int32_t d = 0; d < c; ++d) {
                const int64_t s = (int64_t)v.group_ptr[g] + l + (int64_t)d * b;
                rl.col[(size_t)at] = base + v.lcol[(size_t)s];
                rl.slot[(size_t)at] = (int32_t)s;
                ++at;
            }
        }
    }
    // Groups come in segment order and a lane's slots in local-column order,
    // so rows are already sorted; sort any row that is not (stable, so equal
    // columns keep their slot order).
    parallel_for(M, 4096, nthreads, [&](int64_t rb, int64_t re) {
        std::vector<std::pair<int32_t, int32_t>> tmp;
        for (int64_t r = rb; r < re; ++r) {
            const int64_t a = rl.ptr[(size_t)r], e = rl.ptr[(size_t)r + 1];
            if (std::is_sorted(rl.col.begin() + a, rl.col.begin() + e)) continue;
            tmp.clear();
            for (int64_t i = a; i < e; ++i) tmp.emplace_back(rl.col[(size_t)i], rl.slot[(size_t)i]);
            std::stable_sort(tmp.begin(), tmp.end(),
                             [](const auto& x, const auto& y) { return x.first < y.first; });
            for (int64_t i = a; i < e; ++i) {
                rl.col[(size_t)i] = tmp[(size_t)(i - a)].first;
                rl.slot[(size_t)i] = tmp[(size_t)(i - a)].second;
            }
        }
    });
    return rl;
}

// Sorted multiset union: every column kept with the larger of its two
// multiplicities.
void union_into(const std::vector<int32_t>& a, const int32_t* b, size_t nb,
                std::vector<int32_t>& out) {
    out.clear();
    size_t i = 0, j = 0;
    while (i < a.size() && j < nb) {
        if (a[i] < b[j]) {
            out.push_back(a[i++]);
        } else if (b[j] < a[i]) {
            out.push_back(b[j++]);
        } else {
            out.push_back(a[i]);
            ++i;
            ++j;
        }
    }
    out.insert(out.end(), a.begin() + (int64_t)i, a.end());
    out.insert(out.end(), b + j, b + nb);
}

struct Tile {
    int32_t row0, nrows;
    int64_t nent;  // union size; 1 for a tile of empty rows (one placeholder entry)
};

// Greedy tiles of at most `cap` consecutive rows inside [r0, r1): the next
// row joins the tile while at least half of its columns are already in the
// tile's union (empty rows always join).  With `fixed`, every tile is the
// next `cap` rows whatever their columns (fixed row windows).
void tile_rows(const RowLists& rl, int32_t r0, int32_t r1, int32_t cap, bool fixed,
               std::vector<Tile>& out) {
    std::vector<int32_t> u, w;
    int32_t i = r0;
    while (i < r1) {
        u.assign(rl.col.begin() + rl.ptr[(size_t)i], rl.col.begin() + rl.ptr[(size_t)i + 1]);
        int32_t n = 1;
        while (n < cap && i + n < r1) {
            const int32_t r = i + n;
            const size_t len = (size_t)(rl.ptr[(size_t)r + 1] - rl.ptr[(size_t)r]);
            union_into(u, rl.col.data() + rl.ptr[(size_t)r], len, w);
            if (!fixed && (w.size() - u.size()) * 2 > len) break;
            u.swap(w);
            ++n;
        }
        out.push_back({i, n, std::max<int64_t>(1, (int64_t)u.size())});
        i += n;
    }
}

std::vector<Tile> make_tiles(const RowLists& rl, int32_t M, int32_t cap, bool fixed,
                             int nthreads) {
    const int32_t nblk = (M + kTileRowBlock - 1) / kTileRowBlock;
    std::vector<std::vector<Tile>> per((size_t)nblk);
    parallel_for(nblk, 1, nthreads, [&](int64_t bb, int64_t be) {
        for (int64_t blk = bb; blk < be; ++blk) {
            const int32_t r0 = (int32_t)blk * kTileRowBlock;
            tile_rows(rl, r0, std::min(M, r0 + kTileRowBlock), cap, fixed, per[(size_t)blk]);
        }
    });
    std::vector<Tile> tiles;
    for (auto& p : per) tiles.insert(tiles.end(), p.begin(), p.end());
    return tiles;
}


// Single-row views: the kernel hands work items to the XCDs in eight
// contiguous runs of the item list (one per XCD, device/common.hpp
// xcd_remap), and rows come in order, so each XCD works on an eighth of the
// rows and, for a matrix whose columns cluster near the diagonal, on the
// same eighth of B.  The pieces of very long rows (each an item of its own)
// read B rows all over the matrix, but each covers a narrow column range:
// it is moved into the run whose eighth of B holds its middle column,
// sorted by that column among the run's other items, so that the XCD's L2
// holds its B rows.  Run sizes stay those of the original order.
// Rows cut into 8 or more pieces (more than 448 entries) are moved;
// power-law 322K matrix: O = 8 / 32 / 128 25.6 / 35.9 / 107.8 ->
// 24.9 / 33.9 / 94.8 us per SpMM.  Moving the pieces of every split row
// (more than 64 entries) gave 25.3 / 34.7 / 98.5, from 4 or 16 pieces up
// 25.1 / 34.3 / 95.3 and 24.9 / 34.1 / 95.4, from 32 pieces up 25.0 / 34.2
// / 98.2.
void order_long_pieces_by_column(TileView& tv, int32_t N) {
    constexpr int kSeg = 8;
    constexpr int32_t kMinPieces = 8;
    const int32_t nc = (int32_t)(tv.chunks.size() / 4);
    if (tv.R != 1 || nc < 4 * kSeg || N <= 0 || tv.split.empty()) return;
    std::unordered_map<int32_t, int32_t> npc;
    for (size_t i = 0; i < tv.split.size() / 4; ++i) npc[tv.split[4 * i]] = tv.split[4 * i + 3];
    std::vector<int32_t> fixed;
    std::vector<std::vector<std::pair<int32_t, int32_t>>> mov(kSeg);  // (center, chunk)
    for (int32_t c = 0; c < nc; ++c) {
        const int32_t e0 = tv.chunks[4 * (size_t)c], e1 = tv.chunks[4 * (size_t)c + 1];
        const int32_t p0 = tv.chunks[4 * (size_t)c + 2], p1 = tv.chunks[4 * (size_t)c + 3];
        bool movable = false;
        if (p1 - p0 == 1 && tv.pieces[4 * (size_t)p0 + 3] >= 0) {
            auto it = npc.find(tv.pieces[4 * (size_t)p0]);
            movable = it != npc.end() && it->second >= kMinPieces;
        }
        if (!movable) {
            fixed.push_back(c);
            continue;
        }
        const int32_t center = tv.brow[(size_t)(e0 + (e1 - e0) / 2)];
        const int x = (int)std::min<int64_t>(kSeg - 1, (int64_t)center * kSeg / N);
        mov[(size_t)x].emplace_back(center, c);
    }
    std::vector<int32_t> order;
    order.reserve((size_t)nc);
    size_t f = 0;
    for (int x = 0; x < kSeg; ++x) {
        auto& m = mov[(size_t)x];
        std::stable_sort(m.begin(), m.end());
        const int64_t want = (int64_t)nc * (x + 1) / kSeg - (int64_t)nc * x / kSeg;
        int64_t nf = x == kSeg - 1 ? (int64_t)(fixed.size() - f)
                                   : std::max<int64_t>(0, want - (int64_t)m.size());
        nf = std::min<int64_t>(nf, (int64_t)(fixed.size() - f));
        // Interleave the moved pieces evenly among the run's other items.
        const int64_t K = (int64_t)m.size();
        int64_t j = 0;
        for (int64_t i = 0; i < nf; ++i) {
            while (j < K && (2 * j + 1) * nf < (2 * i + 1) * K) order.push_back(m[(size_t)j++].second);
            order.push_back(fixed[f++]);
        }
        while (j < K) order.push_back(m[(size_t)j++].second);
    }
    while (f < fixed.size()) order.push_back(fixed[f++]);
    TileView out;
    out.R = tv.R;
    out.n_tiles = tv.n_tiles;
    out.split = tv.split;
    out.n_partial_rows = tv.n_partial_rows;
    const size_t E = tv.brow.size();
    out.brow.reserve(E);
    out.slot.reserve(E);
    out.val.reserve(E);
    out.mask.reserve(E);
    out.pieces.reserve(tv.pieces.size());
    out.chunks.reserve(tv.chunks.size());
    for (int32_t c : order) {
        const int32_t e0 = tv.chunks[4 * (size_t)c], e1 = tv.chunks[4 * (size_t)c + 1];
        const int32_t p0 = tv.chunks[4 * (size_t)c + 2], p1 = tv.chunks[4 * (size_t)c + 3];
        const int32_t ne0 = (int32_t)out.brow.size(), np0 = (int32_t)(out.pieces.size() / 4);
        out.brow.insert(out.brow.end(), tv.brow.begin() + e0, tv.brow.begin() + e1);
        out.slot.insert(out.slot.end(), tv.slot.begin() + e0, tv.slot.begin() + e1);
        out.val.insert(out.val.end(), tv.val.begin() + e0, tv.val.begin() + e1);
        out.mask.insert(out.mask.end(), tv.mask.begin() + e0, tv.mask.begin() + e1);
        for (int32_t q = p0; q < p1; ++q)
            out.pieces.insert(out.pieces.end(), {tv.pieces[4 * (size_t)q], tv.pieces[4 * (size_t)q + 1],
                                                 tv.pieces[4 * (size_t)q + 2] - e0 + ne0,
                                                 tv.pieces[4 * (size_t)q + 3]});
        out.chunks.insert(out.chunks.end(), {ne0, ne0 + (e1 - e0), np0, np0 + (p1 - p0)});
    }
    tv = std::move(out);
}

}  // namespace

TileView make_tile_view(const Vcsr& v, int32_t R, int nthreads, bool fixed) {
    if (R != 0 && R != 1 && R != 2 && R != 3 && R != 4 && R != 8 && R != kTileMmaRows)
        throw Error(kEinval, "tile height must be 0, 1, 2, 3, 4, 8 or 16");
    if (fixed && R == 0) throw Error(kEinval, "fixed row windows need a tile height");
    if (nthreads <= 0) nthreads = default_threads();
    const int32_t M = v.M;
    const RowLists rl = row_lists(v, nthreads);

    // Tile height: modelled cost per union entry = one B-row slice load
    // (about 20 cycles of the vector memory pipe) + R accumulator updates on
    // the VALU; 16-row tiles run on the matrix cores, where an entry costs
    // about 4 such updates, but only pay off when the tiles are tall (16-row
    // MFMA operands are wasted on short tiles), so they are considered only
    // when their mean height is at least 12 rows.
    std::vector<Tile> tiles;
    auto pad = [](int32_t cap, int64_t n) {
        return cap == kTileMmaRows ? (n + kTileMmaGroup - 1) / kTileMmaGroup * kTileMmaGroup : n;
    };
    if (R == 0) {
        double best = 0;
        for (int32_t cap : {1, 2, 3, 4, 8, kTileMmaRows}) {
            std::vector<Tile> t = make_tiles(rl, M, cap, false, nthreads);
            int64_t ent = 0;
            for (const Tile& x : t) ent += pad(cap, x.nent);
            if (cap == kTileMmaRows && (int64_t)t.size() * 12 > (int64_t)M) continue;
            const double cost = (double)ent * (16.0 + (cap == kTileMmaRows ? 4 : cap));
            if (R == 0 || cost < best) {
                best = cost;
                R = cap;
                tiles.swap(t);
            }
            // No sharing between neighbouring rows: taller tiles only cost.
            if (cap == 2 && R == 1) break;
        }
    } else {
        tiles = make_tiles(rl, M, R, fixed, nthreads);
    }
    if (R == kTileMmaRows)
        for (Tile& x : tiles) x.nent = pad(R, x.nent);

    TileView tv;
    tv.R = R;
    tv.n_tiles = (int32_t)tiles.size();
    std::vector<int64_t> eoff(tiles.size() + 1, 0);
    for (size_t t = 0; t < tiles.size(); ++t) eoff[t + 1] = eoff[t] + tiles[t].nent;
    const int64_t E = eoff.back();
    if (E > INT32_MAX) throw Error(kErange, "tile view has too many entries");
    tv.brow.resize((size_t)E);
    const size_t stride = (size_t)tile_slot_stride(R);
    tv.slot.assign((size_t)E * stride, -1);
    tv.mask.assign((size_t)E, 0);
    const size_t nval = R == kTileMmaRows ? (size_t)E * kTileMmaRows : (size_t)E * stride;
    tv.val.assign(nval, 0.f);
    parallel_for((int64_t)tiles.size(), 1024, nthreads, [&](int64_t tb, int64_t te) {
        std::vector<int32_t> u, w;
        for (int64_t t = tb; t < te; ++t) {
            const Tile& x = tiles[(size_t)t];
            u.clear();
            for (int32_t r = 0; r < x.nrows; ++r) {
                const int64_t a = rl.ptr[(size_t)(x.row0 + r)], e = rl.ptr[(size_t)(x.row0 + r) + 1];
                union_into(u, rl.col.data() + a, (size_t)(e - a), w);
                u.swap(w);
            }
            const int64_t e0 = eoff[(size_t)t];
            // Placeholder entries (a tile of empty rows, the padding of a
            // 16-row tile) read B row 0 with every slot -1.
            for (int64_t q = 0; q < x.nent; ++q) tv.brow[(size_t)(e0 + q)] = 0;
            if (u.empty()) continue;
            for (size_t q = 0; q < u.size(); ++q) tv.brow[(size_t)e0 + q] = u[q];
            for (int32_t r = 0; r < x.nrows; ++r) {
                int64_t p = rl.ptr[(size_t)(x.row0 + r)];
                const int64_t pe = rl.ptr[(size_t)(x.row0 + r) + 1];
                for (size_t q = 0; q < u.size() && p < pe; ++q) {
                    if (rl.col[(size_t)p] == u[q]) {
                        const size_t k = ((size_t)e0 + q) * stride + (size_t)r;
                        tv.slot[k] = rl.slot[(size_t)p];
                        tv.val[(size_t)tile_val_index(R, e0 + (int64_t)q, r)] =
                            v.val[(size_t)rl.slot[(size_t)p]];
                        tv.mask[(size_t)e0 + q] |= (uint16_t)(1u << r);
                        ++p;
                    }
                }
            }
        }
    });

    // Work items.  A tile longer than half a work item's entry budget gets
    // work items of its own (cut into equal pieces of at most
    // tile_piece_entries that write partial sums when it needs more than
    // one); shorter tiles are packed in row order.
    const int32_t cap_e = tile_chunk_entries(R), cap_p = tile_piece_entries(R);
    int64_t ce0 = 0, cent = 0;
    int32_t cp0 = 0;
    auto close_chunk = [&](int64_t next_e) {
        const int32_t np = (int32_t)(tv.pieces.size() / 4);
        if (np > cp0)
            tv.chunks.insert(tv.chunks.end(), {(int32_t)ce0, (int32_t)(ce0 + cent), cp0, np});
        ce0 = next_e;
        cent = 0;
        cp0 = np;
    };
    int64_t n_partial = 0;
    // 16-row tiles: every tile gets work items of its own, cut at multiples
    // of kTileMmaGroup entries.
    const int64_t align = R == kTileMmaRows ? kTileMmaGroup : 1;
    for (size_t t = 0; t < tiles.size(); ++t) {
        const Tile& x = tiles[t];
        const int64_t e0 = eoff[t];
        if (x.nent > cap_e / 2 || R == kTileMmaRows) {
            close_chunk(e0);
            const int64_t npc = (x.nent + cap_p - 1) / cap_p;
            // Equal pieces in units of `align` entries (x.nent is a multiple).
            const int64_t units = x.nent / align;
            const int64_t base = n_partial;
            for (int64_t j = 0; j < npc; ++j) {
                const int64_t a = align == 1 ? e0 + j * ((x.nent + npc - 1) / npc)
                                             : e0 + align * (j * units / npc);
                const int64_t e = align == 1 ? std::min(e0 + x.nent, a + (x.nent + npc - 1) / npc)
                                             : e0 + align * ((j + 1) * units / npc);
                const int32_t pi = (int32_t)(tv.pieces.size() / 4);
                tv.pieces.insert(tv.pieces.end(),
                                 {x.row0, x.nrows, (int32_t)a,
                                  npc == 1 ? -1 : (int32_t)(base + j * x.nrows)});
                tv.chunks.insert(tv.chunks.end(), {(int32_t)a, (int32_t)e, pi, pi + 1});
            }
            if (npc > 1) {
                for (int32_t r = 0; r < x.nrows; ++r)
                    tv.split.insert(tv.split.end(),
                                    {x.row0 + r, (int32_t)(base + r), x.nrows, (int32_t)npc});
                n_partial += npc * x.nrows;
                if (n_partial > INT32_MAX) throw Error(kErange, "too many partial rows");
            }
            cp0 = (int32_t)(tv.pieces.size() / 4);
            ce0 = e0 + x.nent;
            cent = 0;
            continue;
        }
        if (cent + x.nent > cap_e || (int32_t)(tv.pieces.size() / 4) - cp0 == kTileChunkPieces)
            close_chunk(e0);
        tv.pieces.insert(tv.pieces.end(), {x.row0, x.nrows, (int32_t)e0, -1});
        cent += x.nent;
    }
    close_chunk(E);
    // The reduce kernel takes one split row per block in this order: rows
    // with the most pieces first, so the longest sums are not the last to
    // start (cfg3, 2,740 split rows of up to 264 pieces: 1% faster at O = 8
    // and at O = 128).  Each row's sum does not depend on the order.
    {
        const size_t ns = tv.split.size() / 4;
        std::vector<int32_t> ord(ns);
        std::iota(ord.begin(), ord.end(), 0);
        std::stable_sort(ord.begin(), ord.end(), [&](int32_t a, int32_t b) {
            return tv.split[4 * (size_t)a + 3] > tv.split[4 * (size_t)b + 3];
        });
        std::vector<int32_t> sorted(tv.split.size());
        for (size_t i = 0; i < ns; ++i)
            std::copy_n(tv.split.begin() + 4 * (ptrdiff_t)ord[i], 4,
                        sorted.begin() + 4 * (ptrdiff_t)i);
        tv.split.swap(sorted);
    }
    tv.n_partial_rows = (int32_t)n_partial;
    if (R == 1 && !fixed) order_long_pieces_by_column(tv, v.N);
    return tv;
}

}  // namespace vcsr
