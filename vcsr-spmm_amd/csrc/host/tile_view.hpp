// tile_view.hpp - the row-tile view of a VCSR format that the
// tile-stationary kernel (device/vcsr_tile.hip) walks.
//
// A tile is a run of at most R consecutive rows that share most of their
// columns (the rows of one block row of a block-structured matrix).  Its
// entries are the union of the rows' columns in column order; entry e holds
// the B row it reads and, for every row r of the tile, the VCSR slot whose
// value multiplies that B row for row r (-1 where row r has no such column).
// Each B row slice is then loaded once per tile instead of once per row.
// The view also carries those slots' values in entry order (and a presence
// bit per row), so the kernel reads them with coalesced loads.  Gathered
// through the slot indices at run time (the rows of a tile are scattered
// over the VCSR groups of a segment) the kernel was measured 1.1x (banded,
// O = 128) to 1.9x (FEM, O = 8) slower.  The copy is made at upload; the
// slots stay in the view as the record of where each value comes from.
#pragma once

#include <cstdint>
#include <vector>

#include "core.hpp"

namespace vcsr {

// Entries of one work item, by tile height R: 32 per tile row, measured best
// on MI355X for R = 1 (16..128 tried, power-law rows), R = 3 (64..128, banded
// 3x3 blocks: one tile per wave) and R = 8 (128..256).  Small items keep many
// waves in flight and the rows a XCD works on close together (its L2 holds
// their B rows); for narrow B the kernel merges several consecutive items
// per wave.
constexpr int32_t tile_chunk_entries(int32_t R) { return 32 * R; }
// Tile height of the matrix-core path: a tile of up to 16 rows is one MFMA
// operand (v_mfma_f32_16x16x4f32: 16 rows x 4 entries of A against 4 B-row
// slices).  Its entries come in groups of kTileMmaGroup (four MFMA k-steps;
// a tile's entry count is padded up to a multiple), and every piece is a
// work item of its own.
constexpr int32_t kTileMmaRows = 16;
constexpr int32_t kTileMmaGroup = 16;
// Entries of one piece of a tile longer than half a work item (it gets work
// items of its own): at least 64, so a long row is cut into fewer pieces
// (and partial rows for the reduce kernel); larger pieces for single-row
// tiles measured slower where several work items share a wave (power-law
// 322K matrix, O = 8: 128 / 256 entries 35.1 / 48.9 against 29.2 us: the
// wave's LDS list grows with them and fewer waves fit).  The kernel's LDS
// list holds this many entries per merged work item.
constexpr int32_t tile_piece_entries(int32_t R) {
    return R == kTileMmaRows ? 1024 : (32 * R > 64 ? 32 * R : 64);
}
// Slot indices stored per entry for tile height R (a power of two, so that
// an entry's slots and staged values are one aligned vector).
constexpr int32_t tile_slot_stride(int32_t R) {
    return R <= 2 ? R : (R <= 4 ? 4 : (R <= 8 ? 8 : 16));
}
// Position of the value of entry e, tile row r in the view's value array.
// Up to 8 rows: entry-major (e * stride + r).  16 rows: MFMA operand order,
// so that lane l of a wave reads the A operands of four k-steps as one
// 16-byte vector: within group g = e / 16 of 256 values, entry 16g + 4s + k
// and row r sit at 4 * (16k + r) + s (k-step s, MFMA k-index k).
constexpr int64_t tile_val_index(int32_t R, int64_t e, int32_t r) {
    return R != kTileMmaRows
               ? e * tile_slot_stride(R) + r
               : (e / 16) * 256 + 4 * (16 * ((e % 16) % 4) + r) + (e % 16) / 4;
}
// Tile pieces per work item.
constexpr int32_t kTileChunkPieces = 32;
// B row of a placeholder entry (no tile row present) in the device copy of
// the view's B-row array; the host view keeps 0 there.
constexpr int32_t kTileNoEntry = -1;
// The device copy of the values of 1- and 3-row tiles also holds each
// entry's B row (kTileNoEntry for placeholders), as the bits of one more
// float after its values — for 3 rows in the padding slot of the stride —
// so that one load gives an entry's B row and values.  Floats per entry
// there:
constexpr bool tile_dev_folds_brow(int32_t R) { return R == 1 || R == 3; }
constexpr int32_t tile_dev_stride(int32_t R) { return R == 1 ? 2 : tile_slot_stride(R); }
// Rows are cut into tiles inside fixed blocks of this many rows (so that
// blocks can be tiled in parallel and the view never depends on the thread
// count).
constexpr int32_t kTileRowBlock = 4096;

struct TileView {
    int32_t R = 1;                // accumulator rows per tile: 1, 2, 3, 4, 8 or 16
    int32_t n_tiles = 0;
    // Work items, 4 ints each: first entry, end entry, first piece, end piece.
    std::vector<int32_t> chunks;
    // Tile pieces, 4 ints each: first row, row count, first entry, and the
    // first partial row (pieces of a split tile) or -1 (the piece writes C).
    std::vector<int32_t> pieces;
    std::vector<int32_t> brow;    // per entry: B row = segment base + local column
    // tile_slot_stride(R) per entry: VCSR slot for tile row r, or -1.
    std::vector<int32_t> slot;
    // tile_slot_stride(R) per entry: the value of that slot (0 for -1), at
    // tile_val_index(R, e, r).
    std::vector<float> val;
    // Per entry: bit r set where tile row r has the entry's column.
    std::vector<uint16_t> mask;
    // Rows of split tiles, 4 ints each: row, first partial row, stride
    // between the piece partials of that row, piece count; in decreasing
    // piece count.
    std::vector<int32_t> split;
    int32_t n_partial_rows = 0;
    int64_t n_entries() const { return (int64_t)brow.size(); }
};

// Builds the view.  R = 0 picks the tile height that minimises the modelled
// cost (B-row loads plus accumulator updates); R = 1, 2, 3, 4, 8 or 16 forces
// it.  fixed = true cuts the rows into fixed windows of R consecutive rows
// (aligned to multiples of R from row 0 when R divides kTileRowBlock)
// instead of growing a tile only over rows that share its columns; with
// R = 16 that is the condensed-tile layout of FastSpMM (16-row windows whose
// distinct columns form 16-column blocks, src/fastspmm.cu:129-253).
TileView make_tile_view(const Vcsr& v, int32_t R, int nthreads, bool fixed = false);

}  // namespace vcsr
