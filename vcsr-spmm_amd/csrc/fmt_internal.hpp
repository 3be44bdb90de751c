// fmt_internal.hpp - definition of the opaque handles of include/vcsr_spmm.h,
// shared by the host entry points (capi_host.cpp, g++) and the device entry
// points (device/runtime.hip, hipcc).  Device memory is held as plain
// pointers so this header needs no HIP include.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "host/core.hpp"

// Device copy of a VCSR format plus the derived work list the kernels use.
struct DeviceFmt {
    bool uploaded = false;
    int device = -1;
    int32_t* group_ptr = nullptr;       // G+1
    int32_t* group_depth = nullptr;     // G
    int32_t* group_seg_base = nullptr;  // G
    int32_t* group_rows = nullptr;      // G*bundle
    int32_t* group_nact = nullptr;      // G: lanes with >= 1 entry (a prefix of the lanes)
    int32_t* lcol = nullptr;            // P
    float* val = nullptr;               // P
    int32_t* items = nullptr;           // 2*n_items: [first group, end group) per work item
    int32_t n_items = 0;
    int32_t max_depth = 0;
    // Row-stationary view of the same slots (the inverse of group_rows):
    // for every (group, active lane) pair, {first slot, segment base column,
    // entry count, row}, ordered by row and, within a row, by segment.
    int32_t* pair_rec = nullptr;        // 4*n_pairs
    int64_t n_pairs = 0;
    // Row work items {row, first pair, end pair, partial index or -1}: a row
    // with more pairs than one wave should take is split into chunks whose
    // partial sums a second kernel adds up.
    int32_t* row_items = nullptr;       // 4*n_row_items
    int32_t n_row_items = 0;
    int32_t n_partials = 0;             // chunks of split rows
    int32_t* split_rows = nullptr;      // 3*n_split: {row, first partial, partial count}
    int32_t n_split = 0;
    // Row-tile view (host/tile_view.hpp) walked by the tile-stationary kernel.
    int32_t tv_R = 1;                   // accumulator rows per tile
    int32_t* tv_chunks = nullptr;       // 4*tv_n_chunks: entry range, piece range
    int32_t tv_n_chunks = 0;
    int32_t* tv_pieces = nullptr;       // 4 per piece: row, rows, first entry, partial row
    int32_t* tv_brow = nullptr;         // per entry: B row, kTileNoEntry for placeholders
                                        // (not uploaded for 1- and 3-row tiles)
    float* tv_val = nullptr;            // tile_dev_stride per entry: values (0 where absent),
                                        // then the B row's bits for 1- and 3-row tiles
    uint16_t* tv_mask = nullptr;        // per entry: presence bit per tile row
    int64_t tv_n_entries = 0;
    int32_t* tv_split = nullptr;        // 4*tv_n_split: row, partial row, stride, pieces
    int32_t tv_n_split = 0;
    std::vector<int32_t> tv_split_pieces;  // host copy of the pieces per split row
                                           // (in the split order: decreasing)
    int32_t tv_partial_rows = 0;
    // Partial sums of split rows / tiles (partials_floats floats): sized at
    // upload for every O (split rows and tiles are launched in column slices
    // of at most 256 columns); allocated by the first call that needs it
    // only when the upload ran out of device memory.
    float* partials = nullptr;
    int64_t partials_floats = 0;
};

struct vcsr_coo {
    vcsr::Coo coo;
};
struct vcsr_csr {
    vcsr::Csr csr;
};
struct vcsr_fmt {
    vcsr::Vcsr v;
    DeviceFmt dev;
    int32_t tile_rows = 0;  // requested tile height of the row-tile view (0 = automatic)
    bool tile_fixed = false;  // fixed windows of tile_rows rows instead of shared-column tiles
    int64_t tv_tiles = 0;   // tiles of the uploaded view
};

namespace vcsr {
// Records the message of a failing call for vcsr_last_error() and returns code.
int set_error(int code, const std::string& msg);
void clear_error();
// Releases the device part of a format (device/runtime.hip).
void free_device_fmt(DeviceFmt& d);
}  // namespace vcsr
