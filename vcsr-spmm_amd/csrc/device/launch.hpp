// launch.hpp - internal launchers of the HIP kernels (device/*.hip).
// Each returns the hipError_t of its launch as int (0 = success).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../fmt_internal.hpp"

namespace vcsr {

// csr_naive.hip: C = A*B, one thread per row.
hipError_t launch_csr_naive(int32_t M, const int32_t* rowptr, const int32_t* col,
                            const float* val, const float* B, int32_t O, float* C,
                            hipStream_t st);

// csr_wave.hip: C = A*B on plain CSR, rows spread over wavefront lanes
// (the ASpT-style competitor).  N bounds B's addressing.
hipError_t launch_csr_wave(int32_t M, const int32_t* rowptr, const int32_t* col, const float* val,
                           const float* B, int32_t N, int32_t O, float* C, hipStream_t st);

// vcsr_stream.hip: C += A*B, VCSR segmented streaming on the vector ALUs.
hipError_t launch_vcsr_stream(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                              int32_t tileK, float* C, hipStream_t st);

// vcsr_mfma.hip: C += A*B, every group collapsed to a dense tile and
// multiplied on FP32 MFMA.  tileK <= 0 picks the width from O.
hipError_t launch_vcsr_mfma(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                            int32_t tileK, float* C, hipStream_t st);

// Column-block width (in 32-column MFMA blocks) used for a tileK request.
int mfma_col_blocks(int32_t tileK, int32_t O);

// MFMA instructions launch_vcsr_mfma issues for one SpMM (padding of the
// dense tiles included) and the FLOPs of each.
struct MfmaWork {
    int64_t ops = 0;
    int32_t flops_per_op = 0;
};
MfmaWork mfma_work(const Vcsr& v, int32_t O, int32_t tileK);

// vcsr_rowmajor.hip: row-stationary traversal of the VCSR slots; C = A*B
// (accumulate = 0) or C += A*B (accumulate = 1).  A format with split rows
// is launched in column slices of at most kRowSliceCols columns, whose
// partial rows `partials` holds: rowmajor_partials_floats(d, O) floats.
hipError_t launch_vcsr_rowmajor(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                                float* C, int32_t accumulate, float* partials, hipStream_t st);
constexpr int32_t kRowSliceCols = 256;
int64_t rowmajor_partials_floats(const DeviceFmt& d, int32_t O);

// vcsr_tile.hip: tile-stationary traversal of the VCSR slots through the
// row-tile view; C = A*B (accumulate = 0) or C += A*B (accumulate = 1).
// `partials` holds the partial rows of split tiles: at least
// tile_partials_floats(v, d, B, O, C) floats (none when the view has no
// split tile); every partial row the launch reads it writes first.
hipError_t launch_vcsr_tile(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                            float* C, int32_t accumulate, float* partials, hipStream_t st);
int64_t tile_partials_floats(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                             const float* C);
// Partial-row floats that cover tile_partials_floats for every O, B and C:
// a view with split tiles is launched in column slices of at most 256
// columns, and its partial rows are one slice wide.
int64_t tile_partials_upload_floats(const DeviceFmt& d);
// What launch_vcsr_tile launches for these B and C: floats per lane, column
// slices (one launch each), whether the tiles run on the matrix cores, the
// reduce launches and the partial-row floats.
struct TilePlan {
    int vec = 0;
    int32_t slice_cols = 0, slices = 0;
    bool matrix_cores = false;
    int32_t reduce_launches = 0;
    int64_t partial_floats = 0;
};
TilePlan tile_launch_plan(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                          const float* C);
// MFMA instructions launch_vcsr_tile issues for one SpMM of width O when
// the view has 16-row tiles (none otherwise), as launched for the alignment
// of 16-byte aligned B and C.
MfmaWork tile_mfma_work(const DeviceFmt& d, int32_t O);

// A row-stationary work item covers at most this many (group, lane) pair
// records (one per lane) and entries (the wave's LDS list); longer rows are
// split into chunks whose partial sums a second kernel adds.
constexpr int32_t kRowChunkPairs = 64;
constexpr int32_t kRowChunkEntries = 512;

}  // namespace vcsr
