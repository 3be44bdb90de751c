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

// vcsr_stream.hip: C += A*B, VCSR segmented streaming on the vector ALUs.
hipError_t launch_vcsr_stream(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                              int32_t tileK, float* C, hipStream_t st);

// vcsr_mfma.hip: C += A*B, every group collapsed to a dense tile and
// multiplied on FP32 MFMA.  tileK <= 0 picks the width from O.
hipError_t launch_vcsr_mfma(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                            int32_t tileK, float* C, hipStream_t st);

// Column-block width (in 32-column MFMA blocks) used for a tileK request.
int mfma_col_blocks(int32_t tileK, int32_t O);

}  // namespace vcsr
