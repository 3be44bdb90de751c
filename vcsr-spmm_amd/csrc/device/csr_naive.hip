// csr_naive.hip - naive CSR SpMM on gfx950, the baseline denominator.
//
// Same algorithm and loop order as the reference's csr_spmm_kernel
// (src/kernels.cu:15-33): one thread per row, the row of C zeroed and then
// accumulated in global memory, p ascending outer, k inner, one FMA per term.
// Launch 256 threads (4 wave64) per block as the reference (kernels.cu:109).
// Only HIP hygiene differs: 64-bit row offsets (M*O exceeds 2^31 at 10^6 x
// 256 + headroom) and an explicit fmaf, so the result equals the CPU
// reference (same order, same rounding) bit for bit.
#include "launch.hpp"

namespace vcsr {
namespace {

__global__ __launch_bounds__(256) void csr_naive_kernel(int32_t M, int32_t O,
                                                        const int32_t* __restrict__ rowptr,
                                                        const int32_t* __restrict__ col,
                                                        const float* __restrict__ val,
                                                        const float* __restrict__ B,
                                                        float* __restrict__ C) {
    const int32_t row = (int32_t)(blockIdx.x * 256u + threadIdx.x);
    if (row >= M) return;
    float* crow = C + (int64_t)row * O;
    for (int32_t k = 0; k < O; ++k) crow[k] = 0.f;
    const int32_t s = rowptr[row], e = rowptr[row + 1];
    for (int32_t p = s; p < e; ++p) {
        const float a = val[p];
        const float* brow = B + (int64_t)col[p] * O;
        for (int32_t k = 0; k < O; ++k) crow[k] = __builtin_fmaf(a, brow[k], crow[k]);
    }
}

}  // namespace

hipError_t launch_csr_naive(int32_t M, const int32_t* rowptr, const int32_t* col,
                            const float* val, const float* B, int32_t O, float* C,
                            hipStream_t st) {
    if (M <= 0 || O <= 0) return hipSuccess;
    const unsigned blocks = (unsigned)((M + 255) / 256);
    hipLaunchKernelGGL(csr_naive_kernel, dim3(blocks), dim3(256), 0, st, M, O, rowptr, col, val,
                       B, C);
    return hipGetLastError();
}

}  // namespace vcsr
