// cpu_spmm.cpp - CPU CSR SpMM (FP32), the L2-diff reference of the CLI.
//
// C[r,k] = sum over p in row r (ascending) of val[p]*B[col[p],k], with C's
// row zeroed first and one fused multiply-add per term: the loop order of the
// reference's naive GPU kernel (src/kernels.cu:25-32), which nvcc contracts
// to FMA.  Rows are split over threads; each row is computed by one thread in
// that order, so the result does not depend on the thread count.
// This is an explicit algorithm of its own (--algo cpu); no GPU entry point
// ever calls it.
#include <cmath>
#include <cstring>

#include "core.hpp"
#include "parallel.hpp"

namespace vcsr {

void spmm_csr_cpu(int32_t M, const int32_t* rowptr, const int32_t* col, const float* val,
                  const float* B, int32_t O, float* C, int nthreads) {
    if (M < 0 || O < 0) throw Error(1, "negative shape");
    if (M == 0 || O == 0) return;
    if (!rowptr || !C || (!B && rowptr[M] > 0) || ((!col || !val) && rowptr[M] > 0))
        throw Error(1, "null pointer");
    if (nthreads <= 0) nthreads = default_threads();
    parallel_for(M, 256, nthreads, [&](int64_t rb, int64_t re) {
        for (int64_t r = rb; r < re; ++r) {
            float* c = C + r * (int64_t)O;
            std::memset(c, 0, sizeof(float) * (size_t)O);
            for (int32_t p = rowptr[r]; p < rowptr[r + 1]; ++p) {
                const float a = val[p];
                const float* b = B + (int64_t)col[p] * O;
                for (int32_t k = 0; k < O; ++k) c[k] = std::fma(a, b[k], c[k]);
            }
        }
    });
}

}  // namespace vcsr
