// core.hpp - host-side types and functions of the VCSR SpMM library.
// Everything here is plain C++17 (built with g++); the HIP side lives in
// csrc/device and only sees the flat arrays of these structs.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace vcsr {

// Error carrying one of the VCSR_E* status codes of include/vcsr_spmm.h.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

// Coordinate matrix: the reference's `struct COO` (include/mmio.hpp:15-19).
struct Coo {
    int32_t M = 0, N = 0;
    std::vector<int32_t> rows, cols;
    std::vector<float> vals;
};

// Compressed sparse rows: the reference's `struct CSR` (include/csr.hpp:8-13).
struct Csr {
    int32_t M = 0, N = 0, nnz = 0;
    std::vector<int32_t> row_ptr, col;
    std::vector<float> val;
};

enum Layout : int32_t { kLayoutH = 0, kLayoutS = 1, kLayoutTC = 2 };

// Packed VCSR format; field meaning as VCSRSpMM (include/vcsr.hpp:12-23) and
// VCSRSeg (src/vcsr_seg.cu:10-22).  segment_group_start is filled for every
// layout (the reference keeps it for layout S only).
struct Vcsr {
    int32_t M = 0, N = 0, segw = 0, bundle = 0, layout = kLayoutS;
    int32_t num_segments = 0;
    std::vector<int32_t> group_ptr, group_depth, group_seg_base, group_rows;
    std::vector<int32_t> lcol;
    std::vector<float> val;
    std::vector<int32_t> segment_group_start;
    int32_t num_groups() const { return (int32_t)group_depth.size(); }
};

// mtx.cpp
Coo read_mtx(const std::string& path, bool expand_symmetric);

// csr.cpp
void validate_coo(const Coo& coo);
Csr coo_to_csr(const Coo& coo);
void validate_csr(const Csr& csr);

// vcsr_build.cpp
Vcsr build_vcsr(const Csr& csr, int segw, int bundle, int layout, int nthreads);

// gen.cpp
Coo gen_coo(int cfg, uint64_t seed);
void gen_dense(uint64_t seed, int dist, int64_t rows, int32_t cols, float* out);

// cpu_spmm.cpp
void spmm_csr_cpu(int32_t M, const int32_t* rowptr, const int32_t* col,
                  const float* val, const float* B, int32_t O, float* C,
                  int nthreads);

// Number of worker threads for nthreads <= 0.
int default_threads();

}  // namespace vcsr
