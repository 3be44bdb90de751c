// ref_bridge_h.cpp - exposes the reference's header-only MTX reader, COO->CSR
// converter and layout-H builder (include/mmio.hpp, csr.hpp, vcsr.hpp, used
// unmodified from /root/reference/include) through ref_bridge.h.
#include "mmio.hpp"
#include "csr.hpp"
#include "vcsr.hpp"
#include "ref_bridge_common.inc"

namespace {
thread_local std::string g_err;
}

extern "C" {
const char* ref_last_error(void) { return g_err.c_str(); }
void ref_free(void* p) { std::free(p); }

int ref_read_mtx(const char* path, ref_coo* out) {
    try {
        COO c = read_matrix_market_coo(path);
        out->M = c.M;
        out->N = c.N;
        out->nnz = (long long)c.vals.size();
        out->rows = refbridge::dup(c.rows);
        out->cols = refbridge::dup(c.cols);
        out->vals = refbridge::dup(c.vals);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

int ref_coo_to_csr(int M, int N, long long nnz, const int* rows, const int* cols,
                   const float* vals, ref_csr* out) {
    try {
        COO c;
        c.M = M;
        c.N = N;
        c.rows.assign(rows, rows + nnz);
        c.cols.assign(cols, cols + nnz);
        c.vals.assign(vals, vals + nnz);
        CSR s = coo_to_csr(c);
        out->M = s.M;
        out->N = s.N;
        out->nnz = s.nnz;
        out->row_ptr = refbridge::dup(s.row_ptr);
        out->col = refbridge::dup(s.col);
        out->val = refbridge::dup(s.val);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

int ref_build_h(int M, int N, const int* row_ptr, const int* col, const float* val, int segw,
                int bundle, ref_fmt* out) {
    try {
        CSR c = refbridge::make_csr(M, N, row_ptr, col, val);
        VCSRSpMM v = csr_to_vcsr_spmm(c, segw, bundle);
        refbridge::fill(v, out);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}
}
