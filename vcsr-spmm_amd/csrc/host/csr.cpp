// csr.cpp - COO -> CSR conversion and validation.
//
// Result is identical to coo_to_csr (reference include/csr.hpp:16-37):
//  * row counts + prefix sum, then entries scattered in COO order, so each
//    row starts out in input order (:19-25);
//  * each row is then ordered by column with std::sort and the comparator
//    "column less" (:28-35).  std::sort is not stable, so with duplicate
//    columns in a row the order of the duplicates is whatever libstdc++'s
//    introsort makes of that input; running the same std::sort on a sequence
//    with the same comparison outcomes reproduces it.  Duplicates are kept.
// Rows are independent, so they are sorted in parallel.
#include <algorithm>
#include <numeric>
#include <string>
#include <thread>

#include "core.hpp"
#include "parallel.hpp"

namespace vcsr {

int default_threads() {
    unsigned n = std::thread::hardware_concurrency();
    return n == 0 ? 1 : (int)n;
}

void validate_coo(const Coo& coo) {
    if (coo.M < 0 || coo.N < 0) throw Error(1, "negative matrix dimension");
    if (coo.rows.size() != coo.vals.size() || coo.cols.size() != coo.vals.size())
        throw Error(1, "COO arrays differ in length");
    if (coo.vals.size() > (size_t)INT32_MAX) throw Error(5, "nnz exceeds int32");
}

Csr coo_to_csr(const Coo& coo) {
    validate_coo(coo);
    Csr csr;
    csr.M = coo.M;
    csr.N = coo.N;
    csr.nnz = (int32_t)coo.vals.size();
    csr.row_ptr.assign((size_t)csr.M + 1, 0);
    csr.col.resize(csr.nnz);
    csr.val.resize(csr.nnz);
    for (size_t i = 0; i < coo.rows.size(); ++i) {
        const int32_t r = coo.rows[i];
        if (r < 0 || r >= csr.M) throw Error(5, "row idx out of range");
        const int32_t c = coo.cols[i];
        if (c < 0 || c >= csr.N) throw Error(5, "col idx out of range");
        csr.row_ptr[(size_t)r + 1]++;
    }
    for (int32_t i = 1; i <= csr.M; ++i) csr.row_ptr[i] += csr.row_ptr[i - 1];
    std::vector<int32_t> cursor(csr.row_ptr.begin(), csr.row_ptr.end() - 1);
    for (size_t i = 0; i < coo.vals.size(); ++i) {
        const int32_t dst = cursor[coo.rows[i]]++;
        csr.col[dst] = coo.cols[i];
        csr.val[dst] = coo.vals[i];
    }

    struct ColVal { int32_t c; float v; };
    parallel_for(csr.M, 4096, default_threads(), [&](int64_t rb, int64_t re) {
        std::vector<ColVal> tmp;
        for (int64_t r = rb; r < re; ++r) {
            const int32_t s = csr.row_ptr[r], e = csr.row_ptr[r + 1];
            if (e - s < 2) continue;
            tmp.resize((size_t)(e - s));
            for (int32_t i = s; i < e; ++i) tmp[(size_t)(i - s)] = {csr.col[i], csr.val[i]};
            std::sort(tmp.begin(), tmp.end(),
                      [](const ColVal& a, const ColVal& b) { return a.c < b.c; });
            for (int32_t i = s; i < e; ++i) {
                csr.col[i] = tmp[(size_t)(i - s)].c;
                csr.val[i] = tmp[(size_t)(i - s)].v;
            }
        }
    });
    return csr;
}

void validate_csr(const Csr& csr) {
    if (csr.M < 0 || csr.N < 0 || csr.nnz < 0) throw Error(1, "negative CSR size");
    if (csr.row_ptr.size() != (size_t)csr.M + 1) throw Error(1, "row_ptr must have M+1 entries");
    if (csr.col.size() != (size_t)csr.nnz || csr.val.size() != (size_t)csr.nnz)
        throw Error(1, "col/val must have nnz entries");
    if (csr.row_ptr[0] != 0 || csr.row_ptr[csr.M] != csr.nnz)
        throw Error(5, "row_ptr must start at 0 and end at nnz");
    for (int32_t r = 0; r < csr.M; ++r)
        if (csr.row_ptr[r + 1] < csr.row_ptr[r]) throw Error(5, "row_ptr must be non-decreasing");
    for (int32_t p = 0; p < csr.nnz; ++p)
        if (csr.col[p] < 0 || csr.col[p] >= csr.N) throw Error(5, "col idx out of range");
}

}  // namespace vcsr
