// capi_host.cpp - extern "C" host entry points of include/vcsr_spmm.h.
// Each wrapper catches every exception and turns it into a status code plus
// a thread-local message; no exception crosses the C ABI.
#include <cstring>
#include <memory>
#include <new>
#include <string>

#include "../../include/vcsr_spmm.h"
#include "fmt_internal.hpp"
#include "host/fmt_io.hpp"

namespace vcsr {
namespace {
thread_local std::string g_last_error;
}
int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}
void clear_error() { g_last_error.clear(); }
}  // namespace vcsr

namespace {

template <class F>
int guarded(F&& f) {
    try {
        vcsr::clear_error();
        f();
        return VCSR_OK;
    } catch (const vcsr::Error& e) {
        return vcsr::set_error(e.code, e.what());
    } catch (const std::bad_alloc&) {
        return vcsr::set_error(VCSR_ENOMEM, "host allocation failed");
    } catch (const std::exception& e) {
        return vcsr::set_error(VCSR_EINVAL, e.what());
    } catch (...) {
        return vcsr::set_error(VCSR_EINVAL, "unknown error");
    }
}

void need(bool ok, const char* what) {
    if (!ok) throw vcsr::Error(VCSR_EINVAL, what);
}

}  // namespace

extern "C" {

const char* vcsr_last_error(void) { return vcsr::g_last_error.c_str(); }
const char* vcsr_version(void) { return "vcsr-spmm-mi355x 0.1.0 (gfx950)"; }

int vcsr_mtx_read(const char* path, int32_t expand_symmetric, vcsr_coo** out) {
    return guarded([&] {
        need(path && out, "null argument");
        *out = nullptr;
        auto* h = new vcsr_coo;
        try {
            h->coo = vcsr::read_mtx(path, expand_symmetric != 0);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int vcsr_coo_create(int32_t M, int32_t N, int64_t nnz, const int32_t* rows,
                    const int32_t* cols, const float* vals, vcsr_coo** out) {
    return guarded([&] {
        need(out != nullptr, "null output");
        *out = nullptr;
        need(M >= 0 && N >= 0 && nnz >= 0, "negative size");
        need(nnz == 0 || (rows && cols && vals), "null array");
        auto* h = new vcsr_coo;
        h->coo.M = M;
        h->coo.N = N;
        h->coo.rows.assign(rows, rows + nnz);
        h->coo.cols.assign(cols, cols + nnz);
        h->coo.vals.assign(vals, vals + nnz);
        *out = h;
    });
}

int vcsr_coo_view_get(const vcsr_coo* coo, vcsr_coo_view* out) {
    return guarded([&] {
        need(coo && out, "null argument");
        out->M = coo->coo.M;
        out->N = coo->coo.N;
        out->nnz = (int64_t)coo->coo.vals.size();
        out->rows = coo->coo.rows.data();
        out->cols = coo->coo.cols.data();
        out->vals = coo->coo.vals.data();
    });
}

void vcsr_coo_free(vcsr_coo* coo) { delete coo; }

int vcsr_gen_coo(int32_t cfg, uint64_t seed, vcsr_coo** out) {
    return guarded([&] {
        need(out != nullptr, "null output");
        *out = nullptr;
        auto* h = new vcsr_coo;
        try {
            h->coo = vcsr::gen_coo(cfg, seed);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int vcsr_gen_dense(uint64_t seed, int32_t dist, int64_t rows, int32_t cols, float* out) {
    return guarded([&] { vcsr::gen_dense(seed, dist, rows, cols, out); });
}

int vcsr_coo_to_csr(const vcsr_coo* coo, vcsr_csr** out) {
    return guarded([&] {
        need(coo && out, "null argument");
        *out = nullptr;
        auto* h = new vcsr_csr;
        try {
            h->csr = vcsr::coo_to_csr(coo->coo);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int vcsr_csr_create(int32_t M, int32_t N, const int32_t* row_ptr, const int32_t* col,
                    const float* val, vcsr_csr** out) {
    return guarded([&] {
        need(out != nullptr, "null output");
        *out = nullptr;
        need(M >= 0 && N >= 0, "negative size");
        need(row_ptr != nullptr, "null row_ptr");
        const int32_t nnz = row_ptr[M];
        need(nnz >= 0, "negative nnz");
        need(nnz == 0 || (col && val), "null col/val");
        auto* h = new vcsr_csr;
        h->csr.M = M;
        h->csr.N = N;
        h->csr.nnz = nnz;
        h->csr.row_ptr.assign(row_ptr, row_ptr + (size_t)M + 1);
        h->csr.col.assign(col, col + nnz);
        h->csr.val.assign(val, val + nnz);
        try {
            vcsr::validate_csr(h->csr);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int vcsr_csr_view_get(const vcsr_csr* csr, vcsr_csr_view* out) {
    return guarded([&] {
        need(csr && out, "null argument");
        out->M = csr->csr.M;
        out->N = csr->csr.N;
        out->nnz = csr->csr.nnz;
        out->row_ptr = csr->csr.row_ptr.data();
        out->col = csr->csr.col.data();
        out->val = csr->csr.val.data();
    });
}

void vcsr_csr_free(vcsr_csr* csr) { delete csr; }

int vcsr_build(const vcsr_csr* csr, int32_t segw, int32_t bundle, int32_t layout,
               int32_t nthreads, vcsr_fmt** out) {
    return guarded([&] {
        need(csr && out, "null argument");
        *out = nullptr;
        auto* h = new vcsr_fmt;
        try {
            h->v = vcsr::build_vcsr(csr->csr, segw, bundle, layout, nthreads);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int vcsr_fmt_arrays(const vcsr_fmt* fmt, vcsr_arrays* out) {
    return guarded([&] {
        need(fmt && out, "null argument");
        const vcsr::Vcsr& v = fmt->v;
        out->M = v.M;
        out->N = v.N;
        out->segw = v.segw;
        out->bundle = v.bundle;
        out->layout = v.layout;
        out->num_groups = v.num_groups();
        out->num_segments = v.num_segments;
        out->num_slots = (int64_t)v.lcol.size();
        out->group_ptr = v.group_ptr.data();
        out->group_depth = v.group_depth.data();
        out->group_seg_base = v.group_seg_base.data();
        out->group_rows = v.group_rows.data();
        out->lcol = v.lcol.data();
        out->val = v.val.data();
        out->segment_group_start = v.segment_group_start.data();
    });
}

int vcsr_fmt_save(const vcsr_fmt* fmt, const char* path) {
    return guarded([&] {
        need(fmt && path, "null argument");
        vcsr::save_vcsr(fmt->v, fmt->tile_rows, fmt->tile_fixed, path);
    });
}

int vcsr_fmt_load(const char* path, vcsr_fmt** out) {
    return guarded([&] {
        need(path && out, "null argument");
        *out = nullptr;
        std::unique_ptr<vcsr_fmt> f(new vcsr_fmt());
        f->v = vcsr::load_vcsr(path, &f->tile_rows, &f->tile_fixed);
        *out = f.release();
    });
}

int vcsr_fmt_set_tile_rows(vcsr_fmt* fmt, int32_t rows) {
    return guarded([&] {
        need(fmt != nullptr, "null format");
        need(rows == 0 || rows == 1 || rows == 2 || rows == 3 || rows == 4 || rows == 8 ||
                 rows == 16,
             "tile rows must be 0, 1, 2, 3, 4, 8 or 16");
        if (fmt->dev.uploaded) throw vcsr::Error(VCSR_ESTATE, "format already uploaded");
        fmt->tile_rows = rows;
    });
}

int vcsr_fmt_set_tile_windows(vcsr_fmt* fmt, int32_t fixed) {
    return guarded([&] {
        need(fmt != nullptr, "null format");
        if (fmt->dev.uploaded) throw vcsr::Error(VCSR_ESTATE, "format already uploaded");
        fmt->tile_fixed = fixed != 0;
    });
}

int vcsr_fmt_tile_info(const vcsr_fmt* fmt, int32_t* rows, int64_t* tiles, int64_t* entries) {
    return guarded([&] {
        need(fmt != nullptr, "null format");
        if (!fmt->dev.uploaded) throw vcsr::Error(VCSR_ESTATE, "format not uploaded");
        if (rows) *rows = fmt->dev.tv_R;
        if (tiles) *tiles = fmt->tv_tiles;
        if (entries) *entries = fmt->dev.tv_n_entries;
    });
}

void vcsr_fmt_free(vcsr_fmt* fmt) {
    if (!fmt) return;
    vcsr::free_device_fmt(fmt->dev);
    delete fmt;
}

int spmm_csr_cpu(int32_t M, const int32_t* rowptr, const int32_t* col, const float* val,
                 const float* B, int32_t O, float* C, int32_t nthreads) {
    return guarded([&] { vcsr::spmm_csr_cpu(M, rowptr, col, val, B, O, C, nthreads); });
}

}  // extern "C"
