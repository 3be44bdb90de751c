// vendor.hip - rocSPARSE SpMM as the vendor baseline: CSR (int32 indices,
// FP32 values) times a row-major dense B into a row-major C, default
// algorithm.  The counterpart of the reference's run_cusparse_spmm
// (src/kernels.cu:169-235), which builds a handle, descriptors and a work
// buffer, times only the SpMM call between events, and tears everything
// down.  Here the set-up lives in a plan so that repeated calls do not pay
// for it; spmm_csr_vendor is the one-shot form with the reference's
// behaviour.  For comparison only: no VCSR path calls it.
#include <hip/hip_runtime.h>
#include <rocsparse/rocsparse.h>

#include <string>

#include "entry.hpp"

struct vcsr_vendor_plan {
    rocsparse_handle handle = nullptr;
    rocsparse_spmat_descr A = nullptr;
    rocsparse_dnmat_descr B = nullptr;
    rocsparse_dnmat_descr C = nullptr;
    void* buffer = nullptr;
    size_t buffer_bytes = 0;
    int32_t M = 0, O = 0;
};

namespace {

using namespace vcsr::entry;

void sp_check(rocsparse_status s, const char* where) {
    if (s != rocsparse_status_success)
        throw vcsr::Error(VCSR_EDEVICE, std::string(where) + ": rocSPARSE status " +
                                            std::to_string((int)s));
}

void destroy(vcsr_vendor_plan* p) {
    if (!p) return;
    if (p->A) (void)rocsparse_destroy_spmat_descr(p->A);
    if (p->B) (void)rocsparse_destroy_dnmat_descr(p->B);
    if (p->C) (void)rocsparse_destroy_dnmat_descr(p->C);
    if (p->handle) (void)rocsparse_destroy_handle(p->handle);
    if (p->buffer) (void)hipFree(p->buffer);
    delete p;
}

// C = 1 * A * B + 0 * C, one stage.
rocsparse_status spmm_stage(vcsr_vendor_plan* p, rocsparse_spmm_stage stage, size_t* bytes) {
    const float alpha = 1.f, beta = 0.f;
    return rocsparse_spmm(p->handle, rocsparse_operation_none, rocsparse_operation_none, &alpha,
                          p->A, p->B, &beta, p->C, rocsparse_datatype_f32_r,
                          rocsparse_spmm_alg_default, stage, bytes, p->buffer);
}

}  // namespace

extern "C" {

int vcsr_vendor_plan_create(int32_t M, int32_t N, int32_t nnz, const int32_t* rowptr,
                            const int32_t* col, const float* val, const float* dB, int32_t O,
                            float* dC, void* stream, vcsr_vendor_plan** out) {
    return guarded([&] {
        need(out != nullptr, "null output");
        *out = nullptr;
        need(M >= 0 && N >= 0 && nnz >= 0 && O >= 0, "negative size");
        need(rowptr && (nnz == 0 || (col && val)), "null CSR array");
        need((N == 0 || O == 0 || dB) && (M == 0 || O == 0 || dC), "null dense matrix");
        need_device();
        vcsr_vendor_plan* p = new vcsr_vendor_plan();
        p->M = M;
        p->O = O;
        try {
            sp_check(rocsparse_create_handle(&p->handle), "rocsparse_create_handle");
            sp_check(rocsparse_set_stream(p->handle, (hipStream_t)stream), "rocsparse_set_stream");
            sp_check(rocsparse_create_csr_descr(&p->A, M, N, nnz, const_cast<int32_t*>(rowptr),
                                                const_cast<int32_t*>(col), const_cast<float*>(val),
                                                rocsparse_indextype_i32, rocsparse_indextype_i32,
                                                rocsparse_index_base_zero, rocsparse_datatype_f32_r),
                     "rocsparse_create_csr_descr");
            sp_check(rocsparse_create_dnmat_descr(&p->B, N, O, O, const_cast<float*>(dB),
                                                  rocsparse_datatype_f32_r, rocsparse_order_row),
                     "rocsparse_create_dnmat_descr(B)");
            sp_check(rocsparse_create_dnmat_descr(&p->C, M, O, O, dC, rocsparse_datatype_f32_r,
                                                  rocsparse_order_row),
                     "rocsparse_create_dnmat_descr(C)");
            sp_check(spmm_stage(p, rocsparse_spmm_stage_buffer_size, &p->buffer_bytes),
                     "rocsparse_spmm(buffer size)");
            if (p->buffer_bytes > 0)
                hip_check(hipMalloc(&p->buffer, p->buffer_bytes), "hipMalloc(rocSPARSE buffer)");
            sp_check(spmm_stage(p, rocsparse_spmm_stage_preprocess, &p->buffer_bytes),
                     "rocsparse_spmm(preprocess)");
        } catch (...) {
            destroy(p);
            throw;
        }
        *out = p;
    });
}

int vcsr_vendor_spmm(vcsr_vendor_plan* plan, void* stream, float* ms) {
    return guarded([&] {
        need(plan != nullptr, "null plan");
        sp_check(rocsparse_set_stream(plan->handle, (hipStream_t)stream), "rocsparse_set_stream");
        run_timed((hipStream_t)stream, ms, [&] {
            size_t bytes = plan->buffer_bytes;
            sp_check(spmm_stage(plan, rocsparse_spmm_stage_compute, &bytes), "rocsparse_spmm");
            return hipSuccess;
        });
    });
}

void vcsr_vendor_plan_free(vcsr_vendor_plan* plan) { destroy(plan); }

int spmm_csr_vendor(int32_t M, int32_t N, int32_t nnz, const int32_t* rowptr, const int32_t* col,
                    const float* val, const float* dB, int32_t O, float* dC, void* stream,
                    float* ms) {
    vcsr_vendor_plan* p = nullptr;
    int rc = vcsr_vendor_plan_create(M, N, nnz, rowptr, col, val, dB, O, dC, stream, &p);
    if (rc != VCSR_OK) return rc;
    rc = vcsr_vendor_spmm(p, stream, ms);
    if (rc == VCSR_OK) {
        // The plan's buffer is freed right away: wait for the computation.
        const hipError_t e = hipStreamSynchronize((hipStream_t)stream);
        if (e != hipSuccess)
            rc = vcsr::set_error(VCSR_EDEVICE, std::string("hipStreamSynchronize: ") +
                                                   hipGetErrorString(e));
    }
    destroy(p);
    return rc;
}

}  // extern "C"
