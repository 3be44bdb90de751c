// ref_bridge.h - C ABI of oracle/_ref/libref.so: the reference's own host
// builders (MuuSeoTia/VCSR-SPMM, compiled from /root/reference by
// oracle/Makefile) behind plain-C entry points, so tests can compare the
// oracle and the product with the reference itself.  Test infrastructure
// only; arrays are malloc'ed and released with ref_free.
#pragma once
#ifdef __cplusplus
extern "C" {
#endif
typedef struct {
    int M, N, segw, bundle, num_groups, has_sgs;
    long long num_slots;
    int *group_ptr, *group_depth, *group_seg_base, *group_rows, *lcol;
    float* val;
    int* segment_group_start; /* layout S only (num_groups from the reference) */
    int num_segments;
} ref_fmt;
typedef struct {
    int M, N, nnz;
    int *row_ptr, *col;
    float* val;
} ref_csr;
typedef struct {
    int M, N;
    long long nnz;
    int *rows, *cols;
    float* vals;
} ref_coo;
const char* ref_last_error(void);
void ref_free(void* p);
int ref_read_mtx(const char* path, ref_coo* out);
int ref_coo_to_csr(int M, int N, long long nnz, const int* rows, const int* cols,
                   const float* vals, ref_csr* out);
int ref_build_h(int M, int N, const int* row_ptr, const int* col, const float* val, int segw,
                int bundle, ref_fmt* out);
int ref_build_s(int M, int N, const int* row_ptr, const int* col, const float* val, int segw,
                int bundle, ref_fmt* out);
int ref_build_tc(int M, int N, const int* row_ptr, const int* col, const float* val, int bundle,
                 ref_fmt* out);
#ifdef __cplusplus
}
#endif
