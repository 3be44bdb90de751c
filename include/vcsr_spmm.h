/*
 * vcsr_spmm.h - C ABI of the MI355X (gfx950) VCSR SpMM library.
 *
 * Sparse A (CSR, FP32) x dense B (row-major, FP32) = dense C (row-major).
 * The path: Matrix Market / synthetic load -> COO -> CSR -> VCSR build
 * (column segments of width `segw`, rows of each segment sorted by nnz
 * descending, packed depth-major into bundles of `bundle` lanes) -> HIP kernel.
 *
 * Every entry point returns 0 on success or a nonzero VCSR_E* status; the
 * message of the last failure on the calling thread is vcsr_last_error().
 * No C++ exception crosses this boundary.  Streams and events are passed as
 * `void*` (a hipStream_t / hipEvent_t of the library's own HIP runtime; NULL
 * is the null stream), so the header needs no HIP or framework include.
 *
 * Each declaration names the reference interface it replaces
 * (MuuSeoTia/VCSR-SPMM, path:line).
 */
#ifndef VCSR_SPMM_H
#define VCSR_SPMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status */
enum {
    VCSR_OK = 0,
    VCSR_EINVAL = 1,  /* bad argument (shape, pointer, parameter)            */
    VCSR_EIO = 2,     /* file open / parse failure                           */
    VCSR_ENOMEM = 3,  /* host or device allocation failed                    */
    VCSR_EDEVICE = 4, /* HIP runtime error, or no GPU                        */
    VCSR_ERANGE = 5,  /* index out of range, or a size overflows int32       */
    VCSR_ESTATE = 6   /* object not in the required state (e.g. not uploaded) */
};

/* Thread-local text of the last failing call on this thread ("" if none). */
const char* vcsr_last_error(void);
/* Library version string. */
const char* vcsr_version(void);

/* ------------------------------------------------------- COO (host, owned) */
/* Replaces `struct COO` / `read_matrix_market_coo` (include/mmio.hpp:15-46). */
typedef struct vcsr_coo vcsr_coo;
typedef struct {
    int32_t M, N;
    int64_t nnz;
    const int32_t* rows; /* 0-based */
    const int32_t* cols; /* 0-based */
    const float* vals;
} vcsr_coo_view;

/* Read a coordinate Matrix Market file with the reference's semantics
 * (include/mmio.hpp:22-46): every line starting with '%' and every empty line
 * before the size line is skipped (so `symmetric`/`pattern` qualifiers are
 * ignored), indices are 1-based unless the first entry has a 0 row or column,
 * values are read as double and narrowed to float.  expand_symmetric != 0 is
 * an opt-in extension (not in the reference): when the banner says
 * `symmetric`, every off-diagonal (r,c,v) also yields (c,r,v). */
int vcsr_mtx_read(const char* path, int32_t expand_symmetric, vcsr_coo** out);
/* Wrap caller arrays (copied) as a COO object. */
int vcsr_coo_create(int32_t M, int32_t N, int64_t nnz, const int32_t* rows,
                    const int32_t* cols, const float* vals, vcsr_coo** out);
int vcsr_coo_view_get(const vcsr_coo* coo, vcsr_coo_view* out);
void vcsr_coo_free(vcsr_coo* coo);

/* Synthetic A of BASELINE config `cfg` (1..5) for `seed`, as COO in
 * generation order (rows ascending, columns in draw order).  Deterministic
 * for (cfg, seed).  Not in the reference (it reads SuiteSparse files). */
int vcsr_gen_coo(int32_t cfg, uint64_t seed, vcsr_coo** out);
/* Synthetic dense operand: rows x cols floats, row-major, into `out`
 * (caller-owned host buffer).  dist 0 = U[-1,1) on a 2^-23 grid,
 * dist 1 = N(0,1).  Element i depends only on (seed, i). */
int vcsr_gen_dense(uint64_t seed, int32_t dist, int64_t rows, int32_t cols,
                   float* out);

/* ------------------------------------------------------- CSR (host, owned) */
/* Replaces `struct CSR` / `coo_to_csr` (include/csr.hpp:8-37). */
typedef struct vcsr_csr vcsr_csr;
typedef struct {
    int32_t M, N, nnz;
    const int32_t* row_ptr; /* M+1 */
    const int32_t* col;     /* nnz */
    const float* val;       /* nnz */
} vcsr_csr_view;

/* COO -> CSR with the reference's result: rows bucketed in input order, then
 * each row's entries ordered by column with the same std::sort call as
 * include/csr.hpp:28-35 (duplicates kept, not merged).  Row indices outside
 * [0,M) fail with VCSR_ERANGE (as csr.hpp:19); column indices outside [0,N)
 * also fail (the reference leaves them unchecked). */
int vcsr_coo_to_csr(const vcsr_coo* coo, vcsr_csr** out);
/* Wrap caller CSR arrays (copied, validated) as a CSR object. */
int vcsr_csr_create(int32_t M, int32_t N, const int32_t* row_ptr,
                    const int32_t* col, const float* val, vcsr_csr** out);
int vcsr_csr_view_get(const vcsr_csr* csr, vcsr_csr_view* out);
void vcsr_csr_free(vcsr_csr* csr);

/* ------------------------------------------------------------ VCSR format */
enum {
    VCSR_LAYOUT_H = 0,  /* csr_to_vcsr_spmm, include/vcsr.hpp:25-109          */
    VCSR_LAYOUT_S = 1,  /* csr_to_vcsr_seg / _opt, src/vcsr_seg.cu:24-113    */
    VCSR_LAYOUT_TC = 2  /* csr_to_vcsr_tc (segw=16, bundle=16), src/vcsr_tc.cu:26-106 */
};

typedef struct vcsr_fmt vcsr_fmt;
typedef struct {
    int32_t M, N, segw, bundle, layout;
    int32_t num_groups;   /* G */
    int32_t num_segments; /* S = ceil(N/segw) */
    int64_t num_slots;    /* P = sum_g depth_g * bundle */
    const int32_t* group_ptr;      /* G+1: first slot of group g            */
    const int32_t* group_depth;    /* G                                      */
    const int32_t* group_seg_base; /* G: first column of the group's segment */
    const int32_t* group_rows;     /* G*bundle: row per lane, -1 = padding   */
    const int32_t* lcol;           /* P: column within segment, -1 = padding */
    const float* val;              /* P: value (0 where lcol == -1)          */
    /* S+1: first group of each segment.  The reference keeps it for layout S
     * only (src/vcsr_seg.cu:21,53,109); here it is derived for every layout. */
    const int32_t* segment_group_start;
} vcsr_arrays;

/* Build the VCSR format of a CSR matrix.  Arrays are bit-identical to the
 * reference builder of `layout` on the same CSR (same group order, same row
 * permutation including the order of rows with equal counts, same padding).
 * Layout TC forces segw=16 and bundle=16 like src/vcsr_tc.cu:27-28.
 * nthreads <= 0 uses every hardware thread; segments are built in parallel
 * and concatenated in segment order, which does not change the result. */
int vcsr_build(const vcsr_csr* csr, int32_t segw, int32_t bundle,
               int32_t layout, int32_t nthreads, vcsr_fmt** out);
int vcsr_fmt_arrays(const vcsr_fmt* fmt, vcsr_arrays* out);
/* Write a built format (its host arrays and the row-tile view settings of
 * vcsr_fmt_set_tile_rows / _windows) to a file, and read one back as a new
 * handle that is bit-identical to the saved one and not uploaded, so a
 * matrix's format is built once (the reference rebuilds it every run,
 * src/main.cpp:128-149).  A file that cannot be read is VCSR_EIO; one whose
 * contents break the format's invariants (array sizes, group pointers,
 * rows, columns, segment table) is VCSR_EINVAL.  No reference counterpart. */
int vcsr_fmt_save(const vcsr_fmt* fmt, const char* path);
int vcsr_fmt_load(const char* path, vcsr_fmt** out);
/* Copy the format to the current device (once; later calls are no-ops).
 * Replaces the per-call cudaMallocAsync/cudaMemcpyAsync of
 * src/kernels.cu:139-151 and the one-time static upload of
 * src/vcsr_seg.cu:196-211.  The handle owns the device copy: no globals. */
int vcsr_fmt_upload(vcsr_fmt* fmt, void* stream);
/* Tile height of the row-tile view vcsr_fmt_upload derives for the
 * tile-stationary kernel (VCSR_KERNEL_TILE): rows = 1, 2, 3, 4, 8 or 16
 * forces it, 0 (the default) picks it from the matrix.  16-row tiles run on
 * the FP32 matrix cores (dense sub-blocks, layout TC matrices).  Only before
 * the upload (VCSR_ESTATE after).  No reference counterpart. */
int vcsr_fmt_set_tile_rows(vcsr_fmt* fmt, int32_t rows);
/* fixed != 0: cut the rows into fixed windows of the tile height (which must
 * then be set) instead of tiles of rows that share columns.  With 16
 * rows this is FastSpMM's condensed-tile layout (16-row windows whose
 * distinct columns form 16-column blocks; build_cst_from_csr,
 * src/fastspmm.cu:129-233), computed on FP32 MFMA instead of FP16 WMMA
 * (run_fastspmm_gpu, src/fastspmm.cu:257-303).  Only before the upload
 * (VCSR_ESTATE after); an upload without a tile height is VCSR_EINVAL. */
int vcsr_fmt_set_tile_windows(vcsr_fmt* fmt, int32_t fixed);
/* The uploaded view's tile height, tile count and entry count (B-row slice
 * loads per column tile of one SpMM; nnz for tile height 1).  No reference
 * counterpart. */
int vcsr_fmt_tile_info(const vcsr_fmt* fmt, int32_t* rows, int64_t* tiles, int64_t* entries);
/* Free host and device memory (replaces destroy_vcsr_*_device,
 * src/vcsr_seg.cu:233-243). */
void vcsr_fmt_free(vcsr_fmt* fmt);

/* ----------------------------------------------------------------- SpMM */
/* All GPU entry points take device pointers; B is N x O and C is M x O,
 * row-major with leading dimension O, FP32, int32 indices.
 * If `ms` is non-NULL the call is synchronous like the reference wrappers:
 * it records events around the kernel on `stream`, waits, and stores the
 * kernel-only time in *ms.  If `ms` is NULL the kernel is only enqueued. */

/* C = A*B, one thread per row, C zeroed and accumulated in global memory
 * (the algorithm of csr_spmm_kernel, src/kernels.cu:15-33).  Overwrites C.
 * Replaces run_csr_spmm_gpu (src/kernels.cu:107-118). */
int spmm_csr_naive(int32_t M, const int32_t* d_rowptr, const int32_t* d_col,
                   const float* d_val, const float* dB, int32_t O, float* dC,
                   void* stream, float* ms);

/* C = A*B on plain CSR with rows spread over the lanes of a wavefront: each
 * row's (column, value) pairs are read once and shared by its lanes, C is
 * written once (overwritten; no reset needed).  The ASpT-style competitor:
 * replaces run_aspt_spmm_gpu (src/aspt.cu:144-196), which needs O % 64 == 0;
 * this takes any O and one more argument, N (the rows of B), which bounds
 * B's addressing: a column outside [0, N) contributes nothing. */
int spmm_csr_wave(int32_t M, int32_t N, const int32_t* rowptr, const int32_t* col,
                  const float* val, const float* dB, int32_t O, float* dC, void* stream,
                  float* ms);

/* C += A*B over an uploaded VCSR format (any layout) with the fastest kernel
 * (VCSR_KERNEL_AUTO).  C is accumulated into: zero it first, as
 * main.cpp:126-143 does.  tileK is the C/B column tile of the segment-major
 * kernels (spmm_vcsr_ex); the row- and tile-stationary kernels size their
 * column tiles from O.
 * Replaces run_vcsr_spmm_gpu (src/kernels.cu:120-167),
 * run_vcsr_seg_spmm_gpu (src/vcsr_seg.cu:191-231) and
 * run_vcsr_opt_spmm_gpu (src/vcsr_opt.cu:243-285). */
int spmm_vcsr(const vcsr_fmt* fmt, const float* dB, int32_t O, int32_t tileK,
              float* dC, void* stream, float* ms);

/* Kernel selection of spmm_vcsr_ex (all consume the same uploaded format). */
enum {
    VCSR_KERNEL_AUTO = 0,    /* the fastest kernel for the format (currently TILE) */
    VCSR_KERNEL_SEGMENT = 1, /* segment-major streaming on the vector ALUs, B tile
                                in LDS, C flushed with FP32 atomics per group   */
    VCSR_KERNEL_MFMA = 2,    /* segment-major, group collapsed to a dense tile on
                                FP32 MFMA, C flushed with FP32 atomics          */
    VCSR_KERNEL_ROW = 3,     /* row-stationary: one wavefront per C row walks the
                                row's (group, lane) slots; C written once, no
                                atomics                                         */
    VCSR_KERNEL_TILE = 4     /* tile-stationary: runs of 1, 2, 3, 4 or 8
                                consecutive rows sharing columns are walked
                                together on the vector ALUs, and 16-row tiles
                                (dense sub-blocks) on FP32 MFMA; each B row
                                slice loaded once per tile; C written once    */
};

/* spmm_vcsr with an explicit kernel and C semantics: accumulate = 1 gives
 * C += A*B (the reference's semantics), accumulate = 0 gives C = A*B without
 * a separate reset (the ROW and TILE kernels write every row once; the
 * segment-major kernels clear C on the stream first).  tileK applies to the
 * segment-major kernels.  Calls on one format must not overlap in time: the
 * ROW and TILE kernels keep a scratch buffer in the format for the partial
 * sums of very long rows / tiles.  vcsr_fmt_upload sizes it for every O
 * (a format with split rows or tiles is launched in column slices of at
 * most 256 columns), so with `ms` NULL a call only enqueues kernels — no
 * allocation, memset or synchronisation — and can be captured into a HIP
 * graph.  Only if the upload found too little device memory for that
 * buffer does the first call that needs it wait for the stream and
 * allocate it.
 * No reference counterpart (the reference selects kernels by --algo in
 * src/main.cpp:119-163 and always accumulates). */
int spmm_vcsr_ex(const vcsr_fmt* fmt, const float* dB, int32_t O, int32_t tileK,
                 float* dC, void* stream, float* ms, int32_t kernel,
                 int32_t accumulate);

/* The default kernel (VCSR_KERNEL_TILE, as spmm_vcsr_ex runs it) without any
 * device allocation in the call, for callers that cannot allocate: code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  No counterpart in the reference.  accumulate as in
 * spmm_vcsr_ex (0: C = A*B, 1: C += A*B).  Enqueued on `stream`, not waited
 * for, no timing.  The partial rows of split tiles live in a fixed device
 * array of 16 MiB (4 Mi floats) that each GPU holds until the process ends;
 * a format and O that need more fail with VCSR_ERANGE before any launch
 * (spmm_vcsr_ex has no such limit).  Every call on one GPU uses that GPU's
 * array, so calls that overlap in time on one GPU race; its contents are
 * written before they are read, so a call never sees an earlier one's.
 * The format must be uploaded to the current device; the upload looks up
 * the array's device address, so even the first call may be made under
 * graph capture. */
int spmm_vcsr_noalloc(const vcsr_fmt* fmt, const float* dB, int32_t O, float* dC,
                      void* stream, int32_t accumulate);

/* C += A*B on FP32 MFMA: every group is collapsed to a dense bundle x segw
 * tile and multiplied by the segment's B tile on the matrix cores (FP32 in,
 * FP32 accumulate).  Meant for dense sub-blocks (layout TC); valid for any
 * layout.  Replaces run_vcsr_tc_spmm_gpu (src/vcsr_tc.cu:197-232), which
 * used FP16 WMMA. */
int spmm_vcsr_mfma(const vcsr_fmt* fmt, const float* dB, int32_t O,
                   float* dC, void* stream, float* ms);

/* Work of the FP32-MFMA kernel for one SpMM of width O with column tile
 * tileK (0 as spmm_vcsr_mfma uses): the MFMA instructions it issues (every
 * group as a dense tile, padding included) and the FLOPs of each.  For
 * reporting MFMA utilisation: useful fraction = 2*nnz*O / (ops*flops_per_op),
 * achieved rate = ops*flops_per_op / time against the FP32 MFMA peak.
 * Host only (no upload needed).  No reference counterpart. */
int vcsr_mfma_work(const vcsr_fmt* fmt, int32_t O, int32_t tileK, int64_t* ops,
                   int32_t* flops_per_op);
/* The same for the tile-stationary kernel on an uploaded format whose view
 * has 16-row tiles (v_mfma_f32_16x16x4f32 per four entries, column tile and
 * column part, padding entries included); ops = 0 for other tile heights.
 * No reference counterpart. */
int vcsr_tile_mfma_work(const vcsr_fmt* fmt, int32_t O, int64_t* ops, int32_t* flops_per_op);

/* What one SpMM of width O with `kernel` (VCSR_KERNEL_AUTO resolved) launches
 * on an uploaded format, for reports that name the timed work.  For the
 * tile-stationary kernel: the row-tile view (tile height, tiles, entries =
 * B-row slice loads per column tile), whether its tiles run on the FP32
 * matrix cores, floats per lane, column slices (one launch each) and their
 * width, reduce-kernel launches and split rows, and the partial-row floats
 * of scratch; other kernels report only `kernel`.  As launched on 16-byte
 * aligned B and C.  No reference counterpart. */
typedef struct {
    int32_t kernel;
    int32_t tile_rows;
    int64_t tiles;
    int64_t entries;
    int32_t matrix_cores;
    int32_t vec;
    int32_t column_slices;
    int32_t slice_cols;
    int32_t reduce_launches;
    int32_t split_rows;
    int64_t scratch_floats;
} vcsr_launch_info;
int vcsr_launch_info_get(const vcsr_fmt* fmt, int32_t O, int32_t kernel, vcsr_launch_info* out);

/* ------------------------------------------------------ vendor baseline */
/* rocSPARSE SpMM (CSR int32 x row-major dense, FP32, default algorithm,
 * C = A*B) on caller-owned device arrays: the counterpart of
 * run_cusparse_spmm (src/kernels.cu:169-235), for comparison only.
 * vcsr_vendor_plan_create sets up the handle, descriptors and work buffer
 * (the reference does this inside every call, outside its timed region) and
 * binds the plan to these arrays; vcsr_vendor_spmm computes on `stream` and,
 * if ms is non-NULL, waits and stores the time of the SpMM call alone.
 * spmm_csr_vendor is the one-shot form with the reference's behaviour
 * (returns after the computation).  Failures of the library are
 * VCSR_EDEVICE with its status in vcsr_last_error(). */
typedef struct vcsr_vendor_plan vcsr_vendor_plan;
int vcsr_vendor_plan_create(int32_t M, int32_t N, int32_t nnz, const int32_t* rowptr,
                            const int32_t* col, const float* val, const float* dB,
                            int32_t O, float* dC, void* stream, vcsr_vendor_plan** out);
int vcsr_vendor_spmm(vcsr_vendor_plan* plan, void* stream, float* ms);
void vcsr_vendor_plan_free(vcsr_vendor_plan* plan);
int spmm_csr_vendor(int32_t M, int32_t N, int32_t nnz, const int32_t* rowptr,
                    const int32_t* col, const float* val, const float* dB, int32_t O,
                    float* dC, void* stream, float* ms);

/* CPU CSR SpMM, C = A*B in FP32, for each row: p ascending, k inner, one
 * fused multiply-add per term (the loop order of src/kernels.cu:25-32).
 * nthreads <= 0 uses every hardware thread (rows are independent, so the
 * result does not depend on it).  The reference has no CPU SpMM; its README
 * promises an L2-difference check (README.md:38-39) that needs one. */
int spmm_csr_cpu(int32_t M, const int32_t* rowptr, const int32_t* col,
                 const float* val, const float* B, int32_t O, float* C,
                 int32_t nthreads);

/* --------------------------------------------------- device plumbing */
/* Minimal HIP helpers so hosts (ctypes, the CLI) need no other GPU runtime. */
int vcsr_device_count(int32_t* n);
int vcsr_device_name(char* buf, int32_t len);
int vcsr_dev_malloc(void** ptr, size_t bytes);
int vcsr_dev_free(void* ptr);
int vcsr_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int vcsr_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
/* Device-to-device copy, enqueued on `stream` (not waited for). */
int vcsr_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int vcsr_memset_d(void* dst, int32_t value, size_t bytes, void* stream);
int vcsr_stream_create(void** stream);
int vcsr_stream_destroy(void* stream);
int vcsr_stream_sync(void* stream);
int vcsr_device_sync(void);
int vcsr_event_create(void** event);
int vcsr_event_destroy(void* event);
int vcsr_event_record(void* event, void* stream);
int vcsr_event_elapsed(void* start, void* stop, float* ms);

#ifdef __cplusplus
}
#endif
#endif /* VCSR_SPMM_H */
