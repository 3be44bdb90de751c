// runtime.hip - extern "C" device entry points of include/vcsr_spmm.h:
// format upload, the SpMM launches with optional event timing, and the small
// HIP helpers hosts use instead of a second GPU runtime.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../../include/vcsr_spmm.h"
#include "../fmt_internal.hpp"
#include "../host/tile_view.hpp"
#include "entry.hpp"
#include "launch.hpp"

namespace {

using namespace vcsr::entry;

// Work items: runs of consecutive groups of one segment, at most
// `max_lanes` lanes per run, so a wave's work stays bounded while it reuses
// one B tile across the groups of its run.
std::vector<int32_t> make_items(const vcsr::Vcsr& v, int max_lanes) {
    std::vector<int32_t> items;
    const int per = std::max(1, max_lanes / std::max(1, v.bundle));
    for (int32_t s = 0; s < v.num_segments; ++s) {
        const int32_t a = v.segment_group_start[s], b = v.segment_group_start[s + 1];
        for (int32_t g = a; g < b; g += per) {
            items.push_back(g);
            items.push_back(std::min(b, g + per));
        }
    }
    return items;
}

// Row-stationary view: the inverse of group_rows.  For every group g and
// active lane l (row r = group_rows[g*bundle+l]) one record
// {group_ptr[g]+l, group_seg_base[g], entries of the lane, r}, ordered by r
// and, inside a row, by g (segment order).  A lane with more than
// kRowChunkEntries entries (only possible with duplicate columns) becomes
// several records over consecutive depth ranges.  Each row is cut greedily
// into chunks of at most kRowChunkPairs records and kRowChunkEntries
// entries; a row needing more than one chunk writes per-chunk partial sums
// that a second kernel reduces.
struct RowView {
    std::vector<int32_t> pair_rec, row_items, split_rows;
    int32_t n_partials = 0;
};

RowView make_row_view(const vcsr::Vcsr& v, const std::vector<int32_t>& nact) {
    RowView rv;
    const int32_t G = v.num_groups(), M = v.M, b = v.bundle;
    const int32_t E = vcsr::kRowChunkEntries;
    // Entry count of every active lane (entries are packed from depth 0).
    std::vector<int64_t> lane_off((size_t)G + 1, 0);
    for (int32_t g = 0; g < G; ++g) lane_off[(size_t)g + 1] = lane_off[(size_t)g] + nact[(size_t)g];
    std::vector<int32_t> lane_cnt((size_t)lane_off[(size_t)G]);
    std::vector<int64_t> ptr((size_t)M + 1, 0);
    for (int32_t g = 0; g < G; ++g) {
        const int32_t depth = v.group_depth[g];
        for (int32_t l = 0; l < nact[(size_t)g]; ++l) {
            const int32_t slot0 = v.group_ptr[g] + l;
            int32_t cnt = 0;
            while (cnt < depth && v.lcol[(size_t)slot0 + (size_t)cnt * b] >= 0) ++cnt;
            lane_cnt[(size_t)(lane_off[(size_t)g] + l)] = cnt;
            ptr[(size_t)v.group_rows[(size_t)g * b + l] + 1] += (cnt + E - 1) / E;
        }
    }
    for (int32_t r = 0; r < M; ++r) ptr[(size_t)r + 1] += ptr[(size_t)r];
    const int64_t nrec = ptr[(size_t)M];
    if (nrec > INT32_MAX) throw vcsr::Error(VCSR_ERANGE, "too many (row, segment) pairs");
    rv.pair_rec.resize((size_t)nrec * 4);
    std::vector<int64_t> cur(ptr.begin(), ptr.end() - 1);
    for (int32_t g = 0; g < G; ++g) {
        for (int32_t l = 0; l < nact[(size_t)g]; ++l) {
            const int32_t row = v.group_rows[(size_t)g * b + l];
            const int32_t cnt = lane_cnt[(size_t)(lane_off[(size_t)g] + l)];
            for (int32_t d0 = 0; d0 < cnt; d0 += E) {
                int32_t* rec = rv.pair_rec.data() + 4 * cur[(size_t)row]++;
                rec[0] = v.group_ptr[g] + l + d0 * b;
                rec[1] = v.group_seg_base[g];
                rec[2] = std::min(E, cnt - d0);
                rec[3] = row;
            }
        }
    }
    rv.row_items.reserve((size_t)M * 4);
    std::vector<int32_t> chunk_starts;
    for (int32_t r = 0; r < M; ++r) {
        const int32_t p0 = (int32_t)ptr[(size_t)r], p1 = (int32_t)ptr[(size_t)r + 1];
        chunk_starts.clear();
        chunk_starts.push_back(p0);
        int32_t entries = 0;
        for (int32_t p = p0; p < p1; ++p) {
            const int32_t c = rv.pair_rec[(size_t)p * 4 + 2];
            if (p - chunk_starts.back() == vcsr::kRowChunkPairs || entries + c > E) {
                chunk_starts.push_back(p);
                entries = 0;
            }
            entries += c;
        }
        if (chunk_starts.size() == 1) {
            rv.row_items.insert(rv.row_items.end(), {r, p0, p1, -1});
            continue;
        }
        const int32_t first = rv.n_partials;
        for (size_t q = 0; q < chunk_starts.size(); ++q) {
            const int32_t end = q + 1 < chunk_starts.size() ? chunk_starts[q + 1] : p1;
            rv.row_items.insert(rv.row_items.end(), {r, chunk_starts[q], end, rv.n_partials++});
        }
        rv.split_rows.insert(rv.split_rows.end(), {r, first, rv.n_partials - first});
    }
    return rv;
}

// Scratch of spmm_vcsr_noalloc: the partial rows of split tiles, in a
// file-scope device array instead of memory the call allocates.  Every GPU
// the library runs on holds its own copy until the process ends.  In host
// code `scratch` only names the symbol; its device address on the current
// device comes from hipGetSymbolAddress (scratch_on_current_device), and
// only that address is handed to kernels.
constexpr size_t kScratchFloats = size_t(4) << 20;  // 16 MiB
__device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Address of `scratch` on the current device, looked up once per device
// (by the first format upload there, with that device current, so that a
// first spmm_vcsr_noalloc made under graph capture only reads the cache).
float* scratch_on_current_device() {
    int dev = -1;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw vcsr::Error(VCSR_EDEVICE, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!p) throw vcsr::Error(VCSR_EDEVICE, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    return g_scratch_ptr[dev];
}

// Zeroes n floats: C = A*B for the segment-major kernels, which add into
// C.  A kernel rather than hipMemsetAsync, so that a call captured into a
// HIP graph records kernel nodes only.
__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0.f;
}

hipError_t fill_zero(float* p, int64_t n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, n);
    return hipGetLastError();
}

}  // namespace

namespace vcsr {

void free_device_fmt(DeviceFmt& d) {
    if (!d.uploaded) return;
    int cur = -1;
    (void)hipGetDevice(&cur);
    if (d.device >= 0 && d.device != cur) (void)hipSetDevice(d.device);
    for (void* p : {(void*)d.group_ptr, (void*)d.group_depth, (void*)d.group_seg_base,
                    (void*)d.group_rows, (void*)d.group_nact, (void*)d.lcol, (void*)d.val,
                    (void*)d.items, (void*)d.pair_rec, (void*)d.row_items, (void*)d.split_rows,
                    (void*)d.tv_chunks, (void*)d.tv_pieces, (void*)d.tv_brow, (void*)d.tv_val,
                    (void*)d.tv_mask,
                    (void*)d.tv_split, (void*)d.partials})
        if (p) (void)hipFree(p);
    if (d.device >= 0 && d.device != cur && cur >= 0) (void)hipSetDevice(cur);
    d = DeviceFmt();
}

}  // namespace vcsr

extern "C" {

int vcsr_fmt_upload(vcsr_fmt* fmt, void* stream) {
    return guarded([&] {
        need(fmt != nullptr, "null format");
        if (fmt->dev.uploaded) return;
        need_device();
        const vcsr::Vcsr& v = fmt->v;
        hipStream_t st = (hipStream_t)stream;
        // Derived per-group active-lane count: lanes are sorted by entry count,
        // so the lanes with >= 1 entry are a prefix, and their depth-0 slot is
        // the first real entry.
        const int32_t G = v.num_groups();
        std::vector<int32_t> nact((size_t)G);
        int32_t max_depth = 0;
        for (int32_t g = 0; g < G; ++g) {
            int32_t n = 0;
            for (int32_t l = 0; l < v.bundle; ++l) n += v.lcol[(size_t)v.group_ptr[g] + l] >= 0;
            nact[(size_t)g] = n;
            max_depth = std::max(max_depth, v.group_depth[g]);
        }
        std::vector<int32_t> items = make_items(v, 256);
        RowView rv = make_row_view(v, nact);
        const vcsr::TileView tv = vcsr::make_tile_view(v, fmt->tile_rows, 0, fmt->tile_fixed);
        // Device copy of the entries' B rows: placeholders (no row present)
        // are marked kTileNoEntry, so the kernels tell them apart without
        // reading the presence bits.
        std::vector<int32_t> tv_brow(tv.brow);
        for (size_t q = 0; q < tv_brow.size(); ++q)
            if (tv.mask[q] == 0) tv_brow[q] = vcsr::kTileNoEntry;
        // Device values: for 1- and 3-row tiles each entry's B row follows
        // its values (vcsr::tile_dev_stride).
        std::vector<float> tv_val;
        if (vcsr::tile_dev_folds_brow(tv.R)) {
            const int32_t rs = vcsr::tile_slot_stride(tv.R), ds = vcsr::tile_dev_stride(tv.R);
            const size_t E = tv_brow.size();
            tv_val.assign(E * (size_t)ds, 0.f);
            for (size_t q = 0; q < E; ++q) {
                for (int32_t r = 0; r < tv.R; ++r)
                    tv_val[q * ds + r] = tv.val[q * rs + r];
                std::memcpy(&tv_val[q * ds + ds - 1], &tv_brow[q], sizeof(float));
            }
        }
        DeviceFmt d;
        hip_check(hipGetDevice(&d.device), "hipGetDevice");
        try {
            d.uploaded = true;
            d.group_ptr = upload_array(v.group_ptr, st, "upload group_ptr");
            d.group_depth = upload_array(v.group_depth, st, "upload group_depth");
            d.group_seg_base = upload_array(v.group_seg_base, st, "upload group_seg_base");
            d.group_rows = upload_array(v.group_rows, st, "upload group_rows");
            d.group_nact = upload_array(nact, st, "upload group_nact");
            d.lcol = upload_array(v.lcol, st, "upload lcol");
            d.val = upload_array(v.val, st, "upload val");
            d.items = upload_array(items, st, "upload items");
            d.n_items = (int32_t)(items.size() / 2);
            d.max_depth = max_depth;
            d.pair_rec = upload_array(rv.pair_rec, st, "upload pair records");
            d.n_pairs = (int64_t)(rv.pair_rec.size() / 4);
            d.row_items = upload_array(rv.row_items, st, "upload row items");
            d.n_row_items = (int32_t)(rv.row_items.size() / 4);
            d.split_rows = upload_array(rv.split_rows, st, "upload split rows");
            d.n_split = (int32_t)(rv.split_rows.size() / 3);
            d.n_partials = rv.n_partials;
            d.tv_R = tv.R;
            d.tv_chunks = upload_array(tv.chunks, st, "upload tile chunks");
            d.tv_n_chunks = (int32_t)(tv.chunks.size() / 4);
            d.tv_pieces = upload_array(tv.pieces, st, "upload tile pieces");
            // 1- and 3-row tiles carry the B rows in their value records.
            if (!vcsr::tile_dev_folds_brow(tv.R))
                d.tv_brow = upload_array(tv_brow, st, "upload tile entries");
            d.tv_val = upload_array(vcsr::tile_dev_folds_brow(tv.R) ? tv_val : tv.val, st,
                                    "upload tile values");
            d.tv_mask = upload_array(tv.mask, st, "upload tile masks");
            d.tv_n_entries = tv.n_entries();
            d.tv_split = upload_array(tv.split, st, "upload split tiles");
            d.tv_n_split = (int32_t)(tv.split.size() / 4);
            d.tv_split_pieces.resize((size_t)d.tv_n_split);
            for (int32_t i = 0; i < d.tv_n_split; ++i)
                d.tv_split_pieces[(size_t)i] = tv.split[4 * (size_t)i + 3];
            d.tv_partial_rows = tv.n_partial_rows;
            // Partial rows of split tiles (tile kernel) and split rows (row
            // kernel): both are launched in column slices of at most 256
            // columns when they have any, so this covers every O and no
            // SpMM call needs to allocate.  If the device cannot hold it the
            // format still uploads (kernels without split rows need none)
            // and spmm_vcsr_ex allocates on its first call that needs it.
            const int64_t pf = std::max(vcsr::tile_partials_upload_floats(d),
                                        vcsr::rowmajor_partials_floats(d, vcsr::kRowSliceCols));
            if (pf > 0) {
                hipError_t e = hipMalloc((void**)&d.partials, (size_t)pf * sizeof(float));
                if (e == hipErrorOutOfMemory) {
                    (void)hipGetLastError();  // not a sticky error: later launches check theirs
                    d.partials = nullptr;
                } else {
                    hip_check(e, "hipMalloc partials");
                    d.partials_floats = pf;
                }
            }
            // The host vectors above must outlive the copies.
            hip_check(hipStreamSynchronize(st), "upload sync");
        } catch (...) {
            vcsr::free_device_fmt(d);
            throw;
        }
        fmt->dev = d;
        fmt->tv_tiles = tv.n_tiles;
        // Look up spmm_vcsr_noalloc's scratch array on this device now (it
        // may load the code object), so that the entry point's calls only
        // read the cached address.  A failure here is reported by that
        // entry point, which looks it up again; the upload itself succeeded.
        try {
            (void)scratch_on_current_device();
        } catch (...) {
            (void)hipGetLastError();
        }
    });
}

int spmm_csr_naive(int32_t M, const int32_t* d_rowptr, const int32_t* d_col, const float* d_val,
                   const float* dB, int32_t O, float* dC, void* stream, float* ms) {
    return guarded([&] {
        need(M >= 0 && O >= 0, "negative shape");
        // col, val and B are never read when every row is empty (nnz = 0).
        need(M == 0 || O == 0 || (d_rowptr && dC), "null pointer");
        need_device();
        run_timed((hipStream_t)stream, ms, [&] {
            return vcsr::launch_csr_naive(M, d_rowptr, d_col, d_val, dB, O, dC,
                                          (hipStream_t)stream);
        });
    });
}

int spmm_csr_wave(int32_t M, int32_t N, const int32_t* d_rowptr, const int32_t* d_col,
                  const float* d_val, const float* dB, int32_t O, float* dC, void* stream,
                  float* ms) {
    return guarded([&] {
        need(M >= 0 && N >= 0 && O >= 0, "negative shape");
        need(M == 0 || O == 0 || (d_rowptr && dC), "null pointer");
        need_device();
        run_timed((hipStream_t)stream, ms, [&] {
            return vcsr::launch_csr_wave(M, d_rowptr, d_col, d_val, dB, N, O, dC,
                                         (hipStream_t)stream);
        });
    });
}

int spmm_vcsr_ex(const vcsr_fmt* fmt, const float* dB, int32_t O, int32_t tileK, float* dC,
                 void* stream, float* ms, int32_t kernel, int32_t accumulate) {
    return guarded([&] {
        need(fmt != nullptr, "null format");
        need(O >= 0, "negative O");
        need(kernel >= VCSR_KERNEL_AUTO && kernel <= VCSR_KERNEL_TILE, "unknown kernel");
        need(accumulate == 0 || accumulate == 1, "accumulate must be 0 or 1");
        if (!fmt->dev.uploaded) throw vcsr::Error(VCSR_ESTATE, "format not uploaded");
        need(fmt->v.M == 0 || O == 0 || dC, "null C");
        need(fmt->v.num_groups() == 0 || O == 0 || dB, "null B");
        need_device();
        if (kernel == VCSR_KERNEL_AUTO) kernel = VCSR_KERNEL_TILE;
        hipStream_t st = (hipStream_t)stream;
        DeviceFmt& d = const_cast<vcsr_fmt*>(fmt)->dev;
        // Scratch for the partial sums of split rows / tiles, kept with the
        // format and sized at upload for every O (split rows and tiles are
        // launched in column slices of at most 256 columns), so a call only
        // enqueues kernels.  Only when the upload could not allocate it
        // (out of device memory) is it allocated here, on the first call
        // that needs it, after waiting for the stream.
        const int64_t need = kernel == VCSR_KERNEL_TILE
                                 ? vcsr::tile_partials_floats(fmt->v, d, dB, O, dC)
                                 : kernel == VCSR_KERNEL_ROW ? vcsr::rowmajor_partials_floats(d, O)
                                                             : 0;
        if (need > d.partials_floats) {
            hip_check(hipStreamSynchronize(st), "hipStreamSynchronize");
            if (d.partials) hip_check(hipFree(d.partials), "hipFree");
            d.partials = nullptr;
            d.partials_floats = 0;
            hipError_t e = hipMalloc((void**)&d.partials, (size_t)need * sizeof(float));
            if (e == hipErrorOutOfMemory) throw vcsr::Error(VCSR_ENOMEM, "device allocation failed");
            hip_check(e, "hipMalloc partials");
            d.partials_floats = need;
        }
        run_timed(st, ms, [&]() -> hipError_t {
            if (kernel == VCSR_KERNEL_ROW)
                return vcsr::launch_vcsr_rowmajor(fmt->v, d, dB, O, dC, accumulate, d.partials,
                                                  st);
            if (kernel == VCSR_KERNEL_TILE)
                return vcsr::launch_vcsr_tile(fmt->v, d, dB, O, dC, accumulate, d.partials, st);
            if (!accumulate) {
                hipError_t e = fill_zero(dC, (int64_t)fmt->v.M * O, st);
                if (e != hipSuccess) return e;
            }
            if (kernel == VCSR_KERNEL_SEGMENT)
                return vcsr::launch_vcsr_stream(fmt->v, d, dB, O, tileK, dC, st);
            return vcsr::launch_vcsr_mfma(fmt->v, d, dB, O, tileK, dC, st);
        });
    });
}

int spmm_vcsr_noalloc(const vcsr_fmt* fmt, const float* dB, int32_t O, float* dC, void* stream,
                      int32_t accumulate) {
    return guarded([&] {
        need(fmt != nullptr, "null format");
        need(O >= 0, "negative O");
        need(accumulate == 0 || accumulate == 1, "accumulate must be 0 or 1");
        if (!fmt->dev.uploaded) throw vcsr::Error(VCSR_ESTATE, "format not uploaded");
        need(fmt->v.M == 0 || O == 0 || dC, "null C");
        need(fmt->v.num_groups() == 0 || O == 0 || dB, "null B");
        need_device();
        const DeviceFmt& d = fmt->dev;
        int dev = -1;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        if (dev != d.device)
            throw vcsr::Error(VCSR_ESTATE, "format uploaded to another device than the current one");
        float* sp = scratch_on_current_device();
        const int64_t need_floats = vcsr::tile_partials_floats(fmt->v, d, dB, O, dC);
        if (need_floats > (int64_t)kScratchFloats)
            throw vcsr::Error(VCSR_ERANGE,
                              "split tiles need " + std::to_string(need_floats) +
                                  " floats of scratch at this O; the allocation-free entry point "
                                  "holds " + std::to_string(kScratchFloats) +
                                  " (16 MiB): use spmm_vcsr_ex");
        hip_check(vcsr::launch_vcsr_tile(fmt->v, d, dB, O, dC, accumulate, sp, (hipStream_t)stream),
                  "kernel launch");
    });
}

int spmm_vcsr(const vcsr_fmt* fmt, const float* dB, int32_t O, int32_t tileK, float* dC,
              void* stream, float* ms) {
    return spmm_vcsr_ex(fmt, dB, O, tileK, dC, stream, ms, VCSR_KERNEL_AUTO, 1);
}

int spmm_vcsr_mfma(const vcsr_fmt* fmt, const float* dB, int32_t O, float* dC, void* stream,
                   float* ms) {
    return spmm_vcsr_ex(fmt, dB, O, 0, dC, stream, ms, VCSR_KERNEL_MFMA, 1);
}

int vcsr_launch_info_get(const vcsr_fmt* fmt, int32_t O, int32_t kernel, vcsr_launch_info* out) {
    return guarded([&] {
        need(fmt && out, "null argument");
        need(O >= 0, "negative O");
        need(kernel >= VCSR_KERNEL_AUTO && kernel <= VCSR_KERNEL_TILE, "unknown kernel");
        if (!fmt->dev.uploaded) throw vcsr::Error(VCSR_ESTATE, "format not uploaded");
        std::memset(out, 0, sizeof *out);
        out->kernel = kernel == VCSR_KERNEL_AUTO ? VCSR_KERNEL_TILE : kernel;
        if (out->kernel != VCSR_KERNEL_TILE) return;
        const DeviceFmt& d = fmt->dev;
        // As launched on 16-byte aligned B and C (device allocations are).
        const float* aligned = reinterpret_cast<const float*>(uintptr_t(256));
        const vcsr::TilePlan p = vcsr::tile_launch_plan(fmt->v, d, aligned, O, aligned);
        out->tile_rows = d.tv_R;
        out->tiles = fmt->tv_tiles;
        out->entries = d.tv_n_entries;
        out->matrix_cores = p.matrix_cores ? 1 : 0;
        out->vec = p.vec;
        out->column_slices = p.slices;
        out->slice_cols = p.slice_cols;
        out->reduce_launches = p.reduce_launches;
        out->split_rows = d.tv_n_split;
        out->scratch_floats = p.partial_floats;
    });
}

int vcsr_mfma_work(const vcsr_fmt* fmt, int32_t O, int32_t tileK, int64_t* ops,
                   int32_t* flops_per_op) {
    return guarded([&] {
        need(fmt && ops && flops_per_op, "null argument");
        need(O >= 0, "negative O");
        const vcsr::MfmaWork w = vcsr::mfma_work(fmt->v, O, tileK);
        *ops = w.ops;
        *flops_per_op = w.flops_per_op;
    });
}

int vcsr_tile_mfma_work(const vcsr_fmt* fmt, int32_t O, int64_t* ops, int32_t* flops_per_op) {
    return guarded([&] {
        need(fmt && ops && flops_per_op, "null argument");
        need(O >= 0, "negative O");
        if (!fmt->dev.uploaded) throw vcsr::Error(VCSR_ESTATE, "format not uploaded");
        const vcsr::MfmaWork w = vcsr::tile_mfma_work(fmt->dev, O);
        *ops = w.ops;
        *flops_per_op = w.flops_per_op;
    });
}

int vcsr_device_count(int32_t* n) {
    return guarded([&] {
        need(n != nullptr, "null output");
        int c = 0;
        hipError_t e = hipGetDeviceCount(&c);
        *n = (e == hipSuccess) ? c : 0;
    });
}

int vcsr_device_name(char* buf, int32_t len) {
    return guarded([&] {
        need(buf && len > 0, "bad buffer");
        need_device();
        int dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        hipDeviceProp_t p;
        hip_check(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
        std::string s = std::string(p.gcnArchName) + " cus=" + std::to_string(p.multiProcessorCount);
        std::strncpy(buf, s.c_str(), (size_t)len - 1);
        buf[len - 1] = '\0';
    });
}

int vcsr_dev_malloc(void** ptr, size_t bytes) {
    return guarded([&] {
        need(ptr != nullptr, "null output");
        *ptr = nullptr;
        need_device();
        if (bytes == 0) return;
        hipError_t e = hipMalloc(ptr, bytes);
        if (e == hipErrorOutOfMemory) throw vcsr::Error(VCSR_ENOMEM, "device allocation failed");
        hip_check(e, "hipMalloc");
    });
}

int vcsr_dev_free(void* ptr) {
    return guarded([&] {
        if (ptr) hip_check(hipFree(ptr), "hipFree");
    });
}

int vcsr_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    return guarded([&] {
        if (bytes == 0) return;
        need(dst && src, "null pointer");
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream),
                  "hipMemcpyAsync h2d");
        hip_check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    });
}

int vcsr_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    return guarded([&] {
        if (bytes == 0) return;
        need(dst && src, "null pointer");
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream),
                  "hipMemcpyAsync d2h");
        hip_check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    });
}

int vcsr_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    return guarded([&] {
        if (bytes == 0) return;
        need(dst && src, "null pointer");
        hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream),
                  "hipMemcpyAsync d2d");
    });
}

int vcsr_memset_d(void* dst, int32_t value, size_t bytes, void* stream) {
    return guarded([&] {
        if (bytes == 0) return;
        need(dst != nullptr, "null pointer");
        hip_check(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream), "hipMemsetAsync");
    });
}

int vcsr_stream_create(void** stream) {
    return guarded([&] {
        need(stream != nullptr, "null output");
        need_device();
        hipStream_t s = nullptr;
        hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
        *stream = (void*)s;
    });
}

int vcsr_stream_destroy(void* stream) {
    return guarded([&] {
        if (stream) hip_check(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
    });
}

int vcsr_stream_sync(void* stream) {
    return guarded(
        [&] { hip_check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize"); });
}

int vcsr_device_sync(void) {
    return guarded([&] { hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize"); });
}

int vcsr_event_create(void** event) {
    return guarded([&] {
        need(event != nullptr, "null output");
        need_device();
        hipEvent_t e = nullptr;
        hip_check(hipEventCreate(&e), "hipEventCreate");
        *event = (void*)e;
    });
}

int vcsr_event_destroy(void* event) {
    return guarded([&] {
        if (event) hip_check(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
    });
}

int vcsr_event_record(void* event, void* stream) {
    return guarded([&] {
        need(event != nullptr, "null event");
        hip_check(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
    });
}

int vcsr_event_elapsed(void* start, void* stop, float* ms) {
    return guarded([&] {
        need(start && stop && ms, "null argument");
        hip_check(hipEventSynchronize((hipEvent_t)stop), "hipEventSynchronize");
        hip_check(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop),
                  "hipEventElapsedTime");
    });
}

}  // extern "C"
