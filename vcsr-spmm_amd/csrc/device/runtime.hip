// runtime.hip - extern "C" device entry points of include/vcsr_spmm.h:
// format upload, the SpMM launches with optional event timing, and the small
// HIP helpers hosts use instead of a second GPU runtime.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "../../../include/vcsr_spmm.h"
#include "../fmt_internal.hpp"
#include "launch.hpp"

namespace {

struct HipFail {
    hipError_t e;
    std::string where;
};

void hip_check(hipError_t e, const char* where) {
    if (e != hipSuccess) throw HipFail{e, where};
}

template <class F>
int guarded(F&& f) {
    try {
        vcsr::clear_error();
        f();
        return VCSR_OK;
    } catch (const HipFail& h) {
        return vcsr::set_error(VCSR_EDEVICE,
                               h.where + ": " + hipGetErrorString(h.e) + " (" +
                                   std::to_string((int)h.e) + ")");
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

// The library refuses to run a GPU entry point without a GPU.
void need_device() {
    static const int n = [] {
        int c = 0;
        return hipGetDeviceCount(&c) == hipSuccess ? c : 0;
    }();
    if (n <= 0)
        throw vcsr::Error(VCSR_EDEVICE, "no HIP device available (the VCSR kernels need a GPU)");
}

template <class T>
T* upload_array(const std::vector<T>& h, hipStream_t st, const char* what) {
    if (h.empty()) return nullptr;
    T* d = nullptr;
    hip_check(hipMalloc((void**)&d, h.size() * sizeof(T)), what);
    hipError_t e = hipMemcpyAsync(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice, st);
    if (e != hipSuccess) {
        (void)hipFree(d);
        hip_check(e, what);
    }
    return d;
}

// Runs `launch` between two events when ms != NULL (synchronous, kernel-only
// time, as the reference wrappers do), or just enqueues it.
template <class L>
void run_timed(hipStream_t st, float* ms, L&& launch) {
    if (!ms) {
        hip_check(launch(), "kernel launch");
        return;
    }
    hipEvent_t a = nullptr, b = nullptr;
    hip_check(hipEventCreate(&a), "hipEventCreate");
    hipError_t e = hipEventCreate(&b);
    if (e != hipSuccess) {
        (void)hipEventDestroy(a);
        hip_check(e, "hipEventCreate");
    }
    struct Cleanup {
        hipEvent_t a, b;
        ~Cleanup() {
            (void)hipEventDestroy(a);
            (void)hipEventDestroy(b);
        }
    } cleanup{a, b};
    hip_check(hipEventRecord(a, st), "hipEventRecord");
    hip_check(launch(), "kernel launch");
    hip_check(hipEventRecord(b, st), "hipEventRecord");
    hip_check(hipEventSynchronize(b), "hipEventSynchronize");
    hip_check(hipEventElapsedTime(ms, a, b), "hipEventElapsedTime");
}

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

}  // namespace

namespace vcsr {

void free_device_fmt(DeviceFmt& d) {
    if (!d.uploaded) return;
    int cur = -1;
    (void)hipGetDevice(&cur);
    if (d.device >= 0 && d.device != cur) (void)hipSetDevice(d.device);
    for (void* p : {(void*)d.group_ptr, (void*)d.group_depth, (void*)d.group_seg_base,
                    (void*)d.group_rows, (void*)d.group_nact, (void*)d.lcol, (void*)d.val,
                    (void*)d.items})
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
            // The host vectors above must outlive the copies.
            hip_check(hipStreamSynchronize(st), "upload sync");
        } catch (...) {
            vcsr::free_device_fmt(d);
            throw;
        }
        fmt->dev = d;
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

int spmm_vcsr(const vcsr_fmt* fmt, const float* dB, int32_t O, int32_t tileK, float* dC,
              void* stream, float* ms) {
    return guarded([&] {
        need(fmt != nullptr, "null format");
        need(O >= 0, "negative O");
        if (!fmt->dev.uploaded) throw vcsr::Error(VCSR_ESTATE, "format not uploaded");
        need(fmt->v.M == 0 || O == 0 || dC, "null C");
        need(fmt->v.num_groups() == 0 || O == 0 || dB, "null B");
        need_device();
        run_timed((hipStream_t)stream, ms, [&] {
            return vcsr::launch_vcsr_stream(fmt->v, fmt->dev, dB, O, tileK, dC,
                                            (hipStream_t)stream);
        });
    });
}

int spmm_vcsr_mfma(const vcsr_fmt* fmt, const float* dB, int32_t O, float* dC, void* stream,
                   float* ms) {
    return guarded([&] {
        need(fmt != nullptr, "null format");
        need(O >= 0, "negative O");
        if (!fmt->dev.uploaded) throw vcsr::Error(VCSR_ESTATE, "format not uploaded");
        need(fmt->v.M == 0 || O == 0 || dC, "null C");
        need(fmt->v.num_groups() == 0 || O == 0 || dB, "null B");
        need_device();
        run_timed((hipStream_t)stream, ms, [&] {
            return vcsr::launch_vcsr_mfma(fmt->v, fmt->dev, dB, O, 0, dC, (hipStream_t)stream);
        });
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
