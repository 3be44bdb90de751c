// entry.hpp - error handling shared by the extern "C" device entry points
// (device/*.hip): HIP failures and library errors become return codes with
// a message for vcsr_last_error(), plus the upload and event-timing helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "../../../include/vcsr_spmm.h"
#include "../fmt_internal.hpp"

namespace vcsr {
namespace entry {

struct HipFail {
    hipError_t e;
    std::string where;
};

inline void hip_check(hipError_t e, const char* where) {
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

inline void need(bool ok, const char* what) {
    if (!ok) throw vcsr::Error(VCSR_EINVAL, what);
}

// The library refuses to run a GPU entry point without a GPU.
inline void need_device() {
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

}  // namespace entry
}  // namespace vcsr
