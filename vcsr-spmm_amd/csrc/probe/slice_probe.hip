// slice_probe.hip - measurement probe for bench.py (lib/libvcsr_probe.so),
// not part of the SpMM library: the rate at which waves read B-row-slice
// shaped data through the vector-memory path, for the same slice width and
// per-lane vector as the tile-stationary kernel's B loads.
//
// Every lane of a wave belongs to one of 64 / lps streams of lps lanes; a
// stream reads one slice of slice_floats floats per load (lane k its
// vec floats at offset k * vec), at a pseudo-random slice of a device buffer,
// with 8 loads in flight per lane.  A buffer that fits an XCD's 4 MB L2
// gives the rate of L2-resident slices (each XCD caches its own copy); one
// the size of B gives the rate of uniformly random slices of B, served by
// the MALL or HBM.  The tile kernel reads its slices at B rows the matrix
// chooses, so its rate can be set against the two.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

template <int VEC>
struct VecOf;
template <>
struct VecOf<1> { using T = float; };
template <>
struct VecOf<2> { using T = float2; };
template <>
struct VecOf<4> { using T = float4; };

__device__ inline float hsum(float a) { return a; }
__device__ inline float hsum(float2 a) { return a.x + a.y; }
__device__ inline float hsum(float4 a) { return (a.x + a.y) + (a.z + a.w); }
__device__ inline float add(float a, float b) { return a + b; }
__device__ inline float2 add(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ inline float4 add(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

constexpr int kLoads = 8;      // loads in flight per lane
constexpr int kBlock = 256;    // 4 waves per block

// Slice index s < n_slices, so every load reads inside the buffer
// (n_slices * slice_floats floats); out holds one float per thread.
template <int VEC>
__global__ __launch_bounds__(kBlock) void slice_reads(const float* __restrict__ buf,
                                                      uint32_t n_slices, int32_t slice_floats,
                                                      int32_t lps, int32_t iters,
                                                      float* __restrict__ out) {
    using T = typename VecOf<VEC>::T;
    const uint32_t tid = blockIdx.x * kBlock + threadIdx.x;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t stream = lane / (uint32_t)lps, kl = lane % (uint32_t)lps;
    uint32_t h = (tid >> 6) * 2654435761u + stream * 40503u + 1u;
    T acc{};
    for (int it = 0; it < iters; ++it) {
        T b[kLoads];
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            h = h * 1664525u + 1013904223u;
            const uint32_t s = (h ^ (h >> 15)) % n_slices;
            b[u] = *reinterpret_cast<const T*>(buf + (size_t)s * (size_t)slice_floats +
                                                (size_t)kl * VEC);
        }
#pragma unroll
        for (int u = 0; u < kLoads; ++u) acc = add(acc, b[u]);
    }
    out[tid] = hsum(acc);
}

}  // namespace

extern "C" {

// Times `reps` launches (after two untimed ones) of slice_reads over a
// zeroed buffer of buffer_bytes on a stream of its own, and returns the
// slice bytes read per second and the mean milliseconds per launch.  The
// buffers are allocated and freed here.  Returns 0, 1 for bad arguments, or
// the HIP error code.
int vcsr_probe_slice_reads(uint64_t buffer_bytes, int32_t slice_floats, int32_t vec,
                           int32_t reps, double* bytes_per_s, double* ms_per_launch) {
    if (!bytes_per_s || !ms_per_launch || reps < 1) return 1;
    if (vec != 1 && vec != 2 && vec != 4) return 1;
    if (slice_floats < vec || slice_floats % vec != 0) return 1;
    const int32_t lps = slice_floats / vec;
    if (lps > 64 || (lps & (lps - 1)) != 0) return 1;
    const uint64_t slice_bytes = (uint64_t)slice_floats * 4u;
    const uint64_t n_slices = buffer_bytes / slice_bytes;
    if (n_slices < 1 || n_slices > 0xFFFFFFFFull) return 1;

    const int32_t blocks = 8192, iters = 8;
    float* buf = nullptr;
    float* out = nullptr;
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t err = hipMalloc(&buf, n_slices * slice_bytes);
    if (err == hipSuccess) err = hipMalloc(&out, (size_t)blocks * kBlock * sizeof(float));
    if (err == hipSuccess) err = hipStreamCreate(&st);
    if (err == hipSuccess) err = hipEventCreate(&e0);
    if (err == hipSuccess) err = hipEventCreate(&e1);
    if (err == hipSuccess) err = hipMemsetAsync(buf, 0, n_slices * slice_bytes, st);
    auto launch = [&]() {
        switch (vec) {
            case 4:
                slice_reads<4><<<blocks, kBlock, 0, st>>>(buf, (uint32_t)n_slices, slice_floats,
                                                          lps, iters, out);
                break;
            case 2:
                slice_reads<2><<<blocks, kBlock, 0, st>>>(buf, (uint32_t)n_slices, slice_floats,
                                                          lps, iters, out);
                break;
            default:
                slice_reads<1><<<blocks, kBlock, 0, st>>>(buf, (uint32_t)n_slices, slice_floats,
                                                          lps, iters, out);
                break;
        }
        return hipGetLastError();
    };
    for (int i = 0; i < 2 && err == hipSuccess; ++i) err = launch();
    if (err == hipSuccess) err = hipEventRecord(e0, st);
    for (int i = 0; i < reps && err == hipSuccess; ++i) err = launch();
    if (err == hipSuccess) err = hipEventRecord(e1, st);
    if (err == hipSuccess) err = hipEventSynchronize(e1);
    float ms = 0.f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
    if (err == hipSuccess) {
        const double per = (double)ms / reps;
        const double bytes = (double)blocks * kBlock * iters * kLoads * vec * 4.0;
        *ms_per_launch = per;
        *bytes_per_s = bytes / (per * 1e-3);
    }
    if (st) (void)hipStreamSynchronize(st);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    if (out) (void)hipFree(out);
    if (buf) (void)hipFree(buf);
    return err == hipSuccess ? 0 : (int)err;
}

}  // extern "C"
