// vecops.hpp - per-lane vectors of 1, 2 or 4 floats and the wave-level
// helpers shared by the row- and tile-stationary kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vcsr {

template <int VEC>
struct VecT;
template <>
struct VecT<1> {
    using T = float;
};
template <>
struct VecT<2> {
    using T = float2;
};
template <>
struct VecT<4> {
    using T = float4;
};

__device__ __forceinline__ void fma_vec(float& acc, float a, float b) { acc = __builtin_fmaf(a, b, acc); }
__device__ __forceinline__ void fma_vec(float2& acc, float a, float2 b) {
    acc.x = __builtin_fmaf(a, b.x, acc.x);
    acc.y = __builtin_fmaf(a, b.y, acc.y);
}
__device__ __forceinline__ void fma_vec(float4& acc, float a, float4 b) {
    acc.x = __builtin_fmaf(a, b.x, acc.x);
    acc.y = __builtin_fmaf(a, b.y, acc.y);
    acc.z = __builtin_fmaf(a, b.z, acc.z);
    acc.w = __builtin_fmaf(a, b.w, acc.w);
}
__device__ __forceinline__ float zero_vec(float) { return 0.f; }
__device__ __forceinline__ float2 zero_vec(float2) { return make_float2(0.f, 0.f); }
__device__ __forceinline__ float4 zero_vec(float4) { return make_float4(0.f, 0.f, 0.f, 0.f); }
__device__ __forceinline__ float add_vec(float a, float b) { return a + b; }
__device__ __forceinline__ float2 add_vec(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float4 add_vec(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ float shfl_xor_vec(float x, int m) { return __shfl_xor(x, m); }
__device__ __forceinline__ float2 shfl_xor_vec(float2 x, int m) {
    return make_float2(__shfl_xor(x.x, m), __shfl_xor(x.y, m));
}
__device__ __forceinline__ float4 shfl_xor_vec(float4 x, int m) {
    return make_float4(__shfl_xor(x.x, m), __shfl_xor(x.y, m), __shfl_xor(x.z, m),
                       __shfl_xor(x.w, m));
}

// Non-temporal stores (written once, not read again by this kernel): they do
// not displace B rows from L2.
typedef float nt_float2 __attribute__((ext_vector_type(2)));
typedef float nt_float4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store_nt(float* p, float x) { __builtin_nontemporal_store(x, p); }
__device__ __forceinline__ void store_nt(float2* p, float2 x) {
    __builtin_nontemporal_store(__builtin_bit_cast(nt_float2, x), reinterpret_cast<nt_float2*>(p));
}
__device__ __forceinline__ void store_nt(float4* p, float4 x) {
    __builtin_nontemporal_store(__builtin_bit_cast(nt_float4, x), reinterpret_cast<nt_float4*>(p));
}

// gfx9 raw buffer resource flags: 32-bit data, no swizzle.  Loads past the
// record count return zeros instead of faulting.
constexpr int32_t kRawBufferFlags = 0x00020000;
// B buffers from this size on are addressed with 64-bit pointers instead of
// 32-bit buffer offsets.
constexpr uint64_t kBufferLimit = 0x80000000u;

// VEC floats of B at byte offset `off` through a raw buffer resource.
template <int VEC>
__device__ __forceinline__ typename VecT<VEC>::T load_b_buf(__amdgpu_buffer_rsrc_t rsrc,
                                                            uint32_t off) {
    using V = typename VecT<VEC>::T;
    if constexpr (VEC == 1)
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, 0));
    else if constexpr (VEC == 2)
        return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b64(rsrc, off, 0, 0));
    else
        return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
}

// Orders this wave's LDS writes before its later LDS reads (the wave's
// lanes run in lock step; the fences keep the compiler from reordering).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Inclusive prefix sum over the 64 lanes.
__device__ __forceinline__ int32_t wave_inclusive_scan(int32_t x, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int32_t y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    return x;
}

}  // namespace vcsr
