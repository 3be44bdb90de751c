// common.hpp - small device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vcsr {

// MI355X dispatches workgroup b of a 1-D grid to XCD (b mod 8).  Remapping
// b so that XCD x receives a contiguous range of logical blocks keeps the
// segments one XCD works on next to each other, so the C rows they update
// (row windows overlap for banded matrices) stay in that XCD's 4 MB L2.
// The map is a bijection on [0, nb) for any nb, so correctness never depends
// on the dispatch order; only locality does.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t nb) {
    const uint32_t x = b & 7u, i = b >> 3, base = nb >> 3, rem = nb & 7u;
    return x * base + (x < rem ? x : rem) + i;
}

// FP32 atomic add without return (global_atomic_add_f32).  Float atomics
// are not associative, so C's last bits depend on the order of the flushes;
// results are compared to the CPU reference within tolerance.
__device__ __forceinline__ void atomic_add_f32(float* p, float v) { unsafeAtomicAdd(p, v); }

__device__ __forceinline__ int32_t uniform(int32_t x) {
    return __builtin_amdgcn_readfirstlane(x);
}

}  // namespace vcsr
