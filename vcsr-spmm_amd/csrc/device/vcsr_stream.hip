// vcsr_stream.hip - VCSR segmented-streaming SpMM on the vector ALUs (gfx950).
//
// Computes what the reference's VCSR kernels compute (src/kernels.cu:37-103,
// src/vcsr_seg.cu:124-189, src/vcsr_opt.cu:115-241): for every group g and
// lane l with row r = group_rows[g*bundle+l],
//     C[r, k] += sum_d val[slot] * B[seg_base + lcol[slot], k],
//     slot = group_ptr[g] + d*bundle + l,  lcol[slot] >= 0,
// with C accumulated across groups by FP32 atomics (as vcsr_seg.cu:186-188).
//
// Mapping (one wave64 = one work unit = a run of groups of ONE segment x one
// k-tile of width TK):
//  * the segment's B tile (segw x TK) is read once per unit with coalesced
//    128-bit loads into the wave's LDS slice and reused by all its groups
//    (the reference reloads it per group, serially per row, kernels.cu:67-76);
//  * lane l owns row l of the group; its 32 C columns of the current chunk are
//    stationary in VGPRs over the group's whole depth; B operands come from LDS
//    as float4 (one ds_read_b128 per 4 FMAs), all lanes reading one of segw
//    rows, padded so different rows fall in different banks;
//  * the chunk is flushed through a padded LDS transpose so that each
//    global_atomic_add_f32 covers two 128-byte row segments instead of 64
//    scattered words;
//  * lanes past the group's active prefix (rows with no entry in this
//    segment) are skipped: they would add zeros.
// Work units are ordered (segment, k-tile) and blocks are remapped so each XCD
// sweeps a contiguous segment range (C-row locality in its L2).
#include "common.hpp"
#include "launch.hpp"

namespace vcsr {
namespace {

constexpr int kWaves = 4;        // wave64 per block
constexpr int kChunk = 32;       // C columns per lane held in VGPRs
constexpr int kStagePitch = 33;  // floats per transposed row (bank spread)
constexpr int kStageFloats = 64 * kStagePitch;
constexpr int kLdsFloatsPerWave = 40 * 1024 / 4;  // 40 KB per wave, 160 KB per block

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(256) void vcsr_stream_kernel(
    int32_t n_units, int32_t nkt, int32_t TK, int32_t pitch, int32_t segw, int32_t bundle,
    int32_t N, int32_t O, int32_t vec4, const int32_t* __restrict__ items,
    const int32_t* __restrict__ group_ptr, const int32_t* __restrict__ group_depth,
    const int32_t* __restrict__ group_seg_base, const int32_t* __restrict__ group_rows,
    const int32_t* __restrict__ group_nact, const int32_t* __restrict__ lcol,
    const float* __restrict__ val, const float* __restrict__ B, float* __restrict__ C) {
    extern __shared__ float lds[];
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    const int32_t unit = (int32_t)(xcd_remap(blockIdx.x, gridDim.x) * kWaves) + wave;
    if (unit >= n_units) return;  // whole wave; no block barrier below
    float* Bs = lds + wave * (segw * pitch + kStageFloats);
    float* stage = Bs + segw * pitch;

    const int32_t item = unit / nkt, kt = unit - item * nkt;
    const int32_t g0 = items[2 * item], g1 = items[2 * item + 1];
    const int32_t seg_base = group_seg_base[g0];
    const int32_t k0 = kt * TK;
    const int32_t kn = min(TK, O - k0);

    // Stage the B tile: rows seg_base..seg_base+segw-1 (zero past N).
    if (vec4) {
        const int32_t q = kn >> 2;
        for (int32_t i = lane; i < segw * q; i += 64) {
            const int32_t s = i / q, c4 = i - s * q;
            const int32_t r = seg_base + s;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r < N) x = *reinterpret_cast<const float4*>(B + (int64_t)r * O + k0 + 4 * c4);
            *reinterpret_cast<float4*>(Bs + s * pitch + 4 * c4) = x;
        }
    } else {
        for (int32_t i = lane; i < segw * kn; i += 64) {
            const int32_t s = i / kn, c = i - s * kn;
            const int32_t r = seg_base + s;
            Bs[s * pitch + c] = (r < N) ? B[(int64_t)r * O + k0 + c] : 0.f;
        }
    }
    wave_sync();

    for (int32_t g = g0; g < g1; ++g) {
        const int32_t depth = group_depth[g];
        const int32_t base = group_ptr[g];
        const int32_t nact = group_nact[g];
        for (int32_t l0 = 0; l0 < nact; l0 += 64) {
            const int32_t li = l0 + lane;
            const bool act = li < nact;
            const int32_t row = act ? group_rows[(int64_t)g * bundle + li] : -1;
            const int32_t nrows = min(64, nact - l0);
            for (int32_t kc = 0; kc < kn; kc += kChunk) {
                float acc[kChunk];
#pragma unroll
                for (int j = 0; j < kChunk; ++j) acc[j] = 0.f;
                if (act) {
                    for (int32_t d = 0; d < depth; ++d) {
                        const int64_t slot = (int64_t)base + (int64_t)d * bundle + li;
                        const int32_t lc = lcol[slot];
                        if (lc >= 0 && lc < segw) {
                            const float a = val[slot];
                            const float4* bp = reinterpret_cast<const float4*>(Bs + lc * pitch + kc);
#pragma unroll
                            for (int j = 0; j < kChunk / 4; ++j) {
                                const float4 b = bp[j];
                                acc[4 * j + 0] = __builtin_fmaf(a, b.x, acc[4 * j + 0]);
                                acc[4 * j + 1] = __builtin_fmaf(a, b.y, acc[4 * j + 1]);
                                acc[4 * j + 2] = __builtin_fmaf(a, b.z, acc[4 * j + 2]);
                                acc[4 * j + 3] = __builtin_fmaf(a, b.w, acc[4 * j + 3]);
                            }
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < kChunk; ++j) stage[lane * kStagePitch + j] = acc[j];
                wave_sync();
                const int32_t half = lane >> 5, col = kc + (lane & 31);
                for (int32_t rr = 0; rr < nrows; rr += 2) {
                    const int32_t ri = rr + half;
                    const int32_t rid = __shfl(row, ri);
                    if (ri < nrows && rid >= 0 && col < kn)
                        atomic_add_f32(C + (int64_t)rid * O + k0 + col,
                                       stage[ri * kStagePitch + (lane & 31)]);
                }
                wave_sync();
            }
        }
    }
}

}  // namespace

hipError_t launch_vcsr_stream(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                              int32_t tileK, float* C, hipStream_t st) {
    if (d.n_items == 0 || O <= 0 || v.M == 0) return hipSuccess;
    // k-tile width: multiple of the register chunk, limited by the LDS slice.
    int32_t TK = tileK <= 0 ? 128 : tileK;
    TK = ((TK + kChunk - 1) / kChunk) * kChunk;
    const int32_t cap = ((kLdsFloatsPerWave - kStageFloats) / v.segw - 4) / kChunk * kChunk;
    if (cap < kChunk) return hipErrorInvalidValue;  // segw too wide for the LDS slice
    if (TK > cap) TK = cap;
    const int32_t padded = ((O + kChunk - 1) / kChunk) * kChunk;
    if (TK > padded) TK = padded;
    const int32_t pitch = TK + 4;
    const int32_t nkt = (O + TK - 1) / TK;
    const int64_t units = (int64_t)d.n_items * nkt;
    if (units > INT32_MAX) return hipErrorInvalidValue;
    // TK is a multiple of 32, so k0 % 4 == 0; float4 staging also needs an
    // aligned B base and row pitch.
    const int32_t vec4 = (O % 4 == 0 && ((uintptr_t)B & 15u) == 0) ? 1 : 0;
    const size_t lds = (size_t)kWaves * (v.segw * pitch + kStageFloats) * sizeof(float);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)vcsr_stream_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const unsigned blocks = (unsigned)((units + kWaves - 1) / kWaves);
    hipLaunchKernelGGL(vcsr_stream_kernel, dim3(blocks), dim3(64 * kWaves), lds, st,
                       (int32_t)units, nkt, TK, pitch, v.segw, v.bundle, v.N, O, vec4, d.items,
                       d.group_ptr, d.group_depth, d.group_seg_base, d.group_rows, d.group_nact,
                       d.lcol, d.val, B, C);
    return hipGetLastError();
}

}  // namespace vcsr
