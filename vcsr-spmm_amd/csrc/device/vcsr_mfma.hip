// vcsr_mfma.hip - VCSR SpMM with every group collapsed to a dense tile and
// multiplied on the FP32 matrix cores of gfx950.
//
// The reference's tensor-core kernel (src/vcsr_tc.cu:122-195) scatters one
// nnz per lane into a 16x16 FP16 A tile per depth step and multiplies it by
// the same FP16 B tile every step.  Since the B tile does not change with
// the depth, sum_d A_d * B = (sum_d A_d) * B: a group is one dense
// (bundle x segw) matrix A_g times the segment's (segw x k) B tile.  Here
// A_g is built directly in MFMA operand registers (each lane sums the slots
// of its row whose lcol equals its column; duplicates of a column add up) and
// multiplied in FP32, so no precision is lost (the reference converted A and
// B to half, vcsr_tc.cu:161,170).
//
// Two tile shapes:
//  * bundle > 16: v_mfma_f32_32x32x2f32.  Lane l supplies A[l%32][l/32] and
//    B[l/32][l%32]; accumulator register r holds D[8(r/4)+4(l/32)+r%4][l%32].
//    One MFMA covers 32 group lanes x 2 segment columns x 32 C columns, so a
//    flush instruction writes two full 128-byte C-row segments.
//  * bundle <= 16 (layout TC, 16x16 dense blocks): v_mfma_f32_16x16x4f32.
//    Lane l supplies A[l%16][l/16] and B[l/16][l%16]; register r holds
//    D[4(l/16)+r][l%16].
// Segment columns are processed in passes of 16 (8 K-steps of the 32x32
// shape, 4 of the 16x16 shape), so any segw works.  B operands of a pass are
// loaded once per work unit (a run of groups of one segment) and reused by
// all its groups.  C is accumulated with FP32 atomics like the reference.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"

namespace vcsr {
namespace {

constexpr int kWaves = 4;
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// 32-row tiles.  KS = K-steps (2 segment columns each) per pass; NCB = number
// of 32-column blocks of C per wave.
template <int KS, int NCB>
__global__ __launch_bounds__(256) void vcsr_mfma32_kernel(
    int32_t n_units, int32_t nkt, int32_t segw, int32_t bundle, int32_t N, int32_t O,
    const int32_t* __restrict__ items, const int32_t* __restrict__ group_ptr,
    const int32_t* __restrict__ group_depth, const int32_t* __restrict__ group_seg_base,
    const int32_t* __restrict__ group_rows, const int32_t* __restrict__ group_nact,
    const int32_t* __restrict__ lcol, const float* __restrict__ val,
    const float* __restrict__ B, float* __restrict__ C) {
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    const int32_t unit = (int32_t)(xcd_remap(blockIdx.x, gridDim.x) * kWaves) + wave;
    if (unit >= n_units) return;
    const int32_t item = unit / nkt, kt = unit - item * nkt;
    const int32_t g0 = items[2 * item], g1 = items[2 * item + 1];
    const int32_t seg_base = group_seg_base[g0];
    const int32_t k0 = kt * (32 * NCB);
    const int hi = lane >> 5, lo = lane & 31;

    for (int32_t pass = 0; pass < segw; pass += 2 * KS) {
        // B operands: b[t][cb] = B[seg_base + pass + 2t + hi][k0 + 32cb + lo].
        float b[KS][NCB];
#pragma unroll
        for (int t = 0; t < KS; ++t) {
            const int32_t sc = pass + 2 * t + hi;
            const int32_t r = seg_base + sc;
            const bool rok = sc < segw && r < N;
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                const int32_t c = k0 + 32 * cb + lo;
                b[t][cb] = (rok && c < O) ? B[(int64_t)r * O + c] : 0.f;
            }
        }
        for (int32_t g = g0; g < g1; ++g) {
            const int32_t depth = group_depth[g];
            const int32_t base = group_ptr[g];
            const int32_t nact = group_nact[g];
            for (int32_t l0 = 0; l0 < nact; l0 += 32) {
                const int32_t li = l0 + lo;
                const bool act = li < nact;
                // Dense A operand of this 32-lane block and pass.
                float a[KS];
#pragma unroll
                for (int t = 0; t < KS; ++t) a[t] = 0.f;
                if (act) {
                    for (int32_t d = 0; d < depth; ++d) {
                        const int64_t slot = (int64_t)base + (int64_t)d * bundle + li;
                        const int32_t lc = lcol[slot] - pass - hi;
                        const float v = val[slot];
#pragma unroll
                        for (int t = 0; t < KS; ++t) a[t] += (lc == 2 * t) ? v : 0.f;
                    }
                }
                floatx16 acc[NCB];
#pragma unroll
                for (int cb = 0; cb < NCB; ++cb) acc[cb] = floatx16(0.f);
#pragma unroll
                for (int t = 0; t < KS; ++t)
#pragma unroll
                    for (int cb = 0; cb < NCB; ++cb)
                        acc[cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t], b[t][cb], acc[cb],
                                                                       0, 0, 0);
                const int32_t rowv = act ? group_rows[(int64_t)g * bundle + li] : -1;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int i = 8 * (r >> 2) + 4 * hi + (r & 3);
                    const int32_t rid = __shfl(rowv, i);
                    if (rid >= 0) {
                        float* crow = C + (int64_t)rid * O + k0 + lo;
#pragma unroll
                        for (int cb = 0; cb < NCB; ++cb)
                            if (k0 + 32 * cb + lo < O) atomic_add_f32(crow + 32 * cb, acc[cb][r]);
                    }
                }
            }
        }
    }
}

// 16-row tiles for bundle <= 16.  KS = K-steps (4 segment columns each) per
// pass; NCB = number of 16-column blocks of C per wave.
template <int KS, int NCB>
__global__ __launch_bounds__(256) void vcsr_mfma16_kernel(
    int32_t n_units, int32_t nkt, int32_t segw, int32_t bundle, int32_t N, int32_t O,
    const int32_t* __restrict__ items, const int32_t* __restrict__ group_ptr,
    const int32_t* __restrict__ group_depth, const int32_t* __restrict__ group_seg_base,
    const int32_t* __restrict__ group_rows, const int32_t* __restrict__ group_nact,
    const int32_t* __restrict__ lcol, const float* __restrict__ val,
    const float* __restrict__ B, float* __restrict__ C) {
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    const int32_t unit = (int32_t)(xcd_remap(blockIdx.x, gridDim.x) * kWaves) + wave;
    if (unit >= n_units) return;
    const int32_t item = unit / nkt, kt = unit - item * nkt;
    const int32_t g0 = items[2 * item], g1 = items[2 * item + 1];
    const int32_t seg_base = group_seg_base[g0];
    const int32_t k0 = kt * (16 * NCB);
    const int q = lane >> 4, lo = lane & 15;

    for (int32_t pass = 0; pass < segw; pass += 4 * KS) {
        float b[KS][NCB];
#pragma unroll
        for (int t = 0; t < KS; ++t) {
            const int32_t sc = pass + 4 * t + q;
            const int32_t r = seg_base + sc;
            const bool rok = sc < segw && r < N;
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                const int32_t c = k0 + 16 * cb + lo;
                b[t][cb] = (rok && c < O) ? B[(int64_t)r * O + c] : 0.f;
            }
        }
        for (int32_t g = g0; g < g1; ++g) {
            const int32_t depth = group_depth[g];
            const int32_t base = group_ptr[g];
            const int32_t nact = group_nact[g];
            for (int32_t l0 = 0; l0 < nact; l0 += 16) {
                const int32_t li = l0 + lo;
                const bool act = li < nact;
                float a[KS];
#pragma unroll
                for (int t = 0; t < KS; ++t) a[t] = 0.f;
                if (act) {
                    for (int32_t d = 0; d < depth; ++d) {
                        const int64_t slot = (int64_t)base + (int64_t)d * bundle + li;
                        const int32_t lc = lcol[slot] - pass - q;
                        const float v = val[slot];
#pragma unroll
                        for (int t = 0; t < KS; ++t) a[t] += (lc == 4 * t) ? v : 0.f;
                    }
                }
                floatx4 acc[NCB];
#pragma unroll
                for (int cb = 0; cb < NCB; ++cb) acc[cb] = floatx4(0.f);
#pragma unroll
                for (int t = 0; t < KS; ++t)
#pragma unroll
                    for (int cb = 0; cb < NCB; ++cb)
                        acc[cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t], b[t][cb], acc[cb],
                                                                       0, 0, 0);
                const int32_t rowv = act ? group_rows[(int64_t)g * bundle + li] : -1;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int32_t rid = __shfl(rowv, 4 * q + r);
                    if (rid >= 0) {
                        float* crow = C + (int64_t)rid * O + k0 + lo;
#pragma unroll
                        for (int cb = 0; cb < NCB; ++cb)
                            if (k0 + 16 * cb + lo < O) atomic_add_f32(crow + 16 * cb, acc[cb][r]);
                    }
                }
            }
        }
    }
}

using KernelFn = void (*)(int32_t, int32_t, int32_t, int32_t, int32_t, int32_t,
                          const int32_t*, const int32_t*, const int32_t*, const int32_t*,
                          const int32_t*, const int32_t*, const int32_t*, const float*,
                          const float*, float*);

template <int KS>
KernelFn pick32(int ncb) {
    switch (ncb) {
        case 1: return vcsr_mfma32_kernel<KS, 1>;
        case 2: return vcsr_mfma32_kernel<KS, 2>;
        case 4: return vcsr_mfma32_kernel<KS, 4>;
        default: return vcsr_mfma32_kernel<KS, 8>;
    }
}

template <int KS>
KernelFn pick16(int ncb) {
    switch (ncb) {
        case 1: return vcsr_mfma16_kernel<KS, 1>;
        case 2: return vcsr_mfma16_kernel<KS, 2>;
        case 4: return vcsr_mfma16_kernel<KS, 4>;
        default: return vcsr_mfma16_kernel<KS, 8>;
    }
}

int pow2_at_most(int x, int cap) {
    int p = 1;
    while (p * 2 <= x && p * 2 <= cap) p *= 2;
    return p;
}

}  // namespace

int mfma_col_blocks(int32_t tileK, int32_t O) {
    const int32_t want = tileK > 0 ? tileK : 128;
    const int32_t c = (std::min(want, std::max<int32_t>(O, 1)) + 31) / 32;
    return pow2_at_most(std::max(1, c), 8);
}

namespace {

// Tile shape the launcher uses: 16x16x4 tiles for bundle <= 16, else
// 32x32x2; ks K-steps per pass, ncb column blocks per wave.
struct MfmaShape {
    bool m16;
    int ks, ncb;
    int32_t tile() const { return m16 ? 16 : 32; }   // rows = columns of a tile
    int32_t kstep() const { return m16 ? 4 : 2; }    // segment columns per MFMA
};

MfmaShape mfma_shape(const Vcsr& v, int32_t O, int32_t tileK) {
    MfmaShape s;
    s.m16 = v.bundle <= 16;
    if (s.m16) {
        const int32_t want = tileK > 0 ? tileK : 128;
        s.ncb = pow2_at_most(std::max(1, (std::min(want, std::max<int32_t>(O, 1)) + 15) / 16), 8);
        s.ks = v.segw <= 4 ? 1 : (v.segw <= 8 ? 2 : 4);
    } else {
        s.ncb = mfma_col_blocks(tileK, O);
        s.ks = v.segw <= 2 ? 1 : (v.segw <= 4 ? 2 : (v.segw <= 8 ? 4 : 8));
    }
    return s;
}

}  // namespace

MfmaWork mfma_work(const Vcsr& v, int32_t O, int32_t tileK) {
    MfmaWork w;
    if (O <= 0 || v.M == 0) return w;
    const MfmaShape s = mfma_shape(v, O, tileK);
    const int32_t tile = s.tile(), kw = tile * s.ncb;
    const int64_t passes = (v.segw + s.kstep() * s.ks - 1) / (s.kstep() * s.ks);
    const int64_t colblocks = (int64_t)((O + kw - 1) / kw) * s.ncb;
    int64_t lane_blocks = 0;  // sum over groups of ceil(active lanes / tile)
    for (int32_t g = 0; g < v.num_groups(); ++g) {
        int32_t nact = 0;
        for (int32_t l = 0; l < v.bundle; ++l) nact += v.lcol[(size_t)v.group_ptr[g] + l] >= 0;
        lane_blocks += (nact + tile - 1) / tile;
    }
    w.ops = lane_blocks * passes * s.ks * colblocks;
    w.flops_per_op = 2 * tile * tile * s.kstep();
    return w;
}

hipError_t launch_vcsr_mfma(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                            int32_t tileK, float* C, hipStream_t st) {
    if (d.n_items == 0 || O <= 0 || v.M == 0) return hipSuccess;
    const MfmaShape s = mfma_shape(v, O, tileK);
    KernelFn fn;
    if (s.m16) {
        if (s.ks == 1) fn = pick16<1>(s.ncb);
        else if (s.ks == 2) fn = pick16<2>(s.ncb);
        else fn = pick16<4>(s.ncb);
    } else {
        if (s.ks == 1) fn = pick32<1>(s.ncb);
        else if (s.ks == 2) fn = pick32<2>(s.ncb);
        else if (s.ks == 4) fn = pick32<4>(s.ncb);
        else fn = pick32<8>(s.ncb);
    }
    const int32_t kw = s.tile() * s.ncb;
    const int32_t nkt = (O + kw - 1) / kw;
    const int64_t units = (int64_t)d.n_items * nkt;
    if (units > INT32_MAX) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)((units + kWaves - 1) / kWaves);
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(64 * kWaves), 0, st, (int32_t)units, nkt, v.segw,
                       v.bundle, v.N, O, d.items, d.group_ptr, d.group_depth, d.group_seg_base,
                       d.group_rows, d.group_nact, d.lcol, d.val, B, C);
    return hipGetLastError();
}

}  // namespace vcsr
