// vcsr_rowmajor.hip - row-stationary SpMM over the VCSR format (gfx950).
//
// Same arithmetic as the segmented-streaming kernels (every nonzero is read
// from the packed VCSR slots: val[slot] * B[seg_base + lcol[slot], :]), but
// the work is ordered by C row instead of by segment: one wavefront owns one
// C row (or a chunk of a very long row), keeps its k-slice of that row in
// VGPRs while it walks the row's (group, lane) pairs in segment order, and
// writes the row once with plain coalesced stores.  No atomics: on MI355X a
// global FP32 atomic costs about one element per clock per L2 channel (about
// 10x a plain store) and an LDS FP32 atomic about one element per 3 clocks
// per CU, so the per-group C flush of the segment-major schedule dominates it.
//
// A work item is a row chunk of at most 64 pairs and kRowChunkEntries
// entries.  Phase 1 (lane-parallel): lane i reads pair record i, gathers the
// pair's slots (lcol, val) and writes each entry as (byte offset of its B
// row, value) into the wave's LDS list at the wave-exclusive prefix sum of
// the entry counts.
// Phase 2: the wave streams the list in blocks of 16 load instructions
// issued back to back (all full blocks unpredicated, then one predicated tail
// block), so 16 B-row loads are in flight per wave.  The vector memory pipe takes about 16
// cycles per load instruction whatever its width, so every instruction is a
// 16-byte-per-lane load and, when O is small, serves several entries at
// once (one per group of lanes).  B is read with raw buffer loads: the 32-bit
// byte offset is the only per-entry address arithmetic (one VALU add) and the
// hardware range check turns any read past the end of B into zeros.  B
// buffers of 2 GB or more take the same loop with 64-bit addresses instead.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"
#include "vecops.hpp"

namespace vcsr {
namespace {

constexpr int kWaves = 4;

// VEC floats of B at byte offset `off` (buffer path) or at B + off (64-bit).
template <int VEC, bool BUF>
__device__ __forceinline__ typename VecT<VEC>::T load_b(__amdgpu_buffer_rsrc_t rsrc,
                                                        const float* B, uint32_t off) {
    using V = typename VecT<VEC>::T;
    if constexpr (BUF)
        return load_b_buf<VEC>(rsrc, off);
    else
        return *reinterpret_cast<const V*>(reinterpret_cast<const char*>(B) + off);
}

// One wave per row chunk.  VEC floats per lane (requires O % VEC == 0 and
// B/C aligned to 4*VEC bytes, checked by the launcher); LPE lanes cover one
// B row segment of LPE*VEC columns, so one load instruction serves
// EPI = 64/LPE entries (sub-group s = lane/LPE takes entries t == s mod EPI)
// and moves 64*VEC*4 bytes, the most the vector memory pipe delivers per
// instruction.  The EPI partial sums of a lane's columns are added with
// cross-lane shuffles at the end of each column tile.
// BUF: raw buffer loads with 32-bit byte offsets (B smaller than 2 GB);
// otherwise 64-bit addresses with the entry holding the B row index.
// Columns [0, O) of B and C, whose rows are ld floats apart (ld > O for one
// column slice); partial rows are O floats.
template <int VEC, int LPE, bool BUF>
__global__ __launch_bounds__(256) void vcsr_rowmajor_kernel(
    int32_t n_items, int32_t O, int32_t ld, int32_t bundle, int32_t accumulate, uint32_t b_bytes,
    const int32_t* __restrict__ row_items, const int4* __restrict__ pair_rec,
    const int32_t* __restrict__ lcol, const float* __restrict__ val,
    const float* __restrict__ B, float* __restrict__ C, float* __restrict__ partials) {
    using V = typename VecT<VEC>::T;
    constexpr int EPI = 64 / LPE;                      // entries per load instruction
    constexpr int U = 16;                              // load instructions per block
    __shared__ uint2 list_all[kWaves][kRowChunkEntries];
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    const int32_t item = (int32_t)(xcd_remap(blockIdx.x, gridDim.x) * kWaves) + wave;
    if (item >= n_items) return;
    uint2* list = list_all[wave];
    const int32_t row = uniform(row_items[4 * item + 0]);
    const int32_t p0 = uniform(row_items[4 * item + 1]);
    const int32_t p1 = uniform(row_items[4 * item + 2]);
    const int32_t out = uniform(row_items[4 * item + 3]);
    if (accumulate && p0 == p1) return;  // empty row: nothing to add

    // Phase 1: this chunk's entries as (B-row byte offset or row index, value).
    const uint32_t row_bytes = (uint32_t)ld * 4u;
    const int32_t np = p1 - p0;  // <= 64 by construction
    int32_t cnt = 0, slot0 = 0, seg = 0;
    if (lane < np) {
        const int4 rec = pair_rec[p0 + lane];
        slot0 = rec.x;
        seg = rec.y;
        cnt = rec.z;
    }
    const int32_t incl = wave_inclusive_scan(cnt, lane);
    const int32_t total = uniform(__shfl(incl, 63));  // <= kRowChunkEntries
    const int32_t pos = incl - cnt;
    for (int32_t d = 0; d < cnt; ++d) {
        const int64_t s = (int64_t)slot0 + (int64_t)d * bundle;
        const uint32_t brow = (uint32_t)(seg + lcol[s]);
        list[pos + d] = make_uint2(BUF ? brow * row_bytes : brow,
                                   __builtin_bit_cast(uint32_t, val[s]));
    }
    wave_sync();

    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), (short)0, (int)b_bytes,
                                          kRawBufferFlags);
    const int sub = lane / LPE, kl = lane % LPE;
    // Phase 2: per column tile, stream the list in blocks of U load
    // instructions, all issued before the block's FMAs.  Instructions past
    // the end of the list are skipped by a wave-uniform branch; lanes past it
    // within the last instruction are masked.
    const int32_t ninstr = (total + EPI - 1) / EPI;
    for (int32_t k0 = 0; k0 < O; k0 += LPE * VEC) {
        const int32_t k = k0 + kl * VEC;
        const bool kok = k < O;
        // Lanes past O read data of no use (buffer path: range-checked;
        // 64-bit path: clamped to column 0) and never store.
        const uint32_t koff = (uint32_t)((kok || BUF) ? k : 0) * 4u;
        V acc = zero_vec(V());
        auto load_entry = [&](int32_t t, V& b, float& a) {
            const uint2 e = list[t];
            a = __builtin_bit_cast(float, e.y);
            if constexpr (BUF)
                b = load_b<VEC, true>(rsrc, B, e.x + koff);
            else
                b = *reinterpret_cast<const V*>(B + (int64_t)e.x * ld + koff / 4);
        };
        // Full blocks: every sub-group has an entry in each instruction.
        const int32_t nfull = (total / EPI) / U * U;
        for (int32_t i0 = 0; i0 < nfull; i0 += U) {
            V b[U];
            float a[U];
#pragma unroll
            for (int u = 0; u < U; ++u) load_entry((i0 + u) * EPI + sub, b[u], a[u]);
#pragma unroll
            for (int u = 0; u < U; ++u) fma_vec(acc, a[u], b[u]);
        }
        // Tail: fewer than U instructions, the last one possibly partial.
        if (nfull < ninstr) {
            V b[U];
            float a[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                a[u] = 0.f;
                b[u] = zero_vec(V());
                const int32_t t = (nfull + u) * EPI + sub;
                if (t < total) load_entry(t, b[u], a[u]);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) fma_vec(acc, a[u], b[u]);
        }
#pragma unroll
        for (int sh = LPE; sh < 64; sh <<= 1) acc = add_vec(acc, shfl_xor_vec(acc, sh));
        if (sub != 0 || !kok) continue;
        if (out < 0) {
            V* dst = reinterpret_cast<V*>(C + (int64_t)row * ld + k);
            *dst = accumulate ? add_vec(*dst, acc) : acc;
        } else {
            *reinterpret_cast<V*>(partials + (int64_t)out * O + k) = acc;
        }
    }
}

// Sums the chunk partials of the split rows into C (one wave per split row
// and 64*VEC-column tile).
template <int VEC>
__global__ __launch_bounds__(256) void vcsr_rowmajor_reduce(int32_t n_units, int32_t nkt,
                                                            int32_t O, int32_t ld,
                                                            int32_t accumulate,
                                                            const int32_t* __restrict__ split_rows,
                                                            const float* __restrict__ partials,
                                                            float* __restrict__ C) {
    using V = typename VecT<VEC>::T;
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    const int32_t unit = (int32_t)(blockIdx.x * kWaves) + wave;
    if (unit >= n_units) return;
    const int32_t item = unit / nkt, kt = unit - item * nkt;
    const int32_t row = split_rows[3 * item], q0 = split_rows[3 * item + 1],
                  nq = split_rows[3 * item + 2];
    const int32_t k = kt * 64 * VEC + lane * VEC;
    if (k >= O) return;
    V acc = zero_vec(V());
    for (int32_t q = 0; q < nq; ++q)
        acc = add_vec(acc, *reinterpret_cast<const V*>(partials + (int64_t)(q0 + q) * O + k));
    V* dst = reinterpret_cast<V*>(C + (int64_t)row * ld + k);
    *dst = accumulate ? add_vec(*dst, acc) : acc;
}

template <int VEC, int LPE, bool BUF>
hipError_t launch_one(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O, int32_t ld,
                      float* C, int32_t accumulate, uint32_t b_bytes, float* partials,
                      hipStream_t st) {
    const dim3 grid((unsigned)((d.n_row_items + kWaves - 1) / kWaves)), block(64 * kWaves);
    hipLaunchKernelGGL((vcsr_rowmajor_kernel<VEC, LPE, BUF>), grid, block, 0, st, d.n_row_items,
                       O, ld, v.bundle, accumulate, b_bytes, d.row_items,
                       reinterpret_cast<const int4*>(d.pair_rec), d.lcol, d.val, B, C, partials);
    return hipGetLastError();
}

// Columns [0, O) of B and C, whose rows are ld floats apart.
template <int VEC>
hipError_t launch_vec(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O, int32_t ld,
                      float* C, int32_t accumulate, float* partials, hipStream_t st) {
    if (d.n_row_items > 0) {
        // Bytes from B to the end of its last row.
        const uint64_t b_bytes =
            v.N > 0 ? ((uint64_t)(v.N - 1) * (uint64_t)ld + (uint64_t)O) * 4u : 0u;
        hipError_t e;
        if (b_bytes + 64u * 4u * (uint64_t)VEC >= (uint64_t)kBufferLimit) {
            e = launch_one<VEC, 64, false>(v, d, B, O, ld, C, accumulate, 0u, partials, st);
        } else {
            // Lanes per entry: the smallest power of two covering O.
            const int32_t need = (O + VEC - 1) / VEC;
            const uint32_t bb = (uint32_t)b_bytes;
            if (need <= 1) e = launch_one<VEC, 1, true>(v, d, B, O, ld, C, accumulate, bb, partials, st);
            else if (need <= 2) e = launch_one<VEC, 2, true>(v, d, B, O, ld, C, accumulate, bb, partials, st);
            else if (need <= 4) e = launch_one<VEC, 4, true>(v, d, B, O, ld, C, accumulate, bb, partials, st);
            else if (need <= 8) e = launch_one<VEC, 8, true>(v, d, B, O, ld, C, accumulate, bb, partials, st);
            else if (need <= 16) e = launch_one<VEC, 16, true>(v, d, B, O, ld, C, accumulate, bb, partials, st);
            else if (need <= 32) e = launch_one<VEC, 32, true>(v, d, B, O, ld, C, accumulate, bb, partials, st);
            else e = launch_one<VEC, 64, true>(v, d, B, O, ld, C, accumulate, bb, partials, st);
        }
        if (e != hipSuccess) return e;
    }
    if (d.n_split > 0) {
        const int32_t nkt = (O + 64 * VEC - 1) / (64 * VEC);
        const int64_t ru = (int64_t)d.n_split * nkt;
        if (ru > INT32_MAX) return hipErrorInvalidValue;
        hipLaunchKernelGGL(vcsr_rowmajor_reduce<VEC>, dim3((unsigned)((ru + kWaves - 1) / kWaves)),
                           dim3(64 * kWaves), 0, st, (int32_t)ru, nkt, O, ld, accumulate,
                           d.split_rows, partials, C);
        return hipGetLastError();
    }
    return hipSuccess;
}

// Column-slice width of a launch over O columns: all of them, or slices of
// kRowSliceCols when rows are split (their partial rows are one slice wide,
// so the scratch sized at upload covers every O).
int32_t row_slice_width(const DeviceFmt& d, int32_t O) {
    return d.n_split > 0 ? std::min(O, kRowSliceCols) : O;
}

}  // namespace

int64_t rowmajor_partials_floats(const DeviceFmt& d, int32_t O) {
    if (O <= 0 || d.n_partials == 0) return 0;
    return (int64_t)d.n_partials * row_slice_width(d, O);
}

hipError_t launch_vcsr_rowmajor(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                                float* C, int32_t accumulate, float* partials, hipStream_t st) {
    if (O <= 0 || v.M == 0) return hipSuccess;
    const bool a16 = (((uintptr_t)B | (uintptr_t)C) & 15u) == 0;
    const bool a8 = (((uintptr_t)B | (uintptr_t)C) & 7u) == 0;
    // Slices start at multiples of kRowSliceCols floats, so they keep the
    // alignment of B and C.
    const int32_t width = row_slice_width(d, O);
    for (int32_t c0 = 0; c0 < O; c0 += width) {
        const int32_t w = std::min(width, O - c0);
        hipError_t e;
        if (w % 4 == 0 && O % 4 == 0 && a16)
            e = launch_vec<4>(v, d, B + c0, w, O, C + c0, accumulate, partials, st);
        else if (w % 2 == 0 && O % 2 == 0 && a8)
            e = launch_vec<2>(v, d, B + c0, w, O, C + c0, accumulate, partials, st);
        else
            e = launch_vec<1>(v, d, B + c0, w, O, C + c0, accumulate, partials, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace vcsr
