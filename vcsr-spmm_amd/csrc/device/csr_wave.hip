// csr_wave.hip - wave-per-row CSR SpMM on plain CSR arrays, the ASpT-style
// competitor (src/aspt.cu:38-142): rows are spread over the lanes of a
// wavefront, each row's (column, value) pairs are read once by the lanes and
// shared with the row's other lanes, every lane accumulates its columns of
// C in registers, and C is written once (C = A*B).  No format build.
//
// gfx950 form: a row is a stream of LPE lanes holding VEC consecutive
// columns each (16-byte B loads when O allows), so a wave computes
// S = 64/LPE rows at once; the reference's warp computes one row per
// 64-column chunk with 4-byte loads and needs O % 64 == 0, this kernel takes
// any O.  A stream stages LPE of its row's entries at a time (B-row byte
// offset and value) in the wave's LDS and applies them in blocks of U loads
// issued back to back; B is read with raw buffer loads whose range check
// returns zeros for lanes past the row's end or past O.
#include "common.hpp"
#include "launch.hpp"
#include "vecops.hpp"

namespace vcsr {
namespace {

constexpr int kWaveRowsWaves = 4;
constexpr uint32_t kNoCol = 0x80000000u;  // buffer offset past any B on the buffer path

template <int VEC, int LPE, bool BUF>
__global__ __launch_bounds__(256) void csr_wave_kernel(int32_t M, int32_t N, int32_t O,
                                                       uint32_t b_bytes,
                                                       const int32_t* __restrict__ rowptr,
                                                       const int32_t* __restrict__ col,
                                                       const float* __restrict__ val,
                                                       const float* __restrict__ B,
                                                       float* __restrict__ C) {
    using V = typename VecT<VEC>::T;
    constexpr int S = 64 / LPE;  // rows per wave
    constexpr int U = 8;         // loads per block
    __shared__ uint32_t s_off[kWaveRowsWaves][64];
    __shared__ float s_val[kWaveRowsWaves][64];

    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63), sub = lane / LPE, kl = lane % LPE;
    const int64_t w = (int64_t)xcd_remap(blockIdx.x, gridDim.x) * kWaveRowsWaves + wave;
    const int64_t row = w * S + sub;
    if (w * S >= M) return;
    const bool rowok = row < M;
    const int32_t p0 = rowok ? rowptr[row] : 0, n = rowok ? rowptr[row + 1] - p0 : 0;
    int32_t nmax = n;
#pragma unroll
    for (int sh = LPE; sh < 64; sh <<= 1) nmax = max(nmax, __shfl_xor(nmax, sh));
    nmax = uniform(nmax);
    uint32_t* lo = s_off[wave];
    float* lv = s_val[wave];
    const uint32_t row_bytes = (uint32_t)O * 4u;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), (short)0, (int)b_bytes,
                                          kRawBufferFlags);

    for (int32_t k0 = 0; k0 < O; k0 += LPE * VEC) {
        const int32_t k = k0 + kl * VEC;
        const bool kok = k < O;
        const uint32_t koff = (uint32_t)(kok ? k : 0) * 4u;
        V acc = zero_vec(V());
        for (int32_t c0 = 0; c0 < nmax; c0 += LPE) {
            // Stage this stream's entries c0 .. c0+LPE-1 (lane kl takes one);
            // a column outside [0, N) reads nothing.
            const int32_t i = c0 + kl;
            const int32_t cj = i < n ? col[p0 + i] : -1;
            const bool ok = (uint32_t)cj < (uint32_t)N;
            lo[lane] = ok ? (BUF ? (uint32_t)cj * row_bytes : (uint32_t)cj) : kNoCol;
            lv[lane] = ok ? val[p0 + i] : 0.f;
            wave_sync();
            const int32_t cnt = min(LPE, nmax - c0);
            for (int32_t j0 = 0; j0 < cnt; j0 += U) {
                V b[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int32_t j = min(j0 + u, LPE - 1);
                    const uint32_t off = lo[sub * LPE + j];
                    if constexpr (BUF) {
                        // off + koff < 2^32 (off <= 2^31, koff < 2^31); lanes
                        // past O or past the chunk read "no column" zeros.
                        b[u] = load_b_buf<VEC>(
                            rsrc, (off + koff) | (kok && j0 + u < cnt ? 0u : kNoCol));
                    } else {
                        const bool live = off != kNoCol && kok && j0 + u < cnt;
                        b[u] = live ? *reinterpret_cast<const V*>(B + (int64_t)off * O + k)
                                    : zero_vec(V());
                    }
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int32_t j = min(j0 + u, LPE - 1);
                    const float a = j0 + u < cnt ? lv[sub * LPE + j] : 0.f;
                    fma_vec(acc, a, b[u]);
                }
            }
            wave_sync();
        }
        if (rowok && kok) *reinterpret_cast<V*>(C + row * O + k) = acc;
    }
}

template <int VEC, int LPE>
hipError_t launch_lpe(int32_t M, const int32_t* rowptr, const int32_t* col, const float* val,
                      const float* B, int32_t N, int32_t O, float* C, hipStream_t st) {
    constexpr int S = 64 / LPE;
    const int64_t waves = ((int64_t)M + S - 1) / S;
    const dim3 grid((unsigned)((waves + kWaveRowsWaves - 1) / kWaveRowsWaves)),
        block(64 * kWaveRowsWaves);
    const uint64_t b_bytes = (uint64_t)N * (uint64_t)O * 4u;
    if (b_bytes + 64u * 4u * VEC >= kBufferLimit)
        hipLaunchKernelGGL((csr_wave_kernel<VEC, LPE, false>), grid, block, 0, st, M, N, O, 0u,
                           rowptr, col, val, B, C);
    else
        hipLaunchKernelGGL((csr_wave_kernel<VEC, LPE, true>), grid, block, 0, st, M, N, O,
                           (uint32_t)b_bytes, rowptr, col, val, B, C);
    return hipGetLastError();
}

template <int VEC>
hipError_t launch_vec(int32_t M, const int32_t* rowptr, const int32_t* col, const float* val,
                      const float* B, int32_t N, int32_t O, float* C, hipStream_t st) {
    const int32_t need = (O + VEC - 1) / VEC;
    if (need <= 8) return launch_lpe<VEC, 8>(M, rowptr, col, val, B, N, O, C, st);
    if (need <= 16) return launch_lpe<VEC, 16>(M, rowptr, col, val, B, N, O, C, st);
    if (need <= 32) return launch_lpe<VEC, 32>(M, rowptr, col, val, B, N, O, C, st);
    return launch_lpe<VEC, 64>(M, rowptr, col, val, B, N, O, C, st);
}

}  // namespace

hipError_t launch_csr_wave(int32_t M, const int32_t* rowptr, const int32_t* col, const float* val,
                           const float* B, int32_t N, int32_t O, float* C, hipStream_t st) {
    if (M <= 0 || O <= 0) return hipSuccess;
    const bool a16 = (((uintptr_t)B | (uintptr_t)C) & 15u) == 0;
    const bool a8 = (((uintptr_t)B | (uintptr_t)C) & 7u) == 0;
    if (O % 4 == 0 && a16) return launch_vec<4>(M, rowptr, col, val, B, N, O, C, st);
    if (O % 2 == 0 && a8) return launch_vec<2>(M, rowptr, col, val, B, N, O, C, st);
    return launch_vec<1>(M, rowptr, col, val, B, N, O, C, st);
}

}  // namespace vcsr
