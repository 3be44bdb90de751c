// vcsr_tile.hip - tile-stationary SpMM over the VCSR slots (gfx950).
//
// The arithmetic is the VCSR one: every nonzero is a packed slot s of the
// format, contributing val[s] * B[seg_base + lcol[s], :] to its row.  The
// schedule is the one that suits MI355X: a wavefront owns whole C rows and
// writes them once with plain stores (no FP32 atomics, which cost about ten
// plain stores each here), and rows that share columns are processed
// together as a tile, so each B row slice is loaded once per tile and
// applied to up to R rows held in registers.  On block-structured matrices
// (FEM: the rows of a node's block row have the same columns) this divides
// the B-row traffic through the vector memory pipe, the limiting resource of
// a row-stationary SpMM, by the block height.
//
// Work item (one wave): MERGE consecutive work items of the view, each a run
// of tile pieces with at most tile_piece_entries(R) entries
// (host/tile_view.hpp).
// Phase 1 (lane per entry): read the entry's B row and R values (the view
// stores the values of its slots next to each other, for 1- and 3-row tiles
// in one record with the B row, so these are coalesced loads, not gathers
// from the VCSR value array) and stage (B-row byte offset, values) in the
// wave's LDS list.
// Phase 2, per column tile of LPE*VEC columns: the wave is S = 64/LPE
// streams of LPE lanes; one load instruction serves one entry of every
// stream.
//  - Several pieces: each stream takes a contiguous run of whole pieces
//    (balanced by entry count), accumulates the piece's R rows and stores
//    them when its last entry has been applied.  No cross-lane reduction.
//    Single-row tiles with several work items per wave instead give every
//    stream an equal run of entries; a piece cut between runs is finished
//    by the stream that began it, from the later streams' partial sums in
//    LDS.
//  - One piece (a long tile): the streams interleave over its entries, whose
//    list is padded to whole blocks, and their sums are added with
//    cross-lane shuffles before the store.
// Loads are issued in blocks of U back to back before the block's FMAs; B is
// read with raw buffer loads whose range check turns out-of-range offsets
// into zeros, so inactive lanes and placeholder entries need no branch.
// Rows absent from an entry are updated with a zero value (no per-row
// select); this is exact for finite B.  A piece of a taller tile (or of any
// tile off the buffer path) whose sum comes out non-finite is recomputed
// with the presence bits (read from global memory on that rare path) before
// it is stored, so inf / NaN in B reach exactly the rows the reference's
// loop reaches; single-row tiles on the buffer path need no such check.
//
// The host launcher runs one launch per column slice of at most 256
// columns (128 when B is over 512 MB) for 16-byte vectors, and for any
// vector width when tiles are split (their partial rows are one slice
// wide); tiles of 16 rows go to the MFMA kernel further down.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "../host/tile_view.hpp"
#include "common.hpp"
#include "launch.hpp"
#include "vecops.hpp"

namespace vcsr {
namespace {

// Waves per block of the VALU tile kernel: 2 (1.5% faster than 4 on the
// banded matrix — a freed wave slot waits less for a whole block to fit).
constexpr int kWaves = 2;
// Buffer offset of "no B row": at least 2^31, above any buffer-path B size,
// and still below 2^32 after adding a column offset (< 2^31).
constexpr uint32_t kNoRow = 0x80000000u;
// Compute units of a device (256 on MI355X), read once per device.
int device_cus(int device) {
    static std::atomic<int> cus[64];
    if (device < 0 || device >= 64) return 256;
    int n = cus[device].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[device].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Column slices (launch_vcsr_tile): at most kTileWideCols columns per
// launch, and kTileSliceCols when B is over twice the MALL's 256 MB.
constexpr int32_t kTileWideCols = 256;
constexpr int32_t kTileSliceCols = 128;
constexpr uint64_t kTileSliceBytes = 512ull << 20;

template <int R>
__device__ __forceinline__ void store_vals(float* p, const float (&a)[R]) {
    if constexpr (R == 1) {
        p[0] = a[0];
    } else if constexpr (R == 2) {
        *reinterpret_cast<float2*>(p) = make_float2(a[0], a[1]);
    } else {
#pragma unroll
        for (int q = 0; q < R; q += 4)
            *reinterpret_cast<float4*>(p + q) = make_float4(a[q], a[q + 1], a[q + 2], a[q + 3]);
    }
}

template <int R>
__device__ __forceinline__ void load_vals(const float* p, float (&a)[R]) {
    if constexpr (R == 1) {
        a[0] = p[0];
    } else if constexpr (R == 2) {
        const float2 x = *reinterpret_cast<const float2*>(p);
        a[0] = x.x;
        a[1] = x.y;
    } else {
#pragma unroll
        for (int q = 0; q < R; q += 4) {
            const float4 x = *reinterpret_cast<const float4*>(p + q);
            a[q] = x.x;
            a[q + 1] = x.y;
            a[q + 2] = x.z;
            a[q + 3] = x.w;
        }
    }
}

// z + x * 0 for every component of x, as fused multiply-adds (no rounding:
// x * 0 is a signed zero for finite x, NaN otherwise).
__device__ __forceinline__ float fma_zero_acc(float x, float z) { return __builtin_fmaf(x, 0.f, z); }
__device__ __forceinline__ float fma_zero_acc(float2 x, float z) {
    return __builtin_fmaf(x.y, 0.f, __builtin_fmaf(x.x, 0.f, z));
}
__device__ __forceinline__ float fma_zero_acc(float4 x, float z) {
    return __builtin_fmaf(x.w, 0.f, __builtin_fmaf(x.z, 0.f, __builtin_fmaf(x.y, 0.f,
                          __builtin_fmaf(x.x, 0.f, z))));
}

// Compile-time shape of the per-wave LDS of the VALU tile kernel.
template <int VEC, int LPE, int R, int MERGE>
struct TileShape {
    static constexpr int S = 64 / LPE;                          // streams per wave
    static constexpr int RS = tile_slot_stride(R);              // slots stored per entry
    static constexpr int EMAX = tile_piece_entries(R) * MERGE;  // entries per wave
    static constexpr int PMAX = kTileChunkPieces * MERGE;       // pieces per wave
    // Loads per block: 8, or 4 when 8+ streams split a tall tile's entries
    // (fewer padded entries per block: banded 62K matrix, O = 8 / 32, 3%
    // faster; single-row tiles, which merge four items, measured slower).
    static constexpr int U = (S >= 8 && R > 1) ? 4 : 8;
    // A one-piece item's list is padded with "no row" entries of value 0 up
    // to a multiple of S*UT, so that its blocks are full blocks of U loads
    // per stream and at most one each of U/2, U/4, ... UT (UT = 2).
    static constexpr int UT = U >= 2 ? 2 : U;
    static constexpr int EPAD = (EMAX + S * U - 1) / (S * U) * (S * U);
    // Single-row tiles with several work items per wave: each stream takes
    // an equal run of the wave's entries, cutting pieces where the runs
    // meet (the piece's owner adds the other streams' partial sums after the
    // loop).  Whole pieces per stream leave most streams idle behind a long
    // row's piece: power-law 322K matrix, O = 8 / 32, 41% of the B-load
    // slots busy against 84%, 37.1 / 46.1 against 30.0 / 40.1 us.  A stream
    // that ends a piece begun in an earlier run writes its partial sum to
    // LDS at once (held in registers, the 16-byte-vector build kept it on
    // the stack and ran 1.7x slower).
    static constexpr bool EQ = R == 1 && MERGE > 1;
};

// One wave's LDS: staged entries (B-row byte offsets and values), the piece
// table with its end sentinels, per-piece "not finite" flags and the streams'
// first pieces.
template <int VEC, int LPE, int R, int MERGE>
struct TileLds {
    using Sh = TileShape<VEC, LPE, R, MERGE>;
    __align__(16) float val[Sh::EPAD * Sh::RS];
    // Equal-run streams: per lane, the partial sum of the piece open at its
    // stream's first entry, and per stream that piece (-1: none).
    typename VecT<VEC>::T xs[Sh::EQ ? 64 * R : 1];
    int32_t headp[Sh::EQ ? Sh::S : 1];
    uint32_t brow[Sh::EPAD];
    int4 piece[Sh::PMAX + 2];
    int32_t first[Sh::S + 1];
    uint8_t bad[Sh::PMAX];
};

// Work items c0 .. c1 (MERGE consecutive items of the view, fewer at the end)
// on one wave.  BUF: B smaller than 2 GB, read with raw buffer loads at
// 32-bit byte offsets; otherwise 64-bit addresses from B row indices
// (LPE = 64 only).
template <int VEC, int LPE, int R, int MERGE, bool BUF>
__device__ __forceinline__ void tile_item(
    int32_t c0, int32_t c1, int lane, TileLds<VEC, LPE, R, MERGE>& L, int32_t O, int32_t ld,
    int32_t accumulate, uint32_t b_bytes, const int4* __restrict__ chunks,
    const int4* __restrict__ pieces, const int32_t* __restrict__ ent_brow,
    const uint16_t* __restrict__ ent_mask, const float* __restrict__ ent_val,
    const float* __restrict__ B, float* __restrict__ C, float* __restrict__ partials) {
    using V = typename VecT<VEC>::T;
    using Sh = TileShape<VEC, LPE, R, MERGE>;
    constexpr int S = Sh::S;
    constexpr int RS = Sh::RS;
    constexpr bool FOLD = tile_dev_folds_brow(R);            // B row inside the values
    constexpr int DS = tile_dev_stride(R);                   // floats per entry in ent_val
    constexpr int U = Sh::U;
    constexpr int UT = Sh::UT;
    // Pieces are checked for non-finite sums (and recomputed with the
    // presence bits) because a tile row absent from an entry gets 0 * b,
    // NaN for an infinite b, and because placeholders read B row 0 off the
    // buffer path.  Single-row tiles on the buffer path have neither: every
    // entry is present in its row and placeholders load zeros, so their sums
    // are already the reference's (power-law 322K matrix, O = 8 / 32: 7% /
    // 5% faster without the check at each piece end).
    constexpr bool CHECK = !(R == 1 && BUF);
    uint32_t* lb = L.brow;
    uint8_t* lbad = L.bad;
    float* lv = L.val;
    int4* lp = L.piece;
    int32_t* lf = L.first;
    const int32_t e0 = uniform(chunks[c0].x), ne = uniform(chunks[c1].y) - e0;  // <= EMAX
    const int32_t p0 = uniform(chunks[c0].z), np = uniform(chunks[c1].w) - p0;  // <= PMAX

    // Phase 1: stage the entries (and a one-piece item's padding, buffer
    // path) and the piece table.
    const uint32_t row_bytes = (uint32_t)ld * 4u;
    const bool pad = BUF && np == 1;
    const int32_t ne_pad = pad ? (ne + S * UT - 1) / (S * UT) * (S * UT) : ne;  // <= EPAD
    for (int32_t i = lane; i < ne_pad; i += 64) {
        uint32_t br = (uint32_t)kTileNoEntry;
        float a[RS];
        if (i < ne) {
            const int64_t e = (int64_t)e0 + i;
            if constexpr (FOLD) {
                // One load: the values, then the B row's bits (for 3 rows in
                // the padding slot, which the FMAs never read).
                float rec[DS];
                load_vals<DS>(ent_val + e * DS, rec);
                br = __builtin_bit_cast(uint32_t, rec[DS - 1]);
#pragma unroll
                for (int q = 0; q < RS; ++q) a[q] = rec[q];
            } else {
                br = (uint32_t)ent_brow[e];
                load_vals<RS>(ent_val + e * RS, a);
            }
        } else {
#pragma unroll
            for (int q = 0; q < RS; ++q) a[q] = 0.f;
        }
        // Placeholders: "no row" on the buffer path, else row 0 times 0.
        const bool real = br != (uint32_t)kTileNoEntry;
        const uint32_t off = BUF ? (real ? br * row_bytes : kNoRow) : (real ? br : 0u);
        lb[i] = off;
        // 3-row tiles: the offset also goes into the padding slot of the
        // entry's 4-float value record (the FMAs never read that slot), so
        // the one-piece loop reads each entry with one 16-byte LDS read.
        if constexpr (RS > R) a[RS - 1] = __builtin_bit_cast(float, off);
        store_vals<RS>(lv + i * RS, a);
    }
    if (np > 1) {
        for (int32_t j = lane; j < np; j += 64) {
            int4 pc = pieces[p0 + j];
            pc.z -= e0;
            lp[j] = pc;
            lbad[j] = 0;
        }
        if (lane < 2) lp[np + lane] = make_int4(0, 0, ne, -1);  // end sentinels
    }
    wave_sync();

    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), (short)0, (int)b_bytes,
                                          kRawBufferFlags);
    const int sub = lane / LPE, kl = lane % LPE;

    // One entry's B slice; zeros for "no row" (placeholders, lanes past the
    // end) on the buffer path.  The offset is read for every lane (tc is a
    // valid index) and lanes past the end get the "no row" bit ORed in, so
    // the tail blocks issue their loads back to back like the full ones (a
    // conditional read becomes a branch and an LDS wait per load).
    auto load_b = [&](int32_t tc, bool ok, uint32_t koff) -> V {
        if constexpr (BUF) {
            const uint32_t off = (lb[tc] + koff) | (ok ? 0u : kNoRow);
            return load_b_buf<VEC>(rsrc, off);
        } else {
            const V b = *reinterpret_cast<const V*>(B + (int64_t)lb[tc] * ld + koff / 4);
            return ok ? b : zero_vec(V());
        }
    };
    // acc[r] += a[r] * b for every tile row; absent rows have a[r] = 0, which
    // is exact while b is finite.  A non-finite b reaching an absent row
    // (0 * inf = NaN) shows up as a non-finite row sum at the store, and the
    // piece is then recomputed with the presence bits (redo_piece).
    auto apply = [&](V (&acc)[R], int32_t tc, bool ok, const V& b) {
        float a[RS];
        load_vals<RS>(lv + tc * RS, a);
#pragma unroll
        for (int r = 0; r < R; ++r) fma_vec(acc[r], ok ? a[r] : 0.f, b);
    };
    // Whether every accumulator of this lane is finite (lanes past O hold
    // nothing to store).  z = fma(x, 0, z) over all of them stays finite
    // exactly when every x is (x * 0 is NaN for inf and NaN).  Rows absent
    // from the piece are included: their sums are zero for finite B, so this
    // can only send a piece to the exact recomputation more often.
    auto piece_finite = [&](const V (&acc)[R], bool kok) -> bool {
        float z = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) z = fma_zero_acc(acc[r], z);
        return __builtin_isfinite(z) || !kok;
    };
    // Writes the accumulated rows of piece pc (its first pc.y rows exist) to
    // C or to its partial rows.
    auto store_piece = [&](const int4 pc, const V (&acc)[R], int32_t k, bool kok) {
        if (!kok) return;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r >= pc.y) break;
            if (pc.w < 0) {
                V* dst = reinterpret_cast<V*>(C + (int64_t)(pc.x + r) * ld + k);
                store_nt(dst, accumulate ? add_vec(*dst, acc[r]) : acc[r]);
            } else {
                *reinterpret_cast<V*>(partials + (int64_t)(pc.w + r) * O + k) = acc[r];
            }
        }
    };
    // Exact recomputation of piece pc (entries tb .. te-1) in entry order,
    // skipping absent rows (taken only for pieces whose sum is not finite,
    // which were not stored).
    auto redo_piece = [&](const int4 pc, int32_t tb, int32_t te, int32_t k, uint32_t koff,
                          bool kok) {
        V acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = zero_vec(V());
        for (int32_t t = tb; t < te; ++t) {
            const V b = load_b(t, true, koff);
            float a[RS];
            load_vals<RS>(lv + t * RS, a);
            const uint32_t m = ent_mask[(int64_t)e0 + t];
#pragma unroll
            for (int r = 0; r < R; ++r)
                if ((m >> r) & 1u) fma_vec(acc[r], a[r], b);
        }
        store_piece(pc, acc, k, kok);
    };

    if (np > 1) {
        int32_t pa, pb, tb, te;  // this stream's pieces and entries
        if constexpr (Sh::EQ) {
            // Entries tb .. te-1, and pa the piece holding entry tb (the
            // last piece starting at or before it; pieces are not empty).
            tb = (sub * ne) / S;
            te = ((sub + 1) * ne) / S;
            int32_t lo = 0, hi = np - 1;
            while (lo < hi) {
                const int32_t mid = (lo + hi + 1) >> 1;
                if (lp[mid].z <= tb) lo = mid;
                else hi = mid - 1;
            }
            pa = lo;
            pb = pa;  // set after the loop: the first piece not completed
        } else {
            // Stream s takes the pieces whose entry midpoint falls in the s-th
            // S-quantile of the item: first piece lf[s], end piece lf[s + 1].
            if (lane <= S) {
                int32_t lo = 0, hi = np;
                while (lo < hi) {
                    const int32_t mid = (lo + hi) >> 1;
                    const int32_t sm = ((lp[mid].z + lp[mid + 1].z) * S) / (2 * ne);
                    if (sm < lane) lo = mid + 1;
                    else hi = mid;
                }
                lf[lane] = lo;
            }
            wave_sync();
            pa = lf[sub];
            pb = lf[sub + 1];
            tb = lp[pa].z;
            te = lp[pb].z;
        }
        // Equal runs: piece pa began in an earlier stream's run; this stream
        // only contributes a partial sum to it.
        const bool carry = Sh::EQ && lp[pa].z < tb;
        // Lanes of this lane's stream, for ballots.
        const uint64_t smask =
            LPE == 64 ? ~0ull : (((1ull << (LPE & 63)) - 1ull) << ((sub * LPE) & 63));
        int32_t nmax = te - tb, nmin = te - tb;
#pragma unroll
        for (int sh = LPE; sh < 64; sh <<= 1) {
            nmax = max(nmax, __shfl_xor(nmax, sh));
            nmin = min(nmin, __shfl_xor(nmin, sh));
        }
        nmax = uniform(nmax);
        nmin = uniform(nmin);
        for (int32_t k0 = 0; k0 < O; k0 += LPE * VEC) {
            const int32_t k = k0 + kl * VEC;
            const bool kok = k < O;
            const uint32_t koff = (uint32_t)((kok || BUF) ? k : 0) * 4u;
            V acc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = zero_vec(V());
            int32_t p = pa, pend = lp[pa + 1].z;
            // Without the finiteness check, the row and partial row of piece
            // p are read when the piece starts, so its store waits on no LDS
            // read (power-law 322K matrix, O = 8 / 32 / 128: 2% / 3% / 0.6%).
            int32_t cur_x = lp[pa].x, cur_w = lp[pa].w;
            bool bad = false;
            auto block = [&](auto full_c, int32_t i0) {
                constexpr bool FULL = decltype(full_c)::value;
                V b[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int32_t t = tb + i0 + u;
                    const bool ok = FULL || t < te;
                    b[u] = load_b(ok ? t : 0, ok, koff);
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int32_t t = tb + i0 + u;
                    const bool ok = FULL || t < te;
                    apply(acc, ok ? t : 0, ok, b[u]);
                    if (ok && t + 1 == pend) {
                        if (carry && p == pa) {
                            // The end of a piece begun in an earlier run: its
                            // owner adds this partial sum after the loop.
#pragma unroll
                            for (int r = 0; r < R; ++r) L.xs[lane * R + r] = acc[r];
                        } else if constexpr (CHECK) {
                            // A stream stores a piece only if all its lanes'
                            // sums are finite; otherwise redo_piece computes
                            // and stores it after the loop.
                            const uint64_t bm = __ballot(!piece_finite(acc, kok));
                            if ((bm & smask) != 0) {
                                bad = true;
                                lbad[p] = 1;
                            } else {
                                store_piece(lp[p], acc, k, kok);
                            }
                        } else {
                            store_piece(make_int4(cur_x, 1, 0, cur_w), acc, k, kok);
                        }
#pragma unroll
                        for (int r = 0; r < R; ++r) acc[r] = zero_vec(V());
                        ++p;
                        pend = lp[p + 1].z;
                        if constexpr (!CHECK) {
                            cur_x = lp[p].x;
                            cur_w = lp[p].w;
                        }
                    }
                }
            };
            for (int32_t i0 = 0; i0 < nmax; i0 += U) {
                if (i0 + U <= nmin) block(std::true_type(), i0);
                else block(std::false_type(), i0);
            }
            if constexpr (Sh::EQ) {
                // Piece p is still open at the end of the run when it began
                // before te.  If it is piece pa begun in an earlier run, the
                // whole run was a middle part of it; otherwise this stream
                // owns it and adds the following runs' partial sums (each
                // stream's first piece and its sum up to that piece's end or
                // its run's) in stream order.
                pb = p;
                const bool open = lp[p].z < te || (te == tb && carry);
                const bool middle = open && carry && p == pa;
                if (middle) {
#pragma unroll
                    for (int r = 0; r < R; ++r) L.xs[lane * R + r] = acc[r];
                }
                if (kl == 0) L.headp[sub] = carry ? pa : -1;
                wave_sync();
                if (open && !middle) {
                    for (int32_t s2 = sub + 1; s2 < S && L.headp[s2] == p; ++s2)
#pragma unroll
                        for (int r = 0; r < R; ++r)
                            acc[r] = add_vec(acc[r], L.xs[(s2 * LPE + kl) * R + r]);
                    if constexpr (CHECK) {
                        const uint64_t bm = __ballot(!piece_finite(acc, kok));
                        if ((bm & smask) != 0) redo_piece(lp[p], lp[p].z, lp[p + 1].z, k, koff, kok);
                        else store_piece(lp[p], acc, k, kok);
                    } else {
                        store_piece(lp[p], acc, k, kok);
                    }
                }
                wave_sync();
            }
            if (__any(bad)) {
                wave_sync();
                for (int32_t q = pa; q < pb; ++q)
                    if (lbad[q]) redo_piece(lp[q], lp[q].z, lp[q + 1].z, k, koff, kok);
                wave_sync();
                for (int32_t q = pa; q < pb; ++q) lbad[q] = 0;
                wave_sync();
            }
        }
    } else {
        // One piece: entries t = sub + S*i, summed across streams at the end.
        // Its record is wave-uniform (scalar loads; no LDS table).
        const int4 pc1 = make_int4(uniform(pieces[p0].x), uniform(pieces[p0].y),
                                   uniform(pieces[p0].z) - e0, uniform(pieces[p0].w));
        const int32_t nper = (ne + S - 1) / S, nfull = ne / S;
        for (int32_t k0 = 0; k0 < O; k0 += LPE * VEC) {
            const int32_t k = k0 + kl * VEC;
            const bool kok = k < O;
            const uint32_t koff = (uint32_t)((kok || BUF) ? k : 0) * 4u;
            V acc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = zero_vec(V());
            auto block = [&](auto full_c, int32_t i0) {
                constexpr bool FULL = decltype(full_c)::value;
                V b[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int32_t t = sub + S * (i0 + u);
                    const bool ok = FULL || t < ne;
                    b[u] = load_b(ok ? t : 0, ok, koff);
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int32_t t = sub + S * (i0 + u);
                    const bool ok = FULL || t < ne;
                    apply(acc, ok ? t : 0, ok, b[u]);
                }
            };
            if constexpr (BUF) {
                // Full blocks of U loads per stream, then one of UT if the
                // padded list has that many left.
                auto block_n = [&](auto nu_c, int32_t i0) {
                    constexpr int NU = decltype(nu_c)::value;
                    V b[NU];
                    if constexpr (RS > R) {
                        // One LDS record per entry: values and B-row offset
                        // (banded 62K matrix: O = 8 / 32 5% / 7% faster than
                        // separate offset and value reads, O = 128 2%).
                        static_assert(RS == 4, "padding slot of a 4-float record");
                        float4 rec[NU];
#pragma unroll
                        for (int u = 0; u < NU; ++u)
                            rec[u] = *reinterpret_cast<const float4*>(lv + (sub + S * (i0 + u)) * RS);
#pragma unroll
                        for (int u = 0; u < NU; ++u)
                            b[u] = load_b_buf<VEC>(rsrc, __builtin_bit_cast(uint32_t, rec[u].w) + koff);
#pragma unroll
                        for (int u = 0; u < NU; ++u)
#pragma unroll
                            for (int r = 0; r < R; ++r)
                                fma_vec(acc[r], reinterpret_cast<const float*>(&rec[u])[r], b[u]);
                    } else {
#pragma unroll
                        for (int u = 0; u < NU; ++u) b[u] = load_b(sub + S * (i0 + u), true, koff);
#pragma unroll
                        for (int u = 0; u < NU; ++u) apply(acc, sub + S * (i0 + u), true, b[u]);
                    }
                };
                const int32_t nper_pad = ne_pad / S;
                int32_t i0 = 0;
                for (; i0 + U <= nper_pad; i0 += U) block_n(std::integral_constant<int, U>(), i0);
                if constexpr (U / 2 >= UT) {
                    if (i0 + U / 2 <= nper_pad) {
                        block_n(std::integral_constant<int, U / 2>(), i0);
                        i0 += U / 2;
                    }
                }
                if constexpr (U / 4 >= UT) {
                    if (i0 + U / 4 <= nper_pad) block_n(std::integral_constant<int, U / 4>(), i0);
                }
            } else {
                for (int32_t i0 = 0; i0 < nper; i0 += U) {
                    if (i0 + U <= nfull) block(std::true_type(), i0);
                    else block(std::false_type(), i0);
                }
            }
#pragma unroll
            for (int sh = LPE; sh < 64; sh <<= 1) {
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = add_vec(acc[r], shfl_xor_vec(acc[r], sh));
            }
            // The butterfly leaves every stream the same sums (each step adds
            // the same two values in either order), so stream s stores rows
            // s, s + S, ...: one store instruction per S rows instead of one
            // per row (banded 62K matrix, O = 8: 9.9 -> 9.45 us).  A sum that
            // is not finite is recomputed exactly by stream 0.
            const bool bad = CHECK && !piece_finite(acc, kok);
            if (__any(bad)) {
                if (sub == 0) redo_piece(pc1, pc1.z, ne, k, koff, kok);
            } else if (kok) {
#pragma unroll
                for (int i = 0; i < (R + S - 1) / S; ++i) {
                    const int r = i * S + sub;
                    if (r < R && r < pc1.y) {
                        V x = acc[0];
#pragma unroll
                        for (int q = 1; q < R; ++q)
                            if (q == r) x = acc[q];
                        if (pc1.w < 0) {
                            V* dst = reinterpret_cast<V*>(C + (int64_t)(pc1.x + r) * ld + k);
                            store_nt(dst, accumulate ? add_vec(*dst, x) : x);
                        } else {
                            *reinterpret_cast<V*>(partials + (int64_t)(pc1.w + r) * O + k) = x;
                        }
                    }
                }
            }
        }
    }
}


// One wave per MERGE consecutive work items of the view.  Up to 3 tile rows
// (one work item per wave) the register budget is held to 5 waves per SIMD:
// measured faster than 4 on the banded workload; 6 spills, and so does 5
// with 4 rows.
template <int VEC, int LPE, int R, int MERGE, bool BUF>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu((R <= 3 && MERGE == 1) ? 5 : 1, 8)))
void vcsr_tile_kernel(
    int32_t n_chunks, int32_t O, int32_t ld, int32_t accumulate, uint32_t b_bytes,
    const int4* __restrict__ chunks, const int4* __restrict__ pieces,
    const int32_t* __restrict__ ent_brow, const uint16_t* __restrict__ ent_mask,
    const float* __restrict__ ent_val, const float* __restrict__ B, float* __restrict__ C,
    float* __restrict__ partials) {
    __shared__ TileLds<VEC, LPE, R, MERGE> s_lds[kWaves];
    // Wave-uniform indices, so the work-item records are scalar loads.
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63);
    const int32_t w = (int32_t)(xcd_remap(blockIdx.x, gridDim.x) * kWaves) + wave;
    const int32_t c0 = w * MERGE;
    if (c0 >= n_chunks) return;
    tile_item<VEC, LPE, R, MERGE, BUF>(c0, min(n_chunks, c0 + MERGE) - 1, lane, s_lds[wave], O, ld,
                                       accumulate, b_bytes, chunks, pieces, ent_brow, ent_mask,
                                       ent_val, B, C, partials);
}

// Adds the piece partials of the rows of split tiles into C.  split: {row,
// first partial row, stride, pieces}, in decreasing piece count.  Lanes
// work in groups of cl lanes (the smallest power of two covering the row's
// column vectors, at most 64): lane c of group g sums column vector c of
// partials g, g + groups, ... .
//  - The first n_heavy rows (the most pieces) take a block of 256 threads
//    each (eight loads in flight for 16-byte vectors, four otherwise: cfg3
//    O = 128 1% faster with eight, O = 8 1% slower), whose groups are added
//    in LDS, so a row split into many pieces costs a few load latencies
//    instead of one per piece.
//  - The other rows take one wave each, four per block, whose groups are
//    added with lane shuffles: no LDS and no block barrier.  Most split rows
//    have a few pieces (power-law 322K matrix: 2,740 rows, most with 2 to 8);
//    as a block each they left most of the block idle behind its barriers.
// Each row's sum has a fixed order (the same bits on every call).
template <int VEC>
__global__ __launch_bounds__(256) void vcsr_tile_reduce(int32_t O, int32_t ld, int32_t accumulate,
                                                        int32_t n_heavy, int32_t n_split,
                                                        const int4* __restrict__ split,
                                                        const float* __restrict__ partials,
                                                        float* __restrict__ C) {
    using V = typename VecT<VEC>::T;
    __shared__ V red[256];
    const int32_t nvec = (O + VEC - 1) / VEC;
    int32_t cl = 1;
    while (cl < nvec && cl < 64) cl <<= 1;
    auto part = [&](const int4& s, int32_t j, int32_t cv) {
        return *reinterpret_cast<const V*>(partials + (int64_t)s.y * O +
                                           (int64_t)j * ((int64_t)s.z * O) + (int64_t)cv * VEC);
    };
    // acc += partials g, g + groups, ... of column vector cv of row s.
    auto sum_group = [&](const int4& s, int32_t g, int32_t groups, int32_t cv, V acc) {
        int32_t j = g;
        if constexpr (VEC == 4) {
            for (; j + 7 * groups < s.w; j += 8 * groups) {
                const V x0 = part(s, j, cv), x1 = part(s, j + groups, cv);
                const V x2 = part(s, j + 2 * groups, cv), x3 = part(s, j + 3 * groups, cv);
                const V x4 = part(s, j + 4 * groups, cv), x5 = part(s, j + 5 * groups, cv);
                const V x6 = part(s, j + 6 * groups, cv), x7 = part(s, j + 7 * groups, cv);
                acc = add_vec(acc, add_vec(add_vec(add_vec(x0, x1), add_vec(x2, x3)),
                                           add_vec(add_vec(x4, x5), add_vec(x6, x7))));
            }
        }
        for (; j + 3 * groups < s.w; j += 4 * groups) {
            const V x0 = part(s, j, cv), x1 = part(s, j + groups, cv);
            const V x2 = part(s, j + 2 * groups, cv), x3 = part(s, j + 3 * groups, cv);
            acc = add_vec(acc, add_vec(add_vec(x0, x1), add_vec(x2, x3)));
        }
        for (; j < s.w; j += groups) acc = add_vec(acc, part(s, j, cv));
        return acc;
    };
    auto store = [&](const int4& s, int32_t cv, const V& x) {
        V* dst = reinterpret_cast<V*>(C + (int64_t)s.x * ld + (int64_t)cv * VEC);
        *dst = accumulate ? add_vec(*dst, x) : x;
    };
    if ((int32_t)blockIdx.x < n_heavy) {
        const int4 s = split[blockIdx.x];
        const int32_t groups = 256 / cl;
        const int32_t tid = (int32_t)threadIdx.x, c = tid % cl, g = tid / cl;
        for (int32_t c0 = 0; c0 < nvec; c0 += cl) {
            const int32_t cv = c0 + c;
            red[tid] = cv < nvec ? sum_group(s, g, groups, cv, zero_vec(V())) : zero_vec(V());
            __syncthreads();
            for (int32_t h = groups / 2; h >= 1; h >>= 1) {
                if (g < h) red[tid] = add_vec(red[tid], red[tid + h * cl]);
                __syncthreads();
            }
            if (g == 0 && cv < nvec) store(s, cv, red[tid]);
            __syncthreads();
        }
        return;
    }
    // Light rows: wave w of block b takes row n_heavy + 4 (b - n_heavy) + w.
    const int32_t i = n_heavy + ((int32_t)blockIdx.x - n_heavy) * 4 + (int32_t)(threadIdx.x >> 6);
    if (i >= n_split) return;
    const int4 s = split[i];
    const int32_t lane = (int32_t)(threadIdx.x & 63u), groups = 64 / cl;
    const int32_t c = lane % cl, g = lane / cl;
    for (int32_t c0 = 0; c0 < nvec; c0 += cl) {
        const int32_t cv = c0 + c;
        V acc = cv < nvec ? sum_group(s, g, groups, cv, zero_vec(V())) : zero_vec(V());
        for (int32_t h = cl; h < 64; h <<= 1) acc = add_vec(acc, shfl_xor_vec(acc, h));
        if (g == 0 && cv < nvec) store(s, cv, acc);
    }
}

// ---------------------------------------------------------------------------
// 16-row tiles on the matrix cores (view height kTileMmaRows).
//
// v_mfma_f32_16x16x4f32 computes D[i][j] += sum_k A[i][k] * B[k][j] for a
// 16 x 4 A and a 4 x 16 B, with A[i][k] in lane 16k + i, B[k][j] in lane
// 16k + j and D[4q + v][j] in register v of lane 16q + j (checked on the
// device).  Here A is the tile's values for four entries (k) and its 16 rows
// (i), and B the four entries' B-row slices: lane 16k + j holds VEC columns
// c0 + VEC*j .. + VEC-1 of entry k's B row, and MFMA number c takes
// component c, so D_c[i][j] is C[row i][c0 + VEC*j + c].  A group of 16
// entries is four k-steps; the view stores its values in operand order, so
// lane l reads the A operands of all four as one 16-byte load.
//
// One wave per (piece, column tile of 16*VEC columns).  The grid runs
// column-tile-major with the XCD-aware block order, so each XCD works on one
// column range of B at a time and its L2 holds that slice of B (the B rows a
// block-sparse matrix touches are spread over all of B).  B and C rows are
// ld floats apart (ld > O for one column slice of a wider product); partial
// rows are O floats.
// ---------------------------------------------------------------------------
typedef float mma_acc4 __attribute__((ext_vector_type(4)));
constexpr int kMmaWaves = 4;
constexpr int kMmaPiece = tile_piece_entries(kTileMmaRows);

template <int VEC>
__device__ __forceinline__ float vec_part(const typename VecT<VEC>::T& b, int c) {
    return reinterpret_cast<const float*>(&b)[c];
}

// GU entry groups (of 16) per block of loads.  SB: a scheduling barrier
// keeps the block's loads ahead of its MFMAs (more loads in flight per wave,
// more registers); without it the compiler interleaves them and the kernel
// fits 8 waves per SIMD.
template <int VEC, bool BUF, int GU, bool SB>
__global__ __launch_bounds__(256) void vcsr_tile_mma_kernel(
    int32_t n_items, int32_t n_ctiles, int32_t O, int32_t ld, int32_t accumulate, uint32_t b_bytes,
    const int4* __restrict__ chunks, const int4* __restrict__ pieces,
    const int32_t* __restrict__ ent_brow, const uint16_t* __restrict__ ent_mask,
    const float* __restrict__ ent_val, const float* __restrict__ B, float* __restrict__ C,
    float* __restrict__ partials) {
    using V = typename VecT<VEC>::T;
    __shared__ uint32_t s_brow[kMmaWaves][kMmaPiece];

    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63);
    const int64_t w = (int64_t)xcd_remap(blockIdx.x, gridDim.x) * kMmaWaves + wave;
    if (w >= (int64_t)n_items * n_ctiles) return;
    const int32_t ct = (int32_t)(w / n_items), item = (int32_t)(w - (int64_t)ct * n_items);
    const int32_t e0 = uniform(chunks[item].x), ne = uniform(chunks[item].y) - e0;  // 16 | ne
    const int32_t pidx = uniform(chunks[item].z);
    const int32_t row0 = uniform(pieces[pidx].x), rows = uniform(pieces[pidx].y);
    const int32_t part = uniform(pieces[pidx].w);
    uint32_t* lb = s_brow[wave];

    // Phase 1: B-row byte offsets (row indices without the buffer path) of
    // the piece's entries; placeholders get "no row".
    const uint32_t row_bytes = (uint32_t)ld * 4u;
    for (int32_t i = lane; i < ne; i += 64) {
        const uint32_t br = (uint32_t)ent_brow[e0 + i];
        const bool any = br != (uint32_t)kTileNoEntry;
        lb[i] = BUF ? (any ? br * row_bytes : kNoRow) : (any ? br : kNoRow);
    }
    wave_sync();

    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), (short)0, (int)b_bytes,
                                          kRawBufferFlags);
    const int kq = lane >> 4, jl = lane & 15;  // MFMA k index, column lane
    const int32_t col = ct * 16 * VEC + VEC * jl;
    const bool kok = col < O;
    const uint32_t koff = (uint32_t)(kok ? col : 0) * 4u;
    // Entry t's B slice for this lane; zeros for "no row" and columns past O.
    auto load_b = [&](int32_t t) -> V {
        if constexpr (BUF) {
            return load_b_buf<VEC>(rsrc, (lb[t] + koff) | (kok ? 0u : kNoRow));
        } else {
            const uint32_t br = lb[t];
            if (br == kNoRow || !kok) return zero_vec(V());
            return *reinterpret_cast<const V*>(B + (int64_t)br * ld + col);
        }
    };
    const float* vp = ent_val + (int64_t)e0 * kTileMmaRows + 4 * lane;

    mma_acc4 d[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) d[c] = mma_acc4{0.f, 0.f, 0.f, 0.f};
    auto block = [&](auto n_c, int32_t g0) {
        constexpr int NG = decltype(n_c)::value;
        float4 a[NG];
        V b[NG][4];
#pragma unroll
        for (int gu = 0; gu < NG; ++gu) {
            a[gu] = *reinterpret_cast<const float4*>(vp + (int64_t)(g0 + gu) * 256);
#pragma unroll
            for (int s = 0; s < 4; ++s) b[gu][s] = load_b(16 * (g0 + gu) + 4 * s + kq);
        }
        if constexpr (SB) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int gu = 0; gu < NG; ++gu)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int c = 0; c < VEC; ++c)
                    d[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        reinterpret_cast<const float*>(&a[gu])[s], vec_part<VEC>(b[gu][s], c), d[c],
                        0, 0, 0);
    };
    const int32_t ng = ne / kTileMmaGroup;
    int32_t g0 = 0;
    if constexpr (SB) {
        for (; g0 + GU <= ng; g0 += GU) block(std::integral_constant<int, GU>(), g0);
    } else {
        // Many waves per SIMD, all resident from the start: the SIMD issues
        // oldest first, so with equal work the first waves of a SIMD finish
        // long before its last (cfg5 O = 512: 84 us for the first of 8 against
        // 134 us for the last, slots busy 78% of the kernel).  The wave's
        // priority falls with the quarter of its groups done, so lagging
        // waves issue first: 111-127 us, slots busy 92%, the SpMM 5% faster
        // (O = 256 and 512).
        int32_t lvl = 3;
        __builtin_amdgcn_s_setprio(3);
        for (; g0 + GU <= ng; g0 += GU) {
            const int32_t nl = 3 - min(3, (4 * g0) / ng);
            if (nl != lvl) {
                lvl = nl;
                if (lvl == 2) __builtin_amdgcn_s_setprio(2);
                else if (lvl == 1) __builtin_amdgcn_s_setprio(1);
                else __builtin_amdgcn_s_setprio(0);
            }
            block(std::integral_constant<int, GU>(), g0);
        }
        __builtin_amdgcn_s_setprio(0);
    }
    for (; g0 < ng; ++g0) block(std::integral_constant<int, 1>(), g0);

    // This lane holds rows 4*kq + v of the tile, columns col .. col+VEC-1.
    bool fin = true;
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int c = 0; c < VEC; ++c)
            if (4 * kq + v < rows) fin = fin && __builtin_isfinite(d[c][v]);
    if (__any(!(fin || !kok))) {
        // A non-finite sum: recompute this lane's rows in entry order on the
        // VALU, skipping the rows an entry does not have (0 * inf must not
        // reach them), like the reference's per-row loop.
        V acc[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[v] = zero_vec(V());
        for (int32_t t = 0; t < ne; ++t) {
            const uint32_t m = ent_mask[e0 + t];
            const V b = load_b(t);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = 4 * kq + v;
                if ((m >> r) & 1u)
                    fma_vec(acc[v], ent_val[tile_val_index(kTileMmaRows, (int64_t)e0 + t, r)], b);
            }
        }
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int c = 0; c < VEC; ++c) d[c][v] = reinterpret_cast<const float*>(&acc[v])[c];
    }
    if (!kok) return;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int r = 4 * kq + v;
        if (r >= rows) continue;
        V x;
#pragma unroll
        for (int c = 0; c < VEC; ++c) reinterpret_cast<float*>(&x)[c] = d[c][v];
        if (part < 0) {
            V* dst = reinterpret_cast<V*>(C + (int64_t)(row0 + r) * ld + col);
            store_nt(dst, accumulate ? add_vec(*dst, x) : x);
        } else {
            *reinterpret_cast<V*>(partials + (int64_t)(part + r) * O + col) = x;
        }
    }
}

template <int VEC, bool BUF, int GU, bool SB>
void launch_mma_as(const DeviceFmt& d, dim3 grid, int32_t n_ct, int32_t O, int32_t ld,
                   int32_t accumulate, uint32_t b_bytes, const float* B, float* C, float* partials,
                   hipStream_t st) {
    hipLaunchKernelGGL((vcsr_tile_mma_kernel<VEC, BUF, GU, SB>), grid, dim3(64 * kMmaWaves), 0, st,
                       d.tv_n_chunks, n_ct, O, ld, accumulate, b_bytes,
                       reinterpret_cast<const int4*>(d.tv_chunks),
                       reinterpret_cast<const int4*>(d.tv_pieces), d.tv_brow, d.tv_mask, d.tv_val,
                       B, C, partials);
}

template <int VEC, bool BUF>
void launch_mma_buf(const DeviceFmt& d, dim3 grid, int64_t waves, int32_t n_ct, int32_t O,
                    int32_t ld, int32_t accumulate, uint32_t b_bytes, const float* B, float* C,
                    float* partials, hipStream_t st) {
    // Few waves per SIMD (cfg5-like matrices at O <= 192): each wave's loads
    // in flight bound the time, so its loads go ahead of its MFMAs; with
    // many, 8 waves per SIMD with interleaved loads hide the latency better.
    // Measured on the 16K block-sparse matrix (1,024 tiles): O = 32 / 64,
    // one wave per SIMD, 4 groups with the barrier 27% / 36% faster; O = 128
    // / 192, two or three, 2 groups with the barrier 20% / 4% faster; O >= 256
    // slower with the barrier (O = 512: 236 / 186 against 152 us).  Without
    // it the compiler interleaves loads and MFMAs whatever the block size (42
    // VGPRs); 8 groups measured 1-4% faster than 4 at O = 256 / 512.
    const int64_t simds = 4 * (int64_t)device_cus(d.device);
    if (waves <= simds)
        launch_mma_as<VEC, BUF, 4, true>(d, grid, n_ct, O, ld, accumulate, b_bytes, B, C, partials,
                                         st);
    else if (waves <= 3 * simds)
        launch_mma_as<VEC, BUF, 2, true>(d, grid, n_ct, O, ld, accumulate, b_bytes, B, C, partials,
                                         st);
    else
        launch_mma_as<VEC, BUF, 8, false>(d, grid, n_ct, O, ld, accumulate, b_bytes, B, C,
                                          partials, st);
}

// Columns [0, O) of B and C, whose rows are ld floats apart.
template <int VEC>
hipError_t launch_mma(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O, int32_t ld,
                      float* C, int32_t accumulate, float* partials, hipStream_t st) {
    const int32_t n_ct = (O + 16 * VEC - 1) / (16 * VEC);
    const int64_t waves = (int64_t)d.tv_n_chunks * n_ct;
    const dim3 grid((unsigned)((waves + kMmaWaves - 1) / kMmaWaves));
    // Bytes from B to the end of its last row.
    const uint64_t b_bytes =
        v.N > 0 ? ((uint64_t)(v.N - 1) * (uint64_t)ld + (uint64_t)O) * 4u : 0u;
    if (b_bytes + 64u * 4u * (uint64_t)VEC >= kBufferLimit)
        launch_mma_buf<VEC, false>(d, grid, waves, n_ct, O, ld, accumulate, 0u, B, C, partials, st);
    else
        launch_mma_buf<VEC, true>(d, grid, waves, n_ct, O, ld, accumulate, (uint32_t)b_bytes, B, C,
                                  partials, st);
    return hipGetLastError();
}

template <int VEC, int LPE, int R, bool BUF>
hipError_t launch_one(const DeviceFmt& d, const float* B, int32_t O, int32_t ld, float* C,
                      int32_t accumulate, uint32_t b_bytes, float* partials, hipStream_t st) {
    // Eight streams per wave (B slices of at most 8 columns) and single-row
    // tiles: four work items per wave, so each stream still gets several
    // rows.  Taller tiles stay one per wave (their streams split the tile's
    // entries): measured 1.7x faster than four per wave at O = 8, R = 3.
    constexpr int MERGE = (64 / LPE >= 8 && R == 1) ? 4 : 1;
    const int64_t waves = ((int64_t)d.tv_n_chunks + MERGE - 1) / MERGE;
    const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves)), block(64 * kWaves);
    hipLaunchKernelGGL((vcsr_tile_kernel<VEC, LPE, R, MERGE, BUF>), grid, block, 0, st, d.tv_n_chunks, O,
                       ld, accumulate, b_bytes, reinterpret_cast<const int4*>(d.tv_chunks),
                       reinterpret_cast<const int4*>(d.tv_pieces), d.tv_brow, d.tv_mask, d.tv_val, B,
                       C, partials);
    return hipGetLastError();
}

template <int VEC, int R>
hipError_t launch_r(const DeviceFmt& d, const float* B, int32_t O, int32_t ld, float* C,
                    int32_t accumulate, uint64_t b_bytes, float* partials, hipStream_t st) {
    if (b_bytes + 64u * 4u * (uint64_t)VEC >= kBufferLimit)
        return launch_one<VEC, 64, R, false>(d, B, O, ld, C, accumulate, 0u, partials, st);
    const uint32_t bb = (uint32_t)b_bytes;
    // Lanes per entry: the smallest power of two covering O, at least 8 (at
    // most 8 streams per wave, so every stream gets several tiles); 8 lanes
    // occur for VEC = 4 (O = 32) and VEC = 1 (O <= 8).
    const int32_t need = (O + VEC - 1) / VEC;
    if constexpr (VEC == 1 || VEC == 4) {
        if (need <= 8)
            return launch_one<VEC, 8, R, true>(d, B, O, ld, C, accumulate, bb, partials, st);
    }
    if (need <= 16) return launch_one<VEC, 16, R, true>(d, B, O, ld, C, accumulate, bb, partials, st);
    if (need <= 32) return launch_one<VEC, 32, R, true>(d, B, O, ld, C, accumulate, bb, partials, st);
    return launch_one<VEC, 64, R, true>(d, B, O, ld, C, accumulate, bb, partials, st);
}

// Columns [0, O) of B and C, whose rows are ld floats apart (B and C point
// at the first column; ld > O for one column slice of wider matrices).
template <int VEC>
hipError_t launch_vec(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O, int32_t ld,
                      float* C, int32_t accumulate, float* partials, hipStream_t st) {
    if (d.tv_n_chunks > 0) {
        // Bytes from B to the end of its last row.
        const uint64_t b_bytes = v.N > 0 ? ((uint64_t)(v.N - 1) * (uint64_t)ld + (uint64_t)O) * 4u : 0u;
        hipError_t e;
        switch (d.tv_R) {
            case 1: e = launch_r<VEC, 1>(d, B, O, ld, C, accumulate, b_bytes, partials, st); break;
            case 2: e = launch_r<VEC, 2>(d, B, O, ld, C, accumulate, b_bytes, partials, st); break;
            case 3: e = launch_r<VEC, 3>(d, B, O, ld, C, accumulate, b_bytes, partials, st); break;
            case 4: e = launch_r<VEC, 4>(d, B, O, ld, C, accumulate, b_bytes, partials, st); break;
            case 8: e = launch_r<VEC, 8>(d, B, O, ld, C, accumulate, b_bytes, partials, st); break;
            case kTileMmaRows:
                e = launch_mma<VEC>(v, d, B, O, ld, C, accumulate, partials, st);
                break;
            default: return hipErrorInvalidValue;
        }
        if (e != hipSuccess) return e;
    }
    if (d.tv_n_split > 0) {
        // Narrow B (at most 8 column vectors per row): rows whose pieces
        // would take one wave more than four loads per lane get a block
        // each (the split rows come in decreasing piece count, so they are
        // the first n_heavy), the rest a wave each.  Power-law 322K matrix,
        // O = 8: 29.8 -> 28.6 us per SpMM (eight loads per lane: 29.1-29.4;
        // the kernel's own duration is the same, the gain is the launch of
        // 0.7K blocks instead of 2.7K).  Wider B keeps a block per row: at
        // O = 128 the reduce's duration was 5.9 against 5.3 us.
        const int32_t nvec = (O + VEC - 1) / VEC;
        int32_t cl = 1;
        while (cl < nvec && cl < 64) cl <<= 1;
        const int32_t light_max = cl <= 8 ? 4 * (64 / cl) : 0;
        const auto& pc = d.tv_split_pieces;
        const int32_t n_heavy = (int32_t)(std::partition_point(pc.begin(), pc.end(),
                                                               [&](int32_t x) { return x > light_max; }) -
                                          pc.begin());
        const int64_t blocks = (int64_t)n_heavy + ((int64_t)d.tv_n_split - n_heavy + 3) / 4;
        hipLaunchKernelGGL(vcsr_tile_reduce<VEC>, dim3((unsigned)blocks), dim3(256), 0, st, O, ld,
                           accumulate, n_heavy, d.tv_n_split,
                           reinterpret_cast<const int4*>(d.tv_split), partials, C);
        return hipGetLastError();
    }
    return hipSuccess;
}

}  // namespace

// Floats per lane and B slice: 4 when O allows 8 lanes (16 for 16-row MFMA
// tiles, whose column tiles are 16 lanes wide) of 16-byte vectors and B and
// C are 16-byte aligned, else 2 or 1.  At O = 32, 4 floats per lane measured
// 3% / 8% faster than 2 on the banded / power-law matrices.
static int tile_vec(int32_t O, bool a16, bool a8, bool mma) {
    if (O % 4 == 0 && a16 && O >= (mma ? 64 : 32)) return 4;
    if (O % 2 == 0 && a8 && O >= 32) return 2;
    return 1;
}

// Floats per lane (tile_vec) and column-slice width of a launch over B and
// C of width O.  Tiles of 1 to 8 rows with 16-byte vectors: one launch per
// column slice of at most 256 columns (one column tile of a wave), or 128
// when B is over 512 MB, so that the B bytes live at a time stay small.
// Measured against one launch over all columns: banded 62K matrix, slices of
// 256, O = 512 / 1024 / 2048: same / 16% / 30% faster; slices of 128,
// uniform-random 1M matrix O = 256 (1 GB): 11% faster, power-law 322K
// matrix O = 512 (659 MB): 3% faster, O = 256 (330 MB): 3% slower.
struct TileSlicing {
    int vec;
    int32_t width;
};
static TileSlicing tile_slicing(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                                const float* C) {
    const bool a16 = (((uintptr_t)B | (uintptr_t)C) & 15u) == 0;
    const bool a8 = (((uintptr_t)B | (uintptr_t)C) & 7u) == 0;
    // Narrow B: narrower per-lane vectors give streams of at least 8-16
    // lanes, so fewer streams share a tile's entries (measured at O = 8:
    // 4-byte loads with 8 streams 1.3x faster than 16-byte loads with 32).
    TileSlicing ts{tile_vec(O, a16, a8, d.tv_R == kTileMmaRows), O};
    if (ts.vec == 4 && d.tv_R != kTileMmaRows) {
        if ((uint64_t)v.N * (uint64_t)O * 4u > kTileSliceBytes) ts.width = std::min(O, kTileSliceCols);
        else ts.width = std::min(O, kTileWideCols);
    }
    // Split tiles write partial rows one slice wide: whatever the tile
    // height and vector width, a launch then covers at most the 256 columns
    // the upload sizes the partial rows for, so no O needs more scratch.
    if (d.tv_partial_rows > 0) ts.width = std::min(ts.width, kTileWideCols);
    return ts;
}

int64_t tile_partials_floats(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                             const float* C) {
    if (O <= 0 || v.M == 0 || d.tv_partial_rows == 0) return 0;
    return (int64_t)d.tv_partial_rows * tile_slicing(v, d, B, O, C).width;
}

int64_t tile_partials_upload_floats(const DeviceFmt& d) {
    return (int64_t)d.tv_partial_rows * kTileWideCols;
}

TilePlan tile_launch_plan(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                          const float* C) {
    TilePlan p;
    if (O <= 0 || v.M == 0) return p;
    const TileSlicing ts = tile_slicing(v, d, B, O, C);
    p.vec = ts.vec;
    p.slice_cols = ts.width;
    p.slices = (O + ts.width - 1) / ts.width;
    p.matrix_cores = d.tv_R == kTileMmaRows && d.tv_n_chunks > 0;
    p.reduce_launches = d.tv_n_split > 0 ? p.slices : 0;
    p.partial_floats = tile_partials_floats(v, d, B, O, C);
    return p;
}

hipError_t launch_vcsr_tile(const Vcsr& v, const DeviceFmt& d, const float* B, int32_t O,
                            float* C, int32_t accumulate, float* partials, hipStream_t st) {
    if (O <= 0 || v.M == 0) return hipSuccess;
    const TileSlicing ts = tile_slicing(v, d, B, O, C);
    for (int32_t c0 = 0; c0 < O; c0 += ts.width) {
        const int32_t w = std::min(ts.width, O - c0);
        hipError_t e;
        switch (ts.vec) {
            case 4: e = launch_vec<4>(v, d, B + c0, w, O, C + c0, accumulate, partials, st); break;
            case 2: e = launch_vec<2>(v, d, B + c0, w, O, C + c0, accumulate, partials, st); break;
            default: e = launch_vec<1>(v, d, B + c0, w, O, C + c0, accumulate, partials, st); break;
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

MfmaWork tile_mfma_work(const DeviceFmt& d, int32_t O) {
    MfmaWork w;
    w.flops_per_op = 2 * 16 * 16 * 4;
    if (d.tv_R != kTileMmaRows || O <= 0) return w;
    const int vec = tile_vec(O, true, true, true);
    const int64_t n_ct = (O + 16 * vec - 1) / (16 * vec);
    w.ops = d.tv_n_entries / 4 * n_ct * vec;
    return w;
}

}  // namespace vcsr
