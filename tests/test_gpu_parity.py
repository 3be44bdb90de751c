"""GPU parity: every HIP kernel, called through the C ABI, against the CPU
oracle (oracle/vcsr_oracle.cpp) on the same seeded inputs.

  * naive CSR: same loop order and FMA as the oracle's FP32 SpMM -> bit-exact;
  * VCSR streaming and FP32-MFMA kernels: different summation order and FP32
    atomics -> north-star tolerance (rel L2 <= 1e-5, per-row max-abs <=
    1e-4 * ||A_r||_1 * max|B|) against the oracle's double-accumulated sum,
    and the same against its FP32 sum;
  * full-size configs (every BASELINE config point on the default path):
    every element of C against the oracle's double sum under the same
    bounds, plus the size-independent column-sum identity
    sum_r C[r,:] = (1^T A) B.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import (assert_within_tolerance, block_csr, host_threads, random_csr,
                      row_abs_sums)

pytestmark = pytest.mark.gpu


def _case(vs, orc, rng, M, N, density=0.05, dup_rate=0.0, empty_rows=0.0):
    rows, cols, vals = random_csr(rng, M, N, density, dup_rate, empty_rows)
    coo = vs.Coo.from_arrays(M, N, rows, cols, vals)
    return vs.coo_to_csr(coo)


def _device_csr(vs, csr, st):
    return (vs.DeviceArray.from_numpy(csr.row_ptr, st), vs.DeviceArray.from_numpy(csr.col, st),
            vs.DeviceArray.from_numpy(csr.val, st))


def _run(vs, kind, csr, B, st, layout=1, segw=4, bundle=64, tileK=64, tile_rows=0):
    """Runs one kernel through the C ABI and returns C as numpy."""
    M, O = csr.M, B.shape[1]
    dB = vs.DeviceArray.from_numpy(B, st)
    dC = vs.DeviceArray((M, O), np.float32)
    dC.zero(st)
    if kind == "csr":
        rp, col, val = _device_csr(vs, csr, st)
        ms = vs.run_csr_spmm_gpu(M, rp, col, val, dB, O, dC, st, timed=True)
    else:
        fmt = vs.build_vcsr(csr, segw, bundle, layout)
        fmt.set_tile_rows(tile_rows)
        fmt.upload(st)
        if kind == "vcsr":
            ms = vs.run_vcsr_spmm_gpu(fmt, dB, O, tileK, dC, st, timed=True)
        elif kind == "segment":
            ms = vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, tileK, dC, st, timed=True,
                                         kernel=vs.KERNEL_SEGMENT)
        elif kind == "row":
            ms = vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, tileK, dC, st, timed=True,
                                         kernel=vs.KERNEL_ROW)
        elif kind == "tile":
            ms = vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, tileK, dC, st, timed=True,
                                         kernel=vs.KERNEL_TILE)
        else:
            ms = vs.run_vcsr_tc_spmm_gpu(fmt, dB, O, dC, st, timed=True)
    assert ms is not None and ms >= 0.0
    st.sync()
    return dC.numpy(st)


@pytest.fixture(scope="module")
def st(gpu):
    return gpu.Stream()


# ----------------------------------------------------------- naive CSR
@pytest.mark.parametrize("O", [1, 7, 32, 128])
def test_csr_naive_bit_exact_random(gpu, orc, st, O):
    vs = gpu
    rng = np.random.default_rng(100 + O)
    csr = _case(vs, orc, rng, 300, 257, density=0.04, dup_rate=0.1, empty_rows=0.1)
    B = vs.gen_dense(7, 0, csr.N, O)
    C = _run(vs, "csr", csr, B, st)
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert np.array_equal(C.view(np.uint32), ref.view(np.uint32))


def test_csr_naive_bit_exact_cfg1(gpu, orc, st):
    vs = gpu
    csr = vs.coo_to_csr(vs.generate_coo(1, 0))
    B = vs.gen_dense(1, 0, csr.N, 32)
    C = _run(vs, "csr", csr, B, st)
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert np.array_equal(C.view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------- VCSR kernels, small
KERNELS = [("vcsr", 1), ("vcsr", 0), ("mfma", 1), ("mfma", 0), ("mfma", 2), ("vcsr", 2),
           ("segment", 1), ("segment", 0), ("segment", 2), ("row", 1), ("row", 0), ("row", 2),
           ("tile", 1), ("tile", 0), ("tile", 2)]


@pytest.mark.parametrize("kind,layout", KERNELS)
@pytest.mark.parametrize("O", [1, 8, 33, 128, 200])
def test_vcsr_kernels_random(gpu, orc, st, kind, layout, O):
    vs = gpu
    rng = np.random.default_rng(1000 + 10 * O + layout)
    csr = _case(vs, orc, rng, 257, 203, density=0.05, dup_rate=0.05, empty_rows=0.1)
    B = vs.gen_dense(3, 0, csr.N, O)
    C = _run(vs, kind, csr, B, st, layout=layout, segw=4, bundle=64, tileK=64)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert_within_tolerance(C, ref64, csr.row_ptr, csr.val, B, f"{kind}/L{layout}/O{O}")
    ref32 = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert_within_tolerance(C, ref32.astype(np.float64), csr.row_ptr, csr.val, B, "vs f32")


@pytest.mark.parametrize("kind", ["segment", "mfma", "row", "tile"])
@pytest.mark.parametrize("segw,bundle,tileK", [(1, 64, 32), (3, 64, 100), (8, 64, 128),
                                               (16, 32, 64), (5, 20, 32), (20, 64, 256),
                                               (4, 128, 64), (4, 1, 32), (33, 16, 64)])
def test_vcsr_kernels_shapes(gpu, orc, st, kind, segw, bundle, tileK):
    vs = gpu
    rng = np.random.default_rng(segw * 1000 + bundle * 10 + tileK)
    csr = _case(vs, orc, rng, 190, 150, density=0.08, dup_rate=0.1, empty_rows=0.05)
    O = 70
    B = vs.gen_dense(5, 1, csr.N, O)
    C = _run(vs, kind, csr, B, st, layout=1, segw=segw, bundle=bundle, tileK=tileK)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert_within_tolerance(C, ref64, csr.row_ptr, csr.val, B, f"{kind} segw{segw} b{bundle}")


@pytest.mark.parametrize("kind,layout", KERNELS)
def test_vcsr_kernels_cfg1(gpu, orc, st, kind, layout):
    vs = gpu
    csr = vs.coo_to_csr(vs.generate_coo(1, 0))
    B = vs.gen_dense(1, 0, csr.N, 32)
    C = _run(vs, kind, csr, B, st, layout=layout, segw=4, bundle=64, tileK=64)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert_within_tolerance(C, ref64, csr.row_ptr, csr.val, B, f"cfg1 {kind}/L{layout}")


def test_vcsr_empty_and_degenerate(gpu, orc, st):
    vs = gpu
    # no nonzeros at all, and a matrix whose N is not a multiple of segw
    for M, N in [(5, 3), (64, 1), (1, 17)]:
        csr = vs.Csr.from_arrays(M, N, np.zeros(M + 1, np.int32), np.zeros(0, np.int32),
                                 np.zeros(0, np.float32))
        B = vs.gen_dense(2, 0, N, 9)
        for kind in ("csr", "vcsr", "mfma"):
            C = _run(vs, kind, csr, B, st)
            assert not C.any()
    rng = np.random.default_rng(5)
    csr = _case(vs, orc, rng, 40, 13, density=0.3)
    B = vs.gen_dense(2, 0, csr.N, 9)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    for kind in ("vcsr", "mfma"):
        C = _run(vs, kind, csr, B, st, segw=4)
        assert_within_tolerance(C, ref64, csr.row_ptr, csr.val, B, kind)


def test_vcsr_repeat_runs_agree(gpu, orc, st):
    """Atomic flush order varies between runs; results stay within tolerance."""
    vs = gpu
    csr = vs.coo_to_csr(vs.generate_coo(1, 0))
    B = vs.gen_dense(1, 0, csr.N, 128)
    runs = [_run(vs, "vcsr", csr, B, st) for _ in range(3)]
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    for C in runs:
        assert_within_tolerance(C, ref64, csr.row_ptr, csr.val, B, "repeat")


# ------------------------------------------------- full-size configurations
def _whole_check(orc, csr, B, C, what):
    """Every element of C against the oracle's double-accumulated product
    (rows split over the host's threads; the same sum as one thread)."""
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B, host_threads())
    rel, worst = assert_within_tolerance(C, ref64, csr.row_ptr, csr.val, B, what)
    print(f"{what}: rel L2 {rel:.2e}, max-abs / bound {worst:.4f}", flush=True)
    return ref64


def _colsum_check(csr, B, C):
    """sum_r C[r,:] == (1^T A) B, in double: pins all of C in aggregate."""
    s = np.bincount(csr.col, weights=csr.val.astype(np.float64), minlength=csr.N)
    want = s @ B.astype(np.float64)
    got = C.astype(np.float64).sum(axis=0)
    scale = np.abs(csr.val).astype(np.float64).sum() * float(np.abs(B).max())
    assert np.max(np.abs(got - want)) <= 1e-5 * scale


@pytest.mark.parametrize("cfg,O,segw,tileK,layout", [(2, 128, 4, 64, 1), (3, 128, 4, 128, 1),
                                                     (2, 8, 4, 64, 1), (5, 64, 16, 64, 2)])
@pytest.mark.parametrize("kind", ["segment", "mfma", "row", "tile"])
def test_full_size_configs(gpu, orc, st, cfg, O, segw, tileK, layout, kind):
    vs = gpu
    csr = vs.coo_to_csr(vs.generate_coo(cfg, 0))
    B = vs.gen_dense(cfg, 1 if cfg == 5 else 0, csr.N, O)
    bundle = 16 if layout == 2 else 64
    C = _run(vs, kind, csr, B, st, layout=layout, segw=segw, bundle=bundle, tileK=tileK)
    _whole_check(orc, csr, B, C, f"cfg{cfg} O={O} {kind}")
    _colsum_check(csr, B, C)


@pytest.mark.parametrize("kind", ["segment", "mfma"])
def test_cfg5_o512_segment_major_kernels_whole_c(gpu, orc, st, kind):
    """BASELINE config 5 as it asks: the segmented-streaming kernel and the
    FP32-MFMA dense-group kernel (src/vcsr_seg.cu:191-231,
    src/vcsr_tc.cu:197-232) on the full 16K block-sparse matrix at O = 512,
    layout TC (segw = bundle = 16): every element of C within the north-star
    bounds of the oracle's double sum, and the column-sum identity."""
    vs = gpu
    print(f"cfg5 O=512 {kind}", flush=True)
    csr = vs.coo_to_csr(vs.generate_coo(5, 0))
    B = vs.gen_dense(5, 1, csr.N, 512)
    C = _run(vs, kind, csr, B, st, layout=2, segw=16, bundle=16, tileK=64)
    _whole_check(orc, csr, B, C, f"cfg5 O=512 {kind}")
    _colsum_check(csr, B, C)


# (cfg, O, segw, layout): every O of the BASELINE configs, cfg4 at both segw.
BASELINE_POINTS = [(2, 8, 4, 1), (2, 32, 4, 1), (2, 128, 4, 1), (2, 512, 4, 1), (3, 8, 4, 1),
                   (3, 128, 4, 1), (4, 256, 4, 1), (4, 256, 8, 1), (5, 512, 16, 2)]


@pytest.mark.parametrize("cfg,O,segw,layout", BASELINE_POINTS)
def test_baseline_config_points_whole_c(gpu, orc, st, cfg, O, segw, layout):
    """The default path (spmm_vcsr: VCSR_KERNEL_AUTO, the reference's C +=
    A*B on a zeroed C) at every BASELINE config point and full size: all of
    C within the north-star bounds of the oracle's double sum.  cfg5's
    16-row tiles are never split (816 entries each), so its C is also the
    oracle's FP32 loop bit for bit."""
    vs = gpu
    print(f"baseline point cfg{cfg} O={O} segw={segw} layout={layout}", flush=True)
    csr = vs.coo_to_csr(vs.generate_coo(cfg, 0))
    B = vs.gen_dense(cfg, 1 if cfg == 5 else 0, csr.N, O)
    bundle = 16 if layout == 2 else 64
    C = _run(vs, "vcsr", csr, B, st, layout=layout, segw=segw, bundle=bundle,
             tileK=64 if cfg == 2 else 128)
    _whole_check(orc, csr, B, C, f"cfg{cfg} O={O} segw={segw}")
    _colsum_check(csr, B, C)
    if cfg == 5:
        ref32 = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B, host_threads())
        assert np.array_equal(C.view(np.uint32), ref32.view(np.uint32))


def test_full_size_csr_naive_cfg2(gpu, orc, st):
    vs = gpu
    csr = vs.coo_to_csr(vs.generate_coo(2, 0))
    B = vs.gen_dense(2, 0, csr.N, 128)
    C = _run(vs, "csr", csr, B, st)
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert np.array_equal(C.view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------ row-stationary kernel modes
def _ex(vs, fmt, B, C0, st, kernel, accumulate, tileK=64):
    dB = vs.DeviceArray.from_numpy(B, st)
    dC = vs.DeviceArray.from_numpy(C0, st)
    vs.run_vcsr_spmm_gpu_ex(fmt, dB, B.shape[1], tileK, dC, st, timed=True, kernel=kernel,
                            accumulate=accumulate)
    st.sync()
    return dC.numpy(st)


@pytest.mark.parametrize("kernel", [1, 2, 3, 4])
@pytest.mark.parametrize("O", [5, 64, 130, 256, 300])
def test_accumulate_and_overwrite(gpu, orc, st, kernel, O):
    """accumulate=1 adds A*B to the C it is given; accumulate=0 replaces it."""
    vs = gpu
    rng = np.random.default_rng(77 + O)
    csr = _case(vs, orc, rng, 150, 120, density=0.06, dup_rate=0.05, empty_rows=0.2)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.upload(st)
    B = vs.gen_dense(9, 0, csr.N, O)
    C0 = rng.uniform(-2, 2, size=(csr.M, O)).astype(np.float32)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    got = _ex(vs, fmt, B, C0, st, kernel, True)
    assert_within_tolerance(got - C0, ref64, csr.row_ptr, csr.val, B, "accumulate")
    got = _ex(vs, fmt, B, C0, st, kernel, False)
    assert_within_tolerance(got, ref64, csr.row_ptr, csr.val, B, "overwrite")


@pytest.mark.parametrize("kernel", [3, 4])
@pytest.mark.parametrize("accumulate", [True, False])
def test_row_kernel_split_rows(gpu, orc, st, accumulate, kernel):
    """Rows with more (row, segment) pairs than one wave takes are split into
    chunks and reduced by a second kernel; run it twice (scratch reuse) and
    with a wider O (scratch growth)."""
    vs = gpu
    rng = np.random.default_rng(3)
    M, N = 40, 3000
    rows, cols, vals = random_csr(rng, M, N, density=0.01)
    dense_rows = [0, 7, 39]
    for r in dense_rows:  # every column: N/segw = 750 pairs > one chunk
        rows = np.concatenate([rows, np.full(N, r, np.int32)])
        cols = np.concatenate([cols, np.arange(N, dtype=np.int32)])
        vals = np.concatenate([vals, rng.uniform(-1, 1, N).astype(np.float32)])
    csr = vs.coo_to_csr(vs.Coo.from_arrays(M, N, rows, cols, vals))
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.upload(st)
    for O in (64, 64, 200):
        B = vs.gen_dense(O, 0, N, O)
        C0 = np.ones((M, O), np.float32)
        ref64 = orc.spmm_f64(M, csr.row_ptr, csr.col, csr.val, B)
        got = _ex(vs, fmt, B, C0, st, kernel, accumulate)
        if accumulate:
            got = got - C0
        assert_within_tolerance(got, ref64, csr.row_ptr, csr.val, B, f"split O={O}")


@pytest.mark.parametrize("kind", ["row", "tile"])
@pytest.mark.parametrize("cfg,O,layout", [(3, 128, 1), (4, 256, 1), (5, 512, 2)])
def test_full_size_row_kernel(gpu, orc, st, cfg, O, layout, kind):
    vs = gpu
    csr = vs.coo_to_csr(vs.generate_coo(cfg, 0))
    B = vs.gen_dense(cfg, 1 if cfg == 5 else 0, csr.N, O)
    segw, bundle = (16, 16) if layout == 2 else (4, 64)
    C = _run(vs, kind, csr, B, st, layout=layout, segw=segw, bundle=bundle, tileK=128)
    _whole_check(orc, csr, B, C, f"cfg{cfg} O={O} {kind}")
    _colsum_check(csr, B, C)


# ------------------------------------------------------ tile-stationary kernel
def _block_csr(vs, rng, nbr, bh, N, blocks_per_row, bw, keep):
    return block_csr(vs, rng, nbr, bh, N, blocks_per_row, bw, keep)


@pytest.mark.parametrize("bh,tile_rows", [(2, 0), (3, 0), (4, 0), (8, 0), (16, 0), (3, 1), (3, 2),
                                          (3, 3), (6, 3), (3, 8), (5, 4), (16, 16), (5, 16),
                                          (12, 16)])
@pytest.mark.parametrize("O", [1, 8, 33, 128, 200, 520, 2048])
def test_tile_kernel_block_rows(gpu, orc, st, bh, tile_rows, O):
    vs = gpu
    rng = np.random.default_rng(bh * 100 + tile_rows * 10 + O)
    csr = _block_csr(vs, rng, 37, bh, 300, 7, 3, 0.8)
    B = vs.gen_dense(bh + O, 0, csr.N, O)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.set_tile_rows(tile_rows)
    fmt.upload(st)
    R, tiles, entries = fmt.tile_info()
    if tile_rows:
        assert R == tile_rows
    elif bh >= 2:
        assert R >= 2, "block rows should be tiled"
    assert entries < csr.nnz or R == 1
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    C0 = rng.uniform(-1, 1, size=(csr.M, O)).astype(np.float32)
    for accumulate in (False, True):
        got = _ex(vs, fmt, B, C0, st, vs.KERNEL_TILE, accumulate)
        if accumulate:
            got = got - C0
        assert_within_tolerance(got, ref64, csr.row_ptr, csr.val, B, f"bh{bh} R{R} O{O}")


@pytest.mark.parametrize("tile_rows", [1, 3, 4, 8, 16])
def test_tile_kernel_split_tiles(gpu, orc, st, tile_rows):
    """Block rows wider than one work item: tiles are cut into pieces whose
    partial sums a second kernel adds; wider O grows the scratch."""
    vs = gpu
    rng = np.random.default_rng(tile_rows)
    csr = _block_csr(vs, rng, 6, 8, 4096, 600, 4, 0.9)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.set_tile_rows(tile_rows)
    fmt.upload(st)
    for O in (64, 64, 260):
        B = vs.gen_dense(O, 0, csr.N, O)
        ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
        got = _ex(vs, fmt, B, np.zeros((csr.M, O), np.float32), st, vs.KERNEL_TILE, False)
        assert_within_tolerance(got, ref64, csr.row_ptr, csr.val, B, f"R{tile_rows} O{O}")


@pytest.mark.parametrize("kind,tile_rows,O", [
    ("csr", 4, 36), ("segment", 4, 36), ("row", 4, 36), ("tile", 4, 36), ("tile", 16, 36),
    # 1- and 3-row tiles (B row inside the value record), 8-row tiles, and
    # narrow B: single-row tiles merge four work items per wave at O <= 8
    # and O = 32, and redo non-finite pieces across the merged items.
    ("tile", 1, 36), ("tile", 3, 36), ("tile", 8, 36), ("tile", 1, 8), ("tile", 3, 8),
    ("tile", 1, 32), ("tile", 2, 8), ("row", 4, 8)])
def test_nonfinite_b_stays_in_its_columns(gpu, orc, st, kind, tile_rows, O):
    """Inf and NaN in B reach exactly the C entries whose rows have a nonzero
    in that B row (an absent entry contributes nothing, not 0 * inf).  The
    MFMA kernel is left out: it multiplies every group as a dense tile, so a
    non-finite B value reaches every row of the groups of its segment, as
    with the reference's tensor-core kernel."""
    vs = gpu
    rng = np.random.default_rng(11)
    csr = _block_csr(vs, rng, 20, 4, 120, 5, 3, 0.6)
    B = vs.gen_dense(4, 0, csr.N, O)
    B[5, 3] = np.inf
    B[17, :] = np.nan
    B[40, 7] = -np.inf
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    C = _run(vs, kind, csr, B, st, tile_rows=tile_rows)
    assert np.array_equal(np.isnan(C), np.isnan(ref)), kind
    assert np.array_equal(np.isposinf(C), np.isposinf(ref)), kind
    assert np.array_equal(np.isneginf(C), np.isneginf(ref)), kind
    fin = np.isfinite(ref)
    assert np.allclose(C[fin], ref[fin], rtol=1e-5, atol=1e-4)


def _row_lengths_csr(vs, rng, lengths, N):
    """One row per entry of `lengths`, that many distinct random columns."""
    rows, cols = [], []
    for r, k in enumerate(lengths):
        c = rng.choice(N, size=k, replace=False) if k else np.zeros(0, np.int64)
        rows.extend([r] * k)
        cols.extend(c.tolist())
    vals = rng.uniform(-1, 1, size=len(rows)).astype(np.float32)
    return vs.coo_to_csr(vs.Coo.from_arrays(len(lengths), N, np.array(rows, np.int32),
                                            np.array(cols, np.int32), vals))


# Row lengths that mix short rows (merged into shared work items), rows of
# 17-64 entries (one piece, a work item of their own), rows cut into pieces
# of up to 64 entries (partial rows summed by the reduce kernel) and empty
# rows, so that a wave's four work items hold pieces of every length.
_EQ_PATTERN = [0, 1, 3, 17, 2, 150, 5, 64, 65, 9, 400, 1, 1, 30, 0, 12, 2, 2, 90, 7]


@pytest.mark.parametrize("O", [1, 4, 8, 32])
@pytest.mark.parametrize("accumulate", [False, True])
def test_equal_runs_of_single_row_tiles(gpu, orc, st, O, accumulate):
    """Single-row tiles at O <= 8 and O = 32 run four work items per wave,
    each of 8 streams taking an equal run of the wave's entries; a piece cut
    between runs is finished by the stream that began it from the later
    streams' partial sums.  Rows of every length, pieces spanning up to
    seven runs, and a matrix with fewer entries than streams (empty runs):
    all of C within the north-star bounds, in both C modes, the same bits
    on a second call."""
    vs = gpu
    rng = np.random.default_rng(500 + O)
    cases = [_row_lengths_csr(vs, rng, _EQ_PATTERN * 12, 1000),
             _row_lengths_csr(vs, rng, [1, 0, 2, 0, 1], 9)]
    for csr in cases:
        print(f"equal runs M={csr.M} nnz={csr.nnz} O={O} accumulate={accumulate}", flush=True)
        fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
        fmt.set_tile_rows(1)
        fmt.upload(st)
        li = fmt.launch_info(O, vs.KERNEL_TILE)
        assert li["tile_rows"] == 1 and (li["vec"] == 4 if O == 32 else li["vec"] == 1)
        B = vs.gen_dense(O + 3, 0, csr.N, O)
        C0 = rng.uniform(-2, 2, size=(csr.M, O)).astype(np.float32)
        ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
        got = _ex(vs, fmt, B, C0, st, vs.KERNEL_TILE, accumulate)
        again = _ex(vs, fmt, B, C0, st, vs.KERNEL_TILE, accumulate)
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
        assert_within_tolerance(got - C0 if accumulate else got, ref64, csr.row_ptr, csr.val, B,
                                f"equal runs O={O}")


@pytest.mark.parametrize("O", [8, 32])
def test_equal_runs_nonfinite_b(gpu, orc, st, O):
    """Inf and NaN in B rows read by long rows (pieces cut between streams'
    runs, and split rows) and by short ones reach exactly the C entries the
    reference's loop reaches: the stream that finishes a piece from other
    streams' partial sums recomputes it with the presence bits when the sum
    is not finite."""
    vs = gpu
    rng = np.random.default_rng(900 + O)
    csr = _row_lengths_csr(vs, rng, _EQ_PATTERN * 6, 600)
    B = vs.gen_dense(O, 0, csr.N, O)
    rp, col = csr.row_ptr, csr.col
    long_row = int(np.argmax(np.diff(rp)))
    B[col[rp[long_row] + 3], 0] = np.inf
    B[col[rp[long_row + 13]], :] = np.nan                # a row in another work item
    B[col[rp[3 * len(_EQ_PATTERN) + 8] + 40], O - 1] = -np.inf  # a 65-entry row's second piece
    ref = orc.spmm_f32(csr.M, rp, col, csr.val, B)
    C = _run(vs, "tile", csr, B, st, tile_rows=1)
    assert np.array_equal(np.isnan(C), np.isnan(ref))
    assert np.array_equal(np.isposinf(C), np.isposinf(ref))
    assert np.array_equal(np.isneginf(C), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert np.allclose(C[fin], ref[fin], rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("kind,tile_rows", [("row", 0), ("tile", 0), ("tile", 16)])
def test_b_of_2gb_or_more_uses_64bit_addresses(gpu, orc, st, kind, tile_rows):
    """B of 2^31 bytes or more cannot be addressed with 32-bit buffer
    offsets; the row and tile kernels then take their 64-bit-address path.
    N = 2^19 + 3 rows of O = 1024 floats (2.0 GiB + 12 KiB), 3000 sparse rows
    whose columns reach the last B rows."""
    vs = gpu
    rng = np.random.default_rng(21)
    N, O, M = (1 << 19) + 3, 1024, 3000
    nnz_row = 24
    rows = np.repeat(np.arange(M, dtype=np.int32), nnz_row)
    cols = rng.integers(0, N, size=M * nnz_row).astype(np.int32)
    cols[:nnz_row] = N - 1 - np.arange(nnz_row)  # row 0 reads the end of B
    vals = rng.uniform(-1, 1, size=M * nnz_row).astype(np.float32)
    csr = vs.coo_to_csr(vs.Coo.from_arrays(M, N, rows, cols, vals))
    B = vs.gen_dense(77, 0, N, O)
    assert B.nbytes >= 1 << 31
    C = _run(vs, kind, csr, B, st, layout=1, segw=4, bundle=64, tileK=128, tile_rows=tile_rows)
    _whole_check(orc, csr, B, C, f"2 GiB B {kind} R={tile_rows}")


@pytest.mark.parametrize("accumulate", [False, True])
def test_tile_column_slices_with_split_rows(gpu, orc, st, accumulate):
    """B larger than 512 MB at O > 128 runs in column slices of 128 columns
    (one launch per slice, B and C rows O floats apart); rows too long for
    one work item are cut into pieces whose partial sums the reduce kernel
    adds, slice by slice.  Every element of C is checked.  N = 700,000, O = 200 (560 MB; slices of 128 and
    72 columns), 2,000 rows of which every 50th has 3,000 entries, the
    others 12; columns uniform over N, so the view keeps 1-row tiles."""
    vs = gpu
    rng = np.random.default_rng(5)
    N, O, M = 700_000, 200, 2000
    lens = np.where(np.arange(M) % 50 == 7, 3000, 12)
    rows = np.repeat(np.arange(M, dtype=np.int32), lens)
    cols = rng.integers(0, N, size=rows.size).astype(np.int32)
    vals = rng.uniform(-1, 1, size=rows.size).astype(np.float32)
    csr = vs.coo_to_csr(vs.Coo.from_arrays(M, N, rows, cols, vals))
    B = vs.gen_dense(9, 0, N, O)
    assert B.nbytes > 512 << 20
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.upload(st)
    assert fmt.tile_info()[0] == 1
    C0 = rng.uniform(-1, 1, size=(M, O)).astype(np.float32)
    C = _ex(vs, fmt, B, C0, st, vs.KERNEL_TILE, accumulate)
    if accumulate:
        C = C - C0
    ref64 = orc.spmm_f64(M, csr.row_ptr, csr.col, csr.val, B, host_threads())
    assert_within_tolerance(C, ref64, csr.row_ptr, csr.val, B, "sliced rows")


@pytest.mark.parametrize("O", [8, 32, 100, 512])
def test_tile_mfma_work_counts_the_launch(gpu, orc, st, O):
    """The MFMA instruction count of 16-row tiles: four entries per k-step,
    16*VEC columns per column tile, one MFMA per column part (VEC = 4, 2 or 1
    by O); none for other tile heights.  The result is checked too."""
    vs = gpu
    rng = np.random.default_rng(O)
    csr = _block_csr(vs, rng, 9, 16, 400, 6, 16, 1.0)
    B = vs.gen_dense(O, 0, csr.N, O)
    fmt = vs.build_vcsr(csr, 16, 16, vs.LAYOUT_TC)
    fmt.upload(st)
    R, tiles, entries = fmt.tile_info()
    assert (R, tiles) == (16, 9)
    assert entries % 16 == 0 and entries >= csr.nnz // 16
    vec = 4 if O % 4 == 0 and O >= 64 else (2 if O % 2 == 0 and O >= 32 else 1)
    ops, fpo = vs.tile_mfma_work(fmt, O)
    assert fpo == 2 * 16 * 16 * 4
    assert ops == entries // 4 * -(-O // (16 * vec)) * vec
    got = _ex(vs, fmt, B, np.zeros((csr.M, O), np.float32), st, vs.KERNEL_TILE, False)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert_within_tolerance(got, ref64, csr.row_ptr, csr.val, B, f"O{O}")
    other = vs.build_vcsr(csr, 16, 16, vs.LAYOUT_TC)
    other.set_tile_rows(8)
    other.upload(st)
    assert vs.tile_mfma_work(other, O)[0] == 0


@pytest.mark.parametrize("O", [1, 8, 33, 128])
def test_vendor_baseline_matches_oracle(gpu, orc, st, O):
    """The rocSPARSE baseline (one-shot and plan) computes C = A*B within the
    north-star tolerance, overwriting C, on random and empty-row matrices."""
    vs = gpu
    rng = np.random.default_rng(O)
    csr = _block_csr(vs, rng, 40, 3, 500, 9, 3, 0.7)
    B = vs.gen_dense(O, 0, csr.N, O)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    rp, col, val = _device_csr(vs, csr, st)
    dB = vs.DeviceArray.from_numpy(B, st)
    dC = vs.DeviceArray.from_numpy(np.full((csr.M, O), 7.0, np.float32), st)
    ms = vs.run_vendor_spmm_gpu(csr.M, csr.N, csr.nnz, rp, col, val, dB, O, dC, st, timed=True)
    assert ms >= 0
    assert_within_tolerance(dC.numpy(st), ref64, csr.row_ptr, csr.val, B, f"one-shot O{O}")
    dC2 = vs.DeviceArray.from_numpy(np.full((csr.M, O), -3.0, np.float32), st)
    plan = vs.VendorPlan(csr.M, csr.N, csr.nnz, rp, col, val, dB, O, dC2, st)
    for _ in range(2):
        plan.run(st)
    st.sync()
    assert_within_tolerance(dC2.numpy(st), ref64, csr.row_ptr, csr.val, B, f"plan O{O}")


def _run_wave(vs, st, M, N, row_ptr, col, val, B):
    rp = vs.DeviceArray.from_numpy(np.ascontiguousarray(row_ptr, np.int32), st)
    dcol = vs.DeviceArray.from_numpy(np.ascontiguousarray(col, np.int32), st)
    dval = vs.DeviceArray.from_numpy(np.ascontiguousarray(val, np.float32), st)
    dB = vs.DeviceArray.from_numpy(B, st)
    dC = vs.DeviceArray.from_numpy(np.full((M, B.shape[1]), 5.0, np.float32), st)
    vs.run_csr_wave_spmm_gpu(M, N, rp, dcol, dval, dB, B.shape[1], dC, st, timed=True)
    return dC.numpy(st)


@pytest.mark.parametrize("O", [1, 7, 32, 128, 130, 300])
def test_csr_wave_bit_exact_random(gpu, orc, st, O):
    """The wave-per-row CSR kernel applies each row's entries in CSR order
    with one fused multiply-add per term, like the oracle: bit-exact, with
    duplicates and empty rows; C is overwritten."""
    vs = gpu
    rng = np.random.default_rng(200 + O)
    csr = _case(vs, orc, rng, 300, 257, density=0.04, dup_rate=0.1, empty_rows=0.1)
    B = vs.gen_dense(9, 0, csr.N, O)
    C = _run_wave(vs, st, csr.M, csr.N, csr.row_ptr, csr.col, csr.val, B)
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert np.array_equal(C.view(np.uint32), ref.view(np.uint32))


def test_csr_wave_bit_exact_power_law(gpu, orc, st):
    """cfg3 (rows up to ~17k entries, many rows per wave at O = 8)."""
    vs = gpu
    csr = vs.coo_to_csr(vs.generate_coo(3, 0))
    B = vs.gen_dense(3, 0, csr.N, 8)
    C = _run_wave(vs, st, csr.M, csr.N, csr.row_ptr, csr.col, csr.val, B)
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert np.array_equal(C.view(np.uint32), ref.view(np.uint32))


def test_csr_wave_ignores_columns_outside_b(gpu, orc, st):
    """Columns outside [0, N) contribute nothing (the kernel bounds B's
    addressing by N): the result equals the CSR without those entries."""
    vs = gpu
    rng = np.random.default_rng(5)
    M, N, O = 50, 40, 64
    lens = rng.integers(0, 12, M)
    row_ptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    col = rng.integers(0, N, row_ptr[-1]).astype(np.int32)
    bad = rng.random(col.size) < 0.2
    col[bad] = np.where(rng.random(bad.sum()) < 0.5, -3, N + 7)
    val = rng.uniform(-1, 1, col.size).astype(np.float32)
    B = vs.gen_dense(1, 0, N, O)
    C = _run_wave(vs, st, M, N, row_ptr, col, val, B)
    keep = ~bad
    rp2 = np.concatenate([[0], np.cumsum([keep[row_ptr[r]:row_ptr[r + 1]].sum()
                                          for r in range(M)])]).astype(np.int32)
    ref = orc.spmm_f32(M, rp2, col[keep], val[keep], B)
    assert np.array_equal(C.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("tile_rows", [4, 16])
@pytest.mark.parametrize("O", [8, 64, 200])
def test_fixed_row_windows(gpu, orc, st, tile_rows, O):
    """Fixed row windows (16 rows: FastSpMM's condensed-tile layout) on a
    matrix whose rows share few columns, with empty and duplicate entries:
    C = A*B and C += A*B within the north-star tolerance."""
    vs = gpu
    rng = np.random.default_rng(tile_rows * 1000 + O)
    csr = _case(vs, orc, rng, 333, 290, density=0.03, dup_rate=0.05, empty_rows=0.1)
    B = vs.gen_dense(O + 1, 0, csr.N, O)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.set_tile_rows(tile_rows)
    fmt.set_tile_windows(True)
    fmt.upload(st)
    R, tiles, entries = fmt.tile_info()
    assert R == tile_rows and tiles == -(-csr.M // tile_rows)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    C0 = rng.uniform(-1, 1, size=(csr.M, O)).astype(np.float32)
    for accumulate in (False, True):
        got = _ex(vs, fmt, B, C0, st, vs.KERNEL_TILE, accumulate)
        if accumulate:
            got = got - C0
        assert_within_tolerance(got, ref64, csr.row_ptr, csr.val, B, f"R{R} O{O}")


class _Shifted:
    """A device buffer viewed `off` bytes past its start, so that B and C can
    be handed over with 4- or 8-byte alignment only."""

    def __init__(self, vs, a, off, st):
        import ctypes
        self._lib = vs.load_library()
        self._st = st
        self.shape, self.nbytes, self.dtype = a.shape, a.nbytes, a.dtype
        self._base = vs.DeviceArray((a.nbytes + 64,), np.uint8)
        self.ptr = ctypes.c_void_p(self._base.ptr.value + off)
        a = np.ascontiguousarray(a)
        assert self._lib.vcsr_memcpy_h2d(self.ptr, a.ctypes.data_as(ctypes.c_void_p), a.nbytes,
                                         st.h) == 0
        st.sync()

    def numpy(self):
        import ctypes
        out = np.empty(self.shape, np.float32)
        assert self._lib.vcsr_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), self.ptr,
                                         self.nbytes, self._st.h) == 0
        self._st.sync()
        return out


@pytest.mark.parametrize("off", [4, 8])
@pytest.mark.parametrize("kind", ["tile3", "tile16", "tile1", "row", "wave"])
def test_unaligned_b_and_c(gpu, orc, st, kind, off):
    """B and C that are only 4- or 8-byte aligned take the narrower per-lane
    vectors (1 or 2 floats) of the row, tile and wave kernels."""
    vs = gpu
    rng = np.random.default_rng(off)
    O = 128
    csr = _block_csr(vs, rng, 24, 3, 400, 8, 3, 0.8)
    B = vs.gen_dense(off, 0, csr.N, O)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    dB = _Shifted(vs, B, off, st)
    dC = _Shifted(vs, np.full((csr.M, O), 9.0, np.float32), off, st)
    if kind == "wave":
        rp, col, val = _device_csr(vs, csr, st)
        vs.run_csr_wave_spmm_gpu(csr.M, csr.N, rp, col, val, dB, O, dC, st, timed=True)
    else:
        fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
        if kind.startswith("tile"):
            fmt.set_tile_rows(int(kind[4:]))
        fmt.upload(st)
        kernel = vs.KERNEL_ROW if kind == "row" else vs.KERNEL_TILE
        vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, 64, dC, st, timed=True, kernel=kernel,
                                accumulate=False)
    assert_within_tolerance(dC.numpy(), ref64, csr.row_ptr, csr.val, B, f"{kind} off{off}")


@pytest.mark.parametrize("kind,tile_rows", [("row", 0), ("tile", 1), ("tile", 3), ("tile", 16)])
@pytest.mark.parametrize("off,O", [(4, 301), (8, 522), (0, 301)])
def test_split_rows_in_column_slices_at_any_width(gpu, orc, st, kind, tile_rows, off, O):
    """Formats with split rows (row kernel) or split tiles (tile kernel,
    VALU and 16-row MFMA) run in column slices of at most 256 columns, whose
    partial rows are one slice wide, also when O is not a multiple of 4 or
    B and C are only 4- or 8-byte aligned (1- or 2-float lanes, which used
    to run unsliced): every element of C against the oracle, in both C
    modes, the second call reusing the scratch."""
    vs = gpu
    rng = np.random.default_rng(off * 1000 + O + tile_rows)
    csr = _block_csr(vs, rng, 6, 8, 4096, 600, 4, 0.9)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.set_tile_rows(tile_rows)
    fmt.upload(st)
    kernel = vs.KERNEL_ROW if kind == "row" else vs.KERNEL_TILE
    if kind == "tile":
        li = fmt.launch_info(O, kernel)
        assert li["split_rows"] > 0 and li["column_slices"] == -(-O // 256), li
    B = vs.gen_dense(O + off, 0, csr.N, O)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    C0 = rng.uniform(-1, 1, size=(csr.M, O)).astype(np.float32)
    dB = _Shifted(vs, B, off, st)
    for accumulate in (False, True):
        dC = _Shifted(vs, C0, off, st)
        vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, 64, dC, st, timed=True, kernel=kernel,
                                accumulate=accumulate)
        got = dC.numpy()
        if accumulate:
            got = got - C0
        assert_within_tolerance(got, ref64, csr.row_ptr, csr.val, B,
                                f"{kind} R{tile_rows} off{off} O{O} acc{accumulate}")


@pytest.mark.parametrize("tile_rows", [1, 16])
def test_nonfinite_b_with_split_tiles_in_column_slices(gpu, orc, st, tile_rows):
    """Inf and NaN in B reach exactly the reference's C entries when the
    tiles are split into pieces (partial rows summed by the reduce kernel)
    and the launch is cut into column slices: O = 300, 16-row MFMA tiles and
    1-row tiles."""
    vs = gpu
    rng = np.random.default_rng(17 + tile_rows)
    csr = _block_csr(vs, rng, 6, 8, 4096, 600, 4, 0.9)
    O = 300
    B = vs.gen_dense(23, 0, csr.N, O)
    B[5, 3] = np.inf
    B[17, :] = np.nan
    B[40, 270] = -np.inf
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.set_tile_rows(tile_rows)
    fmt.upload(st)
    li = fmt.launch_info(O)
    assert li["split_rows"] > 0 and li["column_slices"] == 2, li
    C = _ex(vs, fmt, B, np.zeros((csr.M, O), np.float32), st, vs.KERNEL_TILE, False)
    assert np.array_equal(np.isnan(C), np.isnan(ref))
    assert np.array_equal(np.isposinf(C), np.isposinf(ref))
    assert np.array_equal(np.isneginf(C), np.isneginf(ref))
    fin = np.isfinite(ref)
    assert np.allclose(C[fin], ref[fin], rtol=1e-5, atol=1e-4)


def test_loaded_format_computes_the_same(gpu, orc, st, tmp_path):
    """A format saved and loaded back (with its tile settings) uploads and
    gives bit-identical results to the format it was saved from."""
    vs = gpu
    rng = np.random.default_rng(3)
    csr = _block_csr(vs, rng, 30, 16, 500, 6, 16, 0.9)
    O = 96
    B = vs.gen_dense(5, 0, csr.N, O)
    fmt = vs.build_vcsr(csr, 16, 16, vs.LAYOUT_TC)
    fmt.set_tile_rows(16)
    path = str(tmp_path / "f.vcsr")
    vs.save_vcsr(fmt, path)
    back = vs.load_vcsr(path)
    outs = []
    for f in (fmt, back):
        f.upload(st)
        assert f.tile_info()[0] == 16
        outs.append(_ex(vs, f, B, np.zeros((csr.M, O), np.float32), st, vs.KERNEL_TILE, False))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert_within_tolerance(outs[1], ref64, csr.row_ptr, csr.val, B, "loaded")


@pytest.mark.parametrize("fixed", [False, True])
@pytest.mark.parametrize("O", [16, 100, 512])
def test_mfma_tiles_are_bit_exact(gpu, orc, st, fixed, O):
    """v_mfma_f32_16x16x4f32 adds its four products to the accumulator one
    after the other with one rounding each, and the tile kernel feeds each
    row's entries in column order, so 16-row tiles that are not split into
    pieces reproduce the oracle's FP32 loop (one fused multiply-add per term
    in CSR order) bit for bit: dense and partly filled 16x16 blocks, and
    fixed windows over a matrix without block structure."""
    vs = gpu
    rng = np.random.default_rng(O + (7 if fixed else 0))
    if fixed:
        csr = _case(vs, orc, rng, 320, 400, density=0.05, dup_rate=0.0, empty_rows=0.1)
    else:
        csr = _block_csr(vs, rng, 20, 16, 640, 12, 16, 0.85)
    B = vs.gen_dense(O + 3, 1, csr.N, O)
    fmt = vs.build_vcsr(csr, 16, 16, vs.LAYOUT_TC)
    fmt.set_tile_rows(16)
    fmt.set_tile_windows(fixed)
    fmt.upload(st)
    R, tiles, entries = fmt.tile_info()
    assert R == 16 and entries <= tiles * 1024  # no tile is split
    got = _ex(vs, fmt, B, np.zeros((csr.M, O), np.float32), st, vs.KERNEL_TILE, False)
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("O", [64, 128, 512])
def test_mfma_schedules_by_waves_per_simd_are_bit_exact(gpu, orc, st, O):
    """The 16-row MFMA tiles run with one of three load schedules, chosen by
    waves per SIMD (1,024 SIMDs on MI355X): the full cfg5 matrix (1,024 tiles
    of 816 entries) has 1,024 waves at O = 64 (4 groups per block, loads kept
    ahead of the MFMAs), 2,048 at O = 128 (2 groups, kept ahead) and 8,192 at
    O = 512 (8 groups, interleaved by the compiler).  Each gives the oracle's
    FP32 loop bit for bit over all of C."""
    vs = gpu
    csr = vs.coo_to_csr(vs.generate_coo(5, 0))
    B = vs.gen_dense(5, 1, csr.N, O)
    fmt = vs.build_vcsr(csr, 16, 16, vs.LAYOUT_TC)
    fmt.upload(st)
    R, tiles, entries = fmt.tile_info()
    assert (R, tiles) == (16, 1024) and entries <= tiles * 1024
    got = _ex(vs, fmt, B, np.zeros((csr.M, O), np.float32), st, vs.KERNEL_TILE, False)
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B, host_threads())
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as hst


@settings(max_examples=40, deadline=None,
          suppress_health_check=[HealthCheck.function_scoped_fixture, HealthCheck.too_slow])
@given(M=hst.integers(1, 300), N=hst.integers(1, 300), bh=hst.sampled_from([1, 2, 3, 4, 8, 16]),
       keep=hst.floats(0.3, 1.0), tile_rows=hst.sampled_from([0, 1, 2, 3, 4, 8, 16]),
       fixed=hst.booleans(), O=hst.sampled_from([1, 3, 8, 16, 31, 64, 100, 128, 257]),
       accumulate=hst.booleans(), seed=hst.integers(0, 2 ** 31 - 1))
def test_tile_kernel_property(gpu, orc, st, M, N, bh, keep, tile_rows, fixed, O, accumulate,
                              seed):
    """Random shapes, block heights, densities, tile heights (automatic,
    forced, fixed windows), widths and accumulate modes: the tile kernel
    (VALU and MFMA paths) agrees with the oracle within the north-star
    tolerance, widened only by what FP32 arithmetic forces on these corner
    cases — the final rounding of C0 + A*B in accumulate mode, and for the
    relative L2 error of a few cancelling short rows the FP32 summation
    bound (the oracle's own FP32 loop exceeds 1e-5 there too)."""
    vs = gpu
    rng = np.random.default_rng(seed)
    nbr = -(-M // bh)
    rows, cols = [], []
    for br in range(nbr):
        for c0 in rng.choice(max(1, N), size=min(N, int(rng.integers(0, 6))), replace=False):
            rr, cc = np.meshgrid(np.arange(bh) + br * bh, np.arange(min(3, N - c0)) + c0,
                                 indexing="ij")
            m = (rng.random(rr.shape) < keep) & (rr < M)
            rows.append(rr[m]); cols.append(cc[m])
    rows = np.concatenate(rows).astype(np.int32) if rows else np.zeros(0, np.int32)
    cols = np.concatenate(cols).astype(np.int32) if cols else np.zeros(0, np.int32)
    key = np.unique(rows.astype(np.int64) * N + cols)
    rows, cols = (key // N).astype(np.int32), (key % N).astype(np.int32)
    vals = rng.uniform(-1, 1, rows.size).astype(np.float32)
    csr = vs.coo_to_csr(vs.Coo.from_arrays(M, N, rows, cols, vals))
    B = vs.gen_dense(int(seed % 1000), 0, N, O)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.set_tile_rows(tile_rows)
    fmt.set_tile_windows(fixed and tile_rows > 0)
    fmt.upload(st)
    C0 = rng.uniform(-1, 1, size=(M, O)).astype(np.float32)
    got = _ex(vs, fmt, B, C0, st, vs.KERNEL_TILE, accumulate).astype(np.float64)
    ref64 = orc.spmm_f64(M, csr.row_ptr, csr.col, csr.val, B)
    slack = np.zeros_like(ref64)
    if accumulate:
        # C = fl32(C0 + s): the difference to C0 is exact in double, and the
        # final FP32 addition adds up to half an ulp of |C0 + s| to it.
        got -= C0.astype(np.float64)
        slack = 2.0 ** -23 * np.abs(C0.astype(np.float64) + ref64)
    if not csr.nnz:
        assert np.abs(got).max(initial=0.0) <= slack.max(initial=0.0)
        return
    what = f"M{M} N{N} bh{bh} R{tile_rows} fixed{fixed} O{O} acc{accumulate}"
    diff = np.abs(got - ref64)
    tol = 1e-4 * row_abs_sums(csr.row_ptr, csr.val)[:, None] * float(np.abs(B).max()) + slack
    assert (diff <= tol).all(), f"{what}: max-abs error {float((diff - tol).max()):.3e} over tolerance"
    # Relative L2 <= 1e-5, or, where the outputs are small against their
    # terms (cancellation in a few short rows), the error bound of FP32
    # summation in any order, n * 2^-24 * (|A||B|), which the CPU's own FP32
    # loop cannot beat either.
    absref = orc.spmm_f64(M, csr.row_ptr, csr.col, np.abs(csr.val), np.abs(B))
    n = int(np.diff(csr.row_ptr).max())
    bound = max(1e-5 * np.linalg.norm(ref64), n * 2.0 ** -24 * np.linalg.norm(absref))
    assert np.linalg.norm(got - ref64) <= bound + np.linalg.norm(slack), f"{what}: rel L2"


@settings(max_examples=60, deadline=None,
          suppress_health_check=[HealthCheck.function_scoped_fixture, HealthCheck.too_slow])
@given(lengths=hst.lists(hst.one_of(hst.integers(0, 4), hst.integers(5, 70),
                                    hst.integers(60, 700)), min_size=1, max_size=90),
       N=hst.integers(1, 900), O=hst.sampled_from([1, 2, 3, 5, 8, 32]),
       accumulate=hst.booleans(), seed=hst.integers(0, 2 ** 31 - 1))
def test_equal_runs_property(gpu, orc, st, lengths, N, O, accumulate, seed):
    """Random mixes of empty, short, one-piece and split rows on single-row
    tiles at the widths that run four work items per wave with equal stream
    runs (O <= 8, and O = 32 with 16-byte lanes): every element of C within
    the north-star bounds of the oracle's double sum, in both C modes
    (accumulate: C0 + A*B, whose final FP32 rounding is allowed for)."""
    vs = gpu
    rng = np.random.default_rng(seed)
    lengths = [min(k, N) for k in lengths]
    csr = _row_lengths_csr(vs, rng, lengths, N)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.set_tile_rows(1)
    fmt.upload(st)
    B = vs.gen_dense(int(seed % 997), 0, N, O)
    C0 = rng.uniform(-1, 1, size=(csr.M, O)).astype(np.float32)
    got = _ex(vs, fmt, B, C0, st, vs.KERNEL_TILE, accumulate).astype(np.float64)
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    slack = np.zeros_like(ref64)
    if accumulate:
        got -= C0.astype(np.float64)
        slack = 2.0 ** -23 * np.abs(C0.astype(np.float64) + ref64)
    what = f"M{csr.M} N{N} nnz{csr.nnz} O{O} acc{accumulate}"
    diff = np.abs(got - ref64)
    tol = 1e-4 * row_abs_sums(csr.row_ptr, csr.val)[:, None] * float(np.abs(B).max()) + slack
    assert (diff <= tol).all(), f"{what}: max-abs error {float((diff - tol).max()):.3e} over tolerance"


def test_launch_info_names_what_runs(gpu, orc, st):
    """vcsr_launch_info_get reports the default kernel's launch shape: the
    row-tile view, column slices of 256 columns (128 once B exceeds 512 MB),
    the matrix-core path for 16-row tiles, and reduce launches and scratch
    only when tiles are split."""
    vs = gpu
    csr = vs.coo_to_csr(vs.generate_coo(1, 0))
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.upload(st)
    r, tiles, entries = fmt.tile_info()
    li = fmt.launch_info(512)
    assert li["kernel"] == vs.KERNEL_TILE and li["tile_rows"] == r
    assert (li["tiles"], li["entries"]) == (tiles, entries)
    assert (li["column_slices"], li["slice_cols"], li["vec"]) == (2, 256, 4)
    assert li["matrix_cores"] == 0 and li["reduce_launches"] == 0 and li["scratch_floats"] == 0
    assert fmt.launch_info(8)["column_slices"] == 1
    assert fmt.launch_info(64, vs.KERNEL_SEGMENT)["kernel"] == vs.KERNEL_SEGMENT
    # Long rows: split tiles, one reduce launch per slice, partial rows x slice width.
    rng = np.random.default_rng(2)
    lens = np.where(np.arange(200) % 10 == 0, 900, 8)
    rows = np.repeat(np.arange(200, dtype=np.int32), lens)
    cols = np.concatenate([rng.choice(5000, size=n, replace=False) for n in lens]).astype(np.int32)
    long = vs.coo_to_csr(vs.Coo.from_arrays(200, 5000, rows, cols,
                                            rng.uniform(-1, 1, rows.size).astype(np.float32)))
    f2 = vs.build_vcsr(long, 4, 64, vs.LAYOUT_S)
    f2.upload(st)
    li2 = f2.launch_info(300)
    assert li2["column_slices"] == 2 and li2["reduce_launches"] == 2 and li2["split_rows"] == 20
    assert li2["scratch_floats"] > 0 and li2["scratch_floats"] % 256 == 0
    # 16-row dense blocks run on the matrix cores, never column-sliced.
    blk = _block_csr(vs, rng, 8, 16, 256, 4, 16, 1.0)
    f3 = vs.build_vcsr(blk, 16, 16, vs.LAYOUT_TC)
    f3.upload(st)
    li3 = f3.launch_info(512)
    assert li3["tile_rows"] == 16 and li3["matrix_cores"] == 1 and li3["column_slices"] == 1
    # Split 16-row tiles: column slices of 256 and one reduce launch each.
    f4 = vs.build_vcsr(_block_csr(vs, rng, 6, 8, 4096, 600, 4, 0.9), 4, 64, vs.LAYOUT_S)
    f4.set_tile_rows(16)
    f4.upload(st)
    li4 = f4.launch_info(520)
    assert li4["matrix_cores"] == 1 and li4["split_rows"] > 0
    assert li4["column_slices"] == 3 and li4["reduce_launches"] == 3



@pytest.mark.parametrize("where", ["products", "inputs"])
@pytest.mark.parametrize("kind,tile_rows", [("csr", 0), ("tile", 1), ("tile", 3), ("tile", 16),
                                            ("row", 0), ("segment", 0), ("mfma", 0)])
def test_denormals_are_kept(gpu, orc, st, kind, tile_rows, where):
    """FP32 denormals are kept, as by the reference's CUDA kernels (built
    without fast-math).  "products": A and B are normal (~2^-64) but every
    product and partial sum is below the smallest normal, 2^-126;
    "inputs": B itself is denormal (~2^-140) and A ~2^12.  A flush to zero
    anywhere gives a relative L2 error near 1; kept denormals leave the
    north-star bounds met (the denormal grid, 2^-149, is ~2^-20 of these
    sums).  The naive CSR kernel is also the oracle's FP32 loop bit for
    bit."""
    vs = gpu
    print(f"denormals {where} {kind} R={tile_rows}", flush=True)
    rng = np.random.default_rng(77 + tile_rows)
    csr = _block_csr(vs, rng, 12, 16, 160, 4, 16, 0.7)
    a_exp, b_exp = (-64, -64) if where == "products" else (12, -140)
    val = (csr.val * np.float32(2.0 ** a_exp)).astype(np.float32)
    csr = vs.Csr.from_arrays(csr.M, csr.N, csr.row_ptr, csr.col, val)
    O = 40
    B = (vs.gen_dense(78, 0, csr.N, O).astype(np.float64) * 2.0 ** b_exp).astype(np.float32)
    tiny = np.finfo(np.float32).tiny
    if where == "inputs":
        assert np.count_nonzero((B != 0) & (np.abs(B) < tiny)) == np.count_nonzero(B)
    ref32 = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert np.count_nonzero(ref32) > 0.9 * ref32.size
    assert np.median(np.abs(ref32[ref32 != 0])) < tiny
    C = _run(vs, kind, csr, B, st, tile_rows=tile_rows)
    if kind == "csr":
        assert np.array_equal(C.view(np.uint32), ref32.view(np.uint32))
    ref64 = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert_within_tolerance(C, ref64, csr.row_ptr, csr.val, B, f"denormal {where} {kind}")
