"""spmm_vcsr_ex only enqueues kernels: its first call at a new O, with the
row-stationary kernel on split rows or the tile kernel on split 16-row
tiles, is captured into a HIP graph in global capture mode (where a
synchronising call or an allocation in the capture makes it fail), the
graph holds kernel nodes only, and every replay gives the whole C within
the north-star bounds of the oracle and bit for bit what an eager call
gives.  The partial rows of split rows and tiles are sized at upload for
every O (such formats are launched in column slices of at most 256
columns); the reference uploads once and never allocates per call
(src/vcsr_seg.cu:196-211)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_within_tolerance, block_csr, capture, hip_runtime

pytestmark = pytest.mark.gpu


def _dense_rows_csr(vs, rng):
    """40 sparse rows, three of which have every one of 3,000 columns:
    750 (row, segment) pairs each, split over several row work items."""
    M, N = 40, 3000
    rows = np.repeat(np.arange(M, dtype=np.int32), 30)
    cols = rng.integers(0, N, size=rows.size).astype(np.int32)
    for r in (0, 7, 39):
        rows = np.concatenate([rows, np.full(N, r, np.int32)])
        cols = np.concatenate([cols, np.arange(N, dtype=np.int32)])
    vals = rng.uniform(-1, 1, size=rows.size).astype(np.float32)
    return vs.coo_to_csr(vs.Coo.from_arrays(M, N, rows, cols, vals))


@pytest.mark.parametrize("case", ["row kernel, split rows", "tile kernel, split 16-row tiles"])
def test_first_call_at_each_o_captures_into_a_graph(gpu, orc, case):
    vs = gpu
    st = vs.Stream()
    lib = vs.load_library()
    hip = hip_runtime()
    rng = np.random.default_rng(81)
    if case.startswith("row"):
        csr, kernel, rows = _dense_rows_csr(vs, rng), vs.KERNEL_ROW, 0
    else:
        csr, kernel, rows = block_csr(vs, rng, 6, 8, 4096, 600, 4, 0.9), vs.KERNEL_TILE, 16
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.set_tile_rows(rows)
    fmt.upload(st)
    if rows == 16:
        li = fmt.launch_info(520, kernel)
        assert li["matrix_cores"] == 1 and li["split_rows"] > 0, li
    for O in (64, 520):
        print(f"capture: {case}, first call at O={O}", flush=True)
        B = vs.gen_dense(O + 1, 0, csr.N, O)
        dB = vs.DeviceArray.from_numpy(B, st)
        d_graph = vs.DeviceArray((csr.M, O), np.float32)
        d_eager = vs.DeviceArray((csr.M, O), np.float32)
        st.sync()
        graph, kinds = capture(hip, st, lambda: vs.run_vcsr_spmm_gpu_ex(
            fmt, dB, O, 64, d_graph, st, kernel=kernel, accumulate=False))
        gexec = ctypes.c_void_p()
        try:
            print(f"capture: {len(kinds)} nodes, types {kinds}", flush=True)
            assert kinds and all(k == 0 for k in kinds), kinds  # kernel nodes only
            assert hip.hipGraphInstantiateWithFlags(ctypes.byref(gexec), graph, 0) == 0
            want = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
            nan = np.full((csr.M, O), np.nan, np.float32)
            replays = []
            for rep in range(2):
                assert lib.vcsr_memcpy_h2d(d_graph.ptr, nan.ctypes.data, d_graph.nbytes,
                                           st.h) == 0
                assert hip.hipGraphLaunch(gexec, st.h) == 0
                st.sync()
                got = d_graph.numpy(st)
                assert_within_tolerance(got, want, csr.row_ptr, csr.val, B,
                                        f"{case} O={O} replay {rep}")
                replays.append(got)
            vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, 64, d_eager, st, kernel=kernel, accumulate=False)
            st.sync()
            eager = d_eager.numpy(st)
            for got in replays:
                assert np.array_equal(got.view(np.uint32), eager.view(np.uint32))
        finally:
            if gexec.value:
                hip.hipGraphExecDestroy(gexec)
            hip.hipGraphDestroy(graph)


@pytest.mark.parametrize("kernel", [1, 2])
def test_segment_major_overwrite_captures_into_a_graph(gpu, orc, kernel):
    """accumulate = 0 on the segment-major kernels (which add into C) clears
    C with a fill kernel, not a memset node, so the call captures as kernel
    nodes only and a replay over a C full of NaN gives the product."""
    vs = gpu
    st = vs.Stream()
    lib = vs.load_library()
    hip = hip_runtime()
    rng = np.random.default_rng(90 + kernel)
    csr = _dense_rows_csr(vs, rng)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.upload(st)
    O = 96
    B = vs.gen_dense(91, 0, csr.N, O)
    dB = vs.DeviceArray.from_numpy(B, st)
    dC = vs.DeviceArray((csr.M, O), np.float32)
    st.sync()
    graph, kinds = capture(hip, st, lambda: vs.run_vcsr_spmm_gpu_ex(
        fmt, dB, O, 64, dC, st, kernel=kernel, accumulate=False))
    gexec = ctypes.c_void_p()
    try:
        assert kinds and all(k == 0 for k in kinds), kinds
        assert hip.hipGraphInstantiateWithFlags(ctypes.byref(gexec), graph, 0) == 0
        want = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
        nan = np.full((csr.M, O), np.nan, np.float32)
        for rep in range(2):
            assert lib.vcsr_memcpy_h2d(dC.ptr, nan.ctypes.data, dC.nbytes, st.h) == 0
            assert hip.hipGraphLaunch(gexec, st.h) == 0
            st.sync()
            assert_within_tolerance(dC.numpy(st), want, csr.row_ptr, csr.val, B,
                                    f"kernel {kernel} replay {rep}")
    finally:
        if gexec.value:
            hip.hipGraphExecDestroy(gexec)
        hip.hipGraphDestroy(graph)
