"""spmm_vcsr_noalloc (the default kernel with its split-tile scratch in the
library's fixed per-device array instead of allocated memory) against
spmm_vcsr_ex with the same kernel, through the C ABI: two calls in a row,
the second on a smaller input, both C modes; a format whose split tiles
need more than the array holds is refused before any launch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_within_tolerance, block_csr, capture, hip_runtime

pytestmark = pytest.mark.gpu


def _long_row_csr(vs, seed, M, N, every, long_len, short_len):
    """Rows of short_len uniform columns, every `every`-th row long_len:
    the long rows' 1-row tiles are cut into pieces that write partial rows
    (the scratch), summed by the reduce kernel."""
    rng = np.random.default_rng(seed)
    lens = np.where(np.arange(M) % every == 3, long_len, short_len)
    rows = np.repeat(np.arange(M, dtype=np.int32), lens)
    cols = np.concatenate([rng.choice(N, size=n, replace=False) for n in lens]).astype(np.int32)
    vals = rng.uniform(-1, 1, size=rows.size).astype(np.float32)
    return vs.coo_to_csr(vs.Coo.from_arrays(M, N, rows, cols, vals))


def _both(vs, st, csr, O, accumulate, seed):
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.upload(st)
    B = vs.gen_dense(seed, 0, csr.N, O)
    C0 = vs.gen_dense(seed + 1, 0, csr.M, O)
    dB = vs.DeviceArray.from_numpy(B, st)
    d_ref = vs.DeviceArray.from_numpy(C0, st)
    d_got = vs.DeviceArray.from_numpy(C0, st)
    vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, 64, d_ref, st, kernel=vs.KERNEL_TILE,
                            accumulate=accumulate)
    vs.run_vcsr_spmm_gpu_noalloc(fmt, dB, O, d_got, st, accumulate=accumulate)
    st.sync()
    return fmt, B, C0, d_ref.numpy(st), d_got.numpy(st)


@pytest.mark.parametrize("accumulate", [False, True])
def test_noalloc_matches_the_allocating_entry_point(gpu, orc, accumulate):
    vs = gpu
    st = vs.Stream()
    print(f"noalloc: call 1, 600 rows with split tiles, O=200, accumulate={accumulate}", flush=True)
    big = _long_row_csr(vs, 11, 600, 60000, 20, 2500, 16)
    fmt, B, C0, ref, got = _both(vs, st, big, 200, accumulate, 21)
    assert fmt.tile_info()[0] == 1
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # The result is the product (not only the same as the other entry point).
    want = orc.spmm_f64(big.M, big.row_ptr, big.col, big.val, B)
    if accumulate:
        want = want + C0.astype(np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel <= 1e-5, rel
    print(f"noalloc: call 2, 90 rows, O=64, accumulate={accumulate}", flush=True)
    small = _long_row_csr(vs, 12, 90, 9000, 7, 700, 5)
    _, B2, C02, ref2, got2 = _both(vs, st, small, 64, accumulate, 31)
    assert np.array_equal(got2.view(np.uint32), ref2.view(np.uint32))
    want2 = orc.spmm_f64(small.M, small.row_ptr, small.col, small.val, B2)
    if accumulate:
        want2 = want2 + C02.astype(np.float64)
    assert np.linalg.norm(got2 - want2) <= 1e-5 * np.linalg.norm(want2)


def test_noalloc_refuses_more_scratch_than_it_holds(gpu):
    """300 rows of 3,600 columns at O = 256: 17,100 partial rows of 256
    floats (4.38 Mi floats) exceed the 4 Mi-float array: VCSR_ERANGE, C
    untouched; spmm_vcsr_ex (which allocates) still computes it."""
    vs = gpu
    st = vs.Stream()
    csr = _long_row_csr(vs, 13, 300, 100000, 1, 3600, 3600)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.upload(st)
    O = 256
    dB = vs.DeviceArray.from_numpy(vs.gen_dense(41, 0, csr.N, O), st)
    dC = vs.DeviceArray((csr.M, O), np.float32)
    dC.zero(st)
    with pytest.raises(vs.VcsrError) as e:
        vs.run_vcsr_spmm_gpu_noalloc(fmt, dB, O, dC, st)
    assert e.value.code == vs.VCSR_ERANGE
    assert "scratch" in str(e.value)
    st.sync()
    assert not dC.numpy(st).any()
    vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, 64, dC, st, kernel=vs.KERNEL_TILE, accumulate=False)
    st.sync()
    assert np.isfinite(dC.numpy(st)).all() and dC.numpy(st).any()
    # A null format is refused the same way as by the other entry points.
    lib = vs.load_library()
    assert lib.spmm_vcsr_noalloc(None, dB.ptr, O, dC.ptr, st.h, 0) == vs.VCSR_EINVAL


def test_noalloc_replays_in_a_hip_graph(gpu, orc):
    """The caller the entry point is for: spmm_vcsr_noalloc captured into a
    HIP graph (global capture mode, in which an allocation or a
    synchronising call in the capture fails it) holds kernel nodes only,
    and every replay gives the eager call's C bit for bit — with C refilled
    with NaN before each replay and another eager product through the same
    scratch array between replays."""
    vs = gpu
    st = vs.Stream()
    lib = vs.load_library()
    print("noalloc graph: 400 rows with split tiles, O=200", flush=True)
    csr = _long_row_csr(vs, 14, 400, 50000, 9, 2000, 16)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.upload(st)
    O = 200
    B = vs.gen_dense(51, 0, csr.N, O)
    dB = vs.DeviceArray.from_numpy(B, st)
    d_eager = vs.DeviceArray((csr.M, O), np.float32)
    d_graph = vs.DeviceArray((csr.M, O), np.float32)
    # The eager call also looks up the scratch array's address before capture.
    vs.run_vcsr_spmm_gpu_noalloc(fmt, dB, O, d_eager, st)
    st.sync()
    ref = d_eager.numpy(st)
    want = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert np.linalg.norm(ref - want) <= 1e-5 * np.linalg.norm(want)

    other = _long_row_csr(vs, 15, 120, 20000, 5, 900, 8)
    ofmt = vs.build_vcsr(other, 4, 64, vs.LAYOUT_S)
    ofmt.upload(st)
    oB = vs.DeviceArray.from_numpy(vs.gen_dense(52, 0, other.N, 96), st)
    oC = vs.DeviceArray((other.M, 96), np.float32)
    vs.run_vcsr_spmm_gpu_noalloc(ofmt, oB, 96, oC, st)
    st.sync()
    oref = oC.numpy(st)

    hip = hip_runtime()
    graph, gexec = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipStreamBeginCapture(st.h, 0) == 0  # hipStreamCaptureModeGlobal
    try:
        vs.run_vcsr_spmm_gpu_noalloc(fmt, dB, O, d_graph, st)
    finally:
        rc_end = hip.hipStreamEndCapture(st.h, ctypes.byref(graph))
    assert rc_end == 0 and graph.value
    try:
        n = ctypes.c_size_t(0)
        assert hip.hipGraphGetNodes(graph, None, ctypes.byref(n)) == 0
        nodes = (ctypes.c_void_p * n.value)()
        assert hip.hipGraphGetNodes(graph, nodes, ctypes.byref(n)) == 0
        kinds = []
        for i in range(n.value):
            t = ctypes.c_int(-1)
            assert hip.hipGraphNodeGetType(nodes[i], ctypes.byref(t)) == 0
            kinds.append(t.value)
        print(f"noalloc graph: {n.value} nodes, types {kinds}", flush=True)
        assert n.value >= 2 and all(k == 0 for k in kinds)  # tile + reduce kernels only
        assert hip.hipGraphInstantiateWithFlags(ctypes.byref(gexec), graph, 0) == 0
        nan = np.full((csr.M, O), np.nan, np.float32)
        for rep in range(3):
            print(f"noalloc graph: replay {rep}", flush=True)
            assert lib.vcsr_memcpy_h2d(d_graph.ptr, nan.ctypes.data, d_graph.nbytes, st.h) == 0
            vs.run_vcsr_spmm_gpu_noalloc(ofmt, oB, 96, oC, st)
            assert hip.hipGraphLaunch(gexec, st.h) == 0
            st.sync()
            assert np.array_equal(d_graph.numpy(st).view(np.uint32), ref.view(np.uint32)), rep
            assert np.array_equal(oC.numpy(st).view(np.uint32), oref.view(np.uint32)), rep
    finally:
        if gexec.value:
            hip.hipGraphExecDestroy(gexec)
        hip.hipGraphDestroy(graph)


@pytest.mark.parametrize("case", ["1-row tiles, two column slices", "split 16-row tiles"])
def test_noalloc_column_slices_and_16_row_tiles(gpu, orc, case):
    """The scratch array reused across launches of one call: O = 512 on a
    format with split 1-row tiles is two column slices, each a tile launch
    and a reduce through the same array; split 16-row tiles (MFMA) write
    16 partial rows per piece.  Bit for bit against spmm_vcsr_ex, and the
    product within the north-star bounds of the oracle."""
    vs = gpu
    st = vs.Stream()
    rng = np.random.default_rng(61)
    if case.startswith("1-row"):
        csr, O, rows = _long_row_csr(vs, 16, 300, 30000, 10, 2500, 16), 512, 0
    else:
        csr, O, rows = block_csr(vs, rng, 6, 8, 4096, 600, 4, 0.9), 320, 16
    print(f"noalloc: {case}, O={O}", flush=True)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    fmt.set_tile_rows(rows)
    fmt.upload(st)
    li = fmt.launch_info(O)
    assert li["split_rows"] > 0 and li["column_slices"] == 2, li
    assert li["matrix_cores"] == (rows == 16)
    B = vs.gen_dense(62, 0, csr.N, O)
    dB = vs.DeviceArray.from_numpy(B, st)
    d_ref = vs.DeviceArray((csr.M, O), np.float32)
    d_got = vs.DeviceArray((csr.M, O), np.float32)
    nan = np.full((csr.M, O), np.nan, np.float32)
    lib = vs.load_library()
    assert lib.vcsr_memcpy_h2d(d_got.ptr, nan.ctypes.data, d_got.nbytes, st.h) == 0
    vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, 64, d_ref, st, kernel=vs.KERNEL_TILE, accumulate=False)
    vs.run_vcsr_spmm_gpu_noalloc(fmt, dB, O, d_got, st)
    st.sync()
    got, ref = d_got.numpy(st), d_ref.numpy(st)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    want = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert_within_tolerance(got, want, csr.row_ptr, csr.val, B, case)


_FRESH_CAPTURE = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from conftest import capture, hip_runtime, load_product
vs = load_product()
vs.load_library()
rng = np.random.default_rng(71)
M, N, O = 200, 30000, 96
lens = np.where(np.arange(M) % 8 == 3, 1500, 12)
rows = np.repeat(np.arange(M, dtype=np.int32), lens)
cols = np.concatenate([rng.choice(N, size=n, replace=False) for n in lens]).astype(np.int32)
vals = rng.uniform(-1, 1, size=rows.size).astype(np.float32)
csr = vs.coo_to_csr(vs.Coo.from_arrays(M, N, rows, cols, vals))
st = vs.Stream()
fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
fmt.upload(st)
dB = vs.DeviceArray.from_numpy(vs.gen_dense(72, 0, N, O), st)
d_graph = vs.DeviceArray((M, O), np.float32)
d_eager = vs.DeviceArray((M, O), np.float32)
st.sync()
hip = hip_runtime()
# The process's first spmm_vcsr_noalloc call is the captured one.
graph, kinds = capture(hip, st, lambda: vs.run_vcsr_spmm_gpu_noalloc(fmt, dB, O, d_graph, st))
assert kinds and all(k == 0 for k in kinds), kinds
import ctypes
gexec = ctypes.c_void_p()
assert hip.hipGraphInstantiateWithFlags(ctypes.byref(gexec), graph, 0) == 0
assert hip.hipGraphLaunch(gexec, st.h) == 0
st.sync()
vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, 64, d_eager, st, kernel=vs.KERNEL_TILE, accumulate=False)
st.sync()
g, e = d_graph.numpy(st), d_eager.numpy(st)
assert np.array_equal(g.view(np.uint32), e.view(np.uint32))
hip.hipGraphExecDestroy(gexec)
hip.hipGraphDestroy(graph)
print("fresh capture OK", len(kinds), "kernel nodes", flush=True)
"""


def test_noalloc_first_call_under_capture_in_a_fresh_process(gpu):
    """In a process whose first spmm_vcsr_noalloc call is made under graph
    capture (the upload has already looked up the scratch array's address),
    the capture holds kernel nodes only and its replay equals the eager
    spmm_vcsr_ex result bit for bit."""
    import os
    import subprocess
    import sys
    tests_dir = os.path.dirname(os.path.abspath(__file__))
    r = subprocess.run([sys.executable, "-c", _FRESH_CAPTURE, tests_dir], capture_output=True,
                       text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "fresh capture OK" in r.stdout
