"""Shared fixtures: the product binding (vcsr-spmm_amd, via ctypes), the CPU
oracle (test infrastructure), and the tolerance check of the north star."""
from __future__ import annotations

import ctypes
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box only)")


def load_product():
    """Imports vcsr-spmm_amd/ (a directory name with a hyphen) as vcsr_spmm_amd."""
    name = "vcsr_spmm_amd"
    if name in sys.modules:
        return sys.modules[name]
    path = os.path.join(ROOT, "vcsr-spmm_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def vs():
    mod = load_product()
    mod.load_library()
    return mod


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.oracle_lib()
    return oracle


@pytest.fixture(scope="session")
def gpu(vs):
    if vs.device_count() <= 0:
        pytest.fail("no GPU visible to the library (gpu tests run on the GPU box)")
    return vs


def tolerance_report(C, ref64, row_l1, bmax):
    """rel L2 <= 1e-5 and, per row r, max-abs error
    <= 1e-4 * ||A_r||_1 * max|B|.  Returns (rel_l2, worst max-abs/tol)."""
    C = np.asarray(C, dtype=np.float64)
    diff = C - ref64
    den = np.linalg.norm(ref64)
    rel = np.linalg.norm(diff) / den if den > 0 else np.linalg.norm(diff)
    tol = 1e-4 * np.asarray(row_l1, dtype=np.float64)[:, None] * bmax
    err = np.abs(diff)
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(tol > 0, err / tol, np.where(err > 0, np.inf, 0.0))
    return float(rel), float(ratio.max()) if ratio.size else 0.0


def row_abs_sums(row_ptr, val):
    """||A_r||_1 for every row (empty rows give 0)."""
    M = len(row_ptr) - 1
    rows = np.repeat(np.arange(M), np.diff(row_ptr))
    return np.bincount(rows, weights=np.abs(np.asarray(val, dtype=np.float64)), minlength=M)


def host_threads():
    """Threads for the oracle's whole-matrix products: the cores this
    process may use, at most 16 (one GPU's share of the GPU box's host) and
    at most OMP_NUM_THREADS when that is set."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, min(n, 16))


def assert_within_tolerance(C, ref64, row_ptr, val, B, what=""):
    row_l1 = row_abs_sums(row_ptr, val)
    bmax = float(np.abs(B).max()) if B.size else 0.0
    rel, worst = tolerance_report(C, ref64, row_l1, bmax)
    assert rel <= 1e-5, f"{what}: rel L2 {rel:.3e} > 1e-5"
    assert worst <= 1.0, f"{what}: max-abs error {worst:.3f} x tolerance"
    return rel, worst


def random_csr(rng, M, N, density=0.05, dup_rate=0.0, empty_rows=0.0, max_row=None):
    """Random COO arrays (rows, cols, vals), rows ascending and each row's
    columns shuffled, duplicates allowed: the unsorted input the reference's
    COO -> CSR conversion takes."""
    rows, cols = [], []
    for r in range(M):
        if rng.random() < empty_rows:
            continue
        k = rng.binomial(N, density) if max_row is None else rng.integers(0, max_row + 1)
        k = min(k, N)
        c = rng.choice(N, size=k, replace=False) if k else np.zeros(0, np.int64)
        if dup_rate and k:
            extra = c[rng.random(k) < dup_rate]
            c = np.concatenate([c, extra])
        rng.shuffle(c)
        rows.extend([r] * len(c))
        cols.extend(c.tolist())
    rows = np.array(rows, dtype=np.int32)
    cols = np.array(cols, dtype=np.int32)
    vals = rng.uniform(-1, 1, size=len(rows)).astype(np.float32)
    return rows, cols, vals


def hip_runtime():
    """The HIP runtime the library is linked against (already loaded with
    it), for the graph-capture calls the tests make; the library itself
    exports no graph API."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64.so" in parts[-1]:
                paths.add(parts[-1])
    assert len(paths) == 1, paths
    hip = ctypes.CDLL(paths.pop())
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    sigs = {"hipStreamBeginCapture": [vp, ctypes.c_int],
            "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
            "hipGraphGetNodes": [vp, vp, ctypes.POINTER(sz)],
            "hipGraphNodeGetType": [vp, ctypes.POINTER(ctypes.c_int)],
            "hipGraphInstantiateWithFlags": [ctypes.POINTER(vp), vp, ctypes.c_ulonglong],
            "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp],
            "hipGraphDestroy": [vp]}
    for name, args in sigs.items():
        fn = getattr(hip, name)
        fn.argtypes, fn.restype = args, ctypes.c_int
    return hip


def capture(hip, stream, enqueue):
    """Captures what enqueue() puts on `stream` into a HIP graph in global
    capture mode (an allocation or a synchronising call in the capture makes
    it fail) and returns (graph, node types); 0 is a kernel node."""
    graph = ctypes.c_void_p()
    assert hip.hipStreamBeginCapture(stream.h, 0) == 0  # hipStreamCaptureModeGlobal
    try:
        enqueue()
    finally:
        rc_end = hip.hipStreamEndCapture(stream.h, ctypes.byref(graph))
    assert rc_end == 0 and graph.value, f"capture failed: hipStreamEndCapture {rc_end}"
    n = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(graph, None, ctypes.byref(n)) == 0
    nodes = (ctypes.c_void_p * n.value)()
    assert hip.hipGraphGetNodes(graph, nodes, ctypes.byref(n)) == 0
    kinds = []
    for i in range(n.value):
        t = ctypes.c_int(-1)
        assert hip.hipGraphNodeGetType(nodes[i], ctypes.byref(t)) == 0
        kinds.append(t.value)
    return graph, kinds


def block_csr(vs, rng, nbr, bh, N, blocks_per_row, bw, keep):
    """Block-structured matrix: nbr block rows of height bh, each with
    `blocks_per_row` bh x bw blocks at random block columns; every entry is
    kept with probability `keep`, so rows of a block row share most but not
    all of their columns."""
    rows, cols = [], []
    nbc = max(1, N // bw)
    for br in range(nbr):
        for bc in rng.choice(nbc, size=min(blocks_per_row, nbc), replace=False):
            rr, cc = np.meshgrid(np.arange(bh) + br * bh, np.arange(bw) + bc * bw, indexing="ij")
            m = rng.random(rr.shape) < keep
            rows.append(rr[m]); cols.append(cc[m])
    rows = np.concatenate(rows).astype(np.int32)
    cols = np.concatenate(cols).astype(np.int32)
    vals = rng.uniform(-1, 1, rows.size).astype(np.float32)
    return vs.coo_to_csr(vs.Coo.from_arrays(nbr * bh, N, rows, cols, vals))
