"""bench.py's correctness gate, on the CPU: the whole-C check passes the
oracle's own FP32 product and fails a C with one element off by more than
the north-star per-row bound, or with a large relative error; the CPU
baseline's thread count stays within one GPU's share of the host."""
from __future__ import annotations

import importlib.util
import os

import numpy as np
import pytest

from conftest import ROOT


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_whole_c_check(bench, vs, orc):
    csr = vs.coo_to_csr(vs.generate_coo(1, 0))
    B = vs.gen_dense(1, 0, csr.N, 16)
    C = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    rel, worst = bench.full_check(orc, csr, B, C, 2)
    assert rel <= 1e-6 and worst < 0.05
    # One element off by twice its row's bound fails the max-abs test only.
    row_l1 = np.abs(csr.val[csr.row_ptr[7]:csr.row_ptr[8]].astype(np.float64)).sum()
    bad = C.copy()
    bad[7, 3] += np.float32(2e-4 * row_l1 * np.abs(B).max())
    rel, worst = bench.full_check(orc, csr, B, bad, 2)
    assert worst > 1.0
    # A C that is wrong everywhere fails the relative L2 test too.
    rel, worst = bench.full_check(orc, csr, B, C * np.float32(1.001), 2)
    assert rel > 1e-5 and worst > 1.0


def test_cpu_baseline_threads(bench):
    n = bench.host_threads()
    assert 1 <= n <= 16
    d = bench.host_description()
    assert set(d) == {"cpu_model", "nproc", "affinity_cpus"}
