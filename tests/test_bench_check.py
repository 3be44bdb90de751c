"""bench.py's correctness gate, on the CPU: the whole-C check passes the
oracle's own FP32 product and fails a C with one element off by more than
the north-star per-row bound, or with a large relative error; the CPU
baseline's thread count stays within one GPU's share of the host.  On the
GPU: the fields of its one JSON line."""
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


def test_slice_probe_library_rejects_bad_shapes():
    """bench.py's slice-read probe (lib/libvcsr_probe.so, built beside the
    library) loads and refuses, before any GPU call, the shapes its kernel
    cannot read in bounds: a vector width other than 1, 2 or 4 floats, a
    slice that is not a power-of-two number of lanes up to 64, a buffer
    smaller than one slice, and no output pointers."""
    import ctypes as C
    path = os.path.join(ROOT, "vcsr-spmm_amd", "lib", "libvcsr_probe.so")
    if not os.path.exists(path):
        pytest.skip("probe library not built (run __graft_entry__.build())")
    fn = C.CDLL(path).vcsr_probe_slice_reads
    fn.argtypes = [C.c_uint64, C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_double),
                   C.POINTER(C.c_double)]
    fn.restype = C.c_int
    r, m = C.c_double(), C.c_double()
    for nbytes, floats, vec, reps in [(1 << 20, 128, 3, 5), (1 << 20, 96, 4, 5),
                                      (1 << 20, 512, 4, 5), (1 << 20, 2, 4, 5),
                                      (256, 128, 4, 5), (1 << 20, 128, 4, 0)]:
        assert fn(nbytes, floats, vec, reps, C.byref(r), C.byref(m)) == 1, (nbytes, floats, vec)
    assert fn(1 << 20, 128, 4, 5, None, None) == 1


@pytest.mark.gpu
def test_bench_line_contract():
    """On the GPU: bench.py's one JSON line (short run) carries what the
    benchmark contract asks for — the BASELINE metric and unit, steps and
    warm-up as given, a whole-C check that passed, the HBM roofline with
    live and counter-derived figures, and the CPU baseline on this host."""
    import json
    import subprocess
    import sys
    print("bench.py --steps 3 --warmup 1 --cpu-seconds 1", flush=True)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--steps", "3",
                        "--warmup", "1", "--cpu-seconds", "1"],
                       capture_output=True, text=True, timeout=600, cwd=ROOT)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    lines = [x for x in r.stdout.splitlines() if x.startswith("{")]
    assert len(lines) == 1, r.stdout[-2000:]
    d = json.loads(lines[0])
    assert d["metric"].startswith("SpMM GFLOP/s") and d["unit"] == "GFLOP/s"
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1
    assert d["higher_is_better"] is True and d["dtype"] == "f32" and d["vs_baseline"] is None
    assert d["value"] > 0 and d["ms_per_step"] > 0 and d["ms_per_step_median"] > 0
    assert d["config"]["workload"].startswith("cfg2") and "O=128" in d["config"]["workload"]
    assert d["check"]["rows"] == "all" and d["check"]["result"] == "pass"
    roof = d["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert roof["traffic"] and roof["traffic"] > 0
    assert roof["traffic_source"]["commit"] and "kernel_sources_match" in roof["traffic_source"]
    assert roof["copy_gbs"] > 0 and 0 < roof["frac_of_copy"] < 1.5
    # The B-row slice path that binds the tile kernel, against the probe.
    sp = roof["b_slice_path"]
    assert sp["slice_bytes"] == 512 and sp["vec_floats"] == 4
    assert sp["probe_l2_resident_tb_s"] > 0 and sp["probe_b_sized_tb_s"] > 0
    assert 0 < sp["frac_of_l2_resident"] < 1.2
    assert abs(sp["frac_of_l2_resident"] - sp["kernel_tb_s"] / sp["probe_l2_resident_tb_s"]) < 0.02
    cpu = d["cpu_baseline"]
    assert cpu["kind"] == "port" and cpu["value"] > 0 and cpu["cores"] >= 1
    assert cpu["single_thread"]["cores"] == 1 and cpu["host"]
    # The north star's other points, timed in the same run and checked over
    # all of C: config 3 at O = 128, naive CSR on configs 2 and 3 with the
    # VCSR / naive speed-up, config 5 at O = 512 with its MFMA utilisation.
    ex = d["extra"]
    for key in ("cfg2_o128_csr_naive", "cfg2_o128_rocsparse", "cfg3_o128", "cfg3_o128_csr_naive",
                "cfg5_o512"):
        assert ex[key]["check"]["rows"] == "all" and ex[key]["check"]["result"] == "pass", key
        assert ex[key]["kernel_ms"] > 0, key
    assert ex["cfg3_o128"]["workload"].startswith("cfg3") and "O=128" in ex["cfg3_o128"]["workload"]
    assert 0 < ex["cfg3_o128"]["hbm_roofline_frac"] < 1
    assert ex["vcsr_over_naive"]["cfg2_o128"] >= 1.5 and ex["vcsr_over_naive"]["cfg3_o128"] >= 1.5
    assert ex["vcsr_over_rocsparse"]["cfg2_o128"] > 0
    m5 = ex["cfg5_o512"]["mfma"]
    assert "O=512" in ex["cfg5_o512"]["workload"] and 0 < m5["useful_frac_of_peak"] <= 1


def test_traffic_provenance(bench, tmp_path, monkeypatch):
    """roofline.traffic comes with the commit its counters were taken on and
    whether this tree's tile-kernel sources hash to the recorded value; a
    point without a counter set gives none."""
    t, prov = bench.measured_traffic("cfg2", "vcsr")
    assert t and t > 0 and prov["commit"] and prov["profile"]
    assert isinstance(prov["kernel_sources_match"], bool)
    assert bench.measured_traffic("cfg2", "nope") == (None, None)
    h = bench.kernel_sources_sha16()
    assert len(h) == 16 and int(h, 16) >= 0
