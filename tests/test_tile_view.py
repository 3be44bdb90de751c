"""CPU checks of the row-tile view (vcsr-spmm_amd/csrc/host/tile_view.cpp),
the index structure the tile-stationary kernel walks: built from the VCSR
arrays, it must hold exactly the CSR's nonzeros, cover every row once, and
respect the work-item limits the kernel's LDS arrays are sized for; with
fixed 16-row windows it must be FastSpMM's condensed tiles as the oracle
restates them.  The checker (tests/native/tile_view_check.cpp) links the
library's host objects and the oracle's source; no GPU is used."""
from __future__ import annotations

import glob
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vcsr-spmm_amd")
ORACLE_SRC = os.path.join(ROOT, "oracle", "vcsr_oracle.cpp")


def test_tile_view_builder(tmp_path):
    objs = sorted(glob.glob(os.path.join(PKG, "_build", "host", "*.o")))
    if not objs:
        pytest.skip("host objects not built (run __graft_entry__.build())")
    exe = tmp_path / "tile_view_check"
    src = os.path.join(ROOT, "tests", "native", "tile_view_check.cpp")
    subprocess.run(["g++", "-std=c++17", "-O2", "-march=x86-64-v3", "-o", str(exe), src, ORACLE_SRC, *objs,
                    "-lpthread"], check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "ALL OK" in r.stdout, r.stdout[-4000:] + r.stderr[-2000:]


def test_host_code_under_address_and_ub_sanitizers(tmp_path):
    """The host C++ layer (generators, COO->CSR, the three VCSR builders and
    the row-tile view, multi-threaded) built with AddressSanitizer and
    UndefinedBehaviorSanitizer, driven by the view checker: no memory error,
    leak or undefined behaviour on its cases.  g++ only; no HIP code."""
    srcs = [os.path.join(PKG, "csrc", "host", f) for f in
            ("mtx.cpp", "csr.cpp", "vcsr_build.cpp", "gen.cpp", "cpu_spmm.cpp", "tile_view.cpp")]
    exe = tmp_path / "tile_view_check_san"
    check = os.path.join(ROOT, "tests", "native", "tile_view_check.cpp")
    flags = ["-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
             "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
    r = subprocess.run(["g++", *flags, "-o", str(exe), check, ORACLE_SRC, *srcs, "-lpthread"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0 and "ALL OK" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]
