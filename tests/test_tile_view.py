"""CPU checks of the row-tile view (vcsr-spmm_amd/csrc/host/tile_view.cpp),
the index structure the tile-stationary kernel walks: built from the VCSR
arrays, it must hold exactly the CSR's nonzeros, cover every row once, and
respect the work-item limits the kernel's LDS arrays are sized for.  The
checker (tests/native/tile_view_check.cpp) links the library's host objects;
no GPU is used."""
from __future__ import annotations

import glob
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vcsr-spmm_amd")


def test_tile_view_builder(tmp_path):
    objs = sorted(glob.glob(os.path.join(PKG, "_build", "host", "*.o")))
    if not objs:
        pytest.skip("host objects not built (run __graft_entry__.build())")
    exe = tmp_path / "tile_view_check"
    src = os.path.join(ROOT, "tests", "native", "tile_view_check.cpp")
    subprocess.run(["g++", "-std=c++17", "-O2", "-march=x86-64-v3", "-o", str(exe), src, *objs,
                    "-lpthread"], check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "ALL OK" in r.stdout, r.stdout[-4000:] + r.stderr[-2000:]
