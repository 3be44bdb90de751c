"""The C ABI library and the CLI without a GPU: the library loads, exports
every function include/vcsr_spmm.h declares, refuses GPU work cleanly when no
GPU is visible, and the CLI keeps the reference's flag surface and output
line format (src/main.cpp:68-90; reports/a100/*_vcsr_*.txt)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "vcsr_spmm.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(\w+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_api():
    names = declared_functions()
    for n in ("vcsr_build", "vcsr_fmt_arrays", "vcsr_fmt_upload", "vcsr_fmt_free",
              "spmm_csr_naive", "spmm_vcsr", "spmm_vcsr_mfma", "spmm_csr_cpu", "vcsr_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol(vs):
    lib = ctypes.CDLL(vs.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(vs.EXPORTS) == declared_functions()


def test_header_compiles_as_c(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "vcsr_spmm.h"\nint main(void){return VCSR_OK;}\n')
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                        "-c", str(src), "-o", str(tmp_path / "t.o")], capture_output=True)
    assert r.returncode == 0, r.stderr.decode()


def test_gpu_entry_points_without_gpu(vs):
    if vs.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(vs.VcsrError) as e:
        vs.DeviceArray((4,), np.float32)
    assert e.value.code == vs.VCSR_EDEVICE
    fmt = vs.csr_to_vcsr_seg(vs.coo_to_csr(vs.generate_coo(1, 0)), 4, 64)
    with pytest.raises(vs.VcsrError) as e:
        fmt.upload()
    assert e.value.code == vs.VCSR_EDEVICE
    lib = vs.load_library()
    rc = lib.spmm_vcsr(fmt._h, None, 8, 64, None, None, None)
    assert rc == vs.VCSR_ESTATE  # not uploaded: refused before any device work
    with pytest.raises(vs.VcsrError) as e:
        fmt.launch_info(64)
    assert e.value.code == vs.VCSR_ESTATE
    rc = lib.spmm_csr_naive(4, None, None, None, None, 8, None, None, None)
    assert rc == vs.VCSR_EINVAL


class _FakeBuf:
    """Stands in for a device buffer: the Python layer checks shape and type
    before it hands a pointer to the library."""

    def __init__(self, n, dtype=np.float32):
        self.dtype, self.nbytes, self.ptr = np.dtype(dtype), n * np.dtype(dtype).itemsize, None


def test_python_wrappers_check_buffer_sizes(vs):
    """B and C must hold N*O and M*O float32 elements, and CSR arrays must
    be int32/float32 of matching lengths: a short or mistyped buffer is
    VCSR_EINVAL in Python, before the library (and a kernel) sees it."""
    csr = vs.coo_to_csr(vs.generate_coo(1, 0))
    fmt = vs.csr_to_vcsr_seg(csr, 4, 64)
    M, N, O = csr.M, csr.N, 32
    good_b, good_c = _FakeBuf(N * O), _FakeBuf(M * O)
    calls = [
        lambda b, c: vs.run_vcsr_spmm_gpu(fmt, b, O, 64, c),
        lambda b, c: vs.run_vcsr_spmm_gpu_ex(fmt, b, O, 64, c, kernel=vs.KERNEL_TILE),
        lambda b, c: vs.run_vcsr_tc_spmm_gpu(fmt, b, O, c),
    ]
    for call in calls:
        for b, c in ((_FakeBuf(N * O - 1), good_c), (good_b, _FakeBuf(M * O - 4)),
                     (_FakeBuf(N * O, np.float64), good_c), (good_b, _FakeBuf(M * O, np.int32))):
            with pytest.raises(vs.VcsrError) as e:
                call(b, c)
            assert e.value.code == vs.VCSR_EINVAL
    rp, col, val = _FakeBuf(M + 1, np.int32), _FakeBuf(csr.nnz, np.int32), _FakeBuf(csr.nnz)
    for args in ((_FakeBuf(M, np.int32), col, val), (rp, _FakeBuf(csr.nnz), val),
                 (rp, col, _FakeBuf(csr.nnz - 1))):
        for run in (lambda a: vs.run_csr_spmm_gpu(M, *a, good_b, O, good_c),
                    lambda a: vs.run_csr_wave_spmm_gpu(M, N, *a, good_b, O, good_c),
                    lambda a: vs.run_vendor_spmm_gpu(M, N, csr.nnz, *a, good_b, O, good_c)):
            with pytest.raises(vs.VcsrError) as e:
                run(args)
            assert e.value.code == vs.VCSR_EINVAL
    # The vendor library is told nnz and reads that many col / val entries:
    # a larger nnz than the buffers hold (or a negative one) is refused.
    for nnz in (csr.nnz + 1, -1):
        for run in (lambda: vs.run_vendor_spmm_gpu(M, N, nnz, rp, col, val, good_b, O, good_c),
                    lambda: vs.VendorPlan(M, N, nnz, rp, col, val, good_b, O, good_c)):
            with pytest.raises(vs.VcsrError) as e:
                run()
            assert e.value.code == vs.VCSR_EINVAL


def run_cli(vs, *args):
    return subprocess.run([vs.CLI_PATH, *args], capture_output=True, text=True, timeout=300)


def test_cli_usage_errors(vs):
    assert run_cli(vs).returncode == 1                       # no --mtx / --gen
    assert run_cli(vs, "--bogus").returncode == 1            # unknown option
    assert run_cli(vs, "--gen", "cfg1", "--algo", "nope").returncode == 1
    r = run_cli(vs, "--gen", "cfg1", "--algo", "vcsr_naive")
    assert r.returncode == 1 and "not part of this build" in r.stdout
    # cusparse names the vendor baseline (rocSPARSE here), a GPU algorithm.
    r = run_cli(vs, "--gen", "cfg1", "--algo", "cusparse")
    assert r.returncode in (0, 2)
    if r.returncode == 2:
        assert "no GPU visible" in r.stderr


def test_cli_cpu_line_format(vs, tmp_path):
    """The last line carries the tokens the reference's bench parsers take:
    the number before "ms" and before "GFLOP/s" (run_h100_bench.slurm:60-61)."""
    r = run_cli(vs, "--gen", "cfg1", "--O", "32", "--algo", "cpu", "--repeat", "2")
    assert r.returncode == 0, r.stderr
    last = r.stdout.strip().splitlines()[-1]
    tok = last.split()
    ms = float(tok[tok.index("ms") - 1])
    gf = float(tok[tok.index("GFLOP/s") - 1])
    assert ms > 0 and gf > 0
    assert "Matrix: 4096 x 4096, nnz=65536" in r.stdout


def test_cli_reads_mtx(vs, tmp_path):
    p = tmp_path / "a.mtx"
    p.write_text("%%MatrixMarket matrix coordinate real general\n3 3 4\n1 1 1\n2 2 2\n3 3 3\n1 3 4\n")
    r = run_cli(vs, "--mtx", str(p), "--O", "8", "--algo", "cpu")
    assert r.returncode == 0, r.stderr
    assert "Matrix: 3 x 3, nnz=4" in r.stdout
    r = run_cli(vs, "--mtx", str(tmp_path / "missing.mtx"), "--algo", "cpu")
    assert r.returncode != 0 and "Failed to open MTX" in r.stderr


def test_cli_gpu_algo_without_gpu(vs):
    if vs.device_count() > 0:
        pytest.skip("a GPU is visible")
    r = run_cli(vs, "--gen", "cfg1", "--algo", "vcsr")
    assert r.returncode == 2 and "no GPU" in r.stderr


@pytest.mark.gpu
def test_cli_gpu_algorithms_and_format_file(vs, tmp_path):
    """On the GPU: every algorithm's result line parses like the reference's
    bench scripts read it (number before "ms" and before "GFLOP/s"), the L2
    check passes, and --save-fmt / --load-fmt round-trip the VCSR format."""
    if vs.device_count() <= 0:
        pytest.fail("no GPU visible to the library (gpu tests run on the GPU box)")
    fmt = str(tmp_path / "cfg1.vcsr")
    for algo, extra in (("vcsr", ["--save-fmt", fmt]), ("vcsr", ["--load-fmt", fmt]),
                        ("csr", []), ("vcsr_mfma", []), ("vcsr_tc", []), ("rocsparse", []),
                        ("aspt", []), ("fast", [])):
        r = run_cli(vs, "--gen", "cfg1", "--O", "64", "--algo", algo, "--repeat", "2",
                    "--check", *extra)
        assert r.returncode == 0, (algo, r.stdout[-2000:], r.stderr[-2000:])
        last = r.stdout.strip().splitlines()[-1].split()
        ms = float(last[last.index("ms") - 1])
        gf = float(last[last.index("GFLOP/s") - 1])
        assert ms > 0 and gf > 0, (algo, last)
        assert "FAIL" not in r.stdout, (algo, r.stdout[-2000:])
        if "--save-fmt" in extra:
            assert "format: saved to" in r.stdout
        if "--load-fmt" in extra:
            assert "format: loaded from" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", ["cfg2", "cfg3"])
def test_cli_all_algorithms_full_size(vs, cfg):
    """The CLI as the reference's harness drives it, at a headline size:
    --algo all --check on the full banded / power-law matrix at O = 128.
    Every algorithm's L2 check against the CPU CSR SpMM (all of C) passes."""
    if vs.device_count() <= 0:
        pytest.fail("no GPU visible to the library (gpu tests run on the GPU box)")
    print(f"cli --gen {cfg} --O 128 --algo all --check", flush=True)
    r = run_cli(vs, "--gen", cfg, "--O", "128", "--segw", "4", "--bundle", "64", "--tileK", "64",
                "--algo", "all", "--repeat", "2", "--check")
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-2000:])
    checks = [line for line in r.stdout.splitlines() if line.startswith("L2 diff")]
    print("\n".join(checks), flush=True)
    assert len(checks) >= 5, r.stdout[-3000:]
    assert all(line.rstrip().endswith("PASS") for line in checks), checks


def test_integration_shim_compiles(tmp_path):
    """The C++ shim that the repository's integration guide gives a
    maintainer of the reference (its "C++ shim" section, read from the
    guide at the repository root) compiles against include/vcsr_spmm.h,
    with the reference's CSR struct
    (include/csr.hpp:8-13: M, N, nnz, row_ptr, col, val) and an opaque
    hipStream_t, as in the reference's translation unit."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = text[text.index("## 2. C++ shim"):]
    block = sec[sec.index("```cpp") + len("```cpp"):]
    block = block[:block.index("```")]
    prelude = ("#include <vector>\n"
               "struct CSR { int M{0}, N{0}, nnz{0}; std::vector<int> row_ptr; "
               "std::vector<int> col; std::vector<float> val; };\n"
               "typedef struct ihipStream_t* hipStream_t;\n")
    src = tmp_path / "shim.cpp"
    src.write_text(prelude + block + "\nint main() { return 0; }\n")
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-fsyntax-only", "-I",
                        os.path.join(ROOT, "include"), str(src)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
