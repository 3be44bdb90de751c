"""Product host library (through its C ABI) against the pinned oracle and the
reference-made golden fixtures: Matrix Market reader, COO->CSR, the three
VCSR builders (bit-exact, any thread count), the synthetic generators, the
CPU SpMM, and the error behaviour of each entry point."""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from conftest import ROOT, random_csr

ARRAYS = ("group_ptr", "group_depth", "group_seg_base", "group_rows", "lcol", "val")


@pytest.fixture(scope="module")
def golden():
    with open(os.path.join(ROOT, "tests", "golden", "vcsr_golden.json")) as f:
        return json.load(f)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def product_csr(vs, M, N, rows, cols, vals):
    return vs.coo_to_csr(vs.Coo.from_arrays(M, N, rows, cols, vals))


# ------------------------------------------------------------------ builders
@settings(max_examples=60, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(seed=st.integers(0, 2**31 - 1), segw=st.integers(1, 20), bundle=st.integers(1, 80),
       layout=st.sampled_from([0, 1, 2]), threads=st.sampled_from([1, 3, 0]))
def test_builders_match_oracle(vs, orc, seed, segw, bundle, layout, threads):
    rng = np.random.default_rng(seed)
    M, N = int(rng.integers(0, 90)), int(rng.integers(1, 70))
    rows, cols, vals = random_csr(rng, M, N, density=float(rng.uniform(0.0, 0.4)),
                                  dup_rate=float(rng.choice([0.0, 0.3])), empty_rows=0.2)
    csr = product_csr(vs, M, N, rows, cols, vals)
    fmt = vs.build_vcsr(csr, segw, bundle, layout, threads)
    got = fmt.arrays()
    want = orc.build(M, N, csr.row_ptr, csr.col, csr.val, segw, bundle, layout)
    for k in ARRAYS + ("segment_group_start",):
        assert np.array_equal(got[k], want[k]), k
    assert fmt.num_groups == want["num_groups"] and fmt.num_slots == want["num_slots"]


def test_builders_thread_count_invariant(vs):
    csr = vs.coo_to_csr(vs.generate_coo(1, 3))
    for layout in (0, 1, 2):
        ref = vs.build_vcsr(csr, 4, 64, layout, 1).arrays()
        for t in (2, 7, 0):
            got = vs.build_vcsr(csr, 4, 64, layout, t).arrays()
            for k in ref:
                assert np.array_equal(ref[k], got[k]), (layout, t, k)


def test_builders_golden_tiny(vs, golden):
    for name, case in golden["tiny"].items():
        csr = vs.Csr.from_arrays(case["M"], case["N"], case["row_ptr"], case["col"], case["val"])
        for key, fx in case["fmt"].items():
            got = vs.build_vcsr(csr, fx["segw"], fx["bundle"], fx["layout"]).arrays()
            for k in ARRAYS:
                want = np.asarray(fx[k], np.float32 if k == "val" else np.int32)
                assert np.array_equal(got[k], want), f"{name}/{key}/{k}"


def test_builders_golden_large(vs, golden):
    for cfg_name, entry in golden["large"].items():
        csr = vs.coo_to_csr(vs.generate_coo(int(cfg_name[3:]), entry["seed"]))
        assert sha(csr.row_ptr) == entry["csr_sha256"]["row_ptr"]
        assert sha(csr.col) == entry["csr_sha256"]["col"]
        assert sha(csr.val) == entry["csr_sha256"]["val"]
        for key, fx in entry["fmt"].items():
            got = vs.build_vcsr(csr, fx["segw"], fx["bundle"], fx["layout"]).arrays()
            for k in ARRAYS:
                assert sha(got[k]) == fx["sha256"][k], f"{cfg_name}/{key}/{k}"


def test_tc_forces_16x16(vs):
    csr = vs.coo_to_csr(vs.generate_coo(1, 0))
    f = vs.build_vcsr(csr, 3, 7, vs.LAYOUT_TC)
    assert (f.segw, f.bundle) == (16, 16)


# --------------------------------------------------------------- COO -> CSR
@settings(max_examples=40, deadline=None)
@given(seed=st.integers(0, 2**31 - 1))
def test_coo_to_csr_matches_oracle(vs, orc, seed):
    rng = np.random.default_rng(seed)
    M, N = int(rng.integers(0, 60)), int(rng.integers(1, 40))
    n = int(rng.integers(0, 300))
    rows = rng.integers(0, max(M, 1), n).astype(np.int32) if M else np.zeros(0, np.int32)
    cols = rng.integers(0, N, len(rows)).astype(np.int32)
    vals = rng.normal(size=len(rows)).astype(np.float32)
    csr = product_csr(vs, M, N, rows, cols, vals)
    rp, col, val = orc.coo_to_csr(M, N, rows, cols, vals)
    assert np.array_equal(csr.row_ptr, rp)
    assert np.array_equal(csr.col, col)
    assert np.array_equal(csr.val, val)


def test_coo_to_csr_golden(vs, golden):
    for name, case in golden["csr"].items():
        csr = product_csr(vs, case["M"], case["N"], case["rows"], case["cols"], case["vals"])
        assert csr.row_ptr.tolist() == case["row_ptr"], name
        assert csr.col.tolist() == case["col"], name
        assert np.array_equal(csr.val, np.asarray(case["val"], np.float32)), name


# ------------------------------------------------------------- Matrix Market
def test_mtx_golden(vs, golden, tmp_path):
    for name, case in golden["mtx"].items():
        p = tmp_path / f"{name}.mtx"
        p.write_text(case["text"])
        coo = vs.read_matrix_market_coo(str(p))
        assert (coo.M, coo.N) == (case["M"], case["N"])
        assert coo.rows.tolist() == case["rows"] and coo.cols.tolist() == case["cols"]
        assert np.array_equal(coo.vals, np.asarray(case["vals"], np.float32)), name


def test_mtx_matches_oracle_random(vs, orc, tmp_path):
    rng = np.random.default_rng(5)
    for i in range(5):
        M, N, n = 30, 20, 100
        r = rng.integers(1, M + 1, n)
        c = rng.integers(1, N + 1, n)
        v = rng.normal(size=n) * 10.0 ** rng.integers(-8, 8, n)
        lines = ["%%MatrixMarket matrix coordinate real general", "% c", f"{M} {N} {n}"]
        lines += [f"{a} {b} {float(x)!r}" for a, b, x in zip(r, c, v)]
        p = tmp_path / f"r{i}.mtx"
        p.write_text("\n".join(lines) + "\n")
        coo = vs.read_matrix_market_coo(str(p))
        o = orc.read_mtx(str(p))
        assert (coo.M, coo.N) == (o[0], o[1])
        assert np.array_equal(coo.rows, o[2]) and np.array_equal(coo.cols, o[3])
        assert np.array_equal(coo.vals, o[4])


def test_mtx_symmetric_expansion_opt_in(vs, tmp_path):
    p = tmp_path / "s.mtx"
    p.write_text("%%MatrixMarket matrix coordinate real symmetric\n3 3 3\n1 1 2\n3 1 -1\n2 2 4\n")
    plain = vs.read_matrix_market_coo(str(p))
    assert plain.nnz == 3  # the reference does not expand (include/mmio.hpp:29)
    full = vs.read_matrix_market_coo(str(p), expand_symmetric=True)
    assert full.nnz == 4
    trip = sorted(zip(full.rows.tolist(), full.cols.tolist(), full.vals.tolist()))
    assert trip == [(0, 0, 2.0), (0, 2, -1.0), (1, 1, 4.0), (2, 0, -1.0)]


@pytest.mark.parametrize("text,code", [
    ("%%MatrixMarket matrix coordinate real general\n% only comments\n", 2),
    ("", 2),
    ("%%MatrixMarket matrix coordinate real general\n2 2 3\n1 1 1.0\n2 2\n", 2),
    ("%%MatrixMarket matrix coordinate real general\n2 2 1\n1 x 1.0\n", 2),
])
def test_mtx_errors(vs, tmp_path, text, code):
    p = tmp_path / "bad.mtx"
    p.write_text(text)
    with pytest.raises(vs.VcsrError) as e:
        vs.read_matrix_market_coo(str(p))
    assert e.value.code == code


def test_mtx_missing_file(vs):
    with pytest.raises(vs.VcsrError) as e:
        vs.read_matrix_market_coo("/nonexistent/file.mtx")
    assert e.value.code == vs.VCSR_EIO


# ------------------------------------------------------------------- errors
def test_error_behaviour(vs):
    with pytest.raises(vs.VcsrError) as e:  # row out of range (csr.hpp:19)
        vs.coo_to_csr(vs.Coo.from_arrays(2, 2, [2], [0], [1.0]))
    assert e.value.code == vs.VCSR_ERANGE
    with pytest.raises(vs.VcsrError) as e:  # column out of range
        vs.coo_to_csr(vs.Coo.from_arrays(2, 2, [0], [5], [1.0]))
    assert e.value.code == vs.VCSR_ERANGE
    csr = vs.coo_to_csr(vs.Coo.from_arrays(3, 3, [0, 1], [0, 2], [1.0, 2.0]))
    for segw, bundle in [(0, 4), (4, 0), (-1, 4), (4, -3)]:
        with pytest.raises(vs.VcsrError) as e:
            vs.build_vcsr(csr, segw, bundle, vs.LAYOUT_S)
        assert e.value.code == vs.VCSR_EINVAL
    with pytest.raises(vs.VcsrError):
        vs.build_vcsr(csr, 4, 4, 7)
    with pytest.raises(vs.VcsrError) as e:  # invalid CSR
        vs.Csr.from_arrays(2, 2, [0, 2, 1], [0, 1], [1.0, 1.0])
    assert e.value.code == vs.VCSR_ERANGE
    with pytest.raises(vs.VcsrError):
        vs.generate_coo(9, 0)
    assert vs.load_library().vcsr_last_error() != b""


# --------------------------------------------------------------- generators
def test_generators_deterministic(vs):
    a, b = vs.generate_coo(1, 42), vs.generate_coo(1, 42)
    assert np.array_equal(a.cols, b.cols) and np.array_equal(a.vals, b.vals)
    c = vs.generate_coo(1, 43)
    assert not np.array_equal(a.cols, c.cols)
    x, y = vs.gen_dense(7, 0, 100, 9), vs.gen_dense(7, 0, 100, 9)
    assert np.array_equal(x, y)
    assert x.min() >= -1 and x.max() < 1
    # element i depends only on (seed, i): a prefix is the same matrix's prefix
    assert np.array_equal(vs.gen_dense(7, 0, 50, 9), x[:50])
    n = vs.gen_dense(3, 1, 20000, 8)
    assert abs(n.mean()) < 0.02 and abs(n.std() - 1) < 0.02


def test_cfg1_shape(vs):
    coo = vs.generate_coo(1, 0)
    assert (coo.M, coo.N, coo.nnz) == (4096, 4096, 65536)
    cols = coo.cols.reshape(4096, 16)
    assert all(len(set(r.tolist())) == 16 for r in cols)
    assert coo.vals.min() >= -1 and coo.vals.max() < 1


def test_cfg2_shape(vs):
    csr = vs.coo_to_csr(vs.generate_coo(2, 0))
    assert csr.M == csr.N == 62451
    rl = np.diff(csr.row_ptr)
    assert rl.min() >= 40 and rl.max() <= 78 and 60 <= rl.mean() <= 68
    rows = np.repeat(np.arange(csr.M), rl)
    assert np.abs(rows - csr.col).max() <= 3 * 333 + 2  # band
    key = lambda r, c: r.astype(np.int64) * csr.N + c
    fwd = dict(zip(key(rows, csr.col).tolist(), csr.val.tolist()))
    back = [fwd[k] for k in key(csr.col, rows).tolist()]  # symmetric pattern and values
    assert np.array_equal(np.asarray(back, np.float32), csr.val)
    diag = csr.val[rows == csr.col]
    offl1 = np.bincount(rows, weights=np.abs(csr.val) * (rows != csr.col), minlength=csr.M)
    assert np.all(diag >= offl1)  # diagonally dominant


def test_cfg3_shape(vs):
    csr = vs.coo_to_csr(vs.generate_coo(3, 0))
    assert csr.M == 321821
    assert 1.7e6 <= csr.nnz <= 2.1e6
    rl = np.diff(csr.row_ptr)
    assert rl.min() >= 1 and rl.max() >= 5000
    rows = np.repeat(np.arange(csr.M), rl)
    assert np.count_nonzero(rows == csr.col) == csr.M  # full diagonal


def test_cfg5_shape(vs):
    csr = vs.coo_to_csr(vs.generate_coo(5, 0))
    assert csr.M == 16384 and csr.nnz == 1024 * 51 * 256
    rl = np.diff(csr.row_ptr)
    assert np.all(rl == 51 * 16)


# ------------------------------------------------------------------ CPU SpMM
@pytest.mark.parametrize("threads", [1, 4, 0])
def test_cpu_spmm_matches_oracle_bitwise(vs, orc, threads):
    rng = np.random.default_rng(threads)
    rows, cols, vals = random_csr(rng, 200, 150, density=0.05, dup_rate=0.1, empty_rows=0.1)
    csr = product_csr(vs, 200, 150, rows, cols, vals)
    B = vs.gen_dense(1, 0, 150, 37)
    C = vs.spmm_csr_cpu(csr, B, threads)
    ref = orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
    assert np.array_equal(C.view(np.uint32), ref.view(np.uint32))


# --------------------------------------------------- MFMA work accounting
def test_mfma_work_dense_blocks_are_fully_used(vs):
    """cfg5 in layout TC: every group is one dense 16x16 block, so the
    16x16x4 MFMAs the kernel issues carry exactly 2*nnz*O useful FLOPs when O
    is a multiple of the kernel's column tile (16 x up to 8 blocks), and the
    tail tile's padding otherwise (O=520: 5 tiles of 128 columns)."""
    csr = vs.coo_to_csr(vs.generate_coo(5, 0))
    fmt = vs.build_vcsr(csr, 16, 16, vs.LAYOUT_TC)
    for O, issued_cols in ((16, 16), (512, 512), (520, 640)):
        ops, fpo = vs.mfma_work(fmt, O)
        assert fpo == 2 * 16 * 16 * 4
        assert ops * fpo == 2 * csr.nnz * issued_cols


def test_mfma_work_counts_padding(vs):
    """bundle 64 (32x32x2 tiles): a group of n active lanes issues
    ceil(n/32) row blocks x ceil(segw/2) K-steps x the column blocks of
    ceil(O/kw) column tiles (tileK=64: kw = 64 columns = 2 blocks; O=70 -> 4)."""
    rng = np.random.default_rng(2)
    rows, cols, vals = random_csr(rng, 300, 97, density=0.04)
    csr = product_csr(vs, 300, 97, rows, cols, vals)
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    a = fmt.arrays()
    nact = [(a["lcol"][a["group_ptr"][g]:a["group_ptr"][g] + 64] >= 0).sum()
            for g in range(fmt.num_groups)]
    O = 70
    ops, fpo = vs.mfma_work(fmt, O, 64)
    assert fpo == 2 * 32 * 32 * 2
    assert ops == sum(-(-n // 32) for n in nact) * 2 * 4
    assert ops * fpo >= 2 * csr.nnz * O


@pytest.mark.parametrize("layout,segw,bundle", [(0, 4, 32), (1, 4, 64), (1, 3, 7), (2, 16, 16)])
def test_format_file_round_trip(vs, tmp_path, layout, segw, bundle):
    """A saved format loads back with bit-identical arrays and the same
    parameters (a matrix with empty rows, duplicates and ragged rows)."""
    rng = np.random.default_rng(layout * 10 + segw)
    M, N = 200, 150
    rows = rng.integers(0, M, 1500).astype(np.int32)
    rows[rows % 9 == 0] = 3  # one long row, some empty ones
    cols = rng.integers(0, N, 1500).astype(np.int32)
    vals = rng.uniform(-1, 1, 1500).astype(np.float32)
    csr = vs.coo_to_csr(vs.Coo.from_arrays(M, N, rows, cols, vals))
    fmt = vs.build_vcsr(csr, segw, bundle, layout)
    fmt.set_tile_rows(16)
    fmt.set_tile_windows(True)
    path = str(tmp_path / "a.vcsr")
    vs.save_vcsr(fmt, path)
    back = vs.load_vcsr(path)
    a, b = fmt.arrays(), back.arrays()
    assert a.keys() == b.keys()
    for k in a:
        assert np.array_equal(a[k].view(np.uint32) if a[k].dtype == np.float32 else a[k],
                              b[k].view(np.uint32) if b[k].dtype == np.float32 else b[k]), k
    for attr in ("num_groups", "num_slots"):
        assert getattr(fmt, attr) == getattr(back, attr)
    # The tile-view settings travel with the file: a second save is identical.
    path2 = str(tmp_path / "b.vcsr")
    vs.save_vcsr(back, path2)
    assert open(path, "rb").read() == open(path2, "rb").read()


def test_format_file_rejects_bad_files(vs, tmp_path):
    """Unreadable files are VCSR_EIO; files whose header or arrays break the
    format's invariants are VCSR_EINVAL (never a handle the kernels could
    index out of bounds with)."""
    csr = vs.coo_to_csr(vs.generate_coo(1, 0))
    fmt = vs.build_vcsr(csr, 4, 64, vs.LAYOUT_S)
    good = tmp_path / "good.vcsr"
    vs.save_vcsr(fmt, str(good))
    data = bytearray(good.read_bytes())
    G = fmt.num_groups

    def expect(blob, code, name):
        p = tmp_path / name
        p.write_bytes(bytes(blob))
        with pytest.raises(vs.VcsrError) as e:
            vs.load_vcsr(str(p))
        assert e.value.code == code, (name, e.value)

    with pytest.raises(vs.VcsrError) as e:
        vs.load_vcsr(str(tmp_path / "missing.vcsr"))
    assert e.value.code == vs.VCSR_EIO
    expect(data[:20], vs.VCSR_EIO, "short_header")
    bad = bytearray(data); bad[0:8] = b"NOTVCSR!"
    expect(bad, vs.VCSR_EINVAL, "magic")
    expect(data[:-4], vs.VCSR_EINVAL, "truncated")
    expect(data + bytes(4), vs.VCSR_EINVAL, "trailing")
    hdr = 8 + 32 + 16  # magic, 8 int32, 2 int64
    ptr0 = hdr                        # group_ptr
    depth0 = ptr0 + 4 * (G + 1)       # group_depth
    base0 = depth0 + 4 * G            # group_seg_base
    rows0 = base0 + 4 * G             # group_rows
    lcol0 = rows0 + 4 * G * 64        # lcol
    def with_int(off, value, name):
        b = bytearray(data)
        b[off:off + 4] = np.int32(value).tobytes()
        expect(b, vs.VCSR_EINVAL, name)
    with_int(8 + 8, 0, "bundle_zero")             # bundle field of the header
    with_int(8 + 4, 10 ** 6, "n_mismatch")        # N no longer matches segments
    with_int(ptr0 + 4, 7, "group_ptr")            # group 0 no longer depth * bundle
    with_int(depth0, -1, "negative_depth")
    with_int(base0, 4, "segment_base")            # group 0 sits in segment 0
    with_int(rows0, csr.M, "row_out_of_range")
    with_int(lcol0, 4, "lcol_out_of_segment")     # segw = 4
    # Valid arrays under a bad row-tile setting in the header.
    with_int(8 + 24, 5, "tile_height_5")
    with_int(8 + 28, 2, "window_flag_2")
    # An entry after a padding slot of the same lane.
    a = fmt.arrays()
    pad = int(np.nonzero(a["lcol"] < 0)[0][0])
    with_int(lcol0 + 4 * pad, 0, "unpacked_lane")
    # A self-consistent file whose one group has depth 0 (no slots at all):
    # the builders never emit such a group, and the upload reads every
    # group's depth-0 slots.
    zero = bytearray(data[:8])
    zero += np.array([1, 1, 1, 1, vs.LAYOUT_S, 1, 0, 0], np.int32).tobytes()
    zero += np.array([1, 0], np.int64).tobytes()                 # G = 1, P = 0
    zero += np.array([0, 0, 0, 0, 0], np.int32).tobytes()        # ptr, depth, base, rows
    zero += np.array([0, 1], np.int32).tobytes()                 # segment_group_start
    expect(zero, vs.VCSR_EINVAL, "zero_depth")
    ok = bytearray(data[:8])                                     # the same with depth 1
    ok += np.array([1, 1, 1, 1, vs.LAYOUT_S, 1, 0, 0], np.int32).tobytes()
    ok += np.array([1, 1], np.int64).tobytes()
    ok += np.array([0, 1, 1, 0, 0], np.int32).tobytes()
    ok += np.array([0], np.int32).tobytes() + np.array([2.5], np.float32).tobytes()
    ok += np.array([0, 1], np.int32).tobytes()
    p = tmp_path / "one.vcsr"
    p.write_bytes(bytes(ok))
    assert vs.load_vcsr(str(p)).num_groups == 1
    # The untouched file still loads.
    assert vs.load_vcsr(str(good)).num_groups == G
