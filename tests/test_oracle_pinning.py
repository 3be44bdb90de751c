"""Pins the CPU oracle (oracle/vcsr_oracle.cpp) before anything is checked
against it:

  * against the reference's own host code, compiled by oracle/Makefile into
    oracle/_ref/libref.so (skipped where it was not built), on random inputs;
  * against the golden fixtures in tests/golden/vcsr_golden.json, which that
    same reference code produced (these travel without the reference);
  * against closed forms that a plausible mistake would break: tie-independent
    group structure computed from sorted counts, unpacking a format back to A,
    dense products, identity/permutation/diagonal matrices, and an exact
    rational evaluation of the fused multiply-add order on tiny inputs.
"""
from __future__ import annotations

import hashlib
import json
import os
from fractions import Fraction

import numpy as np
import pytest

from conftest import ROOT, random_csr

GOLDEN = os.path.join(ROOT, "tests", "golden", "vcsr_golden.json")
ARRAYS = ("group_ptr", "group_depth", "group_seg_base", "group_rows", "lcol", "val")


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def csr_of(orc, M, N, rows, cols, vals):
    return orc.coo_to_csr(M, N, np.asarray(rows, np.int32), np.asarray(cols, np.int32),
                          np.asarray(vals, np.float32))


needs_ref = pytest.mark.skipif(
    not os.path.exists(os.path.join(ROOT, "oracle", "_ref", "libref.so")),
    reason="reference host code not compiled (needs /root/reference)")


# ------------------------------------------------------- golden fixtures
def test_golden_mtx(orc, golden, tmp_path):
    for name, case in golden["mtx"].items():
        p = tmp_path / f"{name}.mtx"
        p.write_text(case["text"])
        M, N, r, c, v = orc.read_mtx(str(p))
        assert (M, N) == (case["M"], case["N"]), name
        assert r.tolist() == case["rows"] and c.tolist() == case["cols"], name
        assert np.array_equal(v, np.asarray(case["vals"], np.float32)), name


def test_golden_coo_to_csr(orc, golden):
    for name, case in golden["csr"].items():
        rp, col, val = orc.coo_to_csr(case["M"], case["N"], np.asarray(case["rows"], np.int32),
                                      np.asarray(case["cols"], np.int32),
                                      np.asarray(case["vals"], np.float32))
        assert rp.tolist() == case["row_ptr"], name
        assert col.tolist() == case["col"], name
        assert np.array_equal(val, np.asarray(case["val"], np.float32)), name


def test_golden_tiny_formats(orc, golden):
    n = 0
    for name, case in golden["tiny"].items():
        rp = np.asarray(case["row_ptr"], np.int32)
        col = np.asarray(case["col"], np.int32)
        val = np.asarray(case["val"], np.float32)
        for key, fx in case["fmt"].items():
            f = orc.build(case["M"], case["N"], rp, col, val, fx["segw"], fx["bundle"],
                          fx["layout"])
            for k in ARRAYS:
                want = np.asarray(fx[k], np.float32 if k == "val" else np.int32)
                assert np.array_equal(f[k], want), f"{name}/{key}/{k}"
            if "segment_group_start" in fx:
                assert f["segment_group_start"].tolist() == fx["segment_group_start"]
            n += 1
    assert n >= 20


def test_golden_large_formats(orc, vs, golden):
    """The oracle's builders on the full synthetic configs reproduce the
    reference-made SHA-256 of every array (cfg3 and cfg4 are where the tie
    order of unordered_map iteration and std::sort is most exposed).  The
    configs run concurrently (each oracle call is single-threaded and
    releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor

    def csr_of(cfg_name):
        entry = golden["large"][cfg_name]
        coo = vs.generate_coo(int(cfg_name[3:]), entry["seed"])
        rp, col, val = orc.coo_to_csr(coo.M, coo.N, coo.rows, coo.cols, coo.vals)
        assert sha(rp) == entry["csr_sha256"]["row_ptr"], "generator changed"
        assert sha(col) == entry["csr_sha256"]["col"], "generator changed"
        assert sha(val) == entry["csr_sha256"]["val"], "generator changed"
        return coo.M, coo.N, rp, col, val

    def build(task):
        cfg_name, key, (M, N, rp, col, val) = task
        fx = golden["large"][cfg_name]["fmt"][key]
        f = orc.build(M, N, rp, col, val, fx["segw"], fx["bundle"], fx["layout"])
        assert f["num_groups"] == fx["num_groups"], f"{cfg_name}/{key}"
        for k in ARRAYS:
            assert sha(f[k]) == fx["sha256"][k], f"{cfg_name}/{key}/{k}"

    names = sorted(golden["large"])
    assert {"cfg1", "cfg2", "cfg3", "cfg4", "cfg5"} <= set(names)
    workers = min(6, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=workers) as ex:
        csrs = dict(zip(names, ex.map(csr_of, names)))
        # Layout H only on cfg1: the reference's own H builder is O(S*M).
        tasks = [(n, key, csrs[n]) for n in names for key, fx in golden["large"][n]["fmt"].items()
                 if fx["layout"] != 0 or n == "cfg1"]
        assert len(tasks) >= 10
        list(ex.map(build, sorted(tasks, key=lambda t: -len(t[2][3]))))


# -------------------------------------------- the compiled reference itself
@needs_ref
@pytest.mark.parametrize("seed", range(12))
def test_oracle_matches_reference_random(orc, seed):
    rng = np.random.default_rng(seed)
    M, N = int(rng.integers(1, 120)), int(rng.integers(1, 90))
    rows, cols, vals = random_csr(rng, M, N, density=float(rng.uniform(0.01, 0.3)),
                                  dup_rate=0.2 if seed % 3 == 0 else 0.0, empty_rows=0.1)
    rp, col, val = orc.coo_to_csr(M, N, rows, cols, vals)
    r2 = orc.ref_coo_to_csr(M, N, rows, cols, vals)
    assert np.array_equal(rp, r2[0]) and np.array_equal(col, r2[1])
    assert np.array_equal(val, r2[2])
    segw = int(rng.integers(1, 9))
    bundle = int(rng.integers(1, 70))
    for layout in (0, 1, 2):
        a = orc.build(M, N, rp, col, val, segw, bundle, layout)
        b = orc.ref_build(M, N, rp, col, val, segw, bundle, layout)
        for k in ARRAYS:
            assert np.array_equal(a[k], b[k]), (layout, k)
        if layout == 1:
            assert np.array_equal(a["segment_group_start"], b["segment_group_start"])


@needs_ref
def test_oracle_matches_reference_mtx(orc, tmp_path):
    texts = ["%%MatrixMarket matrix coordinate real general\n% x\n4 4 3\n4 4 1e5\n1 2 -3\n2 2 .5\n",
             "%%MatrixMarket matrix coordinate real general\n\n\n3 3 2\n0 0 1\n2 2 -1\n"]
    for i, t in enumerate(texts):
        p = tmp_path / f"m{i}.mtx"
        p.write_text(t)
        a, b = orc.read_mtx(str(p)), orc.ref_read_mtx(str(p))
        assert a[0] == b[0] and a[1] == b[1]
        for x, y in zip(a[2:], b[2:]):
            assert np.array_equal(x, y)


# ----------------------------------------------------------- closed forms
def _closed_form_groups(M, N, rp, col, segw, bundle, layout):
    """group_ptr / depth / seg_base from sorted per-segment counts only."""
    S = (N + segw - 1) // segw
    counts = np.zeros((S, M), np.int64)
    for r in range(M):
        for p in range(rp[r], rp[r + 1]):
            counts[col[p] // segw, r] += 1
    gp, depth, base, sgs = [0], [], [], [0]
    for s in range(S):
        c = np.sort(counts[s])[::-1]
        c = c if layout == 0 else c[c > 0]
        for start in range(0, len(c), bundle):
            d = int(c[start])
            if d == 0:
                continue
            depth.append(d)
            base.append(s * segw)
            gp.append(gp[-1] + d * bundle)
        sgs.append(len(depth))
    return np.array(gp), np.array(depth), np.array(base), np.array(sgs)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("seed", range(6))
def test_tie_independent_arrays_closed_form(orc, layout, seed):
    rng = np.random.default_rng(100 + seed)
    M, N = int(rng.integers(1, 60)), int(rng.integers(1, 50))
    rows, cols, vals = random_csr(rng, M, N, density=0.15, dup_rate=0.1)
    rp, col, val = orc.coo_to_csr(M, N, rows, cols, vals)
    segw, bundle = int(rng.integers(1, 7)), int(rng.integers(1, 20))
    f = orc.build(M, N, rp, col, val, segw, bundle, layout)
    gp, depth, base, sgs = _closed_form_groups(M, N, rp, col, segw, bundle, layout)
    assert np.array_equal(f["group_ptr"], gp)
    assert np.array_equal(f["group_depth"], depth)
    assert np.array_equal(f["group_seg_base"], base)
    assert np.array_equal(f["segment_group_start"], sgs)


@pytest.mark.parametrize("layout", [0, 1, 2])
def test_format_unpacks_to_A(orc, layout):
    """Applying a format to the identity gives back A (values, positions,
    duplicates summed), and each row appears at most once per segment."""
    rng = np.random.default_rng(7 + layout)
    M, N = 45, 38
    rows, cols, vals = random_csr(rng, M, N, density=0.2, dup_rate=0.1, empty_rows=0.1)
    rp, col, val = orc.coo_to_csr(M, N, rows, cols, vals)
    f = orc.build(M, N, rp, col, val, 4, 16, layout)
    A = orc.vcsr_apply(M, N, f, np.eye(N, dtype=np.float32))
    dense = np.zeros((M, N))
    np.add.at(dense, (np.repeat(np.arange(M), np.diff(rp)), col), val.astype(np.float64))
    assert np.allclose(A, dense, rtol=0, atol=1e-6)
    b = f["bundle"]
    gr = f["group_rows"].reshape(-1, b)
    sgs = f["segment_group_start"]
    for s in range(len(sgs) - 1):
        r = gr[sgs[s]:sgs[s + 1]].ravel()
        r = r[r >= 0]
        assert len(r) == len(set(r.tolist()))
    assert np.all((f["lcol"] >= -1) & (f["lcol"] < f["segw"]))
    assert np.all(f["val"][f["lcol"] < 0] == 0)
    assert np.all(f["group_seg_base"] % f["segw"] == 0)
    real = f["lcol"] >= 0
    assert real.sum() == len(val)
    assert np.array_equal(np.sort(f["val"][real]), np.sort(val))


def _fma32(a, b, c):
    """Exact float32 fused multiply-add via rationals (round to nearest even)."""
    x = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    lo = np.float32(float(x))  # nearest double, then nearest float
    # correct a possible double rounding by checking the neighbours exactly
    cands = [lo, np.nextafter(lo, np.float32(np.inf)), np.nextafter(lo, np.float32(-np.inf))]
    best = min(cands, key=lambda f: (abs(Fraction(float(f)) - x),
                                     int(np.float32(f).view(np.uint32)) & 1))
    return np.float32(best)


def test_spmm_f32_is_sequential_fma(orc):
    """The FP32 oracle is C[r,k] = fma(val[p], B[col[p],k], C[r,k]) with p
    ascending: checked exactly against rational arithmetic on a tiny case."""
    rng = np.random.default_rng(3)
    M, N, O = 6, 7, 3
    rows, cols, vals = random_csr(rng, M, N, density=0.5, dup_rate=0.2)
    rp, col, val = orc.coo_to_csr(M, N, rows, cols, vals)
    B = rng.uniform(-1, 1, size=(N, O)).astype(np.float32)
    C = orc.spmm_f32(M, rp, col, val, B)
    for r in range(M):
        for k in range(O):
            acc = np.float32(0)
            for p in range(rp[r], rp[r + 1]):
                acc = _fma32(val[p], B[col[p], k], acc)
            assert C[r, k].view(np.uint32) == acc.view(np.uint32), (r, k)


def test_spmm_closed_forms(orc):
    n, O = 33, 5
    B = np.random.default_rng(1).uniform(-1, 1, (n, O)).astype(np.float32)
    eye = np.arange(n + 1, dtype=np.int32)
    # identity
    C = orc.spmm_f32(n, eye, np.arange(n, dtype=np.int32), np.ones(n, np.float32), B)
    assert np.array_equal(C, B)
    # permutation
    perm = np.random.default_rng(2).permutation(n).astype(np.int32)
    C = orc.spmm_f32(n, eye, perm, np.ones(n, np.float32), B)
    assert np.array_equal(C, B[perm])
    # diagonal scaling by powers of two (exact)
    d = (2.0 ** np.arange(-3, n - 3)).astype(np.float32)
    C = orc.spmm_f32(n, eye, np.arange(n, dtype=np.int32), d, B)
    assert np.array_equal(C, B * d[:, None])
    # empty matrix
    C = orc.spmm_f32(4, np.zeros(5, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32), B)
    assert not C.any()


def test_spmm_dense_reference(orc):
    rng = np.random.default_rng(11)
    M, N, O = 50, 40, 9
    rows, cols, vals = random_csr(rng, M, N, density=0.3, dup_rate=0.1, empty_rows=0.1)
    rp, col, val = orc.coo_to_csr(M, N, rows, cols, vals)
    B = rng.normal(size=(N, O)).astype(np.float32)
    dense = np.zeros((M, N))
    np.add.at(dense, (np.repeat(np.arange(M), np.diff(rp)), col), val.astype(np.float64))
    ref = dense @ B.astype(np.float64)
    C64 = orc.spmm_f64(M, rp, col, val, B)
    assert np.allclose(C64, ref, rtol=1e-13, atol=1e-13)
    C32 = orc.spmm_f32(M, rp, col, val, B)
    assert np.linalg.norm(C32 - ref) <= 1e-6 * np.linalg.norm(ref)


@pytest.mark.parametrize("nthreads", [2, 3, 7, 0])
def test_threaded_spmm_is_the_single_thread_result(orc, nthreads):
    """The row-split oracle SpMM (all-cores CPU baseline, whole-C checks)
    gives the single-thread result bit for bit, in FP32 and in double,
    including empty rows, duplicates and more threads than rows."""
    rng = np.random.default_rng(40 + nthreads)
    for M, N, O in ((300, 200, 17), (5, 9, 3), (0, 4, 2)):
        rows, cols, vals = random_csr(rng, M, N, density=0.1, dup_rate=0.1, empty_rows=0.2)
        rp, col, val = orc.coo_to_csr(M, N, rows, cols, vals)
        B = rng.uniform(-1, 1, size=(N, O)).astype(np.float32)
        one32 = orc.spmm_f32(M, rp, col, val, B)
        one64 = orc.spmm_f64(M, rp, col, val, B)
        assert np.array_equal(orc.spmm_f32(M, rp, col, val, B, nthreads).view(np.uint32),
                              one32.view(np.uint32))
        assert np.array_equal(orc.spmm_f64(M, rp, col, val, B, nthreads).view(np.uint64),
                              one64.view(np.uint64))


# ------------------------------------------------- FastSpMM condensed tiles
def _cst_hand_csr():
    """35 x 40: window 0 (rows 0-15) holds 17 distinct columns (two TCBs),
    with an unsorted row and a row holding column 5 twice; window 1 (rows
    16-31) is empty; window 2 (rows 32-34) is partial."""
    rows = {0: [(20, 2.0), (3, 1.0)], 2: [(5, 4.0), (5, 0.5)],
            7: [(21 + j, 10.0 + j) for j in range(14)], 33: [(39, -1.0), (0, 7.0)]}
    row_ptr, col, val = [0], [], []
    for r in range(35):
        for c, v in rows.get(r, []):
            col.append(c)
            val.append(v)
        row_ptr.append(len(col))
    return (np.array(row_ptr, np.int32), np.array(col, np.int32), np.array(val, np.float32))


def test_cst_hand_case(orc):
    """src/fastspmm.cu:129-251 worked by hand on _cst_hand_csr: window 0's
    columns [3, 5, 20, 21..34] fill TCB 0 (3, 5, 20, 21..33) and TCB 1 (34,
    then padding); entries keep CSR order inside a row (row 0: 20 before 3;
    both column-5 entries of row 2); window 1 adds no TCB; window 2 is TCB 2
    with columns [0, 39]."""
    rp, col, val = _cst_hand_csr()
    s = orc.build_cst(35, 40, rp, col, val)
    assert s["num_windows"] == 3 and s["num_tcb"] == 3
    assert s["window_off"].tolist() == [0, 2, 2, 3]
    assert s["tcb_col_off"].tolist() == [0, 17, 18, 20]
    assert s["tcb_row_off"].tolist() == (
        [0, 2, 2, 4, 4, 4, 4, 4, 17, 17, 17, 17, 17, 17, 17, 17, 17]
        + [17] * 8 + [18] * 9
        + [18, 18] + [20] * 15)
    assert s["col_idx"].tolist() == [2, 0, 1, 1] + list(range(3, 16)) + [0] + [1, 0]
    assert s["value"].tolist() == [2.0, 1.0, 4.0, 0.5] + [10.0 + j for j in range(13)] + [23.0] + [-1.0, 7.0]
    assert s["tcb2b"].tolist() == ([3, 5, 20] + list(range(21, 34)) + [34] + [-1] * 15
                                   + [0, 39] + [-1] * 14)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_cst_properties(orc, seed):
    """What the layout must satisfy, computed independently with numpy:
    each window's TCB columns are its sorted distinct columns padded with -1
    to whole TCBs; the offsets chain (a TCB's first row offset is its first
    entry, its 17th the next TCB's); and walking every TCB row puts every
    nonzero of A back in its row and column exactly once, in CSR order."""
    rng = np.random.default_rng(seed)
    M, N = int(rng.integers(17, 120)), int(rng.integers(20, 300))
    rp, col, val = csr_of(orc, M, N, *random_csr(rng, M, N, density=0.08, dup_rate=0.1,
                                                 empty_rows=0.3))
    # Rows in any column order (the layout keeps CSR order inside a row).
    perm = np.concatenate([rp[r] + rng.permutation(rp[r + 1] - rp[r]) for r in range(M)])
    col, val = col[perm.astype(np.int64)], val[perm.astype(np.int64)]
    # Two empty windows in the middle.
    if M > 48:
        lo, hi = rp[16], rp[48]
        col = np.concatenate([col[:lo], col[hi:]])
        val = np.concatenate([val[:lo], val[hi:]])
        rp = np.concatenate([rp[:17], np.full(32, lo), rp[49:] - (hi - lo)]).astype(np.int32)
    s = orc.build_cst(M, N, rp, col, val)
    W = (M + 15) // 16
    assert s["num_windows"] == W and s["window_off"][0] == 0
    ro, co, t2b = s["tcb_row_off"], s["tcb_col_off"], s["tcb2b"]
    T = s["num_tcb"]
    assert co[0] == 0 and co[-1] == len(s["col_idx"]) == rp[-1]
    for t in range(T):
        assert ro[17 * t] == co[t] and ro[17 * t + 16] == co[t + 1]
        assert np.all(np.diff(ro[17 * t:17 * t + 17]) >= 0)
    dense = np.zeros((M, N))
    want = np.zeros((M, N))
    for r in range(M):
        np.add.at(want[r], col[rp[r]:rp[r + 1]], val[rp[r]:rp[r + 1]].astype(np.float64))
    for w in range(W):
        r0, r1 = 16 * w, min(M, 16 * w + 16)
        cols = np.unique(col[rp[r0]:rp[r1]])
        t0, t1 = s["window_off"][w], s["window_off"][w + 1]
        assert t1 - t0 == (len(cols) + 15) // 16
        padded = np.full(16 * (t1 - t0), -1)
        padded[:len(cols)] = cols
        assert np.array_equal(t2b[16 * t0:16 * t1], padded)
        for lr in range(16):
            got = []
            for t in range(t0, t1):
                for i in range(ro[17 * t + lr], ro[17 * t + lr + 1]):
                    assert lr < r1 - r0
                    c = t2b[16 * t + int(s["col_idx"][i])]
                    assert c >= 0
                    dense[r0 + lr, c] += s["value"][i]
                    got.append((t, c, s["value"][i]))
            if lr < r1 - r0:
                # Per TCB, the row's entries in CSR order.
                r = r0 + lr
                row = list(zip(col[rp[r]:rp[r + 1]].tolist(), val[rp[r]:rp[r + 1]].tolist()))
                for t in range(t0, t1):
                    mine = set(t2b[16 * t:16 * t + 16].tolist())
                    assert [(c, v) for (tt, c, v) in got if tt == t] == \
                        [(c, v) for (c, v) in row if c in mine]
    assert np.array_equal(dense, want)


def test_cst_row_offsets_past_16_bits(orc):
    """The reference stores the absolute row offsets as uint16_t
    (fastspmm.cu:216,225) and its kernel subtracts the TCB's 32-bit first
    entry (fastspmm.cu:61-71): once a matrix passes 65535 entries, the
    16-bit offsets no longer give a TCB row's extent.  The restatement keeps
    int offsets, so every TCB row still indexes its own entries."""
    M, N = 64, 4096
    rng = np.random.default_rng(5)
    rp = np.arange(0, M * 1200 + 1, 1200, dtype=np.int32)
    col = np.concatenate([np.sort(rng.choice(N, 1200, replace=False)) for _ in range(M)]).astype(np.int32)
    val = np.ones(len(col), np.float32)
    s = orc.build_cst(M, N, rp, col, val)
    ro, co = s["tcb_row_off"].astype(np.int64), s["tcb_col_off"].astype(np.int64)
    assert co[-1] == M * 1200 > 65535
    base = np.repeat(co[:-1], 17)
    start = ro - base
    assert np.all((start >= 0) & (start <= np.repeat(np.diff(co), 17)))
    wrapped = (ro & 0xFFFF) - base
    assert np.any(wrapped < 0)
