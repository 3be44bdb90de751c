"""Writes tests/golden/vcsr_golden.json from the REFERENCE's own host code.

The fixtures pin the oracle (oracle/vcsr_oracle.cpp) and the product
builders to what MuuSeoTia/VCSR-SPMM itself produces.  They are made with
oracle/_ref/libref.so, which oracle/Makefile compiles from the reference's
sources where they lie (include/mmio.hpp, csr.hpp, vcsr.hpp and the host
parts of src/vcsr_seg.cu and src/vcsr_tc.cu); no reference source is copied.

Contents (all data, no code):
  * mtx:   Matrix Market texts written by this script and the COO the
           reference reader returns for them (read_matrix_market_coo);
  * csr:   COO inputs (with duplicate and unsorted columns) and the CSR that
           the reference's coo_to_csr returns;
  * tiny:  small CSR matrices and the full VCSR arrays of layouts H, S and TC;
  * large: for synthetic configs cfg1 (seed 0), cfg2, cfg3, cfg4 and cfg5,
           a SHA-256 of the CSR input (to pin the generator) and of every
           VCSR array.  cfg3 and cfg4 have layout S only (segw 4; cfg4 also
           segw 8): the reference's layout-H builder allocates S*M entry
           lists (include/vcsr.hpp:33), 26e9 for cfg3.

Run from the repository root after __graft_entry__.build():
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import importlib.util
import json
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as orc  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "vcsr_golden.json")
ARRAYS = ("group_ptr", "group_depth", "group_seg_base", "group_rows", "lcol", "val")


def product():
    spec = importlib.util.spec_from_file_location(
        "vcsr_spmm_amd", os.path.join(ROOT, "vcsr-spmm_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["vcsr_spmm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def lst(a):
    a = np.asarray(a)
    if a.dtype == np.float32:
        return [float(x) for x in a]  # float32 -> double is exact; JSON keeps it exact
    return [int(x) for x in a]


MTX_CASES = {
    "one_based_general": "%%MatrixMarket matrix coordinate real general\n% comment\n\n"
                         "3 4 5\n1 1 1.5\n2 3 -2.25\n3 4 0.1\n1 4 7e-3\n3 1 -1\n",
    "zero_based_detect": "%%MatrixMarket matrix coordinate real general\n"
                         "2 2 3\n0 1 2.0\n1 0 3.0\n1 1 4.0\n",
    "symmetric_not_expanded": "%%MatrixMarket matrix coordinate real symmetric\n"
                              "3 3 4\n1 1 2.0\n2 1 -1.0\n3 2 -1.0\n3 3 2.0\n",
    "entries_across_lines": "%%MatrixMarket matrix coordinate real general\n"
                            "2 3 3\n1 1\n 0.5 2 3 1.25\n1 2 -0.75\n",
    "double_rounding": "%%MatrixMarket matrix coordinate real general\n"
                       "1 2 2\n1 1 0.1000000000000000055511151231257827\n1 2 3.4028234663852886e38\n",
}


def tiny_cases():
    """Hand-made CSR inputs (as COO, converted by the reference's coo_to_csr)."""
    cases = {}
    rng = np.random.default_rng(20251201)
    # 1: the example of a single segment with ties and an empty row
    cases["ties_and_empty"] = (5, 8, [0, 0, 1, 2, 2, 2, 4, 4], [0, 1, 0, 1, 2, 3, 6, 7],
                               [1, 2, 3, 4, 5, 6, 7, 8])
    # 2: N not a multiple of segw, one dense row
    cases["ragged_n"] = (4, 10, [0] * 10 + [2, 3, 3], list(range(10)) + [9, 0, 9],
                         list(np.arange(1, 14) * 0.5))
    # 3: duplicates (kept, not merged) and unsorted input columns
    cases["duplicates"] = (3, 6, [0, 0, 0, 1, 1, 2, 2, 2], [5, 1, 5, 2, 2, 0, 4, 0],
                           [1, 2, 3, 4, 5, 6, 7, 8])
    # 4-6: random matrices with many equal per-segment counts (tie order)
    for name, (M, N, dens) in {"rand_a": (40, 37, 0.15), "rand_b": (70, 33, 0.08),
                               "rand_c": (130, 48, 0.05)}.items():
        rows, cols = [], []
        for r in range(M):
            k = rng.binomial(N, dens)
            c = rng.choice(N, size=k, replace=False)
            rng.shuffle(c)
            rows += [r] * k
            cols += c.tolist()
        vals = rng.uniform(-1, 1, size=len(rows)).astype(np.float32)
        cases[name] = (M, N, rows, cols, vals.tolist())
    # 7: block-structured (every row of a 16x16 block has the same count)
    rows, cols = [], []
    for I, J in [(0, 2), (1, 0), (1, 2), (2, 1)]:
        for a in range(16):
            for b in range(16):
                rows.append(16 * I + a)
                cols.append(16 * J + b)
    cases["blocks16"] = (48, 48, rows, cols, list(rng.normal(size=len(rows)).astype(np.float32)))
    return cases


def main():
    if not orc.ref_available():
        sys.exit("oracle/_ref/libref.so is not built (needs /root/reference; run "
                 "__graft_entry__.build())")
    vs = product()
    out = {"source": "reference host code compiled by oracle/Makefile (oracle/_ref/libref.so)",
           "mtx": {}, "csr": {}, "tiny": {}, "large": {}}

    with tempfile.TemporaryDirectory() as td:
        for name, text in MTX_CASES.items():
            path = os.path.join(td, name + ".mtx")
            with open(path, "w") as f:
                f.write(text)
            M, N, r, c, v = orc.ref_read_mtx(path)
            out["mtx"][name] = {"text": text, "M": M, "N": N, "rows": lst(r), "cols": lst(c),
                                "vals": lst(v)}

    csr_cases = {"dups_unsorted": (4, 7, [3, 0, 0, 3, 1, 0, 3, 0, 3], [6, 2, 2, 0, 5, 1, 6, 2, 1],
                                   [1, 2, 3, 4, 5, 6, 7, 8, 9]),
                 "long_row_dups": (2, 5, [1] * 40, [(7 * i) % 5 for i in range(40)],
                                   list(np.arange(40, dtype=np.float32) * 0.25)),
                 "empty_rows": (6, 3, [5, 0], [2, 1], [1.0, 2.0])}
    for name, (M, N, r, c, v) in csr_cases.items():
        rp, col, val = orc.ref_coo_to_csr(M, N, r, c, np.asarray(v, np.float32))
        out["csr"][name] = {"M": M, "N": N, "rows": r, "cols": c, "vals": lst(np.float32(v)),
                            "row_ptr": lst(rp), "col": lst(col), "val": lst(val)}

    for name, (M, N, r, c, v) in tiny_cases().items():
        rp, col, val = orc.ref_coo_to_csr(M, N, r, c, np.asarray(v, np.float32))
        entry = {"M": M, "N": N, "row_ptr": lst(rp), "col": lst(col), "val": lst(val), "fmt": {}}
        plan = [(0, "H", [(4, 64), (4, 8), (3, 5)]), (1, "S", [(4, 64), (4, 8), (3, 5), (1, 2)]),
                (2, "TC", [(16, 16)])]
        if name == "blocks16":  # 12k nonzeros: keep the fixture small
            plan = [(1, "S", [(4, 64)]), (2, "TC", [(16, 16)])]
        for layout, lname, params in plan:
            for segw, bundle in params:
                f = orc.ref_build(M, N, rp, col, val, segw, bundle, layout)
                entry["fmt"][f"{lname}_{segw}_{bundle}"] = {
                    "layout": layout, "segw": f["segw"], "bundle": f["bundle"],
                    **{k: lst(f[k]) for k in ARRAYS},
                    **({"segment_group_start": lst(f["segment_group_start"])}
                       if "segment_group_start" in f else {})}
        out["tiny"][name] = entry

    for cfg, fmts in [(1, [(0, 4, 64), (1, 4, 64), (0, 4, 32), (1, 4, 32), (2, 16, 16)]),
                      (2, [(1, 4, 64), (1, 4, 32)]), (3, [(1, 4, 64)]),
                      (4, [(1, 4, 64), (1, 8, 64)]), (5, [(2, 16, 16)])]:
        csr = vs.coo_to_csr(vs.generate_coo(cfg, 0))
        rp, col, val = orc.ref_coo_to_csr(csr.M, csr.N, *[
            np.asarray(x) for x in (vs.generate_coo(cfg, 0).rows, vs.generate_coo(cfg, 0).cols,
                                    vs.generate_coo(cfg, 0).vals)])
        assert np.array_equal(rp, csr.row_ptr) and np.array_equal(col, csr.col)
        entry = {"seed": 0, "M": csr.M, "N": csr.N, "nnz": int(csr.nnz),
                 "csr_sha256": {"row_ptr": sha(rp), "col": sha(col), "val": sha(val)}, "fmt": {}}
        for layout, segw, bundle in fmts:
            f = orc.ref_build(csr.M, csr.N, rp, col, val, segw, bundle, layout)
            key = f"{['H', 'S', 'TC'][layout]}_{segw}_{bundle}"
            entry["fmt"][key] = {"layout": layout, "segw": segw, "bundle": bundle,
                                 "num_groups": int(f["num_groups"]),
                                 "num_slots": int(f["num_slots"]),
                                 "sha256": {k: sha(f[k]) for k in ARRAYS}}
            print(f"cfg{cfg} {key}: G={f['num_groups']} P={f['num_slots']}", flush=True)
        out["large"][f"cfg{cfg}"] = entry

    with open(OUT, "w") as fh:
        json.dump(out, fh, separators=(",", ":"), sort_keys=True)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
