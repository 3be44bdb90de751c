"""ctypes access to the CPU checkers - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker.  The product (vcsr-spmm_amd/) never
imports it.

  liboracle.so     restatement of the reference algorithms (vcsr_oracle.cpp)
  _ref/libref.so   the reference's own host builders compiled from
                   /root/reference by oracle/Makefile (absent if it was never
                   built; tests that need it skip)
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")


class _OrcFmt(C.Structure):
    _fields_ = [("M", C.c_int), ("N", C.c_int), ("segw", C.c_int), ("bundle", C.c_int),
                ("num_groups", C.c_int), ("num_segments", C.c_int), ("num_slots", C.c_longlong),
                ("group_ptr", C.POINTER(C.c_int)), ("group_depth", C.POINTER(C.c_int)),
                ("group_seg_base", C.POINTER(C.c_int)), ("group_rows", C.POINTER(C.c_int)),
                ("lcol", C.POINTER(C.c_int)), ("val", C.POINTER(C.c_float)),
                ("segment_group_start", C.POINTER(C.c_int))]


class _RefFmt(C.Structure):
    _fields_ = [("M", C.c_int), ("N", C.c_int), ("segw", C.c_int), ("bundle", C.c_int),
                ("num_groups", C.c_int), ("has_sgs", C.c_int), ("num_slots", C.c_longlong),
                ("group_ptr", C.POINTER(C.c_int)), ("group_depth", C.POINTER(C.c_int)),
                ("group_seg_base", C.POINTER(C.c_int)), ("group_rows", C.POINTER(C.c_int)),
                ("lcol", C.POINTER(C.c_int)), ("val", C.POINTER(C.c_float)),
                ("segment_group_start", C.POINTER(C.c_int)), ("num_segments", C.c_int)]


class _Csr(C.Structure):
    _fields_ = [("M", C.c_int), ("N", C.c_int), ("nnz", C.c_int),
                ("row_ptr", C.POINTER(C.c_int)), ("col", C.POINTER(C.c_int)),
                ("val", C.POINTER(C.c_float))]


class _Coo(C.Structure):
    _fields_ = [("M", C.c_int), ("N", C.c_int), ("nnz", C.c_longlong),
                ("rows", C.POINTER(C.c_int)), ("cols", C.POINTER(C.c_int)),
                ("vals", C.POINTER(C.c_float))]


class _Cst(C.Structure):
    _fields_ = [("M", C.c_int), ("N", C.c_int), ("num_windows", C.c_int), ("num_tcb", C.c_int),
                ("num_entries", C.c_int), ("window_off", C.POINTER(C.c_int)),
                ("tcb_col_off", C.POINTER(C.c_int)), ("tcb_row_off", C.POINTER(C.c_int)),
                ("col_idx", C.POINTER(C.c_ubyte)), ("value", C.POINTER(C.c_float)),
                ("tcb2b", C.POINTER(C.c_int))]


def _take(lib_free, ptr, n, dtype):
    out = (np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True)
           if n else np.zeros(0, dtype=dtype))
    lib_free(C.cast(ptr, C.c_void_p))
    return out


def _p(a):
    return C.c_void_p(a.ctypes.data) if a.size else C.c_void_p(0)


_orc = None
_ref = None


def oracle_lib():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} not built (run __graft_entry__.build())")
        lib = C.CDLL(ORACLE_SO)
        lib.orc_last_error.restype = C.c_char_p
        lib.orc_free.argtypes = [C.c_void_p]
        lib.orc_read_mtx.argtypes = [C.c_char_p, C.POINTER(_Coo)]
        lib.orc_coo_to_csr.argtypes = [C.c_int, C.c_int, C.c_longlong, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.POINTER(_Csr)]
        lib.orc_build.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                  C.c_int, C.c_int, C.POINTER(_OrcFmt)]
        lib.orc_spmm_f32.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_int, C.c_void_p]
        lib.orc_spmm_f32.restype = None
        lib.orc_spmm_f64.argtypes = lib.orc_spmm_f32.argtypes
        lib.orc_spmm_f64.restype = None
        lib.orc_spmm_f32_mt.argtypes = lib.orc_spmm_f32.argtypes + [C.c_int]
        lib.orc_spmm_f32_mt.restype = None
        lib.orc_spmm_f64_mt.argtypes = lib.orc_spmm_f32_mt.argtypes
        lib.orc_spmm_f64_mt.restype = None
        lib.orc_vcsr_apply.argtypes = [C.c_int] * 5 + [C.c_void_p] * 7 + [C.c_int, C.c_void_p]
        lib.orc_vcsr_apply.restype = None
        lib.orc_build_cst.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.POINTER(_Cst)]
        _orc = lib
    return _orc


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref_lib():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_SO} not built")
        lib = C.CDLL(REF_SO)
        lib.ref_last_error.restype = C.c_char_p
        lib.ref_free.argtypes = [C.c_void_p]
        lib.ref_read_mtx.argtypes = [C.c_char_p, C.POINTER(_Coo)]
        lib.ref_coo_to_csr.argtypes = [C.c_int, C.c_int, C.c_longlong, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.POINTER(_Csr)]
        for n in ("ref_build_h", "ref_build_s"):
            getattr(lib, n).argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_int, C.c_int, C.POINTER(_RefFmt)]
        lib.ref_build_tc.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_int, C.POINTER(_RefFmt)]
        _ref = lib
    return _ref


def _fmt_dict(lib_free, f, with_sgs):
    G, P, b = f.num_groups, f.num_slots, f.bundle
    d = {
        "segw": f.segw, "bundle": f.bundle, "num_groups": G, "num_slots": P,
        "group_ptr": _take(lib_free, f.group_ptr, G + 1, np.int32),
        "group_depth": _take(lib_free, f.group_depth, G, np.int32),
        "group_seg_base": _take(lib_free, f.group_seg_base, G, np.int32),
        "group_rows": _take(lib_free, f.group_rows, G * b, np.int32),
        "lcol": _take(lib_free, f.lcol, P, np.int32),
        "val": _take(lib_free, f.val, P, np.float32),
    }
    if with_sgs:
        d["segment_group_start"] = _take(lib_free, f.segment_group_start, f.num_segments + 1,
                                         np.int32)
    return d


# ------------------------------------------------------------------ oracle
def read_mtx(path):
    lib = oracle_lib()
    c = _Coo()
    if lib.orc_read_mtx(path.encode(), C.byref(c)) != 0:
        raise RuntimeError("oracle read_mtx: " + lib.orc_last_error().decode())
    n = c.nnz
    return (c.M, c.N, _take(lib.orc_free, c.rows, n, np.int32),
            _take(lib.orc_free, c.cols, n, np.int32), _take(lib.orc_free, c.vals, n, np.float32))


def coo_to_csr(M, N, rows, cols, vals):
    lib = oracle_lib()
    rows, cols = np.ascontiguousarray(rows, np.int32), np.ascontiguousarray(cols, np.int32)
    vals = np.ascontiguousarray(vals, np.float32)
    s = _Csr()
    if lib.orc_coo_to_csr(M, N, len(vals), _p(rows), _p(cols), _p(vals), C.byref(s)) != 0:
        raise RuntimeError("oracle coo_to_csr: " + lib.orc_last_error().decode())
    return (_take(lib.orc_free, s.row_ptr, M + 1, np.int32),
            _take(lib.orc_free, s.col, s.nnz, np.int32),
            _take(lib.orc_free, s.val, s.nnz, np.float32))


def build(M, N, row_ptr, col, val, segw, bundle, layout):
    """layout 0 = H, 1 = S, 2 = TC; returns a dict of arrays."""
    lib = oracle_lib()
    row_ptr, col = np.ascontiguousarray(row_ptr, np.int32), np.ascontiguousarray(col, np.int32)
    val = np.ascontiguousarray(val, np.float32)
    f = _OrcFmt()
    if lib.orc_build(M, N, _p(row_ptr), _p(col), _p(val), segw, bundle, layout, C.byref(f)) != 0:
        raise RuntimeError("oracle build: " + lib.orc_last_error().decode())
    return _fmt_dict(lib.orc_free, f, True)


def _spmm(M, row_ptr, col, val, B, dtype, nthreads):
    lib = oracle_lib()
    B = np.ascontiguousarray(B, np.float32)
    out = np.empty((M, B.shape[1]), dtype)
    args = (M, _p(np.ascontiguousarray(row_ptr, np.int32)), _p(np.ascontiguousarray(col, np.int32)),
            _p(np.ascontiguousarray(val, np.float32)), _p(B), B.shape[1], _p(out))
    f32 = dtype == np.float32
    if nthreads == 1:
        (lib.orc_spmm_f32 if f32 else lib.orc_spmm_f64)(*args)
    else:
        (lib.orc_spmm_f32_mt if f32 else lib.orc_spmm_f64_mt)(*args, int(nthreads))
    return out


def spmm_f32(M, row_ptr, col, val, B, nthreads=1):
    """FP32 CSR SpMM in the reference loop order; nthreads != 1 splits the
    rows over threads (<= 0: all hardware threads), same result."""
    return _spmm(M, row_ptr, col, val, B, np.float32, nthreads)


def spmm_f64(M, row_ptr, col, val, B, nthreads=1):
    """The same sum accumulated in double (the tolerance checks' reference)."""
    return _spmm(M, row_ptr, col, val, B, np.float64, nthreads)


def vcsr_apply(M, N, fmt, B):
    """C = A_fmt * B in double, walking the packed format."""
    lib = oracle_lib()
    B = np.ascontiguousarray(B, np.float32)
    O = B.shape[1]
    out = np.zeros((M, O), np.float64)
    a = {k: np.ascontiguousarray(fmt[k]) for k in
         ("group_ptr", "group_depth", "group_seg_base", "group_rows", "lcol", "val")}
    lib.orc_vcsr_apply(M, N, fmt["segw"], fmt["bundle"], len(a["group_depth"]),
                       _p(a["group_ptr"]), _p(a["group_depth"]), _p(a["group_seg_base"]),
                       _p(a["group_rows"]), _p(a["lcol"]), _p(a["val"]), _p(B), O, _p(out))
    return out


def build_cst(M, N, row_ptr, col, val):
    """FastSpMM's condensed sparse tiles (16-row windows, 16-column TCBs) as a
    dict of arrays: window_off (W+1), tcb_col_off (T+1), tcb_row_off (17 T,
    absolute entry numbers), col_idx (uint8), value (float32), tcb2b (16 T)."""
    lib = oracle_lib()
    row_ptr, col = np.ascontiguousarray(row_ptr, np.int32), np.ascontiguousarray(col, np.int32)
    val = np.ascontiguousarray(val, np.float32)
    s = _Cst()
    if lib.orc_build_cst(M, N, _p(row_ptr), _p(col), _p(val), C.byref(s)) != 0:
        raise RuntimeError("oracle build_cst: " + lib.orc_last_error().decode())
    T, E, f = s.num_tcb, s.num_entries, lib.orc_free
    return {"num_windows": s.num_windows, "num_tcb": T,
            "window_off": _take(f, s.window_off, s.num_windows + 1, np.int32),
            "tcb_col_off": _take(f, s.tcb_col_off, T + 1, np.int32),
            "tcb_row_off": _take(f, s.tcb_row_off, 17 * T, np.int32),
            "col_idx": _take(f, s.col_idx, E, np.uint8),
            "value": _take(f, s.value, E, np.float32),
            "tcb2b": _take(f, s.tcb2b, 16 * T, np.int32)}


# -------------------------------------------------------------- reference
def ref_read_mtx(path):
    lib = ref_lib()
    c = _Coo()
    if lib.ref_read_mtx(path.encode(), C.byref(c)) != 0:
        raise RuntimeError("reference read_mtx: " + lib.ref_last_error().decode())
    n = c.nnz
    return (c.M, c.N, _take(lib.ref_free, c.rows, n, np.int32),
            _take(lib.ref_free, c.cols, n, np.int32), _take(lib.ref_free, c.vals, n, np.float32))


def ref_coo_to_csr(M, N, rows, cols, vals):
    lib = ref_lib()
    rows, cols = np.ascontiguousarray(rows, np.int32), np.ascontiguousarray(cols, np.int32)
    vals = np.ascontiguousarray(vals, np.float32)
    s = _Csr()
    if lib.ref_coo_to_csr(M, N, len(vals), _p(rows), _p(cols), _p(vals), C.byref(s)) != 0:
        raise RuntimeError("reference coo_to_csr: " + lib.ref_last_error().decode())
    return (_take(lib.ref_free, s.row_ptr, M + 1, np.int32),
            _take(lib.ref_free, s.col, s.nnz, np.int32),
            _take(lib.ref_free, s.val, s.nnz, np.float32))


def ref_build(M, N, row_ptr, col, val, segw, bundle, layout):
    lib = ref_lib()
    row_ptr, col = np.ascontiguousarray(row_ptr, np.int32), np.ascontiguousarray(col, np.int32)
    val = np.ascontiguousarray(val, np.float32)
    f = _RefFmt()
    if layout == 0:
        rc = lib.ref_build_h(M, N, _p(row_ptr), _p(col), _p(val), segw, bundle, C.byref(f))
    elif layout == 1:
        rc = lib.ref_build_s(M, N, _p(row_ptr), _p(col), _p(val), segw, bundle, C.byref(f))
    else:
        rc = lib.ref_build_tc(M, N, _p(row_ptr), _p(col), _p(val), bundle, C.byref(f))
    if rc != 0:
        raise RuntimeError("reference build: " + lib.ref_last_error().decode())
    return _fmt_dict(lib.ref_free, f, bool(f.has_sgs))
