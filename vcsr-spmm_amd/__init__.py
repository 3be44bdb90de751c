"""Python binding of the gfx950 VCSR SpMM library (lib/libvcsr_spmm.so).

A thin ctypes layer over the C ABI of include/vcsr_spmm.h, with the
reference's function names (MuuSeoTia/VCSR-SPMM) so callers and tests read
like the reference's host code:

    read_matrix_market_coo(path)          include/mmio.hpp:22
    coo_to_csr(coo)                       include/csr.hpp:16
    csr_to_vcsr_spmm(csr, segw, bundle)   include/vcsr.hpp:25    (layout H)
    csr_to_vcsr_seg(csr, segw, bundle)    src/vcsr_seg.cu:24     (layout S)
    csr_to_vcsr_opt(csr, segw, bundle)    src/vcsr_opt.cu:23     (layout S)
    csr_to_vcsr_tc(csr, bundle)           src/vcsr_tc.cu:26      (layout TC)
    run_csr_spmm_gpu(...)                 src/kernels.cu:107
    run_vcsr_spmm_gpu(fmt, dB, O, tileK, dC, stream)   src/kernels.cu:120
    run_vcsr_tc_spmm_gpu(fmt, dB, O, dC, stream)       src/vcsr_tc.cu:197

Errors: the reference throws std::runtime_error from the builders and exits
on CUDA errors; here every failure raises VcsrError carrying the library
status code and message.  GPU calls need a GPU: there is no CPU fallback,
and calling one without a GPU raises VcsrError (status VCSR_EDEVICE).
Device memory and streams are the library's own (DeviceArray, Stream); no
second GPU runtime is loaded into the process.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libvcsr_spmm.so")
CLI_PATH = os.path.join(_HERE, "bin", "spmm_vcsr")

VCSR_OK, VCSR_EINVAL, VCSR_EIO, VCSR_ENOMEM, VCSR_EDEVICE, VCSR_ERANGE, VCSR_ESTATE = range(7)
LAYOUT_H, LAYOUT_S, LAYOUT_TC = 0, 1, 2
KERNEL_AUTO, KERNEL_SEGMENT, KERNEL_MFMA, KERNEL_ROW, KERNEL_TILE = 0, 1, 2, 3, 4

# Every symbol include/vcsr_spmm.h declares (checked by the CPU test suite).
EXPORTS = (
    "vcsr_last_error vcsr_version vcsr_mtx_read vcsr_coo_create vcsr_coo_view_get "
    "vcsr_coo_free vcsr_gen_coo vcsr_gen_dense vcsr_coo_to_csr vcsr_csr_create "
    "vcsr_csr_view_get vcsr_csr_free vcsr_build vcsr_fmt_arrays vcsr_fmt_save vcsr_fmt_load "
    "vcsr_fmt_upload "
    "vcsr_fmt_set_tile_rows vcsr_fmt_set_tile_windows vcsr_fmt_tile_info vcsr_fmt_free spmm_csr_naive spmm_csr_wave spmm_vcsr "
    "spmm_vcsr_ex spmm_vcsr_noalloc spmm_vcsr_mfma vcsr_mfma_work vcsr_launch_info_get vcsr_tile_mfma_work spmm_csr_cpu "
    "vcsr_vendor_plan_create vcsr_vendor_spmm vcsr_vendor_plan_free spmm_csr_vendor "
    "vcsr_device_count vcsr_device_name vcsr_dev_malloc vcsr_dev_free vcsr_memcpy_h2d "
    "vcsr_memcpy_d2h vcsr_memcpy_d2d vcsr_memset_d vcsr_stream_create vcsr_stream_destroy "
    "vcsr_stream_sync vcsr_device_sync vcsr_event_create vcsr_event_destroy "
    "vcsr_event_record vcsr_event_elapsed"
).split()


class VcsrError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class _CooView(C.Structure):
    _fields_ = [("M", C.c_int32), ("N", C.c_int32), ("nnz", C.c_int64),
                ("rows", C.POINTER(C.c_int32)), ("cols", C.POINTER(C.c_int32)),
                ("vals", C.POINTER(C.c_float))]


class _CsrView(C.Structure):
    _fields_ = [("M", C.c_int32), ("N", C.c_int32), ("nnz", C.c_int32),
                ("row_ptr", C.POINTER(C.c_int32)), ("col", C.POINTER(C.c_int32)),
                ("val", C.POINTER(C.c_float))]


class _LaunchInfo(C.Structure):
    _fields_ = [("kernel", C.c_int32), ("tile_rows", C.c_int32), ("tiles", C.c_int64),
                ("entries", C.c_int64), ("matrix_cores", C.c_int32), ("vec", C.c_int32),
                ("column_slices", C.c_int32), ("slice_cols", C.c_int32),
                ("reduce_launches", C.c_int32), ("split_rows", C.c_int32),
                ("scratch_floats", C.c_int64)]


class _Arrays(C.Structure):
    _fields_ = [("M", C.c_int32), ("N", C.c_int32), ("segw", C.c_int32),
                ("bundle", C.c_int32), ("layout", C.c_int32), ("num_groups", C.c_int32),
                ("num_segments", C.c_int32), ("num_slots", C.c_int64),
                ("group_ptr", C.POINTER(C.c_int32)), ("group_depth", C.POINTER(C.c_int32)),
                ("group_seg_base", C.POINTER(C.c_int32)), ("group_rows", C.POINTER(C.c_int32)),
                ("lcol", C.POINTER(C.c_int32)), ("val", C.POINTER(C.c_float)),
                ("segment_group_start", C.POINTER(C.c_int32))]


_lib = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Loads lib/libvcsr_spmm.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise VcsrError(VCSR_EDEVICE, f"{path} not built (run __graft_entry__.build())")
    lib = C.CDLL(path)
    P, I32, I64, U64, F = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float
    pI, pF, pP = C.POINTER(C.c_int32), C.POINTER(C.c_float), C.POINTER(C.c_void_p)
    sig = {
        "vcsr_last_error": (C.c_char_p, []),
        "vcsr_version": (C.c_char_p, []),
        "vcsr_mtx_read": (C.c_int, [C.c_char_p, I32, pP]),
        "vcsr_coo_create": (C.c_int, [I32, I32, I64, P, P, P, pP]),
        "vcsr_coo_view_get": (C.c_int, [P, C.POINTER(_CooView)]),
        "vcsr_coo_free": (None, [P]),
        "vcsr_gen_coo": (C.c_int, [I32, U64, pP]),
        "vcsr_gen_dense": (C.c_int, [U64, I32, I64, I32, P]),
        "vcsr_coo_to_csr": (C.c_int, [P, pP]),
        "vcsr_csr_create": (C.c_int, [I32, I32, P, P, P, pP]),
        "vcsr_csr_view_get": (C.c_int, [P, C.POINTER(_CsrView)]),
        "vcsr_csr_free": (None, [P]),
        "vcsr_build": (C.c_int, [P, I32, I32, I32, I32, pP]),
        "vcsr_fmt_arrays": (C.c_int, [P, C.POINTER(_Arrays)]),
        "vcsr_fmt_upload": (C.c_int, [P, P]),
        "vcsr_fmt_save": (C.c_int, [P, C.c_char_p]),
        "vcsr_fmt_load": (C.c_int, [C.c_char_p, pP]),
        "vcsr_fmt_set_tile_rows": (C.c_int, [P, I32]),
        "vcsr_fmt_set_tile_windows": (C.c_int, [P, I32]),
        "vcsr_fmt_tile_info": (C.c_int, [P, pI, C.POINTER(I64), C.POINTER(I64)]),
        "vcsr_fmt_free": (None, [P]),
        "spmm_csr_naive": (C.c_int, [I32, P, P, P, P, I32, P, P, pF]),
        "spmm_csr_wave": (C.c_int, [I32, I32, P, P, P, P, I32, P, P, pF]),
        "spmm_vcsr": (C.c_int, [P, P, I32, I32, P, P, pF]),
        "spmm_vcsr_ex": (C.c_int, [P, P, I32, I32, P, P, pF, I32, I32]),
        "spmm_vcsr_noalloc": (C.c_int, [P, P, I32, P, P, I32]),
        "spmm_vcsr_mfma": (C.c_int, [P, P, I32, P, P, pF]),
        "vcsr_mfma_work": (C.c_int, [P, I32, I32, C.POINTER(I64), pI]),
        "vcsr_launch_info_get": (C.c_int, [P, I32, I32, C.POINTER(_LaunchInfo)]),
        "vcsr_tile_mfma_work": (C.c_int, [P, I32, C.POINTER(I64), pI]),
        "spmm_csr_cpu": (C.c_int, [I32, P, P, P, P, I32, P, I32]),
        "vcsr_vendor_plan_create": (C.c_int, [I32, I32, I32, P, P, P, P, I32, P, P,
                                              C.POINTER(P)]),
        "vcsr_vendor_spmm": (C.c_int, [P, P, pF]),
        "vcsr_vendor_plan_free": (None, [P]),
        "spmm_csr_vendor": (C.c_int, [I32, I32, I32, P, P, P, P, I32, P, P, pF]),
        "vcsr_device_count": (C.c_int, [pI]),
        "vcsr_device_name": (C.c_int, [C.c_char_p, I32]),
        "vcsr_dev_malloc": (C.c_int, [pP, C.c_size_t]),
        "vcsr_dev_free": (C.c_int, [P]),
        "vcsr_memcpy_h2d": (C.c_int, [P, P, C.c_size_t, P]),
        "vcsr_memcpy_d2h": (C.c_int, [P, P, C.c_size_t, P]),
        "vcsr_memcpy_d2d": (C.c_int, [P, P, C.c_size_t, P]),
        "vcsr_memset_d": (C.c_int, [P, I32, C.c_size_t, P]),
        "vcsr_stream_create": (C.c_int, [pP]),
        "vcsr_stream_destroy": (C.c_int, [P]),
        "vcsr_stream_sync": (C.c_int, [P]),
        "vcsr_device_sync": (C.c_int, []),
        "vcsr_event_create": (C.c_int, [pP]),
        "vcsr_event_destroy": (C.c_int, [P]),
        "vcsr_event_record": (C.c_int, [P, P]),
        "vcsr_event_elapsed": (C.c_int, [P, P, pF]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != VCSR_OK:
        raise VcsrError(rc, load_library().vcsr_last_error().decode())


def _ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data) if a.size else C.c_void_p(0)


def _copy(ptr, n: int, dtype) -> np.ndarray:
    if n == 0:
        return np.zeros(0, dtype=dtype)
    return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True)


# ----------------------------------------------------------------------- COO
class Coo:
    """Owned COO matrix (reference `struct COO`, include/mmio.hpp:15-19)."""

    def __init__(self, handle: C.c_void_p):
        self._h = handle
        v = _CooView()
        _check(load_library().vcsr_coo_view_get(self._h, C.byref(v)))
        self.M, self.N, self.nnz = v.M, v.N, v.nnz
        self.rows = _copy(v.rows, v.nnz, np.int32)
        self.cols = _copy(v.cols, v.nnz, np.int32)
        self.vals = _copy(v.vals, v.nnz, np.float32)

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.vcsr_coo_free(self._h)
            self._h = None

    @staticmethod
    def from_arrays(M, N, rows, cols, vals) -> "Coo":
        rows = np.ascontiguousarray(rows, dtype=np.int32)
        cols = np.ascontiguousarray(cols, dtype=np.int32)
        vals = np.ascontiguousarray(vals, dtype=np.float32)
        h = C.c_void_p()
        _check(load_library().vcsr_coo_create(M, N, len(vals), _ptr(rows), _ptr(cols),
                                             _ptr(vals), C.byref(h)))
        return Coo(h)


def read_matrix_market_coo(path: str, expand_symmetric: bool = False) -> Coo:
    h = C.c_void_p()
    _check(load_library().vcsr_mtx_read(path.encode(), 1 if expand_symmetric else 0, C.byref(h)))
    return Coo(h)


def generate_coo(cfg: int, seed: int = 0) -> Coo:
    """Synthetic A of benchmark config cfg (1..5)."""
    h = C.c_void_p()
    _check(load_library().vcsr_gen_coo(cfg, seed, C.byref(h)))
    return Coo(h)


def gen_dense(seed: int, dist: int, rows: int, cols: int) -> np.ndarray:
    """Synthetic dense operand; dist 0 = U[-1,1), 1 = N(0,1)."""
    out = np.empty((rows, cols), dtype=np.float32)
    _check(load_library().vcsr_gen_dense(seed, dist, rows, cols, _ptr(out)))
    return out


# ----------------------------------------------------------------------- CSR
class Csr:
    """Owned CSR matrix (reference `struct CSR`, include/csr.hpp:8-13)."""

    def __init__(self, handle: C.c_void_p):
        self._h = handle
        v = _CsrView()
        _check(load_library().vcsr_csr_view_get(self._h, C.byref(v)))
        self.M, self.N, self.nnz = v.M, v.N, v.nnz
        self.row_ptr = _copy(v.row_ptr, v.M + 1, np.int32)
        self.col = _copy(v.col, v.nnz, np.int32)
        self.val = _copy(v.val, v.nnz, np.float32)

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.vcsr_csr_free(self._h)
            self._h = None

    @staticmethod
    def from_arrays(M, N, row_ptr, col, val) -> "Csr":
        row_ptr = np.ascontiguousarray(row_ptr, dtype=np.int32)
        col = np.ascontiguousarray(col, dtype=np.int32)
        val = np.ascontiguousarray(val, dtype=np.float32)
        h = C.c_void_p()
        _check(load_library().vcsr_csr_create(M, N, _ptr(row_ptr), _ptr(col), _ptr(val),
                                             C.byref(h)))
        return Csr(h)


def coo_to_csr(coo: Coo) -> Csr:
    h = C.c_void_p()
    _check(load_library().vcsr_coo_to_csr(coo._h, C.byref(h)))
    return Csr(h)


# ---------------------------------------------------------------------- VCSR
class Vcsr:
    """Owned VCSR format; .arrays() returns copies of the packed arrays."""

    def __init__(self, handle: C.c_void_p):
        self._h = handle
        a = _Arrays()
        _check(load_library().vcsr_fmt_arrays(self._h, C.byref(a)))
        self.M, self.N, self.segw, self.bundle = a.M, a.N, a.segw, a.bundle
        self.layout, self.num_groups, self.num_segments = a.layout, a.num_groups, a.num_segments
        self.num_slots = a.num_slots

    def __del__(self):
        self.free()

    def free(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.vcsr_fmt_free(self._h)
            self._h = None

    def arrays(self) -> dict:
        a = _Arrays()
        _check(load_library().vcsr_fmt_arrays(self._h, C.byref(a)))
        G, P, S, b = a.num_groups, a.num_slots, a.num_segments, a.bundle
        return {
            "group_ptr": _copy(a.group_ptr, G + 1, np.int32),
            "group_depth": _copy(a.group_depth, G, np.int32),
            "group_seg_base": _copy(a.group_seg_base, G, np.int32),
            "group_rows": _copy(a.group_rows, G * b, np.int32),
            "lcol": _copy(a.lcol, P, np.int32),
            "val": _copy(a.val, P, np.float32),
            "segment_group_start": _copy(a.segment_group_start, S + 1, np.int32),
        }

    def upload(self, stream: "Stream | None" = None) -> None:
        _check(load_library().vcsr_fmt_upload(self._h, _sp(stream)))

    def set_tile_rows(self, rows: int) -> None:
        """Tile height of the row-tile view (0 = automatic); before upload()."""
        _check(load_library().vcsr_fmt_set_tile_rows(self._h, rows))

    def set_tile_windows(self, fixed: bool) -> None:
        """Fixed row windows of the tile height instead of shared-column
        tiles (16 rows: FastSpMM's condensed tiles); before upload()."""
        _check(load_library().vcsr_fmt_set_tile_windows(self._h, 1 if fixed else 0))

    def launch_info(self, O: int, kernel: int = 0) -> dict:
        """What one SpMM of width O launches (vcsr_launch_info_get): kernel,
        row-tile view, column slices, reduce launches, scratch floats."""
        info = _LaunchInfo()
        _check(load_library().vcsr_launch_info_get(self._h, O, kernel, C.byref(info)))
        return {name: getattr(info, name) for name, _ in _LaunchInfo._fields_}

    def tile_info(self) -> tuple[int, int, int]:
        """(tile height, tiles, entries) of the uploaded row-tile view."""
        r, t, e = C.c_int32(), C.c_int64(), C.c_int64()
        _check(load_library().vcsr_fmt_tile_info(self._h, C.byref(r), C.byref(t), C.byref(e)))
        return r.value, t.value, e.value


def save_vcsr(fmt: "Vcsr", path: str) -> None:
    """Write the format (host arrays, tile-view settings) to a file."""
    _check(load_library().vcsr_fmt_save(fmt._h, os.fsencode(path)))


def load_vcsr(path: str) -> "Vcsr":
    """Read a format file written by save_vcsr (validated; not uploaded)."""
    h = C.c_void_p()
    _check(load_library().vcsr_fmt_load(os.fsencode(path), C.byref(h)))
    return Vcsr(h)


def build_vcsr(csr: Csr, segw: int, bundle: int, layout: int, nthreads: int = 0) -> Vcsr:
    h = C.c_void_p()
    _check(load_library().vcsr_build(csr._h, segw, bundle, layout, nthreads, C.byref(h)))
    return Vcsr(h)


def csr_to_vcsr_spmm(csr: Csr, segw: int = 4, bundle: int = 32) -> Vcsr:
    return build_vcsr(csr, segw, bundle, LAYOUT_H)


def csr_to_vcsr_seg(csr: Csr, segw: int, bundle: int) -> Vcsr:
    return build_vcsr(csr, segw, bundle, LAYOUT_S)


csr_to_vcsr_opt = csr_to_vcsr_seg


def csr_to_vcsr_tc(csr: Csr, bundle: int = 16) -> Vcsr:
    return build_vcsr(csr, 16, bundle, LAYOUT_TC)


def spmm_csr_cpu(csr: Csr, B: np.ndarray, nthreads: int = 0) -> np.ndarray:
    B = np.ascontiguousarray(B, dtype=np.float32)
    O = B.shape[1]
    out = np.empty((csr.M, O), dtype=np.float32)
    _check(load_library().spmm_csr_cpu(csr.M, _ptr(csr.row_ptr), _ptr(csr.col), _ptr(csr.val),
                                       _ptr(B), O, _ptr(out), nthreads))
    return out


# -------------------------------------------------------------------- device
def device_count() -> int:
    n = C.c_int32(0)
    _check(load_library().vcsr_device_count(C.byref(n)))
    return n.value


def device_name() -> str:
    buf = C.create_string_buffer(128)
    _check(load_library().vcsr_device_name(buf, 128))
    return buf.value.decode()


class Stream:
    def __init__(self):
        self.h = C.c_void_p()
        _check(load_library().vcsr_stream_create(C.byref(self.h)))

    def sync(self):
        _check(load_library().vcsr_stream_sync(self.h))

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None and self.h.value:
            _lib.vcsr_stream_destroy(self.h)
            self.h = C.c_void_p()


def _sp(stream):
    return stream.h if stream is not None else C.c_void_p(0)


class Event:
    def __init__(self):
        self.h = C.c_void_p()
        _check(load_library().vcsr_event_create(C.byref(self.h)))

    def record(self, stream=None):
        _check(load_library().vcsr_event_record(self.h, _sp(stream)))

    def elapsed_ms(self, stop: "Event") -> float:
        ms = C.c_float(0)
        _check(load_library().vcsr_event_elapsed(self.h, stop.h, C.byref(ms)))
        return ms.value

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None and self.h.value:
            _lib.vcsr_event_destroy(self.h)
            self.h = C.c_void_p()


class DeviceArray:
    """A device buffer owned by the library's HIP runtime."""

    def __init__(self, shape, dtype):
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = C.c_void_p()
        _check(load_library().vcsr_dev_malloc(C.byref(self.ptr), self.nbytes))

    @staticmethod
    def from_numpy(a: np.ndarray, stream=None) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = DeviceArray(a.shape, a.dtype)
        _check(load_library().vcsr_memcpy_h2d(d.ptr, _ptr(a), d.nbytes, _sp(stream)))
        return d

    def numpy(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _check(load_library().vcsr_memcpy_d2h(_ptr(out), self.ptr, self.nbytes, _sp(stream)))
        return out

    def copy_from(self, other: "DeviceArray", stream=None) -> None:
        """Device-to-device copy of min(nbytes) bytes, enqueued on stream."""
        n = min(self.nbytes, other.nbytes)
        _check(load_library().vcsr_memcpy_d2d(self.ptr, other.ptr, n, _sp(stream)))

    def zero(self, stream=None) -> None:
        _check(load_library().vcsr_memset_d(self.ptr, 0, self.nbytes, _sp(stream)))

    def __del__(self):
        if getattr(self, "ptr", None) and _lib is not None and self.ptr.value:
            _lib.vcsr_dev_free(self.ptr)
            self.ptr = C.c_void_p()


def _need_buf(arr, dtype, count, what):
    """Raises VcsrError(VCSR_EINVAL) unless the device buffer `arr` holds at
    least `count` elements of `dtype`: the kernels index B and C by the
    shapes they are given, so a short or mistyped buffer would be read or
    written past its end on the device."""
    want = np.dtype(dtype)
    have = getattr(arr, "dtype", want)
    if np.dtype(have) != want:
        raise VcsrError(VCSR_EINVAL, f"{what}: dtype {np.dtype(have)}, expected {want}")
    nbytes = getattr(arr, "nbytes", None)
    if nbytes is None or int(nbytes) < int(count) * want.itemsize:
        raise VcsrError(VCSR_EINVAL, f"{what}: {nbytes} bytes, need {int(count) * want.itemsize}")


def _need_csr(M, d_rowptr, d_col, d_val, nnz=0):
    """CSR device buffers: row_ptr of M + 1 entries, col and val of equal
    length and at least `nnz` entries (the vendor library is told nnz and
    reads that many)."""
    if nnz < 0:
        raise VcsrError(VCSR_EINVAL, "negative nnz")
    _need_buf(d_rowptr, np.int32, M + 1, "row_ptr")
    _need_buf(d_col, np.int32, nnz, "col")
    _need_buf(d_val, np.float32, nnz, "val")
    if d_col.nbytes // 4 != d_val.nbytes // 4:
        raise VcsrError(VCSR_EINVAL, "col and val lengths differ")


def _need_bc(N, M, O, dB, dC):
    if O < 0:
        raise VcsrError(VCSR_EINVAL, "negative O")
    _need_buf(dB, np.float32, N * O, "B")
    _need_buf(dC, np.float32, M * O, "C")


def run_csr_spmm_gpu(M, d_rowptr, d_col, d_val, dB, O, dC, stream=None, timed=False):
    """C = A*B (overwrites C).  Returns kernel ms when timed (synchronous)."""
    _need_csr(M, d_rowptr, d_col, d_val)
    _need_bc(0, M, O, dB, dC)
    ms = C.c_float(0)
    _check(load_library().spmm_csr_naive(M, d_rowptr.ptr, d_col.ptr, d_val.ptr, dB.ptr, O,
                                         dC.ptr, _sp(stream), C.byref(ms) if timed else None))
    return ms.value if timed else None


class VendorPlan:
    """rocSPARSE SpMM (C = A*B) bound to device CSR arrays, B and C: the
    vendor baseline (the reference's run_cusparse_spmm, src/kernels.cu:169-235)
    with its set-up done once."""

    def __init__(self, M, N, nnz, d_rowptr, d_col, d_val, dB, O, dC, stream=None):
        _need_csr(M, d_rowptr, d_col, d_val, nnz)
        _need_bc(N, M, O, dB, dC)
        h = C.c_void_p()
        _check(load_library().vcsr_vendor_plan_create(M, N, nnz, d_rowptr.ptr, d_col.ptr,
                                                      d_val.ptr, dB.ptr, O, dC.ptr, _sp(stream),
                                                      C.byref(h)))
        self._h = h
        self._keep = (d_rowptr, d_col, d_val, dB, dC)

    def run(self, stream=None, timed=False):
        """C = A*B; the SpMM call's ms when timed (synchronous)."""
        ms = C.c_float(0)
        _check(load_library().vcsr_vendor_spmm(self._h, _sp(stream),
                                               C.byref(ms) if timed else None))
        return ms.value if timed else None

    def __del__(self):
        if getattr(self, "_h", None) and self._h.value:
            load_library().vcsr_vendor_plan_free(self._h)
            self._h = C.c_void_p()


def run_vendor_spmm_gpu(M, N, nnz, d_rowptr, d_col, d_val, dB, O, dC, stream=None, timed=False):
    """One-shot rocSPARSE C = A*B (set-up, SpMM, tear-down, like the
    reference's cuSPARSE wrapper); the SpMM call's ms when timed."""
    _need_csr(M, d_rowptr, d_col, d_val, nnz)
    _need_bc(N, M, O, dB, dC)
    ms = C.c_float(0)
    _check(load_library().spmm_csr_vendor(M, N, nnz, d_rowptr.ptr, d_col.ptr, d_val.ptr, dB.ptr,
                                          O, dC.ptr, _sp(stream), C.byref(ms) if timed else None))
    return ms.value if timed else None


def run_csr_wave_spmm_gpu(M, N, d_rowptr, d_col, d_val, dB, O, dC, stream=None, timed=False):
    """C = A*B with the wave-per-row CSR kernel (overwrites C); kernel ms
    when timed (synchronous)."""
    _need_csr(M, d_rowptr, d_col, d_val)
    _need_bc(N, M, O, dB, dC)
    ms = C.c_float(0)
    _check(load_library().spmm_csr_wave(M, N, d_rowptr.ptr, d_col.ptr, d_val.ptr, dB.ptr, O,
                                        dC.ptr, _sp(stream), C.byref(ms) if timed else None))
    return ms.value if timed else None


def run_vcsr_spmm_gpu(fmt: Vcsr, dB, O, tileK, dC, stream=None, timed=False):
    """C += A*B (spmm_vcsr: the default kernel, the reference's accumulate
    semantics, so zero C first)."""
    _need_bc(fmt.N, fmt.M, O, dB, dC)
    ms = C.c_float(0)
    _check(load_library().spmm_vcsr(fmt._h, dB.ptr, O, tileK, dC.ptr, _sp(stream),
                                    C.byref(ms) if timed else None))
    return ms.value if timed else None


def run_vcsr_tc_spmm_gpu(fmt: Vcsr, dB, O, dC, stream=None, timed=False):
    """C += A*B with the FP32-MFMA dense-tile kernel; zero C first."""
    _need_bc(fmt.N, fmt.M, O, dB, dC)
    ms = C.c_float(0)
    _check(load_library().spmm_vcsr_mfma(fmt._h, dB.ptr, O, dC.ptr, _sp(stream),
                                         C.byref(ms) if timed else None))
    return ms.value if timed else None


run_vcsr_mfma_spmm_gpu = run_vcsr_tc_spmm_gpu


def mfma_work(fmt: Vcsr, O: int, tileK: int = 0) -> tuple[int, int]:
    """(MFMA instructions, FLOPs per instruction) the FP32-MFMA kernel issues
    for one SpMM of width O (host only)."""
    ops, fpo = C.c_int64(), C.c_int32()
    _check(load_library().vcsr_mfma_work(fmt._h, O, tileK, C.byref(ops), C.byref(fpo)))
    return ops.value, fpo.value


def tile_mfma_work(fmt: Vcsr, O: int) -> tuple[int, int]:
    """(MFMA instructions, FLOPs per instruction) the tile-stationary kernel
    issues for one SpMM of width O on an uploaded format with 16-row tiles
    ((0, flops) for other tile heights)."""
    ops, fpo = C.c_int64(), C.c_int32()
    _check(load_library().vcsr_tile_mfma_work(fmt._h, O, C.byref(ops), C.byref(fpo)))
    return ops.value, fpo.value


def run_vcsr_spmm_gpu_ex(fmt: Vcsr, dB, O, tileK, dC, stream=None, timed=False,
                         kernel=KERNEL_AUTO, accumulate=True):
    """SpMM with an explicit kernel; accumulate=False computes C = A*B."""
    _need_bc(fmt.N, fmt.M, O, dB, dC)
    ms = C.c_float(0)
    _check(load_library().spmm_vcsr_ex(fmt._h, dB.ptr, O, tileK, dC.ptr, _sp(stream),
                                       C.byref(ms) if timed else None, kernel,
                                       1 if accumulate else 0))
    return ms.value if timed else None


def run_vcsr_spmm_gpu_noalloc(fmt: Vcsr, dB, O, dC, stream=None, accumulate=False):
    """The default (tile-stationary) kernel through spmm_vcsr_noalloc: no
    device allocation in the call; the partial rows of split tiles live in
    the library's fixed 16 MiB per-device scratch array (VCSR_ERANGE beyond
    it).  Enqueued only (not waited for); calls that overlap on one GPU race
    on that scratch."""
    _need_bc(fmt.N, fmt.M, O, dB, dC)
    _check(load_library().spmm_vcsr_noalloc(fmt._h, dB.ptr, O, dC.ptr, _sp(stream),
                                            1 if accumulate else 0))
