"""Benchmark of the VCSR SpMM hot path on one MI355X.

Workload (the headline): banded FEM-like A, 62,451^2,
~3.94M nnz (synthetic, seed 0), dense B 62,451 x 128 FP32 U[-1,1), VCSR
layout S with segw=4, bundle=64, tileK=64, built and uploaded before timing.

A step is one complete SpMM C = A*B on device-resident inputs.  The default
kernel (spmm_vcsr_ex, VCSR_KERNEL_AUTO = the tile-stationary VCSR kernel,
16-row tiles on FP32 MFMA where the row-tile view has them, accumulate = 0)
writes every element of C, so a step is its launches alone (one per column
slice, plus the reduce kernel where tiles are split); the kernels that
accumulate into C as the reference's do (--algo segment / mfma) get a C
reset inside the step.  --cols replaces a config's O (column sweeps).  K
steps are timed between HIP events after W warm-up steps; `value` is
2*nnz*O*K / that time.  `kernel_ms` is the kernel alone, K back-to-back
launches between events on its stream (the reference times kernels only,
src/kernels.cu:153-162); the roofline uses it.  `ms_per_step_median` is the
median per-step time of a second pass of K steps timed in 10 groups of K/10.
The default kernel's launch shape (tile height, column slices, reduce
launches) is named in `config`.

The default run also measures, in the same process and each checked over
all of C, the points the north star's targets name besides the headline
(`extra`): the power-law workload (config 3) at O = 128 on the default path,
the naive CSR kernel (src/kernels.cu:15-33) on configs 2 and 3 at O = 128
with the VCSR / naive speed-up, the block-sparse workload (config 5) at
O = 512 with its FP32 MFMA utilisation, and rocSPARSE on the headline
workload (the reference's cuSPARSE comparison).  The reference runs every
algorithm on the same matrix in one process (src/main.cpp:119-163).

Prints ONE JSON line.  Multi-GPU runs are not part of this build.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_FP32_PEAK_TFS = 157.3  # dense FP32 MFMA, MI355X

CONFIGS = {
    # name: (cfg, O, segw, bundle, tileK, layout, B distribution)
    "cfg2": (2, 128, 4, 64, 64, 1, 0),
    "cfg2_o8": (2, 8, 4, 64, 64, 1, 0),
    "cfg2_o32": (2, 32, 4, 64, 64, 1, 0),
    "cfg2_o512": (2, 512, 4, 64, 64, 1, 0),
    "cfg3": (3, 128, 4, 64, 128, 1, 0),
    "cfg3_o8": (3, 8, 4, 64, 128, 1, 0),
    "cfg4": (4, 256, 4, 64, 128, 1, 0),
    "cfg4_segw8": (4, 256, 8, 64, 128, 1, 0),
    "cfg5": (5, 512, 16, 16, 64, 2, 1),
}

# Sources whose code decides the traffic of the dominant (tile) kernel; the
# counter sets in profiles/traffic.json record their hash.
TRAFFIC_SOURCES = ("vcsr-spmm_amd/csrc/device/vcsr_tile.hip",
                   "vcsr-spmm_amd/csrc/device/vecops.hpp",
                   "vcsr-spmm_amd/csrc/device/common.hpp",
                   "vcsr-spmm_amd/csrc/host/tile_view.cpp",
                   "vcsr-spmm_amd/csrc/host/tile_view.hpp")


def _load_product():
    import importlib.util
    name = "vcsr_spmm_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(
        name, os.path.join(ROOT, "vcsr-spmm_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def kernel_sources_sha16():
    """First 16 hex digits of the SHA-256 of TRAFFIC_SOURCES, in order."""
    h = hashlib.sha256()
    for rel in TRAFFIC_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(point, algo):
    """HBM-side bytes per SpMM of the dominant kernel, from the committed
    rocprofv3 counter sets (profiles/traffic.json): FETCH_SIZE and WRITE_SIZE
    per dispatch, each divided by what the same counter reads per byte for a
    device-to-device copy of known size, times the kernel's dispatches per
    SpMM (column slices).  Returns (bytes, provenance) — provenance names
    the commit the counters were taken on and whether this tree's kernel
    sources are the ones profiled — or (None, None) if absent."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        e = t["points"][f"{point}/{algo}"]
        b = e.get("launches", 1) * (e["fetch_kib"] * 1024.0 / t["copy_fetch_factor"] +
                                    e["write_kib"] * 1024.0 / t["copy_write_factor"])
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None, None
    src = e.get("src_sha16")
    return b, {"commit": e.get("commit"), "profile": e.get("profile"),
               "kernel_sources_match": src is not None and src == kernel_sources_sha16()}


def copy_rate_gbs(vs, st, nbytes=512 << 20, reps=10):
    """Read + write bytes per second of a device-to-device copy of `nbytes`
    (hipMemcpyAsync), the rate a kernel that only streams bytes through HBM
    reaches on this GPU; measured in the same run as the SpMM."""
    src = vs.DeviceArray((nbytes // 4,), np.float32)
    dst = vs.DeviceArray((nbytes // 4,), np.float32)
    src.zero(st)
    for _ in range(2):
        dst.copy_from(src, st)
    ev0, ev1 = vs.Event(), vs.Event()
    ev0.record(st)
    for _ in range(reps):
        dst.copy_from(src, st)
    ev1.record(st)
    st.sync()
    ms = ev0.elapsed_ms(ev1) / reps
    return 2.0 * nbytes / (ms * 1e-3) / 1e9


def slice_path_report(w, li, kernel_ms):
    """The rate at which the tile kernel moves its B-row slices (view
    entries x O x 4 bytes per SpMM) from the caches to the CUs, set against
    the probe (lib/libvcsr_probe.so) reading slices of the same width and
    per-lane vector at random from a 2 MiB buffer (L2-resident: the
    practical ceiling of that path) and from a buffer the size of B (served
    by the MALL or HBM).  None where the timed kernel is not the vector-ALU
    tile kernel or its slices are not a power-of-two number of lanes."""
    import ctypes as C
    if li["matrix_cores"] or li["entries"] <= 0 or li["vec"] not in (1, 2, 4):
        return None
    slice_floats = li["slice_cols"]
    lps = slice_floats // li["vec"]
    if slice_floats % li["vec"] or not 1 <= lps <= 64 or lps & (lps - 1):
        return None
    lib = C.CDLL(os.path.join(ROOT, "vcsr-spmm_amd", "lib", "libvcsr_probe.so"))
    fn = lib.vcsr_probe_slice_reads
    fn.argtypes = [C.c_uint64, C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_double),
                   C.POINTER(C.c_double)]
    fn.restype = C.c_int

    def probe(nbytes):
        rate, ms = C.c_double(), C.c_double()
        rc = fn(nbytes, slice_floats, li["vec"], 10, C.byref(rate), C.byref(ms))
        if rc != 0:
            raise RuntimeError(f"slice probe failed ({rc})")
        return rate.value / 1e12

    b_bytes = w.csr.N * slice_floats * 4
    l2 = probe(2 << 20)
    bsz = probe(max(b_bytes, 2 << 20))
    kern = li["entries"] * w.O * 4 / (kernel_ms * 1e-3) / 1e12
    return {"slice_bytes": slice_floats * 4, "vec_floats": li["vec"],
            "kernel_tb_s": round(kern, 2), "probe_l2_resident_tb_s": round(l2, 2),
            "probe_b_sized_tb_s": round(bsz, 2), "frac_of_l2_resident": round(kern / l2, 4),
            "what": "B-row slices moved from the caches to the CUs per second: the timed "
                    "kernel (view entries x O x 4 bytes / kernel time) against a probe "
                    "reading random slices of the same shape from a 2 MiB buffer "
                    "(L2-resident) and from one of B's size (N x slice x 4 bytes)"}


def host_threads():
    """Threads the CPU baseline may use: the cores this process may run on,
    at most 16 (one GPU's share of the GPU box's host) and at most
    OMP_NUM_THREADS when that is set."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, min(n, 16))


def host_description():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": aff}


def cpu_baseline(orc, csr, B, seconds, nthreads):
    """The oracle's FP32 CSR SpMM (reference loop order, rows split over
    `nthreads` threads) on the same matrix and B, repeated until `seconds`
    of wall time after one untimed warm-up run.  Returns (GFLOP/s, reps,
    seconds, median seconds per SpMM)."""
    flop = 2.0 * csr.nnz * B.shape[1]
    orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B, nthreads)
    times = []
    while sum(times) < seconds and len(times) < 1000:
        t0 = time.perf_counter()
        orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B, nthreads)
        times.append(time.perf_counter() - t0)
    t_total = sum(times)
    return flop * len(times) / t_total / 1e9, len(times), t_total, float(np.median(times))


def full_check(orc, csr, B, C, nthreads):
    """Every element of C against the oracle's double-accumulated CSR SpMM:
    north-star relative L2 error <= 1e-5 and, per row r, max-abs error <=
    1e-4 * ||A_r||_1 * max|B|.  Returns (rel_l2, worst max-abs / bound)."""
    ref = orc.spmm_f64(csr.M, csr.row_ptr, csr.col, csr.val, B, nthreads)
    diff = C.astype(np.float64) - ref
    rel = float(np.linalg.norm(diff) / max(np.linalg.norm(ref), 1e-300))
    row_l1 = np.bincount(np.repeat(np.arange(csr.M), np.diff(csr.row_ptr)),
                         weights=np.abs(csr.val.astype(np.float64)), minlength=csr.M)
    bound = 1e-4 * row_l1 * float(np.abs(B).max() if B.size else 0.0)
    err = np.abs(diff).max(axis=1) if diff.size else np.zeros(csr.M)
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(bound > 0, err / bound, np.where(err > 0, np.inf, 0.0))
    return rel, float(ratio.max() if ratio.size else 0.0)


class Workload:
    """One BASELINE config point's synthetic A (CSR, seed 0), B and C,
    with B and C resident on the device."""

    def __init__(self, vs, st, point, O=None):
        cfg, O0, segw, bundle, tileK, layout, dist = CONFIGS[point]
        self.point, self.O = point, O or O0
        self.segw, self.bundle, self.tileK, self.layout = segw, bundle, tileK, layout
        t0 = time.perf_counter()
        self.csr = vs.coo_to_csr(vs.generate_coo(cfg, 0))
        self.B = vs.gen_dense(cfg, dist, self.csr.N, self.O)
        log(f"bench: {point} matrix {self.csr.M}x{self.csr.N} nnz={self.csr.nnz} O={self.O} "
            f"generated in {time.perf_counter() - t0:.2f}s")
        self.dB = vs.DeviceArray.from_numpy(self.B, st)
        self.dC = vs.DeviceArray((self.csr.M, self.O), np.float32)
        c = self.csr
        self.flop = 2.0 * c.nnz * self.O
        self.bytes_alg = 4.0 * (c.M + 1) + 8.0 * c.nnz + 4.0 * c.N * self.O + 4.0 * c.M * self.O


def make_kernel(vs, st, w, algo, tileK):
    """The SpMM of `algo` on workload w: returns (kernel(timed) callable,
    whether a step needs a C reset, the VCSR format or None, format times)."""
    csr, O = w.csr, w.O
    if algo in ("rocsparse", "aspt", "csr"):
        d_rp = vs.DeviceArray.from_numpy(csr.row_ptr, st)
        d_col = vs.DeviceArray.from_numpy(csr.col, st)
        d_val = vs.DeviceArray.from_numpy(csr.val, st)
        keep = (d_rp, d_col, d_val)
        if algo == "rocsparse":
            # The vendor baseline (rocSPARSE SpMM, C = A*B), set up once.
            plan = vs.VendorPlan(csr.M, csr.N, csr.nnz, d_rp, d_col, d_val, w.dB, O, w.dC, st)

            def kernel(timed=False, _k=keep):
                return plan.run(st, timed=timed)
        elif algo == "aspt":
            # Wave-per-row CSR on the plain CSR arrays (overwrites C).
            def kernel(timed=False, _k=keep):
                return vs.run_csr_wave_spmm_gpu(csr.M, csr.N, d_rp, d_col, d_val, w.dB, O, w.dC,
                                                st, timed=timed)
        else:
            # Zeroes its own rows (src/kernels.cu:25): no reset needed.
            def kernel(timed=False, _k=keep):
                return vs.run_csr_spmm_gpu(csr.M, d_rp, d_col, d_val, w.dB, O, w.dC, st,
                                           timed=timed)
        return kernel, False, None, None
    t0 = time.perf_counter()
    fmt = vs.build_vcsr(csr, w.segw, w.bundle, w.layout)
    if algo == "fast":
        # FastSpMM's layout: fixed 16-row windows of condensed columns.
        fmt.set_tile_rows(16)
        fmt.set_tile_windows(True)
    tb = time.perf_counter() - t0
    t0 = time.perf_counter()
    fmt.upload(st)
    tu = time.perf_counter() - t0
    tr, tt, te = fmt.tile_info()
    log(f"bench: VCSR layout={w.layout} groups={fmt.num_groups} slots={fmt.num_slots} "
        f"build {tb*1e3:.1f} ms upload {tu*1e3:.1f} ms; row-tile view: {tt} tiles of <= {tr} "
        f"rows, {te} entries ({csr.nnz / max(te, 1):.2f} nonzeros per B-row load)")
    kern = {"vcsr": vs.KERNEL_AUTO, "tile": vs.KERNEL_TILE, "row": vs.KERNEL_ROW,
            "segment": vs.KERNEL_SEGMENT, "mfma": vs.KERNEL_MFMA, "fast": vs.KERNEL_TILE}[algo]
    overwrite = kern in (vs.KERNEL_AUTO, vs.KERNEL_TILE, vs.KERNEL_ROW)

    def kernel(timed=False):
        return vs.run_vcsr_spmm_gpu_ex(fmt, w.dB, O, tileK, w.dC, st, timed=timed, kernel=kern,
                                       accumulate=not overwrite)
    times = {"build_ms": round(tb * 1e3, 2), "upload_ms": round(tu * 1e3, 2),
             "groups": fmt.num_groups, "slots": fmt.num_slots}
    return kernel, not overwrite, fmt, times


def time_steps(vs, st, w, kernel, needs_reset, steps, warmup, median=True):
    """W warm-up steps, then K steps between two events on the kernel's
    stream (total_ms); C after them; the per-step median of a second pass
    in 10 groups (if `median`); and the kernel alone (kernel_ms: K launches
    back to back without the reset, which equals total_ms / K when a step
    needs no reset)."""
    lib = vs.load_library()

    def step():
        if needs_reset:
            w.dC.zero(st)
        kernel()

    for _ in range(warmup):
        step()
    st.sync()
    ev0, ev1 = vs.Event(), vs.Event()
    lib.vcsr_device_sync()
    ev0.record(st)
    for _ in range(steps):
        step()
    ev1.record(st)
    total_ms = ev0.elapsed_ms(ev1)
    lib.vcsr_device_sync()
    C = w.dC.numpy(st)
    step_ms = None
    if median:
        # Per-step durations: a second pass of K steps in (up to) 10 groups
        # of g consecutive steps with an event between groups, so that an
        # event record (a few us on this device) is spread over g steps.
        g = max(1, steps // 10)
        ngroups = steps // g
        evs = [vs.Event() for _ in range(ngroups + 1)]
        lib.vcsr_device_sync()
        evs[0].record(st)
        for i in range(ngroups):
            for _ in range(g):
                step()
            evs[i + 1].record(st)
        step_ms = [evs[i].elapsed_ms(evs[i + 1]) / g for i in range(ngroups)]
        lib.vcsr_device_sync()
    if needs_reset:
        # The kernel alone, K launches back to back (C is left accumulating;
        # the timing does not depend on its contents).
        e0, e1 = vs.Event(), vs.Event()
        lib.vcsr_device_sync()
        e0.record(st)
        for _ in range(steps):
            kernel()
        e1.record(st)
        kernel_ms = e0.elapsed_ms(e1) / steps
        lib.vcsr_device_sync()
    else:
        kernel_ms = total_ms / steps
    return total_ms, kernel_ms, step_ms, C


def mfma_report(vs, fmt, algo, w, tileK, kernel_ms):
    """Matrix-core utilisation of the timed kernel, or None when it does
    not run on the matrix cores: issued MFMA FLOPs (dense group tiles or
    16-row tiles, padding included) per kernel time against the dense FP32
    MFMA peak, the useful share of the issued FLOPs, and the useful rate."""
    if fmt is None:
        return None
    tile_mma = algo in ("vcsr", "tile", "fast") and fmt.tile_info()[0] == 16
    if not (algo == "mfma" or tile_mma):
        return None
    ops, fpo = vs.tile_mfma_work(fmt, w.O) if tile_mma else vs.mfma_work(fmt, w.O, tileK)
    issued = float(ops) * fpo
    rate = issued / (kernel_ms * 1e-3) / 1e12
    useful = w.flop / (kernel_ms * 1e-3) / 1e12
    return {"instructions": ops, "issued_gflop": round(issued / 1e9, 4),
            "useful_frac": round(w.flop / issued, 4) if issued else None,
            "tflops_issued": round(rate, 2), "tflops_useful": round(useful, 2),
            "peak_tflops": MFMA_FP32_PEAK_TFS,
            "utilization": round(rate / MFMA_FP32_PEAK_TFS, 4),
            "useful_frac_of_peak": round(useful / MFMA_FP32_PEAK_TFS, 4)}


def extra_point(vs, orc, st, w, algo, steps, warmup, nthreads):
    """One more point of the same run: the kernel of `algo` on workload w,
    timed as the headline is (without the median pass) and checked over
    all of C."""
    cfg_tileK = CONFIGS[w.point][4]
    kernel, needs_reset, fmt, _ = make_kernel(vs, st, w, algo, cfg_tileK)
    total_ms, kernel_ms, _, C = time_steps(vs, st, w, kernel, needs_reset, steps, warmup,
                                           median=False)
    rel, worst = full_check(orc, w.csr, w.B, C, nthreads)
    check = "pass" if rel <= 1e-5 and worst <= 1.0 else "FAIL"
    log(f"bench: extra {w.point} {algo}: {kernel_ms * 1e3:.2f} us per SpMM, check {check} "
        f"(rel L2 {rel:.2e}, max-abs / bound {worst:.3f})")
    achieved = w.bytes_alg / (kernel_ms * 1e-3) / 1e9
    out = {"workload": f"{w.point}: {w.csr.M}x{w.csr.N} nnz={w.csr.nnz} O={w.O}", "algo": algo,
           "steps": steps, "warmup": warmup, "kernel_ms": round(kernel_ms, 5),
           "gflops": round(w.flop / (kernel_ms * 1e-3) / 1e9, 2),
           "hbm_roofline_frac": round(achieved / HBM_PEAK_GBS, 4),
           "check": {"rows": "all", "rel_l2": rel, "maxabs_over_bound": round(worst, 4),
                     "result": check}}
    if fmt is not None and algo in ("vcsr", "tile"):
        li = fmt.launch_info(w.O, vs.KERNEL_AUTO)
        out["timed_kernel"] = ("vcsr_tile_mma_kernel (16-row tiles on FP32 MFMA)"
                               if li["matrix_cores"] else "vcsr_tile_kernel (row-tile view)")
        out["reduce_launches"] = li["reduce_launches"]
    m = mfma_report(vs, fmt, algo, w, cfg_tileK, kernel_ms)
    if m is not None:
        out["mfma"] = m
    return out


def north_star_extras(vs, orc, st, head, w2, steps, warmup, nthreads):
    """The north star's other targets, measured in this run: config 3 at
    O = 128 on the default path (its HBM roofline fraction), the naive CSR
    kernel on configs 2 and 3 at O = 128 with the VCSR / naive speed-up
    (target >= 1.5x), config 5 at O = 512 (FP32 MFMA utilisation); and the
    vendor SpMM (rocSPARSE, the counterpart of the reference's cuSPARSE
    column, src/kernels.cu:169-235) on the headline workload."""
    ex = {}
    naive_steps = max(3, steps // 10)
    ex["cfg2_o128_csr_naive"] = extra_point(vs, orc, st, w2, "csr", naive_steps, 1, nthreads)
    ex["cfg2_o128_rocsparse"] = extra_point(vs, orc, st, w2, "rocsparse", steps, warmup, nthreads)
    w3 = Workload(vs, st, "cfg3")
    ex["cfg3_o128"] = extra_point(vs, orc, st, w3, "vcsr", steps, warmup, nthreads)
    ex["cfg3_o128_csr_naive"] = extra_point(vs, orc, st, w3, "csr", 3, 1, nthreads)
    del w3
    w5 = Workload(vs, st, "cfg5")
    ex["cfg5_o512"] = extra_point(vs, orc, st, w5, "vcsr", steps, warmup, nthreads)
    del w5
    ex["vcsr_over_naive"] = {
        "cfg2_o128": round(ex["cfg2_o128_csr_naive"]["kernel_ms"] / head["kernel_ms"], 2),
        "cfg3_o128": round(ex["cfg3_o128_csr_naive"]["kernel_ms"] / ex["cfg3_o128"]["kernel_ms"],
                           2),
        "target": 1.5}
    ex["vcsr_over_rocsparse"] = {
        "cfg2_o128": round(ex["cfg2_o128_rocsparse"]["kernel_ms"] / head["kernel_ms"], 2)}
    return ex


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="cfg2", choices=sorted(CONFIGS))
    ap.add_argument("--algo", default="vcsr",
                    choices=["vcsr", "tile", "row", "segment", "mfma", "fast", "csr", "aspt",
                             "rocsparse"])
    ap.add_argument("--tileK", type=int, default=None)
    ap.add_argument("--cols", type=int, default=None, metavar="O",
                    help="columns of B and C instead of the config's O")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="wall seconds of each CPU baseline mode (1 thread, all threads)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the extra north-star points the default run measures")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only copy a BYTES buffer device-to-device --steps times (the "
                         "known-size kernel that scales the FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.steps < 1 or args.warmup < 0:
        ap.error("--steps must be at least 1 and --warmup at least 0")
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)

    vs = _load_product()
    vs.load_library()
    if vs.device_count() <= 0:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration > 0:
        st = vs.Stream()
        src = vs.DeviceArray((args.copy_calibration // 4,), np.float32)
        dst = vs.DeviceArray((args.copy_calibration // 4,), np.float32)
        src.zero(st)
        ev0, ev1 = vs.Event(), vs.Event()
        ev0.record(st)
        for _ in range(args.steps):
            dst.copy_from(src, st)
        ev1.record(st)
        ms = ev0.elapsed_ms(ev1) / args.steps
        print(json.dumps({"copy_bytes": src.nbytes, "ms_per_copy": round(ms, 5),
                          "gbs_read_plus_write": round(2 * src.nbytes / ms / 1e6, 1)}))
        return
    from oracle import oracle as orc

    tileK = args.tileK or CONFIGS[args.config][4]
    log(f"bench: {args.config} algo={args.algo} O={args.cols or CONFIGS[args.config][1]} "
        f"tileK={tileK} device={vs.device_name()}")
    st = vs.Stream()
    w = Workload(vs, st, args.config, args.cols)
    csr, B, O = w.csr, w.B, w.O
    kernel, needs_reset, fmt, format_times = make_kernel(vs, st, w, args.algo, tileK)
    total_ms, kernel_ms, step_ms, C = time_steps(vs, st, w, kernel, needs_reset, args.steps,
                                                 args.warmup)

    # Correctness of the last step of the first pass: every element of C
    # against the oracle (double), the north-star bounds.
    nthreads = host_threads()
    rel, worst = full_check(orc, csr, B, C, nthreads)
    check = "pass" if rel <= 1e-5 and worst <= 1.0 else "FAIL"
    log(f"bench: whole-C check vs oracle: rel L2 {rel:.2e}, max-abs / bound {worst:.3f} ({check})")

    config = {"workload": f"{args.config}: {csr.M}x{csr.N} nnz={csr.nnz} O={O}",
              "algo": args.algo, "segw": w.segw, "bundle": w.bundle,
              "layout": ["H", "S", "TC"][w.layout] if fmt is not None else "csr",
              "step": "C reset + SpMM kernel (C += A*B)" if needs_reset
              else "SpMM kernel writing C = A*B"}
    if fmt is not None and args.algo in ("vcsr", "tile", "fast"):
        # The tile-stationary kernel walks the row-tile view (derived from the
        # VCSR slots at upload); segw/bundle shape the format it comes from,
        # tileK is the column tile of the segment-major kernels only.
        li = fmt.launch_info(O, vs.KERNEL_TILE)
        config.update({
            "timed_kernel": ("vcsr_tile_mma_kernel (16-row tiles on FP32 MFMA)"
                             if li["matrix_cores"] else "vcsr_tile_kernel (row-tile view)"),
            "tile_rows": li["tile_rows"], "tiles": li["tiles"], "entries": li["entries"],
            "column_slices": li["column_slices"], "slice_cols": li["slice_cols"],
            "reduce_launches": li["reduce_launches"],
            "tileK": f"{tileK} (not used by the timed kernel)"})
    elif fmt is not None:
        config["tileK"] = tileK
    ms_per_step = total_ms / args.steps
    value = w.flop / (ms_per_step * 1e-3) / 1e9
    achieved = w.bytes_alg / (kernel_ms * 1e-3) / 1e9
    default_o = O == CONFIGS[args.config][1]
    traffic, provenance = measured_traffic(args.config, args.algo) if default_o else (None, None)
    out = {
        "metric": "SpMM GFLOP/s (2*nnz*O/t) + % of HBM roofline, FP32, O=128, 1xMI355X",
        "value": round(value, 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "ms_per_step_median": round(float(np.median(step_ms)), 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": config,
        # Host format build (all host threads) and upload, outside the timed
        # region as in the reference (src/main.cpp:128-149), reported beside it.
        "format": format_times,
        "kernel_ms": round(kernel_ms, 5),
        "kernel_gflops": round(w.flop / (kernel_ms * 1e-3) / 1e9, 2),
        "check": {"rows": "all", "rel_l2": rel, "maxabs_over_bound": round(worst, 4),
                  "result": check},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": provenance,
                     "bytes_alg": w.bytes_alg},
    }
    m = mfma_report(vs, fmt, args.algo, w, tileK, kernel_ms)
    if m is not None:
        # The roofline that binds is then the FP32 MFMA peak (useful FLOPs).
        out["mfma"] = m
        useful = w.flop / (kernel_ms * 1e-3) / 1e12
        out["roofline"] = {"bound": "mfma", "achieved": round(useful, 2),
                           "peak": MFMA_FP32_PEAK_TFS, "unit": "TFLOP/s",
                           "frac": round(useful / MFMA_FP32_PEAK_TFS, 4),
                           "traffic": traffic, "traffic_source": provenance,
                           "bytes_alg": w.bytes_alg}
    if out["roofline"]["bound"] == "hbm":
        # Context for frac: the copy rate is the practical ceiling of any
        # kernel that moves its bytes through HBM once.
        copy = copy_rate_gbs(vs, st)
        out["roofline"]["copy_gbs"] = round(copy, 1)
        out["roofline"]["frac_of_copy"] = round(achieved / copy, 4)
        if fmt is not None and args.algo in ("vcsr", "tile", "fast"):
            # The path that binds the tile kernel: B-row slices from the
            # caches.  A context figure only: a probe that cannot run is
            # reported as such, not allowed to drop the line.
            try:
                sp = slice_path_report(w, fmt.launch_info(O, vs.KERNEL_TILE), kernel_ms)
            except (OSError, RuntimeError) as e:
                sp = {"error": str(e)}
                log(f"bench: slice probe not run: {e}")
            if sp is not None:
                out["roofline"]["b_slice_path"] = sp
    checks = [check]
    if (not args.no_extras and args.config == "cfg2" and args.algo == "vcsr"
            and args.cols is None):
        extra_steps = max(5, min(args.steps, 20))
        out["extra"] = north_star_extras(vs, orc, st, out, w, extra_steps,
                                         min(args.warmup, 3), nthreads)
        checks += [v["check"]["result"] for v in out["extra"].values() if "check" in v]
    if not args.no_cpu_baseline:
        # The oracle's FP32 CSR SpMM (the reference's loop order; the
        # reference has no CPU SpMM of its own) on the same matrix and B:
        # all of this process's host threads (value), and one thread.
        gf, reps, secs, med = cpu_baseline(orc, csr, B, args.cpu_seconds, nthreads)
        gf1, reps1, secs1, med1 = cpu_baseline(orc, csr, B, args.cpu_seconds, 1)
        out["cpu_baseline"] = {
            "value": round(gf, 3), "unit": "GFLOP/s", "cores": nthreads, "kind": "port",
            "sample": f"full {args.config} matrix x B (O={O}), {reps} SpMMs in {secs:.1f}s "
                      f"(median {med * 1e3:.1f} ms), oracle FP32 CSR SpMM, rows split over "
                      f"{nthreads} threads",
            "single_thread": {"value": round(gf1, 3), "cores": 1,
                              "sample": f"{reps1} SpMMs in {secs1:.1f}s (median "
                                        f"{med1 * 1e3:.1f} ms)"},
            "host": host_description()}
    print(json.dumps(out), flush=True)
    if any(c != "pass" for c in checks):
        sys.exit(1)


if __name__ == "__main__":
    main()
