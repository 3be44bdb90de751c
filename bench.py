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
reset inside the step.  --cols replaces a config's O (column sweeps).  K steps are timed between HIP events after W
warm-up steps; `value` is 2*nnz*O*K / that time.  `kernel_ms` is the kernel
alone, K back-to-back launches between events on its stream (the reference
times kernels only, src/kernels.cu:153-162); the roofline uses it.
`ms_per_step_median` is the median per-step time of a second pass of K
steps timed in 10 groups of K/10.  The default kernel's launch shape (tile
height, column slices, reduce launches) is named in `config`.

Prints ONE JSON line.  Multi-GPU runs are not part of this build.
"""
from __future__ import annotations

import argparse
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


def measured_traffic(config, algo):
    """HBM-side bytes per SpMM of the dominant kernel, from the committed
    rocprofv3 counter summary (profiles/traffic.json): FETCH_SIZE and
    WRITE_SIZE per dispatch, each divided by what the same counter reads per
    byte for a device-to-device copy of known size, times the kernel's
    dispatches per SpMM (column slices).  None if absent."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        e = t["kernels"][f"{config}/{algo}"]
        return e.get("launches", 1) * (e["fetch_kib"] * 1024.0 / t["copy_fetch_factor"] +
                                       e["write_kib"] * 1024.0 / t["copy_write_factor"])
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None


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

    cfg, O, segw, bundle, tileK, layout, dist = CONFIGS[args.config]
    if args.tileK:
        tileK = args.tileK
    if args.cols:
        O = args.cols
    log(f"bench: {args.config} algo={args.algo} O={O} segw={segw} bundle={bundle} "
        f"tileK={tileK} device={vs.device_name()}")
    t0 = time.perf_counter()
    csr = vs.coo_to_csr(vs.generate_coo(cfg, 0))
    B = vs.gen_dense(cfg, dist, csr.N, O)
    log(f"bench: matrix {csr.M}x{csr.N} nnz={csr.nnz} generated in {time.perf_counter()-t0:.2f}s")
    st = vs.Stream()
    dB = vs.DeviceArray.from_numpy(B, st)
    dC = vs.DeviceArray((csr.M, O), np.float32)
    fmt = None
    # Kernels that write every C element themselves need no reset per step;
    # the accumulate-into-C kernels get a C reset inside the timed step.
    needs_reset = True
    if args.algo == "rocsparse":
        # The vendor baseline (rocSPARSE SpMM, C = A*B), set up once.
        d_rp = vs.DeviceArray.from_numpy(csr.row_ptr, st)
        d_col = vs.DeviceArray.from_numpy(csr.col, st)
        d_val = vs.DeviceArray.from_numpy(csr.val, st)
        plan = vs.VendorPlan(csr.M, csr.N, csr.nnz, d_rp, d_col, d_val, dB, O, dC, st)
        needs_reset = False

        def kernel(timed=False):
            return plan.run(st, timed=timed)
    elif args.algo == "aspt":
        # Wave-per-row CSR on the plain CSR arrays (overwrites C).
        d_rp = vs.DeviceArray.from_numpy(csr.row_ptr, st)
        d_col = vs.DeviceArray.from_numpy(csr.col, st)
        d_val = vs.DeviceArray.from_numpy(csr.val, st)
        needs_reset = False

        def kernel(timed=False):
            return vs.run_csr_wave_spmm_gpu(csr.M, csr.N, d_rp, d_col, d_val, dB, O, dC, st,
                                            timed=timed)
    elif args.algo == "csr":
        d_rp = vs.DeviceArray.from_numpy(csr.row_ptr, st)
        d_col = vs.DeviceArray.from_numpy(csr.col, st)
        d_val = vs.DeviceArray.from_numpy(csr.val, st)
        needs_reset = False  # zeroes its own rows (src/kernels.cu:25)

        def kernel(timed=False):
            return vs.run_csr_spmm_gpu(csr.M, d_rp, d_col, d_val, dB, O, dC, st, timed=timed)
    else:
        t0 = time.perf_counter()
        fmt = vs.build_vcsr(csr, segw, bundle, layout)
        if args.algo == "fast":
            # FastSpMM's layout: fixed 16-row windows of condensed columns.
            fmt.set_tile_rows(16)
            fmt.set_tile_windows(True)
        tb = time.perf_counter() - t0
        t0 = time.perf_counter()
        fmt.upload(st)
        tu = time.perf_counter() - t0
        log(f"bench: VCSR layout={layout} groups={fmt.num_groups} slots={fmt.num_slots} "
            f"build {tb*1e3:.1f} ms upload {tu*1e3:.1f} ms")
        tr, tt, te = fmt.tile_info()
        log(f"bench: row-tile view: {tt} tiles of <= {tr} rows, {te} entries "
            f"({csr.nnz / max(te, 1):.2f} nonzeros per B-row load)")
        kern = {"vcsr": vs.KERNEL_AUTO, "tile": vs.KERNEL_TILE, "row": vs.KERNEL_ROW,
                "segment": vs.KERNEL_SEGMENT, "mfma": vs.KERNEL_MFMA,
                "fast": vs.KERNEL_TILE}[args.algo]
        overwrite = kern in (vs.KERNEL_AUTO, vs.KERNEL_TILE, vs.KERNEL_ROW)
        needs_reset = not overwrite

        def kernel(timed=False):
            return vs.run_vcsr_spmm_gpu_ex(fmt, dB, O, tileK, dC, st, timed=timed, kernel=kern,
                                           accumulate=not overwrite)

    def step():
        if needs_reset:
            dC.zero(st)
        kernel()

    for _ in range(args.warmup):
        step()
    st.sync()
    ev0, ev1 = vs.Event(), vs.Event()
    lib = vs.load_library()
    lib.vcsr_device_sync()
    ev0.record(st)
    for _ in range(args.steps):
        step()
    ev1.record(st)
    total_ms = ev0.elapsed_ms(ev1)
    lib.vcsr_device_sync()
    C = dC.numpy(st)

    # Per-step durations for the median: a second pass of K steps in (up to)
    # 10 groups of g consecutive steps with an event between groups, so that
    # an event record (a few us on this device) is spread over g steps; the
    # median is taken over the groups' per-step times (the headline uses
    # the first pass).
    g = max(1, args.steps // 10)
    ngroups = args.steps // g
    evs = [vs.Event() for _ in range(ngroups + 1)]
    lib.vcsr_device_sync()
    evs[0].record(st)
    for i in range(ngroups):
        for _ in range(g):
            step()
        evs[i + 1].record(st)
    step_ms = [evs[i].elapsed_ms(evs[i + 1]) / g for i in range(ngroups)]
    lib.vcsr_device_sync()

    # Correctness of the last step of the first pass: every element of C
    # against the oracle (double), the north-star bounds.
    nthreads = host_threads()
    rel, worst = full_check(orc, csr, B, C, nthreads)
    check = "pass" if rel <= 1e-5 and worst <= 1.0 else "FAIL"
    log(f"bench: whole-C check vs oracle: rel L2 {rel:.2e}, max-abs / bound {worst:.3f} ({check})")

    # Kernel-only duration: the kernel alone, K launches back to back between
    # two events on the stream it runs on (C is left accumulating; the
    # timing does not depend on its contents).  Without a reset in the step
    # this equals ms_per_step.
    if needs_reset:
        e0, e1 = vs.Event(), vs.Event()
        lib.vcsr_device_sync()
        e0.record(st)
        for _ in range(args.steps):
            kernel()
        e1.record(st)
        kernel_ms = e0.elapsed_ms(e1) / args.steps
        lib.vcsr_device_sync()
    else:
        kernel_ms = total_ms / args.steps

    config = {"workload": f"{args.config}: {csr.M}x{csr.N} nnz={csr.nnz} O={O}",
              "algo": args.algo, "segw": segw, "bundle": bundle,
              "layout": ["H", "S", "TC"][layout] if fmt is not None else "csr",
              "step": "C reset + SpMM kernel (C += A*B)" if needs_reset
              else "SpMM kernel writing C = A*B"}
    if fmt is not None and kern in (vs.KERNEL_AUTO, vs.KERNEL_TILE):
        # The tile-stationary kernel walks the row-tile view (derived from the
        # VCSR slots at upload); segw/bundle shape the format it comes from,
        # tileK is the column tile of the segment-major kernels only.
        li = fmt.launch_info(O, kern)
        config.update({
            "timed_kernel": ("vcsr_tile_mma_kernel (16-row tiles on FP32 MFMA)"
                             if li["matrix_cores"] else "vcsr_tile_kernel (row-tile view)"),
            "tile_rows": li["tile_rows"], "tiles": li["tiles"], "entries": li["entries"],
            "column_slices": li["column_slices"], "slice_cols": li["slice_cols"],
            "reduce_launches": li["reduce_launches"],
            "tileK": f"{tileK} (not used by the timed kernel)"})
    elif fmt is not None:
        config["tileK"] = tileK
    # Host format build (all host threads) and upload, outside the timed
    # region as in the reference (src/main.cpp:128-149), reported beside it.
    format_times = ({"build_ms": round(tb * 1e3, 2), "upload_ms": round(tu * 1e3, 2),
                     "groups": fmt.num_groups, "slots": fmt.num_slots}
                    if fmt is not None else None)
    flop = 2.0 * csr.nnz * O
    ms_per_step = total_ms / args.steps
    value = flop / (ms_per_step * 1e-3) / 1e9
    bytes_alg = 4.0 * (csr.M + 1) + 8.0 * csr.nnz + 4.0 * csr.N * O + 4.0 * csr.M * O
    achieved = bytes_alg / (kernel_ms * 1e-3) / 1e9
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
        "format": format_times,
        "kernel_ms": round(kernel_ms, 5),
        "kernel_gflops": round(flop / (kernel_ms * 1e-3) / 1e9, 2),
        "check": {"rows": "all", "rel_l2": rel, "maxabs_over_bound": round(worst, 4),
                  "result": check},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (measured_traffic(args.config, args.algo)
                                 if O == CONFIGS[args.config][1] else None),
                     "bytes_alg": bytes_alg},
    }
    # The tile-stationary kernel runs 16-row tiles on the matrix cores.
    tile_mma = args.algo in ("vcsr", "tile", "fast") and tr == 16
    if args.algo == "mfma" or tile_mma:
        # Matrix-core utilisation: issued MFMA FLOPs (dense group tiles or
        # 16-row tiles, padding included) per kernel time against the dense
        # FP32 MFMA peak, and the useful share of the issued FLOPs.  The
        # roofline that binds is then the FP32 MFMA peak (useful FLOPs).
        ops, fpo = vs.tile_mfma_work(fmt, O) if tile_mma else vs.mfma_work(fmt, O, tileK)
        issued = float(ops) * fpo
        rate = issued / (kernel_ms * 1e-3) / 1e12
        out["mfma"] = {"instructions": ops, "issued_gflop": round(issued / 1e9, 4),
                       "useful_frac": round(flop / issued, 4) if issued else None,
                       "tflops_issued": round(rate, 2), "peak_tflops": MFMA_FP32_PEAK_TFS,
                       "utilization": round(rate / MFMA_FP32_PEAK_TFS, 4)}
        useful = flop / (kernel_ms * 1e-3) / 1e12
        out["roofline"] = {"bound": "mfma", "achieved": round(useful, 2),
                           "peak": MFMA_FP32_PEAK_TFS, "unit": "TFLOP/s",
                           "frac": round(useful / MFMA_FP32_PEAK_TFS, 4),
                           "traffic": out["roofline"]["traffic"], "bytes_alg": bytes_alg}
    if out["roofline"]["bound"] == "hbm":
        # Context for frac: the copy rate is the practical ceiling of any
        # kernel that moves its bytes through HBM once.
        copy = copy_rate_gbs(vs, st)
        out["roofline"]["copy_gbs"] = round(copy, 1)
        out["roofline"]["frac_of_copy"] = round(achieved / copy, 4)
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
    if check != "pass":
        sys.exit(1)


if __name__ == "__main__":
    main()
