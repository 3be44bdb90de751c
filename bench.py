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


def cpu_baseline(orc, csr, B, seconds):
    """The oracle's single-thread FP32 CSR SpMM (reference loop order) on the
    same matrix and B, repeated until `seconds` of CPU work."""
    flop = 2.0 * csr.nnz * B.shape[1]
    reps, t_total = 0, 0.0
    while t_total < seconds and reps < 1000:
        t0 = time.perf_counter()
        orc.spmm_f32(csr.M, csr.row_ptr, csr.col, csr.val, B)
        t_total += time.perf_counter() - t0
        reps += 1
    return flop * reps / t_total / 1e9, reps, t_total


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
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only copy a BYTES buffer device-to-device --steps times (the "
                         "known-size kernel that scales the FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
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
        log(f"bench: VCSR layout={layout} groups={fmt.num_groups} slots={fmt.num_slots} "
            f"build {tb*1e3:.1f} ms upload {(time.perf_counter()-t0)*1e3:.1f} ms")
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

    # Correctness of the last step: sampled rows against the oracle (double).
    rng = np.random.default_rng(0)
    rows = np.unique(rng.choice(csr.M, size=min(512, csr.M), replace=False))
    rp = np.concatenate([[0], np.cumsum(np.diff(csr.row_ptr)[rows])]).astype(np.int32)
    cols = np.concatenate([csr.col[csr.row_ptr[r]:csr.row_ptr[r + 1]] for r in rows])
    vals = np.concatenate([csr.val[csr.row_ptr[r]:csr.row_ptr[r + 1]] for r in rows])
    ref = orc.spmm_f64(len(rows), rp, cols.astype(np.int32), vals.astype(np.float32), B)
    rel = float(np.linalg.norm(C[rows] - ref) / max(np.linalg.norm(ref), 1e-300))
    check = "pass" if rel <= 1e-5 else "FAIL"
    log(f"bench: sampled-row rel L2 vs oracle {rel:.2e} ({check})")

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
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{args.config}: {csr.M}x{csr.N} nnz={csr.nnz} O={O}",
                   "algo": args.algo, "segw": segw, "bundle": bundle, "tileK": tileK,
                   "layout": ["H", "S", "TC"][layout] if args.algo not in ("csr", "aspt", "rocsparse")
                   else "csr",
                   "step": "C reset + SpMM kernel (C += A*B)" if needs_reset
                   else "SpMM kernel writing C = A*B"},
        "kernel_ms": round(kernel_ms, 5),
        "kernel_gflops": round(flop / (kernel_ms * 1e-3) / 1e9, 2),
        "check": {"rel_l2_sampled_rows": rel, "result": check},
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
    if not args.no_cpu_baseline:
        gf, reps, secs = cpu_baseline(orc, csr, B, args.cpu_seconds)
        out["cpu_baseline"] = {"value": round(gf, 3), "unit": "GFLOP/s", "cores": 1,
                               "kind": "port",
                               "sample": f"full {args.config} matrix x B (O={O}), {reps} reps, "
                                         f"{secs:.1f}s, oracle FP32 CSR SpMM single thread"}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
