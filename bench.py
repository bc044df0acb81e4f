"""Benchmark driver: SpMM TFLOPS (2*nnz*colB/t) and % of the MI355X HBM
roofline for one synthetic configuration, on one GPU.

A step is one full tiled SpMM C = A*B (the row-block class kernels, each on
its own stream, forked from and joined on the plan's main stream; a plan
with one class launches it on the main stream) with A's tiles, the schedule,
B and C already resident in HBM.  Default workload: configuration 2
(5-point Laplacian 512x512, fp16, colB 128).  Prints ONE JSON line.

  python bench.py [--steps K] [--warmup W] [--config 1..5] [--prec fp16|tf32]
                  [--colB N] [--no-cpu] [--no-vendor] [--cold-reps N] [--gpus 1]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
NAMES = {1: "C1 uniform 4096^2 8/row", 2: "C2 5-pt Laplacian 512x512", 3: "C3 power-law 2^20 mean 16",
         4: "C4 block-sparse 65536^2", 5: "C5 RMAT scale 22"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def alg_bytes(rows, nnz, s_a, k_rows, n, s_b):
    """Compulsory bytes: CSR A (rowptr + colidx + values), the B rows the
    product touches read once, C written once in fp32."""
    return 4 * (rows + 1) + nnz * (4 + s_a) + k_rows * n * s_b + rows * n * 4


def gather_calibration(hip, reps):
    """Random 128/256-byte row gathers from tables of 2 MB .. 2 GB, and
    16-64-byte rows from 1 GB (tsp_gather_kernel): the bandwidth ceiling of
    B-row gathers, and its unit (one request per cache line, whatever the
    row's size)."""
    import ctypes as C
    maxb = 2 << 30
    tab, sink = C.c_void_p(), C.c_void_p()
    assert hip.tsp_malloc(C.byref(tab), maxb) == 0 and hip.tsp_malloc(C.byref(sink), 8192 * 256 * 4) == 0
    hip.tsp_memset(tab, 1, maxb)
    e0, e1 = C.c_void_p(), C.c_void_p()
    hip.tsp_event_create(C.byref(e0))
    hip.tsp_event_create(C.byref(e1))
    iters = 64
    cases = [(rowb, mb) for rowb in (128, 256) for mb in (2, 8, 32, 128, 256, 512, 1024, 2048)]
    cases += [(rowb, 1024) for rowb in (16, 32, 64)]
    for rowb, mb in cases:
        nb = mb << 20
        for w in range(3):
            assert hip.tsp_gather_kernel(tab, nb, rowb, iters, w, sink, None) == 0
        hip.tsp_event_record(e0, None)
        for r in range(reps):
            hip.tsp_gather_kernel(tab, nb, rowb, iters, 100 + r, sink, None)
        hip.tsp_event_record(e1, None)
        hip.tsp_event_sync(e1)
        ms = C.c_float()
        hip.tsp_event_elapsed_ms(C.byref(ms), e0, e1)
        t = ms.value / reps
        nbytes = 8192 * 256 * 16 * iters
        print(json.dumps({"gather_row_bytes": rowb, "table_mb": mb, "ms": round(t, 5),
                          "gbs": round(nbytes / (t * 1e-3) / 1e9, 1),
                          "g_rows_per_s": round(nbytes / rowb / (t * 1e-3) / 1e9, 2)}), flush=True)
    hip.tsp_free(tab)
    hip.tsp_free(sink)


def copy_calibration(hip, nbytes, reps):
    """Plain 16-byte-vector copy of nbytes (dst = src): its FETCH_SIZE /
    WRITE_SIZE per dispatch calibrate the HBM byte counters, its time gives the
    achievable copy bandwidth."""
    import ctypes as C
    nbytes = (nbytes + 15) // 16 * 16
    src, dst = C.c_void_p(), C.c_void_p()
    assert hip.tsp_malloc(C.byref(src), nbytes) == 0 and hip.tsp_malloc(C.byref(dst), nbytes) == 0
    hip.tsp_memset(src, 1, nbytes)
    e0, e1 = C.c_void_p(), C.c_void_p()
    hip.tsp_event_create(C.byref(e0))
    hip.tsp_event_create(C.byref(e1))
    for _ in range(3):
        hip.tsp_copy_kernel(dst, src, nbytes, None)
    hip.tsp_event_record(e0, None)
    for _ in range(reps):
        hip.tsp_copy_kernel(dst, src, nbytes, None)
    hip.tsp_event_record(e1, None)
    hip.tsp_event_sync(e1)
    ms = C.c_float()
    hip.tsp_event_elapsed_ms(C.byref(ms), e0, e1)
    t = ms.value / reps
    print(json.dumps({"copy_bytes": nbytes, "ms": round(t, 5),
                      "gbs_read_plus_write": round(2 * nbytes / (t * 1e-3) / 1e9, 1)}), flush=True)
    hip.tsp_free(src)
    hip.tsp_free(dst)


def cold_steps(hip, plan, reps, stream_bytes, flush_bytes=512 << 20):
    """Median time of one step after a plain copy over 2 x flush_bytes of
    other memory, which evicts L2 (8 x 4 MB) and the 256 MB MALL, so A, B and
    C come from HBM; of the same single step repeated right after it, with
    the caches warm; and of a plain copy moving stream_bytes (half read, half
    written) after the same eviction, the cold streaming rate at that size.
    The headline steps are back to back, as the reference times them: these
    medians separate what caches carry across steps from the fixed cost of
    timing one step alone."""
    import ctypes as C
    half = max(16, stream_bytes // 32 * 16)
    bufs = [C.c_void_p() for _ in range(4)]
    sizes = (flush_bytes, flush_bytes, half, half)
    if any(hip.tsp_malloc(C.byref(b), n) for b, n in zip(bufs, sizes)):
        raise SystemExit("bench.py: cannot allocate the cache-flush buffers")
    src, dst, csrc, cdst = bufs
    hip.tsp_memset(src, 1, flush_bytes)
    hip.tsp_memset(csrc, 1, half)
    e0, e1 = C.c_void_p(), C.c_void_p()
    hip.tsp_event_create(C.byref(e0))
    hip.tsp_event_create(C.byref(e1))

    def flush():
        if hip.tsp_copy_kernel(dst, src, flush_bytes, None) or hip.tsp_device_sync():
            raise SystemExit("bench.py: cache-flush copy failed")

    cold, warm, copy = [], [], []
    try:
        for _ in range(reps):
            flush()
            cold.append(plan.time(1))
            warm.append(plan.time(1))
            flush()
            hip.tsp_event_record(e0, None)
            hip.tsp_copy_kernel(cdst, csrc, half, None)
            hip.tsp_event_record(e1, None)
            hip.tsp_event_sync(e1)
            ms = C.c_float()
            hip.tsp_event_elapsed_ms(C.byref(ms), e0, e1)
            copy.append(ms.value)
    finally:
        for b in bufs:
            hip.tsp_free(b)
        hip.tsp_event_destroy(e0)
        hip.tsp_event_destroy(e1)
    return float(np.median(cold)), float(np.median(warm)), float(np.median(copy)), 2 * half


def default_width(hip, bm, prec, cbp):
    """Output columns one wave covers when the plan keeps the library default."""
    import ctypes as C
    import tilespmm_amd as tsp
    k = tsp.KernelInfo()
    assert hip.tsp_kernel_probe(bm, prec, cbp, C.byref(k)) == 0
    return k.cols_per_task


def sweep(plan, tiles, cbp, args):
    """Time every kernel variant (chunk width W, pipeline stages S, tasks per
    wave) of each active class; one JSON line per class."""
    for t, bm in zip(tiles, (64, 16, 8)):
        if t.tilenum == 0:
            continue
        widths = [w for w in ((32, 64) if bm == 64 else (32, 64, 128)) if cbp % w == 0]
        res = {}
        plan.set_variant(bm)
        res["default"] = plan.time_class(bm, args.class_reps)
        for w in widths:
            for s in (1, 2, 3, 4):
                for tpw in (1, 4):
                    for order in ((1, 2) if cbp > w else (1,)):
                        plan.set_variant(bm, w, s, tpw, order)
                        plan.time_class(bm, 3)
                        res[f"w{w}_s{s}_t{tpw}_o{order}"] = plan.time_class(bm, args.class_reps)
        plan.set_variant(bm)
        best = min(res, key=res.get)
        print(json.dumps({"sweep": args.config, "bm": bm, "tiles": t.tilenum, "best": best,
                          "best_ms": round(res[best], 5), "default_ms": round(res["default"], 5),
                          "ms": {k: round(v, 5) for k, v in res.items()}}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--prec", choices=["fp16", "tf32"], default=None)
    ap.add_argument("--colB", type=int, default=-1)
    ap.add_argument("--gamma", type=float, default=None)
    ap.add_argument("--delta", type=float, default=None)
    ap.add_argument("--no-tune", action="store_true")
    ints3 = lambda s: [int(x) for x in s.split(",")]
    ap.add_argument("--th", type=ints3, default=None, help="pin thresholds TH64,TH16,TH8 (after tuning, if any)")
    ap.add_argument("--format", type=ints3, default=None,
                    help="pin the A format per class 64,16,8 (1 dense, 2 packed, 0 keep)")
    ap.add_argument("--order", type=ints3, default=None,
                    help="pin the chunk order per class 64,16,8 (1 side by side, 2 chunk-major, 0 keep)")
    ap.add_argument("--tpw", type=ints3, default=None,
                    help="pin the tasks per wave per class 64,16,8 (0 keep)")
    ap.add_argument("--width", type=ints3, default=None,
                    help="pin the chunk width per class 64,16,8 (32, 64, 128; 0 keep)")
    ap.add_argument("--stages", type=ints3, default=None,
                    help="pin the pipeline depth per class 64,16,8 (1-4; 0 keep)")
    ap.add_argument("--place", type=ints3, default=None,
                    help="pin the XCD placement per class 64,16,8 (1 contiguous, 2 interleaved, 0 keep)")
    ap.add_argument("--hot-bytes", type=int, default=None,
                    help="pin the hot B row budget in bytes after tuning (0: no hot rows)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-vendor", action="store_true")
    ap.add_argument("--class-reps", type=int, default=200,
                    help="launches per class in the class-alone timing (at least)")
    ap.add_argument("--class-min-ms", type=float, default=20.0,
                    help="lengthen the class-alone timing to span at least this long")
    ap.add_argument("--cold-reps", type=int, default=50,
                    help="single steps timed after evicting L2 and MALL (0 skips)")
    ap.add_argument("--sweep", action="store_true", help="time every kernel variant per class instead")
    ap.add_argument("--gather", action="store_true",
                    help="only run the random row-gather probe (gather bandwidth ceiling)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run the plain copy kernel on this many bytes (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the SpMM is not split across GPUs", file=sys.stderr)
        sys.exit(2)

    import tilespmm_amd as tsp
    hip, host = tsp.load()
    if not tsp.device_available():
        raise SystemExit("bench.py: no gfx950 device")
    if args.gather:
        gather_calibration(hip, min(args.steps, 20))
        return
    if args.copy_bytes:
        copy_calibration(hip, args.copy_bytes, args.steps)
        return

    prec = {"fp16": 0, "tf32": 1, None: -1}[args.prec]
    t0 = time.time()
    A, B, colB, cbp = tsp.gen_config(args.config, prec, args.colB)
    prec = A.prec
    s = 2 if prec == 0 else 4
    log(f"generated {NAMES[args.config]}: {A.rows} rows, nnz {A.nnz}, colB {colB} ({time.time() - t0:.1f}s)")

    t0 = time.time()
    f = tsp.features(A, 9.5, colB)
    g, d = tsp.predict(f, prec)
    if args.gamma is not None:
        g = args.gamma
    if args.delta is not None:
        d = args.delta
    subs = tsp.matrix_split(A, g, d)
    split_ms = (time.time() - t0) * 1e3
    t0 = time.time()
    tiles = [tsp.tile_create(sb, A.cols, bm, prec) for sb, bm in zip(subs, (64, 16, 8))]
    host_tiles_ms = (time.time() - t0) * 1e3
    log(f"split gamma={g} delta={d} ({split_ms:.0f} ms); host tiles: tilenum {[t.tilenum for t in tiles]} "
        f"({host_tiles_ms:.0f} ms)")

    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
    th, model_ms, tune_ms = plan.tune(not args.no_tune)
    if args.th:
        plan.set_th(*args.th)
        th = tuple(args.th)
    for bm, f in zip((64, 16, 8), args.format or ()):
        if f:
            plan.set_format(bm, f)
    for bm, o in zip((64, 16, 8), args.order or ()):
        if o:
            w, st, tpw, _ = plan.get_variant(bm)
            plan.set_variant(bm, w, st, tpw, o)
    for bm, n in zip((64, 16, 8), args.tpw or ()):
        if n:
            w, st, _, o = plan.get_variant(bm)
            plan.set_variant(bm, w, st, n, o)
    for bm, wd in zip((64, 16, 8), args.width or ()):
        if wd:
            _, st, n, o = plan.get_variant(bm)
            plan.set_variant(bm, wd, st, n, o)
    for bm, sg in zip((64, 16, 8), args.stages or ()):
        if sg:
            wd, _, n, o = plan.get_variant(bm)
            plan.set_variant(bm, wd, sg, n, o)
    for bm, pl in zip((64, 16, 8), args.place or ()):
        if pl:
            plan.set_placement(bm, pl - 1)
    if args.hot_bytes is not None:
        plan.set_hot_rows(args.hot_bytes)
    hot_n, hot_b = plan.get_hot_rows()
    log(f"thresholds {th} (model {model_ms:.1f} ms, tuning {tune_ms:.1f} ms), hot B rows {hot_n} ({hot_b} bytes)")

    if args.sweep:
        sweep(plan, tiles, cbp, args)
        plan.close()
        return

    # warmup, then K timed steps bracketed by device syncs and main-stream events
    plan.warmup(args.warmup)
    plan.run(zero_c=True)
    hip.tsp_device_sync()
    ms = plan.time(args.steps)
    hip.tsp_device_sync()
    tflops = 2.0 * A.nnz * colB / (ms * 1e-3) / 1e12
    # per-class kernel time (each class alone on its own stream)
    cls = {}
    for t, sb, bm in zip(tiles, subs, (64, 16, 8)):
        if t.tilenum == 0:
            continue
        # one untimed round first (the clock drops while the device idles),
        # then enough launches to span at least --class-min-ms
        warm = plan.time_class(bm, args.class_reps)
        reps = int(min(20000, max(args.class_reps, args.class_min_ms / max(warm, 1e-4))))
        cms = plan.time_class(bm, reps)
        k_rows = int(np.unique(t.arrays()["tile_colidx"]).size)
        b = alg_bytes(sb.rows, sb.nnz, s, k_rows, colB, s)
        cls[bm] = {"ms": cms, "reps": reps, "rows": sb.rows, "nnz": int(sb.nnz), "tiles": t.tilenum,
                   "format": {1: "dense", 2: "packed"}.get(plan.get_format(bm), "?"),
                   "order": {0: "side-by-side", 1: "side-by-side", 2: "chunk-major"}[plan.get_variant(bm)[3]],
                   "tasks_per_wave": max(1, plan.get_variant(bm)[2]),
                   "stages": max(1, plan.get_variant(bm)[1]),
                   "chunk_width": plan.get_variant(bm)[0] or default_width(hip, bm, prec, cbp),
                   "placement": {0: "contiguous", 1: "interleaved"}.get(plan.get_placement(bm), "?"),
                   "alg_bytes": b, "gbs": b / (cms * 1e-3) / 1e9}
    dom = max(cls, key=lambda k: cls[k]["ms"])
    k_all = int(np.unique(A.colidx).size)
    step_bytes = alg_bytes(A.rows, A.nnz, s, k_all, colB, s)
    step_gbs = step_bytes / (ms * 1e-3) / 1e9

    # the dominant kernel's instantiation spmm_kernel<BM, W, PREC, S, PK>; the
    # profiled HBM traffic applies only to the same instantiation
    dk = cls[dom]
    kname = (f"spmm_kernel<{dom}, {dk['chunk_width']}, {prec}, {dk['stages']}, "
             f"{'true' if dk['format'] == 'packed' else 'false'}>")
    traffic, traffic_note = None, "no profile of this workload in profiles/"
    prof = os.path.join(ROOT, "profiles", f"traffic_config{args.config}_{'fp16' if prec == 0 else 'tf32'}_{colB}.json")
    if os.path.exists(prof):
        with open(prof) as fh:
            tp = json.load(fh).get(f"bm{dom}", {})
        if tp.get("kernel", "").endswith(kname):
            traffic, traffic_note = tp.get("hbm_bytes_per_launch"), os.path.relpath(prof, ROOT)
        else:
            traffic_note = f"{os.path.relpath(prof, ROOT)} profiles {tp.get('kernel', '?')}, not the tuned {kname}"

    roof = {"bound": "hbm", "achieved": round(cls[dom]["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(cls[dom]["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
            "traffic_source": traffic_note, "kernel": kname, "kernel_ms": round(cls[dom]["ms"], 5),
            "alg_bytes_per_launch": cls[dom]["alg_bytes"],
            "step_achieved": round(step_gbs, 2), "step_frac": round(step_gbs / HBM_PEAK_GBS, 4),
            "step_alg_bytes": step_bytes}

    # the same tiles built on the GPU (upload of the class sub-CSRs + device
    # conversion), the alternative to the host conversion timed above
    dplan = tsp.Plan.from_csr(subs, A.rows, A.cols, cbp, prec, B)
    dev_tiles_ms = dplan.tile_ms
    dplan.close()

    # after every other device measurement: the eviction copies must not
    # disturb the class timings above
    cold = None
    if args.cold_reps > 0:
        sb = step_bytes
        cms, wms, cpms, cpb = cold_steps(hip, plan, args.cold_reps, sb)
        cold = {"ms_per_step": round(cms, 6), "tflops": round(2.0 * A.nnz * colB / (cms * 1e-3) / 1e12, 4),
                "alg_gbs": round(sb / (cms * 1e-3) / 1e9, 1), "warm_single_ms": round(wms, 6),
                "copy_cold_ms": round(cpms, 6), "copy_cold_gbs": round(cpb / (cpms * 1e-3) / 1e9, 1),
                "reps": args.cold_reps,
                "protocol": "median of single steps, each after a 1 GB copy that evicts L2 and the 256 MB MALL; "
                            "warm_single_ms: the same single step again right after; copy_cold: a plain copy "
                            "moving the step's algorithmic bytes after the same eviction"}

    vendor = None
    if not args.no_vendor:
        import ctypes as C
        vp, vm = C.c_double(), C.c_double()
        Cv = np.zeros((A.rows, colB), dtype=np.float32)
        st = hip.tsp_vendor_spmm(prec, A.rows, A.cols, A.nnz, A.rowptr.ctypes.data_as(C.c_void_p),
                                 A.colidx.ctypes.data_as(C.c_void_p), A.val.ctypes.data_as(C.c_void_p), colB, cbp,
                                 np.ascontiguousarray(B).ctypes.data_as(C.c_void_p),
                                 Cv.ctypes.data_as(C.c_void_p), 20, 200, C.byref(vp), C.byref(vm))
        if st == 0:
            vendor = {"lib": "rocSPARSE spmm (CSR, alg default)", "ms": round(vm.value, 5),
                      "tflops": round(2.0 * A.nnz * colB / (vm.value * 1e-3) / 1e12, 4)}
        else:
            vendor = {"lib": "rocSPARSE", "status": st}
        del Cv

    cpu = None
    if not args.no_cpu:
        import oracle
        a32 = oracle.values_f64(A.val, prec).astype(np.float32)
        b32 = oracle.values_f64(B[:, :colB].reshape(-1), prec).astype(np.float32).reshape(A.cols, colB)
        # bounded sample: the first rows holding ~min(nnz, 4M) entries
        lim = min(A.nnz, 4_000_000)
        r_end = int(np.searchsorted(A.rowptr, lim, side="right")) - 1
        r_end = max(1, min(A.rows, r_end))
        nz = int(A.rowptr[r_end])
        out = np.zeros((r_end, colB), dtype=np.float32)
        oracle.spmm_f32_omp(r_end, A.rowptr[:r_end + 1], A.colidx, a32, b32, colB, out)   # warmup
        times = []
        used = 1
        for _ in range(5):
            t1 = time.perf_counter()
            _, used = oracle.spmm_f32_omp(r_end, A.rowptr[:r_end + 1], A.colidx, a32, b32, colB, out)
            times.append(time.perf_counter() - t1)
        tm = float(np.median(times))
        nproc = len(os.sched_getaffinity(0))
        cpu = {"value": round(2.0 * nz * colB / tm / 1e12, 5), "unit": "TFLOPS", "cores": int(used), "kind": "port",
               "sample": f"rows 0..{r_end} ({nz} of {A.nnz} nnz), colB {colB}, fp32 accumulate, "
                         f"OpenMP dynamic(64) on {used} threads ({nproc} cpus usable, "
                         f"OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS', 'unset')}), "
                         f"median of 5 after 1 warmup, {tm * 1e3:.2f} ms"}

    line = {
        "metric": "SpMM TFLOPS (2*nnz*colB/t) + % HBM roofline",
        "value": round(tflops, 4), "unit": "TFLOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp16" if prec == 0 else "tf32", "data": "synthetic",
        "config": {"workload": f"{NAMES[args.config]}, {'fp16' if prec == 0 else 'tf32'}, colB {colB}",
                   "config_id": args.config, "rows": A.rows, "nnz": A.nnz, "colB": colB, "colB_padded": cbp,
                   "gamma": g, "delta": d, "th": list(th), "tilenum": [t.tilenum for t in tiles],
                   "hot_rows": hot_n, "hot_bytes": hot_b,
                   "parallelism": "single GPU"},
        "roofline": roof,
        "classes": {f"bm{k}": {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in cls.items()},
        "cold_cache": cold,
        "vendor": vendor,
        "cpu_baseline": cpu,
        "pre_ms": {"split": round(split_ms, 1), "tiles_host": round(host_tiles_ms, 1),
                   "tiles_device": round(dev_tiles_ms, 1), "model": round(model_ms, 2), "tune": round(tune_ms, 1)},
    }
    plan.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
