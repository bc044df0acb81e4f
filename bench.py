"""Benchmark driver: SpMM TFLOPS (2*nnz*colB/t) and % of the MI355X HBM
roofline for one synthetic configuration, on one GPU.

A step is one full tiled SpMM C = A*B (the row-block class kernels, each on
its own stream, forked from and joined on the plan's main stream; a plan
with one class launches it on the main stream) with A's tiles, the schedule,
B and C already resident in HBM.  Default workload: configuration 5 as
stated (RMAT scale 22, tf32, colB 64), the largest single-GPU configuration;
the fp16 / colB 128 targets on the configuration 3 and 5 structures (T3, T5)
are timed in the same run and reported under "targets".  Prints ONE JSON
line.

  python bench.py [--steps K] [--warmup W] [--config 1..5] [--prec fp16|tf32]
                  [--colB N] [--targets 3,5] [--no-cpu] [--no-vendor]
                  [--cold-reps N] [--gpus 1]

Experiments (other JSON lines): --gather (gather bandwidth by row size and
table size), --copy-bytes N (copy calibration), --hub-split H (the hub-row
experiment), --gather-stream (the gathers of the workload's own B-row index
stream alone, against its tuned step), --sweep (variant sweep).
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
    """Compulsory bytes: CSR A (rowptr + colidx + values), k_rows rows of B
    read once, C written once in fp32.  The roofline figure takes k_rows = K,
    all of B's rows (4(M+1) + nnz(4+s_A) + K*N*s_B + M*N*4); with k_rows =
    the distinct columns of A it is the touched-row figure reported beside
    it."""
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


def copy_calibration(hip, nbytes, reps, quiet=False):
    """Plain 16-byte-vector copy of nbytes (dst = src): its FETCH_SIZE /
    WRITE_SIZE per dispatch calibrate the HBM byte counters, its time gives the
    achievable copy bandwidth (returned in GB/s, read plus write)."""
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
    gbs = 2 * nbytes / (t * 1e-3) / 1e9
    if not quiet:
        print(json.dumps({"copy_bytes": nbytes, "ms": round(t, 5), "gbs_read_plus_write": round(gbs, 1)}), flush=True)
    hip.tsp_event_destroy(e0)
    hip.tsp_event_destroy(e1)
    hip.tsp_free(src)
    hip.tsp_free(dst)
    return gbs


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


def sweep(plan, tilenum, cbp, args):
    """Time every kernel variant (chunk width W, pipeline stages S, tasks per
    wave) of each active class; one JSON line per class."""
    for tn, bm in zip(tilenum, (64, 16, 8)):
        if tn == 0:
            continue
        widths = [w for w in ((32, 64) if bm == 64 else (32, 64, 128)) if cbp % w == 0]
        res = {}
        plan.set_variant(bm)
        res["default"] = plan.time_class(bm, args.class_reps)
        for w in widths:
            for s in (1, 2, 3):
                for tpw in (1, 4):
                    for order in ((1, 2) if cbp > w else (1,)):
                        plan.set_variant(bm, w, s, tpw, order)
                        plan.time_class(bm, 3)
                        res[f"w{w}_s{s}_t{tpw}_o{order}"] = plan.time_class(bm, args.class_reps)
        plan.set_variant(bm)
        best = min(res, key=res.get)
        print(json.dumps({"sweep": args.config, "bm": bm, "tiles": tn, "best": best,
                          "best_ms": round(res[best], 5), "default_ms": round(res["default"], 5),
                          "ms": {k: round(v, 5) for k, v in res.items()}}), flush=True)


def gather_ceiling(hip, reps=5):
    """Uniform random 128-byte row gathers from a 1 GB table: the line-request
    rate (G lines/s) that the B-row gathers of a uniform-column matrix can
    reach, measured in the same process as the headline."""
    import ctypes as C
    nb = 1 << 30
    tab, sink = C.c_void_p(), C.c_void_p()
    if hip.tsp_malloc(C.byref(tab), nb) or hip.tsp_malloc(C.byref(sink), 8192 * 256 * 4):
        raise SystemExit("bench.py: cannot allocate the gather probe")
    try:
        hip.tsp_memset(tab, 1, nb)
        e0, e1 = C.c_void_p(), C.c_void_p()
        hip.tsp_event_create(C.byref(e0))
        hip.tsp_event_create(C.byref(e1))
        iters = 64
        for w in range(2):
            hip.tsp_gather_kernel(tab, nb, 128, iters, w, sink, None)
        hip.tsp_event_record(e0, None)
        for r in range(reps):
            hip.tsp_gather_kernel(tab, nb, 128, iters, 10 + r, sink, None)
        hip.tsp_event_record(e1, None)
        hip.tsp_event_sync(e1)
        ms = C.c_float()
        hip.tsp_event_elapsed_ms(C.byref(ms), e0, e1)
        hip.tsp_event_destroy(e0)
        hip.tsp_event_destroy(e1)
    finally:
        hip.tsp_free(tab)
        hip.tsp_free(sink)
    lines = 8192 * 256 * 16 * iters / 128
    return lines / (ms.value / reps * 1e-3) / 1e9


def apply_pins(plan, args):
    """--th / --format / --order / --tpw / --width / --stages / --place /
    --hot-bytes pin what the tuning chose (profiling runs replay a tuned
    configuration with --no-tune)."""
    th = None
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
    for bm, li in zip((64, 16, 8), args.lane_idx or ()):
        if li:
            plan.set_lane_indices(bm, li - 1)
    for bm, pr in zip((64, 16, 8), args.pairs or ()):
        if pr:
            plan.set_pairs(bm, pr - 1)
    for bm, b3 in zip((64, 16, 8), args.b3 or ()):
        if b3:
            plan.set_b_3byte(bm, b3 - 1)
    lags = args.panel_lag or (2, 2, 2)
    for bm, pr, lg in zip((64, 16, 8), args.panels or (), lags):
        if pr:
            plan.set_panels(bm, pr, lg)
    if args.hot_bytes is not None:
        plan.set_hot_rows(args.hot_bytes)
    return th


def variant_of(c):
    """The runtime choices of one class beyond its kernel instantiation, as a
    traffic profile records them."""
    return {"order": c["order"], "placement": c["placement"], "tasks_per_wave": c["tasks_per_wave"],
            "panel_rows": c["panel_rows"], "panel_lag": c["panel_lag"] if c["panel_rows"] else 0}


def pins_of(plan, th, cls):
    """The bench flags that replay this plan's tuned configuration."""
    f, o, t, w, s, p, li, pr, lg, tp, b3 = [], [], [], [], [], [], [], [], [], [], []
    for bm in (64, 16, 8):
        c = cls.get(bm)
        f.append({"dense": 1, "packed": 2}[c["format"]] if c else 0)
        o.append({"side-by-side": 1, "chunk-major": 2}[c["order"]] if c else 0)
        t.append(c["tasks_per_wave"] if c else 0)
        w.append(c["chunk_width"] if c else 0)
        s.append(c["stages"] if c else 0)
        p.append({"contiguous": 1, "interleaved": 2, "chunk-xcd": 3}[c["placement"]] if c else 0)
        li.append(c["lane_indices"] + 1 if c else 0)
        pr.append(c["panel_rows"] if c else 0)
        lg.append(c["panel_lag"] if c else 0)
        tp.append(c["tile_pairs"] + 1 if c else 0)
        b3.append(c["b_3byte"] + 1 if c else 0)
    j = lambda v: ",".join(str(x) for x in v)
    return (f"--no-tune --th {j(th)} --format {j(f)} --order {j(o)} --tpw {j(t)} --width {j(w)} "
            f"--stages {j(s)} --place {j(p)} --lane-idx {j(li)} --pairs {j(tp)} --b3 {j(b3)} --panels {j(pr)} "
            f"--panel-lag {j(lg)} --hot-bytes {plan.get_hot_rows()[1]}")


def measure(tsp, hip, config, prec, colB, args, headline):
    """Build, tune and time one workload.  headline=True also runs the host
    tiling, the device tiling comparison, the cold-cache leg and rocSPARSE;
    returns (record, A, subs, plan) with the plan still open."""
    t0 = time.time()
    A, B, colB, cbp = tsp.gen_config(config, prec, colB)
    prec = A.prec
    s = 2 if prec == 0 else 4
    pname = "fp16" if prec == 0 else "tf32"
    log(f"generated {NAMES[config]}: {A.rows} rows, nnz {A.nnz}, {pname}, colB {colB} ({time.time() - t0:.1f}s)")

    t0 = time.time()
    f = tsp.features(A, 9.5, colB)
    g, d = tsp.predict(f, prec)
    if args.gamma is not None:
        g = args.gamma
    if args.delta is not None:
        d = args.delta
    subs = tsp.matrix_split(A, g, d)
    split_ms = (time.time() - t0) * 1e3
    pre = {"split": round(split_ms, 1)}
    if headline:
        t0 = time.time()
        tiles = [tsp.tile_create(sb, A.cols, bm, prec) for sb, bm in zip(subs, (64, 16, 8))]
        pre["tiles_host"] = round((time.time() - t0) * 1e3, 1)
        tilenum = [t.tilenum for t in tiles]
        kcols = {bm: int(np.unique(t.arrays()["tile_colidx"]).size) for t, bm in zip(tiles, (64, 16, 8))
                 if t.tilenum}
        plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
        del tiles
        # the same tiles built on the GPU (upload of the class sub-CSRs +
        # device conversion), the alternative to the host conversion above
        dplan = tsp.Plan.from_csr(subs, A.rows, A.cols, cbp, prec, B)
        pre["tiles_device"] = round(dplan.tile_ms, 1)
        dplan.close()
    else:
        plan = tsp.Plan.from_csr(subs, A.rows, A.cols, cbp, prec, B)
        pre["tiles_device"] = round(plan.tile_ms, 1)
        tilenum = [plan.tilenum(bm) for bm in (64, 16, 8)]
        kcols = {bm: int(np.unique(sb.colidx).size) for sb, bm in zip(subs, (64, 16, 8)) if sb.nnz}
    if not headline:
        del B
    log(f"split gamma={g} delta={d} ({split_ms:.0f} ms); tilenum {tilenum}")

    if args.tune_cold:
        plan.set_tune_mode(True)
    th, model_ms, tune_ms = plan.tune(not args.no_tune)
    th = apply_pins(plan, args) or th
    hot_n, hot_b = plan.get_hot_rows()
    pre.update({"model": round(model_ms, 2), "tune": round(tune_ms, 1)})
    log(f"thresholds {th} (model {model_ms:.1f} ms, tuning {tune_ms:.1f} ms), hot B rows {hot_n} ({hot_b} bytes)")

    # W untimed warm-up steps, a clock-stable warm-up (batches until the GFX
    # clock settles, at most 1000 steps), then exactly K timed steps between
    # device syncs and events on the plan's main stream
    for _ in range(args.warmup):
        plan.run(zero_c=False)
    hip.tsp_device_sync()
    wit, mhz = plan.warmup(1000)
    plan.run(zero_c=True)
    hip.tsp_device_sync()
    ms = plan.time(args.steps)
    hip.tsp_device_sync()
    # a cross-check over a long window (at least 200 ms)
    long_reps = int(min(100000, max(args.steps, np.ceil(200.0 / max(ms, 1e-4)))))
    ms_long, submit_long = plan.time_ex(long_reps)
    tflops = 2.0 * A.nnz * colB / (ms * 1e-3) / 1e12

    # per-class kernel time, each class alone on the stream a step launches it on
    cls = {}
    for sb, bm, tn in zip(subs, (64, 16, 8), tilenum):
        if tn == 0:
            continue
        warm = plan.time_class(bm, args.class_reps)
        reps = int(min(20000, max(args.class_reps, args.class_min_ms / max(warm, 1e-4))))
        cms = plan.time_class(bm, reps)
        b = alg_bytes(sb.rows, sb.nnz, s, A.cols, colB, s)
        b_touched = alg_bytes(sb.rows, sb.nnz, s, kcols[bm], colB, s)
        v = plan.get_variant(bm)
        w = v[0] or default_width(hip, bm, prec, cbp)
        bn = tsp.tile_bn(bm, prec)
        b3 = max(0, plan.get_b_3byte(bm))
        lines = tn * bn * (cbp // w) * max(1, -(-w * (3 if b3 else s) // 128))
        cls[bm] = {"ms": cms, "reps": reps, "rows": sb.rows, "nnz": int(sb.nnz), "tiles": tn,
                   "format": {1: "dense", 2: "packed"}.get(plan.get_format(bm), "?"),
                   "order": {0: "side-by-side", 1: "side-by-side", 2: "chunk-major"}[v[3]],
                   "tasks_per_wave": max(1, v[2]), "stages": max(1, v[1]), "chunk_width": w,
                   "lane_indices": max(0, plan.get_lane_indices(bm)),
                   "tile_pairs": max(0, plan.get_pairs(bm)), "b_3byte": b3,
                   "placement": {0: "contiguous", 1: "interleaved", 2: "chunk-xcd"}.get(plan.get_placement(bm), "?"),
                   "panel_rows": plan.get_panels(bm)[0], "panel_lag": plan.get_panels(bm)[1],
                   "alg_bytes": b, "gbs": b / (cms * 1e-3) / 1e9, "alg_bytes_touched": b_touched,
                   "gathered_lines": lines, "glines_per_s": lines / (cms * 1e-3) / 1e9}
    dom = max(cls, key=lambda k: cls[k]["ms"])
    dk = cls[dom]
    k_all = int(np.unique(A.colidx).size)
    step_bytes = alg_bytes(A.rows, A.nnz, s, A.cols, colB, s)
    step_gbs = step_bytes / (ms * 1e-3) / 1e9

    # the dominant kernel's instantiation spmm_kernel<BM, W, PREC, S, PK, LI, SY, PR>;
    # the profiled HBM traffic applies only to the same instantiation and hot
    # rows (plans launch tf32 on operands they rounded once: kernel precision
    # code 2, or 3 with B in the 3-byte form)
    tf = lambda b: "true" if b else "false"
    kcode = (3 if dk["b_3byte"] else 2) if prec == 1 else 0
    kname = (f"spmm_kernel<{dom}, {dk['chunk_width']}, {kcode}, {dk['stages']}, "
             f"{tf(dk['format'] == 'packed')}, {tf(dk['lane_indices'])}, {tf(dk['panel_rows'])}, "
             f"{tf(dk['tile_pairs'])}>")
    traffic, traffic_note = None, "no profile of this workload in profiles/"
    prof = os.path.join(ROOT, "profiles", f"traffic_config{config}_{pname}_{colB}.json")
    if os.path.exists(prof):
        with open(prof) as fh:
            pj = json.load(fh)
        # the tuned instantiation may be the profile's main entry or one of
        # the alternatives profiled beside it
        entries = [pj.get(f"bm{dom}", {})] + [e for e in pj.get("alternatives", []) if e.get("bm") == dom]
        # the same instantiation, hot rows and runtime variant (chunk order,
        # XCD placement, tasks per wave, panel sweep), as the profile's
        # replay flags ran it
        run_variant = variant_of(dk)
        hit = [e for e in entries if e.get("kernel", "").endswith(kname) and e.get("hot_rows", 0) == hot_n
               and e.get("variant") == run_variant]
        if hit:
            traffic, traffic_note = hit[0].get("hbm_bytes_per_launch"), os.path.relpath(prof, ROOT)
        else:
            traffic_note = (f"{os.path.relpath(prof, ROOT)} profiles {len(entries)} variants of the {dom}-row "
                            f"class, not the tuned {kname} {json.dumps(run_variant)} with {hot_n} hot rows")
    roof = {"bound": "hbm", "achieved": round(dk["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(dk["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
            "traffic_over_alg": round(traffic / dk["alg_bytes"], 3) if traffic else None,
            "traffic_source": traffic_note, "kernel": kname, "kernel_ms": round(dk["ms"], 5),
            "alg_bytes_per_launch": dk["alg_bytes"],
            "alg_bytes_touched_per_launch": dk["alg_bytes_touched"],
            "frac_touched": round(dk["alg_bytes_touched"] / (dk["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "step_achieved": round(step_gbs, 2), "step_frac": round(step_gbs / HBM_PEAK_GBS, 4),
            "step_alg_bytes": step_bytes}

    rec = {"workload": f"{NAMES[config]}, {pname}, colB {colB}", "config_id": config, "dtype": pname,
           "tune_mode": "cold" if args.tune_cold else "back-to-back",
           "rows": A.rows, "nnz": A.nnz, "colB": colB, "colB_padded": cbp, "gamma": g, "delta": d,
           "th": list(th), "tilenum": tilenum, "hot_rows": hot_n, "hot_bytes": hot_b,
           "ms_per_step": ms, "tflops": tflops, "steps": args.steps, "window_ms": ms * args.steps,
           "long_window": {"steps": long_reps, "ms_per_step": round(ms_long, 6),
                           "tflops": round(2.0 * A.nnz * colB / (ms_long * 1e-3) / 1e12, 4),
                           # host wall time per step to submit the launches: about
                           # ms_per_step when the steps are bound by the launch rate
                           "host_submit_ms_per_step": round(submit_long, 6)},
           "warmup_clock": {"steps": wit, "gfx_mhz": mhz},
           "roofline": roof, "classes": cls, "pre_ms": pre,
           "replay": pins_of(plan, th, cls)}

    # the same steps replayed from one HIP graph: one submission per graph
    # instead of one launch per kernel (reported beside the eager protocol,
    # which stays the value, as the reference times it)
    if headline and not args.no_graph:
        gsteps = max(10, args.steps)
        plan.graph_capture(gsteps)
        greps = max(3, min(1000, int(round(50.0 / (gsteps * ms)))))
        plan.graph_time(1)
        gms = plan.graph_time(greps)
        plan.graph_free()
        rec["graph"] = {
            "steps_per_graph": gsteps, "replays": greps, "ms_per_step": round(gms, 6),
            "tflops": round(2.0 * A.nnz * colB / (gms * 1e-3) / 1e12, 4),
            "note": "the same steps captured once (tsp_plan_graph_capture) and replayed as HIP graphs; "
                    "`value` and `ms_per_step` are eager back-to-back launches"}
    # the cold-cache leg runs for the headline and for the target records
    if args.cold_reps > 0:
        cms, wms, cpms, cpb = cold_steps(hip, plan, args.cold_reps, step_bytes)
        rec["cold_cache"] = {
            "ms_per_step": round(cms, 6), "tflops": round(2.0 * A.nnz * colB / (cms * 1e-3) / 1e12, 4),
            "alg_gbs": round(step_bytes / (cms * 1e-3) / 1e9, 1), "warm_single_ms": round(wms, 6),
            "copy_cold_ms": round(cpms, 6), "copy_cold_gbs": round(cpb / (cpms * 1e-3) / 1e9, 1),
            "reps": args.cold_reps,
            "protocol": "median of single steps, each after a 1 GB copy that evicts L2 and the 256 MB "
                        "MALL; warm_single_ms: the same single step again right after; copy_cold: a "
                        "plain copy moving the step's algorithmic bytes after the same eviction"}
    if headline:
        if not args.no_vendor:
            rec["vendor"] = vendor_spmm(hip, A, B, colB, cbp, prec)
        if not args.no_cpu:
            rec["cpu_baseline"] = cpu_baseline(A, B, colB, prec)
    return rec, A, subs, plan


def vendor_spmm(hip, A, B, colB, cbp, prec):
    """rocSPARSE spmm (CSR, alg default) on the same A and B."""
    import ctypes as C
    vp, vm = C.c_double(), C.c_double()
    Cv = np.zeros((A.rows, colB), dtype=np.float32)
    st = hip.tsp_vendor_spmm(prec, A.rows, A.cols, A.nnz, A.rowptr.ctypes.data_as(C.c_void_p),
                             A.colidx.ctypes.data_as(C.c_void_p), A.val.ctypes.data_as(C.c_void_p), colB, cbp,
                             np.ascontiguousarray(B).ctypes.data_as(C.c_void_p),
                             Cv.ctypes.data_as(C.c_void_p), 20, 200, C.byref(vp), C.byref(vm))
    if st:
        return {"lib": "rocSPARSE", "status": st}
    return {"lib": "rocSPARSE spmm (CSR, alg default)", "ms": round(vm.value, 5),
            "tflops": round(2.0 * A.nnz * colB / (vm.value * 1e-3) / 1e12, 4)}


def cpu_baseline(A, B, colB, prec):
    """The oracle's OpenMP CSR SpMM (fp32 accumulate, dynamic(64)) over the
    WHOLE matrix on the host's cores: one warm-up run, then five timed runs
    (fewer only if they would pass 30 s); the median is reported."""
    import oracle
    a32 = oracle.values_f64(A.val, prec).astype(np.float32)
    b32 = oracle.values_f64(B[:, :colB].reshape(-1), prec).astype(np.float32).reshape(A.cols, colB)
    out = np.zeros((A.rows, colB), dtype=np.float32)
    t1 = time.perf_counter()
    _, used = oracle.spmm_f32_omp(A.rows, A.rowptr, A.colidx, a32, b32, colB, out)
    first = time.perf_counter() - t1
    times, spent = [], 0.0
    while len(times) < 5 and spent + first < 30.0:
        t1 = time.perf_counter()
        oracle.spmm_f32_omp(A.rows, A.rowptr, A.colidx, a32, b32, colB, out)
        times.append(time.perf_counter() - t1)
        spent += times[-1]
    tm = float(np.median(times))
    nproc = len(os.sched_getaffinity(0))
    return {"value": round(2.0 * A.nnz * colB / tm / 1e12, 5), "unit": "TFLOPS", "cores": int(used), "kind": "port",
            "sample": f"whole matrix: {A.rows} rows, {A.nnz} nnz, colB {colB}, fp32 accumulate, OpenMP "
                      f"dynamic(64) on {used} threads ({nproc} cpus usable, OMP_NUM_THREADS="
                      f"{os.environ.get('OMP_NUM_THREADS', 'unset')}), median of {len(times)} after one warm-up "
                      f"run ({first * 1e3:.0f} ms), {tm * 1e3:.1f} ms per run"}


def hub_split(tsp, hip, args):
    """The hub-row experiment: split A by column into the entries whose
    columns are the H most gathered (distinct (8-row block, column) pairs)
    and the rest, and time three plans -- the whole matrix, the hub part and
    the cold part -- each tuned as the headline is, with the policy split of
    the whole matrix.  If L2 reuse of the hub rows were what bounds the
    kernel, the hub part (every gather from an L2-sized set of rows) would
    run far faster per tile and hub + cold would beat the whole; a real
    two-phase kernel would also pay a read-modify-write of C.  One JSON line
    per H, after lines for each plan.  Between the timed launches of the
    three plans a 16-byte copy kernel marks the boundary (for profilers)."""
    import ctypes as C
    prec = {"fp16": 0, "tf32": 1, None: -1}[args.prec]
    A, B, colB, cbp = tsp.gen_config(args.config, prec, args.colB)
    prec = A.prec
    g, d = tsp.predict(tsp.features(A, 9.5, colB), prec)
    rows = np.repeat(np.arange(A.rows, dtype=np.int64), np.diff(A.rowptr))
    pairs = np.unique((rows // 8) * A.cols + A.colidx)
    cnt = np.bincount((pairs % A.cols).astype(np.int64), minlength=A.cols)
    del pairs
    order = np.argsort(-cnt, kind="stable")
    mark_src, mark_dst = C.c_void_p(), C.c_void_p()
    assert hip.tsp_malloc(C.byref(mark_src), 256) == 0 and hip.tsp_malloc(C.byref(mark_dst), 256) == 0

    def part(mask):
        rp = np.concatenate([[0], np.cumsum(np.bincount(rows[mask], minlength=A.rows))]).astype(np.int32)
        return tsp.Csr(A.rows, A.cols, rp, A.colidx[mask], A.val[mask], prec)

    def plan_of(Ap):
        plan = tsp.Plan.from_csr(tsp.matrix_split(Ap, g, d), Ap.rows, Ap.cols, cbp, prec, B)
        th, _, _ = plan.tune(True)
        plan.warmup(300)
        plan.run(zero_c=True)
        return plan, th

    def timed(name, plan, th, Ap):
        hip.tsp_copy_kernel(mark_dst, mark_src, 16, None)
        hip.tsp_device_sync()
        ms = plan.time(args.steps)
        rec = {"hub_split": name, "nnz": Ap.nnz, "tiles": [plan.tilenum(bm) for bm in (64, 16, 8)],
               "ms_per_step": round(ms, 5), "tiles_per_us": round(sum(plan.tilenum(bm) for bm in (64, 16, 8))
                                                                    / (ms * 1e3), 1),
               "th": list(th), "hot_rows": plan.get_hot_rows()[0]}
        print(json.dumps(rec), flush=True)
        return ms

    for H in args.hub_split:
        hub = np.zeros(A.cols, bool)
        hub[order[:H]] = True
        m = hub[A.colidx]
        parts = [("whole", A), ("hub", part(m)), ("cold", part(~m))]
        plans = [plan_of(Ap) for _, Ap in parts]
        ms = [timed(f"{n} H={H}", p, th, Ap) for (n, Ap), (p, th) in zip(parts, plans)]
        for p, _ in plans:
            p.close()
        print(json.dumps({"hub_split_summary": H, "workload": NAMES[args.config], "prec": prec, "colB": colB,
                          "hub_share_of_gathers": round(float(cnt[order[:H]].sum() / cnt.sum()), 4),
                          "hub_share_of_nnz": round(float(m.mean()), 4), "whole_ms": round(ms[0], 5),
                          "hub_ms": round(ms[1], 5), "cold_ms": round(ms[2], 5),
                          "hub_plus_cold_ms": round(ms[1] + ms[2], 5)}), flush=True)
    hip.tsp_free(mark_src)
    hip.tsp_free(mark_dst)


def stream_floor(tsp, hip, A, subs, prec, cbp, b3=False):
    """Gathers the B rows of every tile column index of every class of the
    split `subs`, in tile order, with nothing else in the loop
    (tsp_gather_index_stream: one colB_p-wide row per index, 8 loads in
    flight per lane), once from B's rows in place and once with the hot rows
    a plan copies (the most gathered columns gathered at least 4 times, up to
    16 MB, at rows colA + slot); tf32 also with the hot rows in the 3-byte
    form (rows of colB_p x 3 bytes).  The faster of the first two is the
    floor of the step's own gathers, or the third when the step's dominant
    class reads B in the 3-byte form (b3).  Beside it, the time to write C
    once (rows x colB_p fp32, a memset of that size): the other compulsory
    stream of a step, which shares the memory system with the gathers."""
    import ctypes as C
    stream = np.concatenate([tsp.tile_create(sb, A.cols, bm, prec).arrays()["tile_colidx"].astype(np.int32)
                             for sb, bm in zip(subs, (64, 16, 8)) if sb.rows > 0])
    row_bytes = cbp * (2 if prec == 0 else 4)
    if row_bytes not in (64, 128, 256, 512):
        return {"row_bytes": row_bytes, "indices": int(stream.size),
                "skipped": "the index-stream probe reads rows of 64 to 512 bytes"}
    cnt = np.bincount(stream, minlength=A.cols)
    H = min(int((16 << 20) // row_bytes), int((cnt >= 4).sum()))
    order = np.argsort(-cnt, kind="stable")[:H]
    slot = np.full(A.cols, -1, np.int64)
    slot[order] = np.arange(H)
    nrows = A.cols + H
    tab, sink, didx = C.c_void_p(), C.c_void_p(), C.c_void_p()
    if (hip.tsp_malloc(C.byref(tab), nrows * row_bytes) or hip.tsp_malloc(C.byref(sink), 1024)
            or hip.tsp_malloc(C.byref(didx), stream.nbytes)):
        raise SystemExit("bench.py: cannot allocate the gather stream probe")
    e0, e1 = C.c_void_p(), C.c_void_p()
    hip.tsp_event_create(C.byref(e0))
    hip.tsp_event_create(C.byref(e1))
    out = {"row_bytes": row_bytes, "indices": int(stream.size),
           "hot_share_of_gathers": round(float(cnt[order].sum() / max(stream.size, 1)), 4)}
    try:
        hip.tsp_memset(tab, 1, nrows * row_bytes)
        forms = [("canonical", row_bytes), ("hot_rows", row_bytes)]
        if prec == 1 and 3 * cbp in (96, 192, 384):
            forms.append(("hot_rows_3byte", 3 * cbp))
        for name, rb in forms:
            idx = stream if name == "canonical" else np.where(slot[stream] >= 0, A.cols + slot[stream],
                                                              stream).astype(np.int32)
            assert hip.tsp_memcpy_h2d(didx, idx.ctypes.data_as(C.c_void_p), idx.nbytes) == 0
            assert hip.tsp_gather_index_stream(tab, nrows, rb, didx, idx.size, sink, None) == 0
            reps = 5
            hip.tsp_event_record(e0, None)
            for _ in range(reps):
                hip.tsp_gather_index_stream(tab, nrows, rb, didx, idx.size, sink, None)
            hip.tsp_event_record(e1, None)
            hip.tsp_event_sync(e1)
            ms = C.c_float()
            hip.tsp_event_elapsed_ms(C.byref(ms), e0, e1)
            t = ms.value / reps
            out[name] = {"ms": round(t, 5), "g_rows_per_s": round(idx.size / (t * 1e-3) / 1e9, 2)}
    finally:
        hip.tsp_event_destroy(e0)
        hip.tsp_event_destroy(e1)
        for p in (tab, sink, didx):
            hip.tsp_free(p)
    out["hot_rows"]["rows"] = H
    out["floor_ms"] = (out["hot_rows_3byte"]["ms"] if b3 and "hot_rows_3byte" in out
                       else min(out["canonical"]["ms"], out["hot_rows"]["ms"]))
    out["floor_form"] = "hot rows, 3-byte B" if b3 and "hot_rows_3byte" in out else "4-byte B"
    cbytes = A.rows * cbp * 4
    cbuf = C.c_void_p()
    if hip.tsp_malloc(C.byref(cbuf), cbytes) == 0:
        try:
            hip.tsp_event_create(C.byref(e0))
            hip.tsp_event_create(C.byref(e1))
            hip.tsp_memset_async(cbuf, 0, cbytes, None)
            reps = 5
            hip.tsp_event_record(e0, None)
            for _ in range(reps):
                hip.tsp_memset_async(cbuf, 0, cbytes, None)
            hip.tsp_event_record(e1, None)
            hip.tsp_event_sync(e1)
            ms = C.c_float()
            hip.tsp_event_elapsed_ms(C.byref(ms), e0, e1)
            out["c_write_ms"] = round(ms.value / reps, 5)
            out["floor_plus_c_write_ms"] = round(out["floor_ms"] + out["c_write_ms"], 5)
        finally:
            hip.tsp_event_destroy(e0)
            hip.tsp_event_destroy(e1)
            hip.tsp_free(cbuf)
    return out


def gather_stream(tsp, hip, args):
    """The gather floor of a workload's own B-row stream (stream_floor) beside
    the tuned plan's step time: their ratio is how close the kernels run to
    the rate at which the memory system serves their gathers.  One JSON
    line."""
    prec = {"fp16": 0, "tf32": 1, None: -1}[args.prec]
    A, B, colB, cbp = tsp.gen_config(args.config, prec, args.colB)
    prec = A.prec
    g, d = tsp.predict(tsp.features(A, 9.5, colB), prec)
    subs = tsp.matrix_split(A, g, d)
    plan = tsp.Plan.from_csr(subs, A.rows, A.cols, cbp, prec, B)
    plan.tune(True)
    plan.warmup(300)
    plan.run(zero_c=True)
    step_ms = plan.time(args.steps)
    hot_tuned = plan.get_hot_rows()[0]
    b3 = any(plan.get_b_3byte(bm) == 1 for bm in (64, 16, 8))
    plan.close()
    del B
    out = stream_floor(tsp, hip, A, subs, prec, cbp, b3=b3)
    print(json.dumps({"gather_stream": NAMES[args.config], "prec": prec, "colB": colB,
                      "tuned_step_ms": round(step_ms, 5), "tuned_hot_rows": hot_tuned, **out,
                      "gather_floor_over_step": round(out["floor_ms"] / step_ms, 4) if "floor_ms" in out else None,
                      "floor_plus_c_write_over_step": round(out.get("floor_plus_c_write_ms", 0.0) / step_ms, 4)}),
          flush=True)


TARGETS = {3: "T3", 5: "T5"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", type=int, default=5,
                    help="headline configuration (default 5: RMAT scale 22, tf32, colB 64, the largest)")
    ap.add_argument("--prec", choices=["fp16", "tf32"], default=None)
    ap.add_argument("--colB", type=int, default=-1)
    ap.add_argument("--targets", default="3,5",
                    help="configurations also run as fp16 / colB 128 targets (T3, T5); empty for none")
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
                    help="pin the pipeline depth per class 64,16,8 (1-3; 0 keep)")
    ap.add_argument("--place", type=ints3, default=None,
                    help="pin the XCD placement per class 64,16,8 (1 contiguous, 2 interleaved, 3 one column "
                         "chunk per XCD group, 0 keep)")
    ap.add_argument("--lane-idx", type=ints3, default=None,
                    help="pin lane-loaded column indices per class 64,16,8 (1 off, 2 on, 0 keep)")
    ap.add_argument("--pairs", type=ints3, default=None,
                    help="pin tile pairs per class 64,16,8 (1 off, 2 on, 0 keep; fp16 8-/16-row classes, tf32 8-row class)")
    ap.add_argument("--b3", type=ints3, default=None,
                    help="pin B in the 3-byte form per class 64,16,8 (1 off, 2 on, 0 keep; tf32)")
    ap.add_argument("--panels", type=ints3, default=None,
                    help="pin the panel-synchronised sweep per class: B rows per panel (0 = off)")
    ap.add_argument("--panel-lag", type=ints3, default=None,
                    help="lead in panels a wave may have on the slowest (with --panels; default 2)")
    ap.add_argument("--hot-bytes", type=int, default=None,
                    help="pin the hot B row budget in bytes after tuning (0: no hot rows)")
    ap.add_argument("--tune-cold", action="store_true",
                    help="tune for single steps from a cold cache (TSP_TUNE_COLD) instead of back-to-back steps")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-vendor", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP graph replay leg")
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
    ap.add_argument("--gather-stream", action="store_true",
                    help="only time the gathers of the workload's own B-row index stream against its tuned step")
    ap.add_argument("--hub-split", type=lambda v: [int(x) for x in v.split(",")], default=None,
                    help="only run the hub-row experiment for these hub set sizes (columns), e.g. 16384")
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
    if args.hub_split:
        hub_split(tsp, hip, args)
        return
    if args.gather_stream:
        gather_stream(tsp, hip, args)
        return

    prec = {"fp16": 0, "tf32": 1, None: -1}[args.prec]
    if args.sweep:
        args.no_vendor = args.no_cpu = True
        args.cold_reps = 0
    rec, A, subs, plan = measure(tsp, hip, args.config, prec, args.colB, args, headline=True)
    if args.sweep:
        sweep(plan, rec["tilenum"], rec["colB_padded"], args)
        plan.close()
        return
    plan.close()
    # the floor of the headline step's own B-row gathers (stream_floor)
    dk = rec["classes"][max(rec["classes"], key=lambda k: rec["classes"][k]["ms"])]
    floor = stream_floor(tsp, hip, A, subs, A.prec, rec["colB_padded"], b3=bool(dk.get("b_3byte")))
    if "floor_ms" in floor:
        floor["floor_over_step"] = round(floor["floor_ms"] / rec["ms_per_step"], 4)
    if "floor_plus_c_write_ms" in floor:
        floor["floor_plus_c_write_over_step"] = round(floor["floor_plus_c_write_ms"] / rec["ms_per_step"], 4)
    rec["gather_floor"] = floor
    del A, subs
    ceiling = gather_ceiling(hip)
    # the measured copy-bandwidth peak (a 512 MB copy back to back, read plus
    # write), beside the 8 TB/s spec peak the roofline fraction uses
    copy_gbs = copy_calibration(hip, 512 << 20, 10, quiet=True)

    def vs_copy(roof):
        roof["copy_peak_gbs"] = round(copy_gbs, 1)
        roof["frac_of_copy"] = round(roof["achieved"] / copy_gbs, 4)
        return roof

    vs_copy(rec["roofline"])

    def gather_stats(r):
        dk = r["classes"][max(r["classes"], key=lambda k: r["classes"][k]["ms"])]
        return {"glines_per_s": round(dk["glines_per_s"], 2), "ceiling_glines_per_s": round(ceiling, 2),
                "frac_of_ceiling": round(dk["glines_per_s"] / ceiling, 3)}

    targets = {}
    for cfg in [int(x) for x in args.targets.split(",") if x.strip()]:
        targ = argparse.Namespace(**vars(args))
        for k in ("th", "format", "order", "tpw", "width", "stages", "place", "lane_idx", "pairs", "b3", "panels",
                  "panel_lag",
                  "hot_bytes",
                  "gamma",
                  "delta"):
            setattr(targ, k, None)
        targ.no_tune = False
        targ.tune_cold = False
        t, _, _, tplan = measure(tsp, hip, cfg, 0, 128, targ, headline=False)
        tplan.close()
        targets[TARGETS.get(cfg, f"C{cfg}")] = {
            "workload": t["workload"], "ms_per_step": round(t["ms_per_step"], 6), "tflops": round(t["tflops"], 4),
            "long_window": t["long_window"], "kernel": t["roofline"]["kernel"],
            "kernel_ms": t["roofline"]["kernel_ms"], "frac": t["roofline"]["frac"],
            "frac_of_copy": vs_copy(t["roofline"])["frac_of_copy"],
            "alg_bytes_per_launch": t["roofline"]["alg_bytes_per_launch"], "traffic": t["roofline"]["traffic"],
            "traffic_over_alg": t["roofline"]["traffic_over_alg"], "traffic_source": t["roofline"]["traffic_source"],
            "gather": gather_stats(t), "cold_cache": t.get("cold_cache"),
            "hot_rows": t["hot_rows"], "th": t["th"], "tilenum": t["tilenum"],
            "classes": {f"bm{k}": {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                        for k, v in t["classes"].items()},
            "replay": t["replay"]}

    line = {
        "metric": "SpMM TFLOPS (2*nnz*colB/t) + % HBM roofline",
        "value": round(rec["tflops"], 4), "unit": "TFLOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(rec["ms_per_step"], 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": rec["dtype"], "data": "synthetic",
        "config": {"workload": rec["workload"], "config_id": rec["config_id"], "rows": rec["rows"],
                   "nnz": rec["nnz"], "colB": rec["colB"], "colB_padded": rec["colB_padded"],
                   "gamma": rec["gamma"], "delta": rec["delta"], "th": rec["th"], "tilenum": rec["tilenum"],
                   "hot_rows": rec["hot_rows"], "hot_bytes": rec["hot_bytes"], "parallelism": "single GPU"},
        "roofline": rec["roofline"],
        "cpu_baseline": rec.get("cpu_baseline"),
        "gather": gather_stats(rec),
        "gather_floor": rec.get("gather_floor"),
        "targets": targets,
        "window_ms": round(rec["window_ms"], 3),
        "long_window": rec["long_window"],
        "warmup_clock": rec["warmup_clock"],
        "classes": {f"bm{k}": {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in rec["classes"].items()},
        "cold_cache": rec.get("cold_cache"),
        "graph": rec.get("graph"),
        "tune_mode": rec["tune_mode"],
        "vendor": rec.get("vendor"),
        "pre_ms": rec["pre_ms"],
        "replay": rec["replay"],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
