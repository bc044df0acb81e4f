"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Tolerances (element-wise, normalised by the magnitude sum |A|.|B| of the
entry): fp16 path 1e-3, tf32 path 1e-4 -- the north-star bounds.  Inputs are
exact in the kernels' arithmetic (fp16 values; tf32-rounded fp32 values), so
the only error is fp32 accumulation.  With the CLI's integer value stream the
result is an exact integer and the comparison is exact equality.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

from parity_checks import TOL, assert_checksums

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def gpu(tsp):
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    return tsp


def run_tiles(tsp, A, B, colB_p, gamma, delta, th=(8, 8, 8), tune=False):
    subs = tsp.matrix_split(A, gamma, delta)
    tiles = [tsp.tile_create(s, A.cols, bm, A.prec) for s, bm in zip(subs, (64, 16, 8))]
    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, colB_p, A.prec, B)
    try:
        if tune:
            plan.tune(True)
        else:
            plan.set_th(*th)
        plan.run(zero_c=True)
        Cg = plan.download_c()
    finally:
        plan.close()
    return Cg, tiles


def reference(orc, A, B, colB, rows=None):
    """fp64 CSR SpMM of the kernel's exact inputs; optionally a row subset."""
    tf = A.prec == 1
    a = orc.values_f64(A.val, A.prec, tf32_round=tf)
    b = orc.values_f64(B[:, :colB].reshape(-1), A.prec, tf32_round=tf).reshape(B.shape[0], colB)
    rp, ci = A.rowptr, A.colidx
    if rows is not None:
        rows = np.asarray(rows)
        lens = rp[rows + 1] - rp[rows]
        sel = np.concatenate([np.arange(rp[r], rp[r + 1]) for r in rows]) if len(rows) else np.zeros(0, int)
        rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        ci, a = ci[sel], a[sel]
    n = len(rp) - 1
    Cref = orc.spmm_f64(n, rp, ci, a, b, colB)
    Cabs = orc.spmm_f64(n, rp, ci, np.abs(a), np.abs(b), colB)
    return Cref, Cabs


def assert_close(Cg, Cref, Cabs, prec, what=""):
    err = np.abs(Cg.astype(np.float64) - Cref)
    bound = TOL[prec] * Cabs + 1e-30
    bad = err > bound
    assert np.isfinite(Cg).all(), what
    if bad.any():
        i = np.argwhere(bad)[0]
        pytest.fail(f"{what}: {bad.sum()} entries out of tolerance, first {tuple(i)}: "
                    f"gpu={Cg[tuple(i)]!r} ref={Cref[tuple(i)]!r} bound={bound[tuple(i)]!r}")


def random_matrix(tsp, rng, rows, cols, maxlen, prec, empty_frac=0.1, heavy_rows=0):
    lens = rng.integers(0, maxlen + 1, rows)
    lens[rng.random(rows) < empty_frac] = 0
    if heavy_rows:
        lens[rng.choice(rows, heavy_rows, replace=False)] = min(cols, 40 * maxlen)
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ci = np.concatenate([rng.choice(cols, size=int(l), replace=False) for l in lens]).astype(np.int32) \
        if rp[-1] else np.zeros(0, np.int32)
    v = rng.uniform(-1, 1, rp[-1]).astype(np.float32)
    val = v.astype(np.float16).view(np.uint16) if prec == 0 else v
    return tsp.Csr(rows, cols, rp, ci, val, prec)


def random_b(tsp, rng, cols, colB, prec):
    cbp = tsp.colB_padded(colB)
    b = np.zeros((cols, cbp), dtype=np.float32)
    b[:, :colB] = rng.uniform(-1, 1, (cols, colB))
    return (b.astype(np.float16).view(np.uint16) if prec == 0 else b), cbp


@pytest.mark.parametrize("prec", [0, 1])
@pytest.mark.parametrize("colB", [8, 32, 64, 100, 128, 192, 256, 320, 512])
def test_random_all_classes(gpu, orc, prec, colB):
    tsp = gpu
    rng = np.random.default_rng(prec * 1000 + colB)
    A = random_matrix(tsp, rng, 777, 613, 40, prec, heavy_rows=5)
    B, cbp = random_b(tsp, rng, A.cols, colB, prec)
    Cref, Cabs = reference(orc, A, B, colB)
    for g, d in [(2.0, 1.5), (0.0, 1.5), (5.0, 0.0), (5.0, 3.0), (1.0, 1.0)]:
        for th in ((8, 8, 8), (128, 128, 128)):
            say(f"random prec={prec} colB={colB} gamma={g} delta={d} th={th}")
            Cg, _ = run_tiles(tsp, A, B, cbp, g, d, th)
            assert_close(Cg[:, :colB], Cref, Cabs, prec, f"g={g} d={d} th={th}")
            if colB < cbp:
                assert (Cg[:, colB:] == 0).all()


@pytest.mark.parametrize("prec", [0, 1])
def test_every_kernel_variant(gpu, orc, prec):
    """Every (chunk width, pipeline depth, tasks per wave, scalar or
    lane-loaded column indices) variant of every class and A format, with
    every XCD placement its chunk count allows, gives the oracle's result,
    split tasks included."""
    tsp = gpu
    rng = np.random.default_rng(50 + prec)
    A = random_matrix(tsp, rng, 611, 509, 45, prec, heavy_rows=4)
    colB = 128
    B, cbp = random_b(tsp, rng, A.cols, colB, prec)
    Cref, Cabs = reference(orc, A, B, colB)
    for g, d, bm in [(0.0, 1.5, 64), (5.0, 0.0, 16), (5.0, 3.0, 8)]:
        subs = tsp.matrix_split(A, g, d)
        tiles = [tsp.tile_create(s, A.cols, b, prec) for s, b in zip(subs, (64, 16, 8))]
        plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
        try:
            plan.set_th(8, 8, 8)
            for fmt in ((1,) if bm == 64 else (1, 2)):
                plan.set_format(bm, fmt)
                assert plan.get_format(bm) == fmt
                for w in ((32, 64) if bm == 64 else (32, 64, 128)):
                    for s, li in [(s, li) for s in (1, 2, 3) for li in ((0,) if bm == 64 else (0, 1))]:
                        for tpw, order in ((1, 1), (3, 2), (0, 0)):
                            for place in ((0, 1, 2) if cbp // w in (2, 4, 8) else (0, 1)):
                                tag = (f"prec={prec} bm={bm} fmt={fmt} w={w} s={s} lane_idx={li} tpw={tpw} "
                                       f"order={order} place={place}")
                                say("variant " + tag)
                                plan.set_variant(bm, w, s, tpw, order)
                                plan.set_lane_indices(bm, li)
                                assert plan.get_lane_indices(bm) == li
                                plan.set_placement(bm, place)
                                assert plan.get_placement(bm) == place
                                plan.run(zero_c=True)
                                Cg = plan.download_c()
                                assert_close(Cg[:, :colB], Cref, Cabs, prec, tag)
        finally:
            plan.close()


def test_tile_pairs(gpu, orc):
    """Tile pairs (two tiles of a task per K = 32 MFMA; fp16 8- and 16-row
    classes, 64- and 128-column chunks): every depth, format, index mode,
    tasks per wave, order and placement gives the oracle's result, with
    thresholds that leave tasks of odd and even tile counts (the last unit of
    an odd task holds one tile) and split tasks; the panel sweep with pairs
    is bit-identical to the unsynchronised pair launch.  Chunk widths without
    pair kernels refuse them."""
    tsp = gpu
    prec = 0
    rng = np.random.default_rng(91)
    A = random_matrix(tsp, rng, 611, 509, 45, prec, heavy_rows=4)
    colB = 128
    B, cbp = random_b(tsp, rng, A.cols, colB, prec)
    Cref, Cabs = reference(orc, A, B, colB)
    for g, d, bm in [(5.0, 0.0, 16), (5.0, 3.0, 8)]:
        subs = tsp.matrix_split(A, g, d)
        tiles = [tsp.tile_create(s, A.cols, b, prec) for s, b in zip(subs, (64, 16, 8))]
        plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
        try:
            for th in ((3, 3, 3), (8, 8, 8), (4096, 4096, 4096)):
                plan.set_th(*th)
                for fmt in (1, 2):
                    plan.set_format(bm, fmt)
                    for w in (64, 128):
                        for st, li in [(st, li) for st in ((1, 2, 3) if fmt == 2 else (1, 2))
                                       for li in ((0, 1) if fmt == 2 else (0,))]:
                            for tpw, order in ((1, 1), (3, 2)):
                                for place in ((0, 1, 2) if cbp // w == 2 else (0, 1)):
                                    tag = (f"pairs bm={bm} th={th[0]} fmt={fmt} w={w} s={st} lane_idx={li} "
                                           f"tpw={tpw} order={order} place={place}")
                                    say(tag)
                                    plan.set_variant(bm, w, st, tpw, order)
                                    plan.set_lane_indices(bm, li)
                                    plan.set_placement(bm, place)
                                    plan.set_pairs(bm, 1)
                                    assert plan.get_pairs(bm) == 1
                                    plan.run(zero_c=True)
                                    Cg = plan.download_c()
                                    assert_close(Cg[:, :colB], Cref, Cabs, prec, tag)
                                    plan.set_pairs(bm, 0)
                # the panel sweep over pair units (dense format, one task per wave)
                if th[0] == 4096:
                    plan.set_format(bm, 1)
                    plan.set_lane_indices(bm, 0)
                    for w in (64, 128):
                        plan.set_variant(bm, w, 1, 1, 1)
                        plan.set_placement(bm, 1)
                        plan.set_pairs(bm, 1)
                        plan.set_panels(bm, 0, 1)
                        plan.run(zero_c=True)
                        C0 = plan.download_c()
                        for pr, lag in ((256, 1), (512, 2)):
                            say(f"pairs bm={bm} panels={pr} lag={lag} w={w}")
                            plan.set_panels(bm, pr, lag)
                            for rep in range(2):
                                plan.run(zero_c=True)
                                Cg = plan.download_c()
                                assert np.array_equal(Cg, C0), f"pairs bm={bm} w={w} panels={pr} rep={rep}"
                        plan.set_panels(bm, 0, 1)
                        assert_close(C0[:, :colB], Cref, Cabs, prec, f"pairs bm={bm} w={w} unsynchronised")
                        plan.set_pairs(bm, 0)
            # a width without pair kernels: the launch refuses
            plan.set_variant(bm, 32, 1, 1, 1)
            plan.set_pairs(bm, 1)
            with pytest.raises(tsp.TspError):
                plan.run(zero_c=True)
            plan.set_pairs(bm, 0)
        finally:
            plan.close()


def test_tile_pairs_tf32(gpu, orc):
    """tf32 tile pairs (8-row tiles, 64-column chunks): split-bf16 products on
    v_mfma_f32_16x16x32_bf16 against B in split words.  Every depth, format,
    index mode, tasks per wave, order and placement gives the oracle's
    result within the tf32 tolerance, with odd and even task lengths and
    split tasks, and with hot B rows (the plan refills the split form's hot
    slots); the split form converts back exactly."""
    tsp = gpu
    hip = tsp.load()[0]
    prec = 1
    rng = np.random.default_rng(93)
    A = random_matrix(tsp, rng, 613, 509, 45, prec, heavy_rows=4)
    colB = 128
    B, cbp = random_b(tsp, rng, A.cols, colB, prec)
    Cref, Cabs = reference(orc, A, B, colB)
    subs = tsp.matrix_split(A, 5.0, 3.0)
    tiles = [tsp.tile_create(sb, A.cols, b, prec) for sb, b in zip(subs, (64, 16, 8))]
    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
    try:
        with pytest.raises(tsp.TspError):
            plan.set_pairs(16, 1)                       # tf32 pairs: 8-row tiles only
        for hot in (0, 1 << 16):
            plan.set_hot_rows(hot)
            for th in ((3, 3, 3), (8, 8, 8), (4096, 4096, 4096)):
                plan.set_th(*th)
                for fmt in (1, 2):
                    plan.set_format(8, fmt)
                    for st, li in [(st, li) for st in ((1, 2, 3) if fmt == 2 else (1, 2))
                                   for li in ((0, 1) if fmt == 2 else (0,))]:
                        for tpw, order in ((1, 1), (3, 2)):
                            for place in (0, 1, 2):
                                tag = (f"tf32 pairs hot={hot} th={th[0]} fmt={fmt} s={st} lane_idx={li} tpw={tpw} "
                                       f"order={order} place={place}")
                                say(tag)
                                plan.set_variant(8, 64, st, tpw, order)
                                plan.set_lane_indices(8, li)
                                plan.set_placement(8, place)
                                plan.set_pairs(8, 1)
                                plan.run(zero_c=True)
                                Cg = plan.download_c()
                                assert_close(Cg[:, :colB], Cref, Cabs, prec, tag)
                                plan.set_pairs(8, 0)
        plan.set_variant(8, 128, 1, 1, 1)
        plan.set_pairs(8, 1)
        with pytest.raises(tsp.TspError):
            plan.run(zero_c=True)                       # 128-column chunks have no tf32 pair kernel
    finally:
        plan.close()
    # the split words: host and device conversions agree and sum back exactly
    bits = np.concatenate([np.frombuffer(np.float32(rng.uniform(-1e3, 1e3, 4000)).tobytes(), np.uint32),
                           np.array([0x7F800000, 0xFF800000, 0x7F800001, 0x7FFFFFFF, 0, 0x80000000], np.uint32)])
    tf = np.zeros_like(bits)
    assert hip.tsp_round_tf32_bits(bits.ctypes.data, tf.ctypes.data, bits.size) == 0
    host = np.zeros_like(tf)
    assert hip.tsp_split_bf16_bits(tf.ctypes.data, host.ctypes.data, tf.size) == 0
    d = tsp._DevBuf(tf)
    try:
        assert hip.tsp_split_bf16_device(d.p, d.p, tf.size, None) == 0
        assert np.array_equal(tsp._d2h(d.p, tf.size, np.uint32), host)
    finally:
        d.free()
    hi = (host & 0xFFFF0000).view(np.float32).astype(np.float64)
    lo = (host << 16).view(np.float32).astype(np.float64)
    fin = np.isfinite(tf.view(np.float32))
    assert np.array_equal(hi[fin] + lo[fin], tf.view(np.float32)[fin].astype(np.float64))
    assert np.isposinf(hi[-6]) and lo[-6] == 0 and np.isneginf(hi[-5]) and lo[-5] == 0
    assert np.isnan(hi[-4]) and np.isnan(lo[-4]) and np.isnan(hi[-3]) and np.isnan(lo[-3])


@pytest.mark.parametrize("prec", [0, 1])
def test_nan_and_inf_propagate_with_tile_pairs(gpu, prec):
    """NaN and Inf propagate through the tile-pair kernels exactly as through
    the single-tile ones (every row in the 8-row class, 64-column chunks;
    tf32 through the split words), with tasks of odd tile counts (whose last
    unit has no second tile), even counts and split tasks: a NaN in A reaches
    its row; a NaN / +Inf in a B row reaches, as NaN / +Inf, the rows whose
    CSR rows hold it and, as NaN, the other rows of the row-blocks whose
    tiles gather it; a -Inf in A meets finite B values as -Inf; every other
    entry stays finite."""
    tsp = gpu
    rng = np.random.default_rng(19)
    rows, cols, colB = 256, 128, 64
    rp = np.concatenate([[0], np.cumsum(np.full(rows, 4))]).astype(np.int32)
    ci = np.concatenate([np.sort(rng.choice(cols, 4, replace=False)) for _ in range(rows)]).astype(np.int32)
    v = rng.uniform(0.5, 1, rp[-1]).astype(np.float32)
    bv = rng.uniform(0.5, 1, (cols, colB)).astype(np.float32)
    if prec == 0:
        val, B = v.astype(np.float16).view(np.uint16), bv.astype(np.float16).view(np.uint16)
        nan_a, ninf_a, nan_b, inf_b = np.uint16(0x7E01), np.uint16(0xFC00), np.uint16(0x7C01), np.uint16(0x7C00)
    else:
        val, B = v.copy(), bv.copy()
        nan_a, ninf_a = np.uint32(0x7FFFFFFF), np.uint32(0xFF800000)
        nan_b, inf_b = np.uint32(0x7F800001), np.uint32(0x7F800000)
    bits = np.uint16 if prec == 0 else np.uint32
    val.view(bits)[rp[10] + 1] = nan_a
    val.view(bits)[rp[100] + 2] = ninf_a
    cnan, cinf = 77, 91
    B.view(bits)[cnan, 5] = nan_b
    B.view(bits)[cinf, 9] = inf_b
    A = tsp.Csr(rows, cols, rp, ci, val, prec)
    subs = tsp.matrix_split(A, 5.0, 3.0)
    assert [s.rows for s in subs] == [0, 0, rows]
    tiles = [tsp.tile_create(s, A.cols, b, prec) for s, b in zip(subs, (64, 16, 8))]
    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, colB, prec, B)
    has = lambda c: np.array([c in ci[rp[r]:rp[r + 1]] for r in range(rows)])
    block = lambda c: np.repeat([has(c)[i:i + 8].any() for i in range(0, rows, 8)], 8)
    a_inf = ci[rp[100] + 2]                     # the B row the -Inf of row 100 meets
    try:
        for th in (1, 3, 8, 4096):
            plan.set_th(0, 0, th)
            plan.set_variant(8, 64, 1, 1, 1)
            plan.set_pairs(8, 0)
            plan.run(zero_c=True)
            C1 = plan.download_c()[:, :colB]
            plan.set_pairs(8, 1)
            plan.run(zero_c=True)
            C = plan.download_c()[:, :colB]
            tag = f"prec={prec} th={th}"
            assert np.array_equal(np.isnan(C), np.isnan(C1)), tag
            assert np.array_equal(np.isposinf(C), np.isposinf(C1)), tag
            assert np.array_equal(np.isneginf(C), np.isneginf(C1)), tag
            other = np.ones(rows, bool)
            other[[10, 100]] = False
            assert np.isnan(C[10]).all(), tag
            assert np.isnan(C[has(cnan) & other, 5]).all(), tag
            assert np.isposinf(C[has(cinf) & other, 9]).all(), tag
            assert np.isnan(C[block(cinf) & ~has(cinf) & other, 9]).all(), tag
            rest = np.delete(np.arange(colB), [5, 9])
            assert np.isneginf(C[100, rest]).all(), tag
            assert np.isfinite(C[other][:, rest]).all(), tag
            assert np.isfinite(C[~block(cnan) & other, 5]).all(), tag
            assert np.isfinite(C[~block(cinf) & other, 9]).all(), tag
            assert a_inf not in (cnan, cinf)
    finally:
        plan.close()


@pytest.mark.parametrize("prec", [0, 1])
def test_zero_results_not_stored_until_c_is_shared(gpu, orc, prec):
    """A plan's launches skip storing exact-zero results: its C starts at zero
    and only its launches write it, so empty rows and B's padded columns stay
    zero and every other entry is right, step after step (split tasks, whose
    atomic adds accumulate across steps, with C zeroed before each).  Once the caller takes C's device pointer the plan stores
    every result again: garbage written into C is overwritten by the next
    step wherever a row-block has tiles (rows of row-blocks without any tile
    are written by no step, as in the reference)."""
    import ctypes as C
    tsp = gpu
    hip, host = tsp.load()
    rng = np.random.default_rng(123 + prec)
    A = random_matrix(tsp, rng, 700, 509, 30, prec, empty_frac=0.4, heavy_rows=2)
    colB = 100
    B, cbp = random_b(tsp, rng, A.cols, colB, prec)
    Cref, Cabs = reference(orc, A, B, colB)
    subs = tsp.matrix_split(A, 2.0, 1.5)
    tiles = [tsp.tile_create(sb, A.cols, bm, prec) for sb, bm in zip(subs, (64, 16, 8))]
    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
    empty = np.diff(A.rowptr) == 0
    assert empty.sum() > 100
    written = np.zeros(A.rows, bool)               # rows of row-blocks that have tiles
    for sb, bm in zip(subs, (64, 16, 8)):
        lens = np.diff(sb.rowptr) if sb.rows else np.zeros(0)
        for b0 in range(0, sb.rows, bm):
            if lens[b0:b0 + bm].any():
                written[sb.orig_row[b0:b0 + bm]] = True
    try:
        for th in ((1 << 20,) * 3, (8, 8, 8)):
            plan.set_th(*th)
            for rep in range(2):
                plan.run(zero_c=th[0] == 8)
                Cg = plan.download_c()
                tag = f"prec={prec} th={th[0]} rep={rep}"
                assert_close(Cg[:, :colB], Cref, Cabs, prec, tag)
                assert (Cg[:, colB:] == 0).all() and (Cg[empty] == 0).all(), tag
        plan.set_th(*((1 << 20,) * 3))
        plan.run(zero_c=True)
        C0 = plan.download_c()
        dc = C.c_void_p()
        assert host.tsp_plan_device_c(plan.p, C.byref(dc)) == 0
        assert hip.tsp_memset(dc, 0x7f, A.rows * cbp * 4) == 0      # 0x7f7f7f7f: a large finite value
        plan.run(zero_c=False)
        C1 = plan.download_c()
        assert np.array_equal(C1[written].view(np.uint32), C0[written].view(np.uint32))
        assert (C1[~written].view(np.uint32) == 0x7f7f7f7f).all()
    finally:
        plan.close()


@pytest.mark.parametrize("prec", [0, 1])
def test_panel_sweep_and_wide_chunks(gpu, orc, prec):
    """The panel-synchronised sweep (tsp_plan_set_panels, dense format) and
    the 256-column chunks: every class, chunk width, depth, order, placement
    and panel size gives the oracle's result; without split tasks the result
    is bit-identical to the unsynchronised launch of the same variant (the
    sweep only changes when a wave loads), and repeated launches (the
    counters clear themselves) repeat it.  The 8-row class holds enough
    row-blocks for several generations of the capped grid."""
    tsp = gpu
    rng = np.random.default_rng(70 + prec)
    A = random_matrix(tsp, rng, 20000, 6000, 24, prec, heavy_rows=6)
    colB = 256
    B, cbp = random_b(tsp, rng, A.cols, colB, prec)
    rows = np.unique(np.concatenate([rng.choice(A.rows, 3000, replace=False),
                                     np.argsort(np.diff(A.rowptr))[-20:]]))
    Cref, Cabs = reference(orc, A, B, colB, rows)
    for g, d, bm in [(0.0, 1.5, 64), (5.0, 0.0, 16), (5.0, 3.0, 8)]:
        subs = tsp.matrix_split(A, g, d)
        tiles = [tsp.tile_create(s, A.cols, b, prec) for s, b in zip(subs, (64, 16, 8))]
        plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
        try:
            plan.set_format(bm, 1)
            for th in ((4096, 4096, 4096), (8, 8, 8)):
                plan.set_th(*th)
                full = th[0] == 4096
                for w in ((64,) if bm == 64 else (64, 128, 256) if full else (128, 256)):
                    for s, order, place in ((1, 1, 0), (2, 2, 1), (1, 2, 1)) if full else ((1, 2, 1),):
                        plan.set_variant(bm, w, s, 1, order)
                        plan.set_placement(bm, place)
                        plan.set_panels(bm, 0, 1)
                        plan.run(zero_c=True)
                        C0 = plan.download_c()
                        tag = f"prec={prec} bm={bm} th={th[0]} w={w} s={s} order={order} place={place}"
                        assert_close(C0[rows, :colB], Cref, Cabs, prec, tag + " unsynchronised")
                        for pr, lag in ((256, 1), (4096, 2), (512, 4)) if full else ((512, 2),):
                            say(f"panels {tag} panel_rows={pr} lag={lag}")
                            plan.set_panels(bm, pr, lag)
                            assert plan.get_panels(bm) == (pr, lag)
                            for rep in range(2):
                                plan.run(zero_c=True)
                                Cg = plan.download_c()
                                assert_close(Cg[rows, :colB], Cref, Cabs, prec, f"{tag} panels={pr} rep={rep}")
                                if full:
                                    assert np.array_equal(Cg, C0), f"{tag} panels={pr} rep={rep} differs"
            plan.set_panels(bm, 0, 1)
        finally:
            plan.close()


@pytest.mark.parametrize("prec", [0, 1])
@pytest.mark.parametrize("colB", [32, 128])
def test_cli_integer_stream_dc2_exact(gpu, orc, dc2_path, prec, colB):
    """The reference CLI's inputs on its shipped matrix: exact integers."""
    tsp = gpu
    m, n, rp, ci, _, _ = tsp.mm_read(dc2_path)
    libc = C.CDLL("libc.so.6")
    libc.srand(1325)
    a = np.array([1 + libc.rand() % 3 for _ in range(len(ci))], dtype=np.float32)
    cbp = tsp.colB_padded(colB)
    b = np.zeros((n, cbp), dtype=np.float32)
    draws = np.array([1 + libc.rand() % 3 for _ in range(n * colB)], dtype=np.float32)
    b[:, :colB] = draws.reshape(n, colB)
    val = a.astype(np.float16).view(np.uint16) if prec == 0 else a
    B = b.astype(np.float16).view(np.uint16) if prec == 0 else b
    A = tsp.Csr(m, n, rp, ci, val, prec)
    Cref = orc.spmm_f64(m, rp, ci, a.astype(np.float64), b[:, :colB].astype(np.float64), colB)
    for g, d in [(2.0, 1.5), (1.0, 1.0), (5.0, 3.0)]:
        say(f"dc2 prec={prec} colB={colB} gamma={g} delta={d}")
        Cg, _ = run_tiles(tsp, A, B, cbp, g, d, th=(16, 16, 16))
        assert np.array_equal(Cg[:, :colB].astype(np.float64), Cref)


@pytest.mark.parametrize("exe,colB,tiling", [("tilespmm_fp16", 32, "device"), ("tilespmm_fp16", 128, "device"),
                                             ("tilespmm_tf32", 32, "device"), ("tilespmm_tf32", 128, "device"),
                                             ("tilespmm_fp16", 128, "host"), ("tilespmm_tf32", 32, "host")])
def test_cli_end_to_end(gpu, dc2_path, tmp_path, exe, colB, tiling):
    """The reference's test.sh run: CLI on dc2, check passes, 19-field CSV row;
    tiles built on the device (default) or by the host library."""
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    binary = os.path.join(root, "tilespmm_amd", "bin", exe)
    say(f"cli {exe} colB={colB} tiling={tiling}")
    env = dict(os.environ, TSP_TILING=tiling)
    r = subprocess.run([binary, "-d", "0", dc2_path, str(colB)], cwd=tmp_path, capture_output=True, text=True,
                       timeout=240, env=env)
    assert r.returncode == 0, r.stderr
    assert "Check... PASS!" in r.stdout, r.stdout[-2000:]
    csv = tmp_path / ("TileSpMM-FP16.csv" if exe.endswith("fp16") else "TileSpMM-TF32.csv")
    fields = csv.read_text().strip().split(",")
    assert len(fields) == 19 and fields[0] == dc2_path
    assert int(fields[1]) == 116835 and int(fields[3]) == 766396 and int(fields[4]) == colB
    assert all(float(x) > 0 for x in (fields[14], fields[15], fields[17], fields[18]))


def test_direct_kernel_boundary(gpu, orc):
    """tsp_switch_v16 called directly on device buffers (the kernel ABI), and
    tsp_spmm_launch_placed with both XCD placements on the same buffers."""
    tsp = gpu
    hip, _ = tsp.load()
    rng = np.random.default_rng(2)
    A = random_matrix(tsp, rng, 64, 300, 30, 0)
    colB = 64
    B, cbp = random_b(tsp, rng, A.cols, colB, 0)
    sub = tsp.Csr(A.rows, A.cols, A.rowptr, A.colidx, A.val, 0)
    sub.orig_row = np.arange(A.rows, dtype=np.int32)
    t = tsp.tile_create(sub, A.cols, 16, 0)
    arr = t.arrays()
    rows, cs = tsp.pretreatment(t, 3)          # small TH: several split tasks
    assert (rows & 0x80000000).any()
    bufs = {}

    def up(name, a):
        p = C.c_void_p()
        assert hip.tsp_malloc(C.byref(p), max(a.nbytes, 4)) == 0
        assert hip.tsp_memcpy_h2d(p, a.ctypes.data_as(C.c_void_p), a.nbytes) == 0
        bufs[name] = p
        return p

    try:
        up("val", arr["dense"]); up("col", arr["tile_colidx"]); up("rows", rows); up("cs", cs); up("B", B)
        Cz = np.zeros((A.rows, cbp), dtype=np.float32)
        up("C", Cz)
        outs = []
        for place in (None, 0, 1):
            assert hip.tsp_memcpy_h2d(bufs["C"], Cz.ctypes.data_as(C.c_void_p), Cz.nbytes) == 0
            if place is None:
                st = hip.tsp_switch_v16(0, len(rows), cbp, bufs["val"], bufs["rows"], bufs["cs"], bufs["B"],
                                        bufs["C"], bufs["col"], A.rows, None)
            else:
                st = hip.tsp_spmm_launch_placed(16, 0, len(rows), cbp, bufs["val"], None, None, bufs["rows"],
                                                bufs["cs"], bufs["B"], bufs["C"], bufs["col"], A.rows, None,
                                                0, 0, 0, 0, place)
            assert st == 0
            assert hip.tsp_device_sync() == 0
            out = np.zeros_like(Cz)
            assert hip.tsp_memcpy_d2h(out.ctypes.data_as(C.c_void_p), bufs["C"], out.nbytes) == 0
            outs.append(out)
        # an unknown placement is rejected before any launch
        assert hip.tsp_spmm_launch_placed(16, 0, len(rows), cbp, bufs["val"], None, None, bufs["rows"], bufs["cs"],
                                          bufs["B"], bufs["C"], bufs["col"], A.rows, None, 0, 0, 0, 0, 2) != 0
    finally:
        for p in bufs.values():
            hip.tsp_free(p)
    Cref, Cabs = reference(orc, A, B, colB)
    for place, out in zip(("switch", "contiguous", "interleaved"), outs):
        assert_close(out[:, :colB], Cref, Cabs, 0, f"direct v16 {place}")


def test_split_tasks_in_any_order(gpu, orc):
    """A split task (bit 31) is added atomically whatever the order of the
    schedule, as in the reference: every row-block is cut in two pieces, all
    first pieces come before all second pieces (tiles laid out in task
    order), and tsp_switch_v8 / tsp_spmm_launch_placed (one task per wave)
    still match the oracle."""
    tsp = gpu
    hip, _ = tsp.load()
    rng = np.random.default_rng(12)
    A = random_matrix(tsp, rng, 200, 400, 40, 0)
    colB = 64
    B, cbp = random_b(tsp, rng, A.cols, colB, 0)
    sub = tsp.Csr(A.rows, A.cols, A.rowptr, A.colidx, A.val, 0)
    sub.orig_row = np.arange(A.rows, dtype=np.int32)
    t = tsp.tile_create(sub, A.cols, 8, 0)
    arr = t.arrays()
    tp, orig, bn = arr["tile_ptr"], arr["orig_tile_row_idx"], 16
    first, second = [], []
    for rb in range(len(tp) - 1):
        t0, t1 = int(tp[rb]), int(tp[rb + 1])
        if t1 - t0 >= 2:
            mid = (t0 + t1) // 2
            first.append((rb, t0, mid, True))
            second.append((rb, mid, t1, True))
        elif t1 > t0:
            first.append((rb, t0, t1, False))
    tasks = first + second
    assert sum(sp for *_, sp in tasks) >= 20
    perm = np.concatenate([np.arange(a, b) for _, a, b, _ in tasks])
    rows = np.array([int(orig[rb]) | (0x80000000 if sp else 0) for rb, _, _, sp in tasks], dtype=np.uint32)
    cs = np.concatenate([[0], np.cumsum([b - a for _, a, b, _ in tasks])]).astype(np.int32)
    val = arr["dense"].reshape(t.tilenum, 8 * bn)[perm]
    col = arr["tile_colidx"].reshape(t.tilenum, bn)[perm]
    bufs = {}

    def up(name, a):
        a = np.ascontiguousarray(a)
        p = C.c_void_p()
        assert hip.tsp_malloc(C.byref(p), max(a.nbytes, 4)) == 0
        assert hip.tsp_memcpy_h2d(p, a.ctypes.data_as(C.c_void_p), a.nbytes) == 0
        bufs[name] = p

    outs = []
    try:
        up("val", val); up("col", col); up("rows", rows); up("cs", cs); up("B", B)
        Cz = np.zeros((A.rows, cbp), dtype=np.float32)
        up("C", Cz)
        for place in (None, 0, 1):
            say(f"split tasks in any order: placement {place}")
            assert hip.tsp_memcpy_h2d(bufs["C"], Cz.ctypes.data_as(C.c_void_p), Cz.nbytes) == 0
            if place is None:
                st = hip.tsp_switch_v8(0, len(rows), cbp, bufs["val"], bufs["rows"], bufs["cs"], bufs["B"],
                                       bufs["C"], bufs["col"], A.rows, None)
            else:
                st = hip.tsp_spmm_launch_placed(8, 0, len(rows), cbp, bufs["val"], None, None, bufs["rows"],
                                                bufs["cs"], bufs["B"], bufs["C"], bufs["col"], A.rows, None,
                                                0, 0, 1, 0, place)
            assert st == 0
            assert hip.tsp_device_sync() == 0
            out = np.zeros_like(Cz)
            assert hip.tsp_memcpy_d2h(out.ctypes.data_as(C.c_void_p), bufs["C"], out.nbytes) == 0
            outs.append(out)
    finally:
        for p in bufs.values():
            hip.tsp_free(p)
    Cref, Cabs = reference(orc, A, B, colB)
    for place, out in zip(("switch", "contiguous", "interleaved"), outs):
        assert_close(out[:, :colB], Cref, Cabs, 0, f"split tasks in any order, {place}")


def test_edge_shapes(gpu, orc):
    tsp = gpu
    rng = np.random.default_rng(9)
    for rows, cols, maxlen in [(1, 1, 1), (7, 3, 3), (65, 1000, 0), (129, 17, 17), (1000, 5, 5)]:
        for prec in (0, 1):
            A = random_matrix(tsp, rng, rows, cols, maxlen, prec, empty_frac=0.3)
            B, cbp = random_b(tsp, rng, cols, 32, prec)
            Cref, Cabs = reference(orc, A, B, 32)
            for g, d in [(2.0, 1.5), (0.0, 1.5), (5.0, 0.0), (5.0, 3.0)]:
                say(f"edge rows={rows} cols={cols} prec={prec} g={g} d={d}")
                Cg, _ = run_tiles(tsp, A, B, cbp, g, d, th=(8, 8, 8))
                assert_close(Cg[:, :32], Cref, Cabs, prec, f"edge {rows}x{cols}")


def test_tuned_plan_and_determinism(gpu, orc):
    tsp = gpu
    A, B, colB, cbp = tsp.gen_config(1)
    Cref, Cabs = reference(orc, A, B, colB)
    C1, _ = run_tiles(tsp, A, B, cbp, 2.0, 1.5, tune=True)
    assert_close(C1[:, :colB], Cref, Cabs, 0, "C1 tuned")
    C2, _ = run_tiles(tsp, A, B, cbp, 2.0, 1.5, th=(128, 128, 128))
    # no split tasks at TH=128 here -> plain stores -> bit-identical reruns
    C3, _ = run_tiles(tsp, A, B, cbp, 2.0, 1.5, th=(128, 128, 128))
    assert np.array_equal(C2, C3)


def test_time_ex_reports_host_submission(gpu):
    """tsp_plan_time_ex: the event time per step and the host's submission
    time per step, both positive; the host cannot finish submitting much
    later than the GPU finishes running what it submitted, and a step's
    submission stays within a launch's few microseconds (the plan adds no
    host work of its own per step)."""
    tsp = gpu
    A, B, colB, cbp = tsp.gen_config(1)
    subs = tsp.matrix_split(A, 5.0, 3.0)
    tiles = [tsp.tile_create(s, A.cols, b, 0) for s, b in zip(subs, (64, 16, 8))]
    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, 0, B)
    try:
        plan.set_th(8, 8, 8)
        plan.run(zero_c=True)
        ms, sub = plan.time_ex(500)
        assert plan.time(10) > 0
        say(f"C1 step {ms * 1e3:.2f} us, host submission {sub * 1e3:.2f} us")
        assert ms > 0 and sub > 0
        assert sub < 1.5 * ms + 0.002
        assert sub < 0.05
    finally:
        plan.close()


@pytest.mark.parametrize("config", [2, 3])
def test_config_full_parity(gpu, orc, config):
    tsp = gpu
    say(f"config {config}: generating")
    A, B, colB, cbp = tsp.gen_config(config)
    Cref, Cabs = reference(orc, A, B, colB)
    g, d = tsp.predict(tsp.features(A, 9.5, colB), A.prec)
    for gd in [(g, d), (1.0, 1.0), (5.0, 3.0)]:
        say(f"config {config}: gamma/delta {gd}")
        Cg, _ = run_tiles(tsp, A, B, cbp, *gd, tune=True)
        assert_close(Cg[:, :colB], Cref, Cabs, A.prec, f"config {config} {gd}")


@pytest.mark.parametrize("config,prec,colB", [(4, -1, -1), (5, -1, -1), (3, 0, 128), (5, 0, 128)])
def test_config_sampled_rows(gpu, orc, config, prec, colB):
    """Large configurations: full GPU run with the runtime tuning (the variant
    the bench ships), oracle on a row sample that includes the heaviest rows
    and a uniform stride, and the row-sum and column-sum identities over all
    of C."""
    tsp = gpu
    say(f"config {config} prec {prec} colB {colB}: generating")
    A, B, colB, cbp = tsp.gen_config(config, prec, colB)
    g, d = tsp.predict(tsp.features(A, 9.5, colB), A.prec)
    say(f"config {config}: split+tiles+run gamma={g} delta={d}")
    Cg, _ = run_tiles(tsp, A, B, cbp, g, d, tune=True)
    lens = np.diff(A.rowptr)
    rows = np.unique(np.concatenate([np.argsort(lens)[-64:], np.arange(0, A.rows, max(1, A.rows // 3000))]))
    Cref, Cabs = reference(orc, A, B, colB, rows)
    assert_close(Cg[rows, :colB], Cref, Cabs, A.prec, f"config {config} sampled")
    say(f"config {config}: row and column sums over all of C")
    assert_checksums(orc, A, B, colB, Cg, f"config {config}")


def skewed_matrix(tsp, rng, rows, cols, maxlen, prec):
    """Rows of random length whose columns follow an RMAT-like marginal:
    each bit of the column index is set with probability 0.24, so columns
    with few set bits are gathered far more often than the rest."""
    bits = int(np.log2(cols))
    lens = rng.integers(0, maxlen + 1, rows)
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ci = []
    for ln in lens:
        draw = (rng.random((4 * int(ln) + 8, bits)) < 0.24).astype(np.int64) @ (1 << np.arange(bits))
        ci.append(np.unique(draw)[: int(ln)])
    lens = np.array([len(c) for c in ci])
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ci = np.concatenate(ci).astype(np.int32)
    v = rng.uniform(-1, 1, rp[-1]).astype(np.float32)
    val = v.astype(np.float16).view(np.uint16) if prec == 0 else v
    return tsp.Csr(rows, cols, rp, ci, val, prec)


@pytest.mark.parametrize("prec", [0, 1])
def test_hot_rows_bit_identical(gpu, orc, prec):
    """Hot B rows (copies of the most-gathered rows in spare rows of B) leave
    C bit-identical to the plan without them: the kernels multiply the same
    values in the same order.  Budgets change in sequence, so slot indices of
    one selection are decoded before the next is applied; one plan has every
    class (fork/join path), one a single class; B changes between steps."""
    tsp = gpu
    rng = np.random.default_rng(77 + prec)
    A = skewed_matrix(tsp, rng, 3000, 4096, 60, prec)
    for colB in (32, 128):
        B, cbp = random_b(tsp, rng, A.cols, colB, prec)
        Cref, Cabs = reference(orc, A, B, colB)
        unsplit = (1 << 20,) * 3        # no split tasks: no atomics, so C is reproducible bit for bit
        for g, d in [(2.0, 1.5), (5.0, 3.0)]:
            base, _ = run_tiles(tsp, A, B, cbp, g, d, unsplit)
            assert_close(base[:, :colB], Cref, Cabs, prec, f"no hot rows colB={colB} g={g}")
            subs = tsp.matrix_split(A, g, d)
            tiles = [tsp.tile_create(s, A.cols, bm, A.prec) for s, bm in zip(subs, (64, 16, 8))]
            plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, A.prec, B)
            try:
                rb = cbp * (2 if prec == 0 else 4)
                for budget in (rb, 4096, 1 << 20, 0, 32 << 20, 64 * rb):
                    say(f"hot rows prec={prec} colB={colB} g={g} d={d} budget={budget}")
                    plan.set_th(*unsplit)
                    plan.set_hot_rows(budget)
                    n, nb = plan.get_hot_rows()
                    assert nb == n * rb and nb <= max(budget, 0) and (budget == 0) == (n == 0)
                    plan.run(zero_c=True)
                    Cg = plan.download_c()
                    assert np.array_equal(Cg.view(np.uint32), base.view(np.uint32)), f"budget {budget}"
                    # hot rows are re-copied every step
                    plan.time(3)
                    plan.run(zero_c=True)
                    assert np.array_equal(plan.download_c().view(np.uint32), base.view(np.uint32))
                    # split tasks (atomic flushes) read the same slots
                    plan.set_th(8, 8, 8)
                    plan.run(zero_c=True)
                    assert_close(plan.download_c()[:, :colB], Cref, Cabs, prec, f"split, budget {budget}")
            finally:
                plan.close()


@pytest.mark.parametrize("prec", [0, 1])
def test_graph_replay_matches_eager_steps(gpu, orc, prec):
    """Steps replayed from a HIP graph (tsp_plan_graph_*) give the eager
    step's C bit for bit (unsplit schedule: plain stores), replay after
    replay with eager work in between: every class (fork/join across the
    class streams), hot B rows re-copied inside each step, and a dense class
    on the panel-synchronised sweep.  A configuration change makes the graph
    stale until it is captured again; split tasks stay within tolerance."""
    tsp = gpu
    hip, host = tsp.load()
    rng = np.random.default_rng(88 + prec)
    A = skewed_matrix(tsp, rng, 3000, 4096, 60, prec)
    colB = 128
    B, cbp = random_b(tsp, rng, A.cols, colB, prec)
    Cref, Cabs = reference(orc, A, B, colB)
    subs = tsp.matrix_split(A, 1.0, 1.0)
    assert all(s.rows > 0 for s in subs)
    tiles = [tsp.tile_create(s, A.cols, bm, A.prec) for s, bm in zip(subs, (64, 16, 8))]
    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, A.prec, B)
    dc = C.c_void_p()
    assert host.tsp_plan_device_c(plan.p, C.byref(dc)) == 0
    cbytes = A.rows * cbp * 4
    try:
        unsplit = (1 << 20,) * 3
        cases = [("default", lambda: None),
                 ("hot rows", lambda: plan.set_hot_rows(1 << 20)),
                 ("panel sweep", lambda: (plan.set_format(16, 1), plan.set_panels(16, 256, 2)))]
        if prec == 1:
            # B in the 3-byte form for the 64- and 8-row classes (the 16-row
            # class stays on the panel sweep, which reads 4-byte rows): each
            # step re-copies the hot rows into the spare rows of both forms
            def b3_setup():
                for bm in (64, 16, 8):
                    plan.set_b_3byte(bm, True)
                assert [plan.get_b_3byte(bm) for bm in (64, 16, 8)] == [1, 0, 1]
                assert plan.get_hot_rows()[0] > 0
            cases.append(("3-byte B rows", b3_setup))
        for label, setup in cases:
            say(f"graph replay prec={prec}: {label}")
            plan.set_th(*unsplit)
            setup()
            plan.run(zero_c=True)
            eager = plan.download_c()
            assert_close(eager[:, :colB], Cref, Cabs, prec, label)
            plan.graph_capture(3)
            for rnd in range(3):
                assert hip.tsp_memset(dc, 0, cbytes) == 0
                plan.graph_run(1 + rnd)
                assert hip.tsp_device_sync() == 0
                got = plan.download_c()
                assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), (label, rnd)
                plan.run(zero_c=True)             # eager work between replays
                plan.time(2)
            assert plan.graph_time(2) > 0
            # a configuration change makes the captured graph stale
            plan.set_th(*unsplit)
            with pytest.raises(tsp.TspError):
                plan.graph_run(1)
        # split tasks (atomic flushes): one zeroed replay of one step
        plan.set_th(8, 8, 8)
        plan.graph_capture(1)
        assert hip.tsp_memset(dc, 0, cbytes) == 0
        plan.graph_run(1)
        assert hip.tsp_device_sync() == 0
        assert_close(plan.download_c()[:, :colB], Cref, Cabs, prec, "split tasks, graph")
        plan.graph_free()
        with pytest.raises(tsp.TspError):
            plan.graph_run(1)
    finally:
        plan.close()


def test_hot_row_device_helpers(gpu):
    """tsp_colidx_count / tsp_colidx_remap / tsp_hot_rows_gather against numpy."""
    tsp = gpu
    hip = tsp.load()[0]
    rng = np.random.default_rng(5)
    colA, n, rb = 1000, 50000, 48
    ci = (rng.pareto(1.2, n) * 20).astype(np.int64) % colA
    ci = ci.astype(np.int32)
    hot = np.sort(rng.choice(colA, 37, replace=False)).astype(np.int32)
    mp = np.arange(colA, dtype=np.int32)
    mp[hot] = colA + np.arange(len(hot), dtype=np.int32)
    Bh = rng.integers(0, 2 ** 32, (colA + len(hot)) * rb // 4, dtype=np.uint64).astype(np.uint32)
    bufs = {k: tsp._DevBuf(v) for k, v in
            dict(ci=ci, hot=hot, mp=mp, cnt=np.zeros(colA, np.uint32), B=Bh).items()}
    try:
        P = lambda k: bufs[k].p
        get = lambda k, m, dt: tsp._d2h(bufs[k].p, m, dt)
        assert hip.tsp_colidx_count(P("ci"), n, colA, None, 0, P("cnt"), None) == 0
        assert hip.tsp_device_sync() == 0
        assert np.array_equal(get("cnt", colA, np.uint32), np.bincount(ci, minlength=colA))
        assert hip.tsp_colidx_remap(P("ci"), n, colA, None, 0, P("mp"), None) == 0
        assert hip.tsp_device_sync() == 0
        assert np.array_equal(get("ci", n, np.int32), mp[ci])
        # counting decodes remapped entries
        hip.tsp_memset(P("cnt"), 0, colA * 4)
        assert hip.tsp_colidx_count(P("ci"), n, colA, P("hot"), len(hot), P("cnt"), None) == 0
        assert hip.tsp_device_sync() == 0
        assert np.array_equal(get("cnt", colA, np.uint32), np.bincount(ci, minlength=colA))
        assert hip.tsp_colidx_remap(P("ci"), n, colA, P("hot"), len(hot), None, None) == 0
        assert hip.tsp_device_sync() == 0
        assert np.array_equal(get("ci", n, np.int32), ci)
        assert hip.tsp_hot_rows_gather(P("B"), colA, rb, P("hot"), len(hot), None) == 0
        assert hip.tsp_device_sync() == 0
        got = get("B", Bh.size, np.uint32).reshape(colA + len(hot), rb // 4)
        want = Bh.reshape(colA + len(hot), rb // 4).copy()
        want[colA:] = want[hot]
        assert np.array_equal(got, want)
        assert hip.tsp_hot_rows_gather(P("B"), colA, 40, P("hot"), len(hot), None) != 0   # not 16-byte rows
    finally:
        for b in bufs.values():
            b.free()


def test_tf32_raw_fp32_inputs_error_bound(gpu, orc):
    """fp32 inputs that are NOT tf32 values.  The kernels round both operands
    to tf32 (nearest-even, relative error <= 2^-11 each), so against the fp64
    product of the UNROUNDED inputs every entry is within
    (2 * 2^-11 + 2^-22 + fp32 accumulation) of sum |A||B|: bounded here by
    1.0e-3, and checked to be above the exact-input tolerance (the rounding
    really happens).  The reference instead hands raw fp32 bits to tf32
    tensor cores (src/utils.h:233-246), which ignore the low 13 bits, so its
    per-operand error reaches 2^-10.  Against the oracle on tf32-rounded
    inputs the result stays within the 1e-4 tf32 tolerance."""
    tsp = gpu
    rng = np.random.default_rng(2024)
    A = random_matrix(tsp, rng, 600, 500, 50, 1, heavy_rows=3)
    A.val = (rng.uniform(-1, 1, A.nnz) * (1 + rng.random(A.nnz) * 2 ** -12)).astype(np.float32)
    assert ((A.val.view(np.uint32) & 0x1FFF) != 0).mean() > 0.99
    colB = 64
    B, cbp = random_b(tsp, rng, A.cols, colB, 1)
    B[:, :colB] = (B[:, :colB] * (1 + rng.random((A.cols, colB)) * 2 ** -12)).astype(np.float32)
    Cg, _ = run_tiles(tsp, A, B, cbp, 2.0, 1.5, (16, 16, 16))
    a = A.val.astype(np.float64)
    b = B[:, :colB].astype(np.float64)
    Craw = orc.spmm_f64(A.rows, A.rowptr, A.colidx, a, b, colB)
    Cabs = orc.spmm_f64(A.rows, A.rowptr, A.colidx, np.abs(a), np.abs(b), colB)
    err = np.abs(Cg[:, :colB] - Craw) / (Cabs + 1e-30)
    say(f"tf32 on raw fp32 inputs: max normalised error {err.max():.3e}")
    assert err.max() <= 1.0e-3
    assert err.max() > 1e-4
    Cref, Cabs_r = reference(orc, A, B, colB)
    assert_close(Cg[:, :colB], Cref, Cabs_r, 1, "tf32 vs oracle on rounded inputs")


@pytest.mark.parametrize("prec", [0, 1])
def test_nan_and_inf_propagate(gpu, prec):
    """Non-finite operands propagate as through the reference's raw operands;
    NaN payloads that a rounding bias would carry into the exponent or sign
    (0x7f800001, 0x7fffffff) stay NaN in the tf32 path.
    * A NaN in A reaches exactly its own row of C (every column).
    * A NaN / +Inf in B row c, column j reaches C[r, j] of every row r whose
      CSR row holds c (NaN / +Inf with positive operands) -- and, because the
      tiles are dense zero-padded blocks (as the reference's are), also
      C[r', j] of the other rows r' of those row-blocks as NaN (0 * Inf and
      0 * NaN are NaN).  Every other entry stays finite."""
    tsp = gpu
    rng = np.random.default_rng(9)
    rows, cols, colB = 256, 128, 64
    lens = np.full(rows, 4)
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ci = np.concatenate([np.sort(rng.choice(cols, 4, replace=False)) for _ in range(rows)]).astype(np.int32)
    v = rng.uniform(0.5, 1, rp[-1]).astype(np.float32)
    bv = rng.uniform(0.5, 1, (cols, colB)).astype(np.float32)
    if prec == 0:
        val = v.astype(np.float16).view(np.uint16)
        B = bv.astype(np.float16).view(np.uint16)
        nan_a, nan_b, inf_b = np.uint16(0x7E01), np.uint16(0x7C01), np.uint16(0x7C00)
    else:
        val = v.copy()
        B = bv.copy()
        nan_a, nan_b, inf_b = np.uint32(0x7FFFFFFF), np.uint32(0x7F800001), np.uint32(0x7F800000)
    vb = val.view(np.uint16 if prec == 0 else np.uint32)
    Bb = B.view(np.uint16 if prec == 0 else np.uint32)
    vb[rp[10] + 1] = nan_a                 # row 10
    cnan, cinf = 77, 91
    Bb[cnan, 5] = nan_b
    Bb[cinf, 9] = inf_b
    A = tsp.Csr(rows, cols, rp, ci, val, prec)
    for th in ((8, 8, 8), (128, 128, 128)):
        Cg, _ = run_tiles(tsp, A, B, colB, 2.0, 1.5, th)
        C = Cg[:, :colB]
        has = lambda c: np.array([c in ci[rp[r]:rp[r + 1]] for r in range(rows)])
        other = np.ones(rows, bool)
        other[10] = False
        assert np.isnan(C[10]).all()
        assert np.isnan(C[has(cnan) & other, 5]).all()
        assert np.isposinf(C[has(cinf) & other, 9]).all()
        # rows of C other than 10 are finite outside columns 5 and 9, and
        # columns 5 / 9 hold no Inf / NaN of the wrong kind
        rest = np.delete(np.arange(colB), [5, 9])
        assert np.isfinite(C[other][:, rest]).all()
        assert not np.isinf(C[other, 5]).any()
        assert not np.isneginf(C[other, 9]).any()


@pytest.mark.parametrize("bm", [64, 16, 8])
def test_tf32_prerounded_launch_matches_rounding_launch(gpu, orc, bm):
    """The plan rounds its copies of A and B to tf32 once and launches with
    TSP_LAUNCH_OPERANDS_TF32 (no per-operand rounding in the kernel); the
    reference-compatible launch (tsp_switch_v*) rounds in the kernel.  On raw
    fp32 inputs, NaN included, both give the same C bit for bit (unsplit
    schedule: no atomics), and tsp_round_tf32_device equals the host
    rounding.  The same holds for the packed format with lane-loaded column
    indices (whose 64-column kernels take their B operands straight from
    the gathered registers), rounding or pre-rounded."""
    tsp = gpu
    hip, _ = tsp.load()
    rng = np.random.default_rng(40 + bm)
    A = random_matrix(tsp, rng, 3 * bm + 5, 400, 40, 1)
    A.val = (rng.uniform(-1, 1, A.nnz) * (1 + rng.random(A.nnz) * 2 ** -12)).astype(np.float32)
    A.val.view(np.uint32)[3] = 0x7FFFFFFF                                   # NaN whose rounding would carry
    colB = 64
    B, cbp = random_b(tsp, rng, A.cols, colB, 1)
    B[:, :colB] = (B[:, :colB] * (1 + rng.random((A.cols, colB)) * 2 ** -12)).astype(np.float32)
    sub = tsp.Csr(A.rows, A.cols, A.rowptr, A.colidx, A.val, 1)
    sub.orig_row = np.arange(A.rows, dtype=np.int32)
    t = tsp.tile_create(sub, A.cols, bm, 1)
    arr = t.arrays()
    rows, cs = tsp.pretreatment(t, 1 << 20)
    assert not (rows & 0x80000000).any()
    bufs = {}

    def up(name, a):
        p = C.c_void_p()
        assert hip.tsp_malloc(C.byref(p), max(a.nbytes, 4)) == 0
        assert hip.tsp_memcpy_h2d(p, a.ctypes.data_as(C.c_void_p), a.nbytes) == 0
        bufs[name] = p
        return p

    def down(name, like):
        out = np.zeros_like(like)
        assert hip.tsp_memcpy_d2h(out.ctypes.data_as(C.c_void_p), bufs[name], out.nbytes) == 0
        return out

    switch = {64: hip.tsp_switch_v64, 16: hip.tsp_switch_v16, 8: hip.tsp_switch_v8}[bm]
    try:
        dense = np.ascontiguousarray(arr["dense"]).view(np.float32)
        up("val", dense); up("col", arr["tile_colidx"]); up("rows", rows); up("cs", cs); up("B", B)
        up("valr", dense); up("Br", B)
        Cz = np.zeros((A.rows, cbp), dtype=np.float32)
        up("C1", Cz); up("C2", Cz)
        assert switch(1, len(rows), cbp, bufs["val"], bufs["rows"], bufs["cs"], bufs["B"], bufs["C1"], bufs["col"],
                      A.rows, None) == 0
        assert hip.tsp_round_tf32_device(bufs["valr"], dense.size, None) == 0
        assert hip.tsp_round_tf32_device(bufs["Br"], B.size, None) == 0
        assert hip.tsp_device_sync() == 0
        host_r = np.zeros(dense.size, np.uint32)
        assert hip.tsp_round_tf32_bits(dense.ctypes.data_as(C.c_void_p), host_r.ctypes.data_as(C.c_void_p),
                                       dense.size) == 0
        assert np.array_equal(down("valr", dense).view(np.uint32).reshape(-1), host_r)
        assert hip.tsp_spmm_launch_ex(bm, 1, len(rows), cbp, bufs["valr"], None, None, bufs["rows"], bufs["cs"],
                                      bufs["Br"], bufs["C2"], bufs["col"], A.rows, None, 0, 0, 0, 0, 0, 1) == 0
        assert hip.tsp_device_sync() == 0
        c1, c2 = down("C1", Cz), down("C2", Cz)
        assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))
        row3 = int(np.searchsorted(A.rowptr, 3, side="right") - 1)
        assert np.isnan(c1[row3, :colB]).all()
        ok = np.ones(A.rows, bool)
        ok[row3] = False
        Cref, Cabs = reference(orc, A, B, colB)
        assert_close(c1[ok, :colB], Cref[ok], Cabs[ok], 1, f"bm {bm}")
        # an unknown flag is refused before any launch, and so are lane-loaded
        # indices where no kernel has them (64-row tiles)
        assert hip.tsp_spmm_launch_ex(bm, 1, len(rows), cbp, bufs["valr"], None, None, bufs["rows"], bufs["cs"],
                                      bufs["Br"], bufs["C2"], bufs["col"], A.rows, None, 0, 0, 0, 0, 0, 64) != 0
        li = hip.tsp_spmm_launch_ex(bm, 1, len(rows), cbp, bufs["valr"], None, None, bufs["rows"], bufs["cs"],
                                    bufs["Br"], bufs["C2"], bufs["col"], A.rows, None, 0, 0, 0, 0, 0, 3)
        if bm == 64:
            assert li != 0
        else:
            # dense tiles with lane-loaded indices: the same result bit for bit
            assert li == 0 and hip.tsp_device_sync() == 0
            assert np.array_equal(down("C2", Cz).view(np.uint32), c1.view(np.uint32))
        # TSP_LAUNCH_SKIP_ZERO_STORES (16): exact-zero results are not stored,
        # so a C full of garbage keeps it exactly there (NaN is stored)
        junk = np.full_like(Cz, 0).view(np.uint32)
        junk[:] = 0x7f7f7f7f
        up("C3", junk.view(np.float32))
        assert hip.tsp_spmm_launch_ex(bm, 1, len(rows), cbp, bufs["valr"], None, None, bufs["rows"], bufs["cs"],
                                      bufs["Br"], bufs["C3"], bufs["col"], A.rows, None, 0, 0, 0, 0, 0, 1 | 16) == 0
        assert hip.tsp_device_sync() == 0
        c3 = down("C3", Cz).view(np.uint32)
        zero = c1.view(np.uint32) == 0
        assert (~zero).any()
        assert (c3[zero] == 0x7f7f7f7f).all() and np.array_equal(c3[~zero], c1.view(np.uint32)[~zero])
        if bm != 64:
            # packed A with lane-loaded indices and 64-column chunks (the
            # gathered B registers are the MFMA operands, no LDS panel): the
            # rounding launch on the raw values and the pre-rounded launch
            # both equal the dense rounding launch bit for bit
            bn = tsp.tile_bn(bm, 1)
            up("bmp", np.ascontiguousarray(arr["bitmap"]))
            for src, flags, cname in (("val", 2, "C3"), ("valr", 3, "C4")):
                nv = C.c_longlong()
                pv, vp = C.c_void_p(), C.c_void_p()
                assert hip.tsp_tiles_pack_device(t.tilenum, bm, bn, 1, bufs[src], bufs["bmp"], C.byref(nv),
                                                 C.byref(pv), C.byref(vp), None) == 0
                bufs[src + "_pv"], bufs[src + "_vp"] = pv, vp
                up(cname, Cz)
                for s in (1, 2, 3):
                    say(f"packed tf32 lane indices bm={bm} flags={flags} stages={s}")
                    assert hip.tsp_spmm_launch_ex(bm, 1, len(rows), cbp, pv, bufs["bmp"], vp, bufs["rows"],
                                                  bufs["cs"], bufs["B" if src == "val" else "Br"], bufs[cname],
                                                  bufs["col"], A.rows, None, 64, s, 0, 0, 0, flags) == 0
                    assert hip.tsp_device_sync() == 0
                    c = down(cname, Cz)
                    assert np.array_equal(c.view(np.uint32), c1.view(np.uint32)), (flags, s)
    finally:
        for p in bufs.values():
            hip.tsp_free(p)


def same_bits_or_nan(a, b):
    """Equal bit for bit, except that NaN equals NaN whatever its payload."""
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb])


@pytest.mark.parametrize("colB", [64, 128, 256])
@pytest.mark.parametrize("bm", [64, 16, 8])
def test_b_3byte_launch_matches_4byte_launch(gpu, orc, bm, colB):
    """TSP_LAUNCH_B_3BYTE: B's tf32 values as the top 3 bytes of their fp32
    words (tsp_pack_3byte_device, equal byte for byte to the host packing)
    give the C of the 4-byte launch of the same operands bit for bit, for
    every variant the 4-byte form has (chunk widths 32-256 -- 64 gathers
    into the MFMA operands, the others widen into the LDS panel -- dense
    and packed A, depth 1-3, scalar and lane-loaded indices), with later
    column chunks at 3-byte offsets.  An Inf and a NaN whose payload lies
    only in the dropped low byte (it becomes a quiet NaN) reach the same
    rows of C as NaN / Inf.  Tile pairs, the panel sweep, fp16 and operands
    not declared tf32 refuse the form."""
    tsp = gpu
    hip, _ = tsp.load()
    rng = np.random.default_rng(90 + bm + colB)
    A = random_matrix(tsp, rng, 3 * bm + 5, 400, 40, 1)
    B, cbp = random_b(tsp, rng, A.cols, colB, 1)
    nan_row, inf_row = int(A.colidx[0]), int(A.colidx[A.nnz // 2])
    if inf_row == nan_row:
        inf_row = int(A.colidx[-1])
    Bu = B.view(np.uint32)
    Bu[nan_row, 3] = 0x7f800001
    Bu[inf_row, 5] = 0x7f800000
    sub = tsp.Csr(A.rows, A.cols, A.rowptr, A.colidx, A.val, 1)
    sub.orig_row = np.arange(A.rows, dtype=np.int32)
    t = tsp.tile_create(sub, A.cols, bm, 1)
    arr = t.arrays()
    rows, cs = tsp.pretreatment(t, 1 << 20)
    assert not (rows & 0x80000000).any()
    bufs = {}

    def alloc(name, nbytes):
        p = C.c_void_p()
        assert hip.tsp_malloc(C.byref(p), max(nbytes, 4)) == 0
        bufs[name] = p
        return p

    def up(name, a):
        p = alloc(name, a.nbytes)
        assert hip.tsp_memcpy_h2d(p, a.ctypes.data_as(C.c_void_p), a.nbytes) == 0
        return p

    def down(name, like):
        out = np.zeros_like(like)
        assert hip.tsp_memcpy_d2h(out.ctypes.data_as(C.c_void_p), bufs[name], out.nbytes) == 0
        return out

    try:
        dense = np.ascontiguousarray(arr["dense"]).view(np.float32)
        up("val", dense); up("col", arr["tile_colidx"]); up("rows", rows); up("cs", cs); up("B", B)
        assert hip.tsp_round_tf32_device(bufs["val"], dense.size, None) == 0
        assert hip.tsp_round_tf32_device(bufs["B"], B.size, None) == 0
        alloc("B3", B.size * 3)
        assert hip.tsp_pack_3byte_device(bufs["B"], bufs["B3"], B.size, None) == 0
        assert hip.tsp_device_sync() == 0
        Br = down("B", B)
        host3 = np.zeros(B.size * 3, np.uint8)
        assert hip.tsp_pack_3byte_bits(Br.ctypes.data_as(C.c_void_p), host3.ctypes.data_as(C.c_void_p), B.size) == 0
        assert np.array_equal(down("B3", host3), host3)
        Cz = np.zeros((A.rows, cbp), dtype=np.float32)
        alloc("C4", Cz.nbytes)
        alloc("C3", Cz.nbytes)
        variants = [(False, None, None)]
        if bm != 64:
            bn = tsp.tile_bn(bm, 1)
            up("bmp", np.ascontiguousarray(arr["bitmap"]))
            nv, pv, vp = C.c_longlong(), C.c_void_p(), C.c_void_p()
            assert hip.tsp_tiles_pack_device(t.tilenum, bm, bn, 1, bufs["val"], bufs["bmp"], C.byref(nv),
                                             C.byref(pv), C.byref(vp), None) == 0
            bufs["pv"], bufs["vp"] = pv, vp
            variants.append((True, pv, vp))

        def launch(cname, packed, pv, vp, b, s, flags, w=64):
            assert hip.tsp_memset(bufs[cname], 0, Cz.nbytes) == 0
            return hip.tsp_spmm_launch_ex(bm, 1, len(rows), cbp, pv if packed else bufs["val"],
                                          bufs["bmp"] if packed else None, vp if packed else None, bufs["rows"],
                                          bufs["cs"], b, bufs[cname], bufs["col"], A.rows, None, w, s, 0, 0, 0,
                                          flags)
        first = None
        ran = 0
        for w in (32, 64, 128, 256):
            if cbp % w:
                continue
            for packed, pv, vp in variants:
                for li in ((0, 2) if bm != 64 else (0,)):
                    for s in (1, 2, 3):
                        say(f"3-byte B bm={bm} colB={colB} w={w} packed={packed} lane indices={li} stages={s}")
                        st4 = launch("C4", packed, pv, vp, bufs["B"], s, 1 | li, w)
                        st3 = launch("C3", packed, pv, vp, bufs["B3"], s, 1 | li | 32, w)
                        assert (st3 == 0) == (st4 == 0), (w, packed, li, s, st4, st3)
                        if st4:
                            continue      # a variant neither form has
                        assert hip.tsp_device_sync() == 0
                        c4, c3 = down("C4", Cz), down("C3", Cz)
                        assert same_bits_or_nan(c3, c4), (w, packed, li, s)
                        first = c4 if first is None else first
                        ran += 1
        assert ran >= (6 if bm == 64 else 12)
        # the NaN and the Inf reached C, and every other entry is within
        # the tf32 tolerance of the fp64 reference (a tile multiplies its
        # zeros too, and 0 x NaN = 0 x Inf = NaN: every row of a row-block
        # with a tile on those columns is hit, as in the reference's tiles)
        assert np.isnan(first[:, 3]).any() and np.isinf(first).any()
        uses = np.array([np.isin(A.colidx[A.rowptr[r]:A.rowptr[r + 1]], (nan_row, inf_row)).any()
                         for r in range(A.rows)])
        hit = np.repeat(np.add.reduceat(uses, np.arange(0, A.rows, bm)) > 0, bm)[:A.rows]
        Bf = B.copy()
        Bf.view(np.uint32)[nan_row, 3] = 0
        Bf.view(np.uint32)[inf_row, 5] = 0
        Cref, Cabs = reference(orc, A, Bf, colB)
        assert_close(first[~hit, :colB], Cref[~hit], Cabs[~hit], 1, f"bm {bm}")
        # refused: the panel sweep, fp16, tile pairs, and operands not
        # declared tf32 -- all before any launch
        assert hip.tsp_spmm_launch_panels(bm, 1, len(rows), cbp, bufs["val"], None, None, bufs["rows"], bufs["cs"],
                                          bufs["B3"], bufs["C3"], bufs["col"], A.rows, None, 64, 1, 0, 0, 0, 1 | 32,
                                          A.cols, 256, 2, bufs["C4"], 1024) != 0
        assert launch("C3", False, None, None, bufs["B3"], 1, 32) != 0
        assert launch("C3", False, None, None, bufs["B3"], 1, 1 | 8 | 32) != 0
        assert hip.tsp_spmm_launch_ex(bm, 0, len(rows), cbp, bufs["val"], None, None, bufs["rows"], bufs["cs"],
                                      bufs["B3"], bufs["C3"], bufs["col"], A.rows, None, 64, 1, 0, 0, 0, 1 | 32) != 0
    finally:
        for p in bufs.values():
            hip.tsp_free(p)


def test_plan_b_3byte(gpu, orc):
    """A tf32 plan whose classes read B in the 3-byte form computes C bit for
    bit as with the 4-byte form -- with hot rows too, whose slots in the
    3-byte copy are refilled every step -- at any chunk width; with tile
    pairs the class reads the split form instead.  Split tasks (atomic
    flushes) stay within tolerance.  fp16 plans refuse the form."""
    tsp = gpu
    rng = np.random.default_rng(123)
    A = skewed_matrix(tsp, rng, 3000, 4096, 60, 1)
    unsplit = (1 << 20,) * 3
    for colB in (64, 128):
        B, cbp = random_b(tsp, rng, A.cols, colB, 1)
        Cref, Cabs = reference(orc, A, B, colB)
        subs = tsp.matrix_split(A, 2.0, 1.5)
        tiles = [tsp.tile_create(s, A.cols, bm, 1) for s, bm in zip(subs, (64, 16, 8))]
        active = [bm for t, bm in zip(tiles, (64, 16, 8)) if t.tilenum]
        assert len(active) == 3
        plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, 1, B)
        try:
            plan.set_th(*unsplit)
            for bm in active:
                plan.set_variant(bm, 64)
            plan.run(zero_c=True)
            base = plan.download_c()
            assert_close(base[:, :colB], Cref, Cabs, 1, f"4-byte B colB={colB}")
            for bm in active:
                assert plan.get_b_3byte(bm) == 0
                plan.set_b_3byte(bm, True)
                assert plan.get_b_3byte(bm) == 1
            for budget in (0, 1 << 20):
                say(f"plan 3-byte B colB={colB} hot budget={budget}")
                plan.set_hot_rows(budget)
                plan.run(zero_c=True)
                assert np.array_equal(plan.download_c().view(np.uint32), base.view(np.uint32)), budget
                plan.time(3)
                plan.run(zero_c=True)
                assert np.array_equal(plan.download_c().view(np.uint32), base.view(np.uint32)), budget
            for w in (32, 128):
                if cbp % w == 0:
                    plan.set_variant(8, w)
                    assert plan.get_b_3byte(8) == 1
                    plan.run(zero_c=True)
                    assert np.array_equal(plan.download_c().view(np.uint32), base.view(np.uint32)), w
            plan.set_variant(8, 64)
            plan.set_pairs(8, True)
            assert plan.get_b_3byte(8) == 0 and plan.get_pairs(8) == 1
            plan.run(zero_c=True)
            assert_close(plan.download_c()[:, :colB], Cref, Cabs, 1, f"tile pairs beside 3-byte B, colB={colB}")
            plan.set_pairs(8, False)
            assert plan.get_b_3byte(8) == 1
            plan.set_th(8, 8, 8)
            plan.run(zero_c=True)
            assert_close(plan.download_c()[:, :colB], Cref, Cabs, 1, f"3-byte B, split tasks, colB={colB}")
        finally:
            plan.close()
    Af = skewed_matrix(tsp, rng, 500, 1024, 20, 0)
    Bf, cbp = random_b(tsp, rng, Af.cols, 64, 0)
    subs = tsp.matrix_split(Af, 2.0, 1.5)
    tiles = [tsp.tile_create(s, Af.cols, bm, 0) for s, bm in zip(subs, (64, 16, 8))]
    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], Af.rows, Af.cols, cbp, 0, Bf)
    try:
        with pytest.raises(Exception):
            plan.set_b_3byte(8, True)
        assert plan.get_b_3byte(8) == 0
    finally:
        plan.close()


@pytest.mark.parametrize("prec", [0, 1])
def test_chunk_xcd_placement_chunk_counts(gpu, orc, prec):
    """One column chunk per XCD group with 2, 4 and 8 chunks (colB 64, 128,
    256 at 32-column chunks) for every class, split tasks included; a chunk
    count that does not divide the 8 XCDs (colB 192 at 64 columns: 3) is
    refused."""
    tsp = gpu
    rng = np.random.default_rng(70 + prec)
    A = random_matrix(tsp, rng, 900, 700, 40, prec, heavy_rows=4)
    for colB in (64, 128, 256, 192):
        B, cbp = random_b(tsp, rng, A.cols, colB, prec)
        Cref, Cabs = reference(orc, A, B, colB)
        subs = tsp.matrix_split(A, 2.0, 1.5)
        tiles = [tsp.tile_create(s, A.cols, b, prec) for s, b in zip(subs, (64, 16, 8))]
        plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
        try:
            plan.set_th(8, 8, 8)
            w = 64 if colB == 192 else 32
            for bm in (64, 16, 8):
                plan.set_variant(bm, w, 1, 1, 1)
                plan.set_placement(bm, 2)
            say(f"chunk-xcd prec={prec} colB={colB} w={w} chunks={cbp // w}")
            if cbp // w in (2, 4, 8):
                plan.run(zero_c=True)
                assert_close(plan.download_c()[:, :colB], Cref, Cabs, prec, f"colB {colB}")
            else:
                with pytest.raises(tsp.TspError):
                    plan.run(zero_c=True)
        finally:
            plan.close()


def test_cold_tune_mode(gpu, orc):
    """TSP_TUNE_COLD: the tuning times single launches after evicting L2 and
    the MALL; the tuned plan still gives the oracle's result, and the mode
    can be switched back (freeing the eviction buffer)."""
    tsp = gpu
    rng = np.random.default_rng(12)
    A = random_matrix(tsp, rng, 2000, 1500, 30, 0, heavy_rows=3)
    colB = 128
    B, cbp = random_b(tsp, rng, A.cols, colB, 0)
    Cref, Cabs = reference(orc, A, B, colB)
    subs = tsp.matrix_split(A, 2.0, 1.5)
    tiles = [tsp.tile_create(s, A.cols, b, 0) for s, b in zip(subs, (64, 16, 8))]
    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, 0, B)
    try:
        assert plan.get_tune_mode() == 0
        plan.set_tune_mode(True)
        assert plan.get_tune_mode() == 1
        plan.tune(True)
        plan.run(zero_c=True)
        assert_close(plan.download_c()[:, :colB], Cref, Cabs, 0, "cold-tuned plan")
        plan.set_tune_mode(False)
        assert plan.get_tune_mode() == 0
        plan.run(zero_c=True)
        assert_close(plan.download_c()[:, :colB], Cref, Cabs, 0, "after switching back")
    finally:
        plan.close()
