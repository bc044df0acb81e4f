"""GPU-side CSR -> tiles (tsp_tile_create_device) against the CPU oracle's
tile restatement and the host library's tsp_tile_create: every array
(tile_ptr, tile_colidx, tile_nnz, canonical values, occupancy bitmap) must be
bit-identical, including the per-add rounding of duplicate entries."""
import sys

import numpy as np
import pytest

from test_host_parity import random_csr, values_for

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def gpu(tsp):
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    return tsp


def assert_same(d, ref, prec, what):
    assert np.array_equal(d["tile_ptr"], ref["tile_ptr"]), f"{what}: tile_ptr"
    assert np.array_equal(d["tile_colidx"], ref["tile_colidx"]), f"{what}: tile_colidx"
    assert np.array_equal(d["tile_nnz"], ref["tile_nnz"]), f"{what}: tile_nnz"
    vt = np.uint16 if prec == 0 else np.uint32
    rv = np.asarray(ref["dense"])
    # host tile arrays hold float32 values for tf32 (compare their bits); the
    # oracle returns the bit patterns already
    rv = rv.view(vt) if rv.dtype.itemsize == np.dtype(vt).itemsize else rv.astype(vt)
    dv = d["dense"].view(vt)
    if not np.array_equal(dv, rv):
        i = int(np.argwhere(dv != rv)[0][0])
        pytest.fail(f"{what}: value bits differ at {i}: {dv[i]:#x} vs {rv[i]:#x}")
    assert np.array_equal(d["bitmap"], ref["bitmap"]), f"{what}: bitmap"


def check_vs_oracle(tsp, orc, rows, cols, rp, ci, prec, bm, store, bits, what):
    bn = tsp.tile_bn(bm, prec)
    sub = tsp.Csr(rows, cols, rp, ci, store, prec)
    say(f"device tiles vs oracle: {what} rows={rows} cols={cols} nnz={len(ci)} bm={bm} prec={prec}")
    d = tsp.tile_create_device(sub, cols, bm, prec)
    o = orc.tile_create(rows, cols, rp, ci, bits, prec, bm, bn)
    assert len(d["tile_ptr"]) == o["tilem"] + 1
    assert_same(d, o, prec, what)


@pytest.mark.parametrize("prec", [0, 1])
@pytest.mark.parametrize("bm", [64, 16, 8])
@pytest.mark.parametrize("seed", range(4))
def test_device_tiles_random(gpu, orc, prec, bm, seed):
    rng = np.random.default_rng(5000 + 100 * bm + 10 * seed + prec)
    rows = int(rng.integers(1, 700))          # ragged last row-block
    cols = int(rng.integers(1, 5000))
    rp, ci = random_csr(rng, rows, cols, int(rng.integers(1, 120)), dup=(seed >= 2), empty_frac=0.15 * seed)
    store, bits = values_for(rng, len(ci), prec)
    check_vs_oracle(gpu, orc, rows, cols, rp, ci, prec, bm, store, bits, f"random seed {seed}")


@pytest.mark.parametrize("prec", [0, 1])
def test_device_tiles_duplicate_rounding(gpu, orc, prec):
    # many entries on few slots, spread over 24 binades: the order and the
    # rounding of every add show in the result
    rng = np.random.default_rng(78)
    rows, cols = 70, 5
    rp, ci = random_csr(rng, rows, cols, 80, dup=True)
    v = (rng.uniform(-1, 1, len(ci)) * 2.0 ** rng.integers(-12, 12, len(ci))).astype(np.float32)
    if prec == 0:
        store = v.astype(np.float16).view(np.uint16)
        bits = store.astype(np.uint32)
    else:
        store, bits = v, v.view(np.uint32)
    for bm in (64, 16, 8):
        check_vs_oracle(gpu, orc, rows, cols, rp, ci, prec, bm, store, bits, "duplicates")


def test_device_tiles_edges(gpu, orc):
    # all rows empty; one row; one column; a row block wider than 32 tiles
    cases = []
    cases.append((100, 10, np.zeros(101, np.int32), np.zeros(0, np.int32)))
    cases.append((1, 7, np.array([0, 3], np.int32), np.array([6, 0, 3], np.int32)))
    cases.append((9, 1, np.arange(10, dtype=np.int32), np.zeros(9, np.int32)))
    wide = np.arange(2000, dtype=np.int32)[::-1].copy()
    cases.append((3, 4000, np.array([0, 0, 2000, 2000], np.int32), wide))
    rng = np.random.default_rng(3)
    for k, (rows, cols, rp, ci) in enumerate(cases):
        for prec in (0, 1):
            store, bits = values_for(rng, len(ci), prec)
            for bm in (64, 16, 8):
                check_vs_oracle(gpu, orc, rows, cols, rp, ci, prec, bm, store, bits, f"edge case {k}")


def test_device_tiles_dc2(gpu, orc, dc2_path):
    m, n, rp, ci, v, sym = orc.mm_read(dc2_path)
    for prec in (0, 1):
        if prec == 0:
            store = v.astype(np.float16).view(np.uint16)
            bits = store.astype(np.uint32)
        else:
            store = orc.round_tf32_array(v.astype(np.float32))
            bits = store.view(np.uint32)
        for bm in (64, 16, 8):
            check_vs_oracle(gpu, orc, m, n, rp, ci, prec, bm, store, bits, "dc2")


@pytest.mark.parametrize("config,prec", [(2, 0), (3, 1), (4, 0), (3, 0), (5, 0), (5, 1)])
def test_device_tiles_config_classes(gpu, config, prec):
    """Every class sub-CSR of a full synthetic config, split at the shipped
    policy's (gamma, delta): device tiles == host tiles (the host conversion
    is pinned against the oracle by the CPU tests)."""
    tsp = gpu
    A, B, colB, _ = tsp.gen_config(config, prec=prec)
    g, dl = tsp.predict(tsp.features(A, 9.5, colB), prec)
    del B
    subs = tsp.matrix_split(A, g, dl)
    for s, bm in zip(subs, (64, 16, 8)):
        if s.rows == 0:
            continue
        say(f"config {config} prec {prec} class {bm}: rows={s.rows} nnz={s.nnz}")
        h = tsp.tile_create(s, A.cols, bm, prec).arrays()
        d = tsp.tile_create_device(s, A.cols, bm, prec)
        assert_same(d, h, prec, f"config {config} class {bm}")


def test_device_tiles_rejects_out_of_range_column(gpu):
    # the fill kernel finds no slot for a column outside [0, colA): the call
    # reports TSP_EINVAL and frees its outputs
    rows, cols = 20, 64
    rp = np.arange(0, 41, 2, dtype=np.int32)
    ci = np.tile(np.array([3, 9], np.int32), 20)
    ci[17] = cols
    sub = gpu.Csr(rows, cols, rp, ci, np.ones(40, np.float32), 1)
    with pytest.raises(gpu.TspError) as e:
        gpu.tile_create_device(sub, cols, 16, 1)
    assert e.value.status == 1001


def plan_c(plan, th, fmt16=1, fmt8=1):
    plan.set_th(*th)
    plan.set_format(16, fmt16)
    plan.set_format(8, fmt8)
    plan.run(zero_c=True)
    return plan.download_c()


@pytest.mark.parametrize("config,prec", [(2, 0), (3, 1)])
def test_plan_from_csr_matches_host_tiles(gpu, config, prec):
    """A plan whose tiles were built on the device computes the same C, bit
    for bit, as a plan over the host library's tiles (same thresholds and A
    format, no split tasks so no atomics), in the dense and the device-packed
    format."""
    tsp = gpu
    A, B, colB, cbp = tsp.gen_config(config, prec=prec)
    g, dl = tsp.predict(tsp.features(A, 9.5, colB), prec)
    subs = tsp.matrix_split(A, g, dl)
    tiles = [tsp.tile_create(s, A.cols, bm, prec) for s, bm in zip(subs, (64, 16, 8))]
    th = []
    for t in tiles:
        lens = np.diff(t.arrays()["tile_ptr"]) if t.tilenum else np.zeros(1, np.int64)
        th.append(int(max(8, -(-int(lens.max()) // 8) * 8)))     # >= every row-block: no split tasks
    say(f"config {config} prec {prec}: thresholds {th}")
    host_plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
    dev_plan = tsp.Plan.from_csr(subs, A.rows, A.cols, cbp, prec, B)
    try:
        say(f"device tiling {dev_plan.tile_ms:.2f} ms")
        hip, host = tsp.load()
        for bm, t in zip((64, 16, 8), tiles):
            assert host.tsp_plan_tilenum(dev_plan.p, bm) == t.tilenum
        for fmt in (1, 2):
            Ch = plan_c(host_plan, th, fmt, fmt)
            Cd = plan_c(dev_plan, th, fmt, fmt)
            assert np.array_equal(Ch.view(np.uint32), Cd.view(np.uint32)), f"format {fmt}"
    finally:
        host_plan.close()
        dev_plan.close()
