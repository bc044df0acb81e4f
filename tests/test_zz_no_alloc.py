"""The allocation-free packing entry point (tsp_tiles_pack_device_noalloc)
against the allocating one (tsp_tiles_pack_device), through the C ABI: the
same vptr and packed values bit for bit, on two calls in a row (the second on
a smaller input, so stale scratch from the first would show), plus its
refusals (no room for the values, more tiles than its scratch covers, and
-- for both entry points -- more packed values than the int offsets hold)."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def host_tiles(tsp, rng, rows, cols, maxlen, prec, bm):
    lens = rng.integers(0, maxlen + 1, rows)
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ci = np.concatenate([rng.choice(cols, size=int(l), replace=False) for l in lens]).astype(np.int32)
    v = rng.uniform(-1, 1, rp[-1]).astype(np.float32)
    val = v.astype(np.float16).view(np.uint16) if prec == 0 else v
    A = tsp.Csr(rows, cols, rp, ci, val, prec)
    subs = tsp.matrix_split(A, 5.0, 3.0 if bm == 8 else 0.0)      # all rows in one 8- or 16-row class
    sub = subs[2 if bm == 8 else 1]
    assert sub.rows == rows
    t = tsp.tile_create(sub, cols, bm, prec)
    return t.tilenum, t.arrays()


def packed_by_alloc(tsp, hip, tilenum, bm, bn, prec, d_val, d_bmp):
    nv = C.c_longlong()
    pv, vp = C.c_void_p(), C.c_void_p()
    assert hip.tsp_tiles_pack_device(tilenum, bm, bn, prec, d_val, d_bmp, C.byref(nv), C.byref(pv), C.byref(vp),
                                     None) == 0
    try:
        dt = np.uint16 if prec == 0 else np.uint32
        return nv.value, tsp._d2h(vp, tilenum + 1, np.int32), tsp._d2h(pv, nv.value + 4, dt)
    finally:
        hip.tsp_free(pv)
        hip.tsp_free(vp)


@pytest.mark.parametrize("prec", [0, 1])
def test_pack_noalloc_matches_allocating_entry(tsp, prec):
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    hip = tsp.load()[0]
    assert hip.tsp_device_init(0) == 0
    rng = np.random.default_rng(11 + prec)
    dt = np.uint16 if prec == 0 else np.uint32
    # first a larger input, then a smaller one (the second call must not see
    # the first call's scratch contents)
    for case, (rows, cols, maxlen, bm) in enumerate([(9000, 5000, 90, 16), (1500, 700, 30, 8)]):
        bn = tsp.tile_bn(bm, prec)
        tilenum, arr = host_tiles(tsp, rng, rows, cols, maxlen, prec, bm)
        say(f"no-alloc pack: call {case + 1}, prec={prec} bm={bm} tilenum={tilenum}")
        assert tilenum > 2048 or case == 1      # the first input spans several scan blocks
        dense = np.ascontiguousarray(arr["dense"]).view(dt)
        bmp = np.ascontiguousarray(arr["bitmap"])
        bufs = [tsp._DevBuf(dense), tsp._DevBuf(bmp)]
        try:
            d_val, d_bmp = bufs[0].p, bufs[1].p
            nv, vptr_ref, pval_ref = packed_by_alloc(tsp, hip, tilenum, bm, bn, prec, d_val, d_bmp)
            # the packed stream restated on the host: tile values at set bits, in bit order
            words = bmp.reshape(tilenum, -1)
            bits = np.unpackbits(words.view(np.uint8), bitorder="little").reshape(tilenum, -1)[:, : bm * bn]
            want = dense.reshape(tilenum, bm * bn)[bits.astype(bool)]
            assert nv == want.size and np.array_equal(pval_ref[:nv], want)
            # caller-owned outputs, filled with garbage first
            out_v = tsp._DevBuf(np.full(tilenum + 1, -7, np.int32))
            out_p = tsp._DevBuf(np.full(nv + 4, 0xABCD, dt))
            try:
                got_n = C.c_longlong(-1)
                st = hip.tsp_tiles_pack_device_noalloc(tilenum, bm, bn, prec, d_val, d_bmp, out_p.p, nv + 4,
                                                       out_v.p, C.byref(got_n), None)
                assert st == 0 and got_n.value == nv
                assert np.array_equal(tsp._d2h(out_v.p, tilenum + 1, np.int32), vptr_ref)
                assert np.array_equal(tsp._d2h(out_p.p, nv + 4, dt), pval_ref)
                # no room for the padding: refused, the needed count reported
                got_n.value = -1
                st = hip.tsp_tiles_pack_device_noalloc(tilenum, bm, bn, prec, d_val, d_bmp, out_p.p, nv + 3,
                                                       out_v.p, C.byref(got_n), None)
                assert st != 0 and got_n.value == nv
                # more tiles than the scratch covers: refused on the host, nothing launched
                big = (2 ** 18 - 3) * 2048 + 1
                assert hip.tsp_tiles_pack_device_noalloc(big, bm, bn, prec, d_val, d_bmp, out_p.p, nv + 4,
                                                         out_v.p, C.byref(got_n), None) != 0
            finally:
                out_v.free()
                out_p.free()
        finally:
            for b in bufs:
                b.free()


def test_pack_noalloc_empty(tsp):
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    hip = tsp.load()[0]
    out_v = tsp._DevBuf(np.full(1, -7, np.int32))
    out_p = tsp._DevBuf(np.full(4, 0xABCD, np.uint16))
    try:
        n = C.c_longlong(-1)
        assert hip.tsp_tiles_pack_device_noalloc(0, 16, 16, 0, None, None, out_p.p, 4, out_v.p, C.byref(n), None) == 0
        assert n.value == 0
        assert tsp._d2h(out_v.p, 1, np.int32)[0] == 0
        assert (tsp._d2h(out_p.p, 4, np.uint16) == 0).all()
    finally:
        out_v.free()
        out_p.free()


def test_pack_refuses_counts_past_int_max(tsp):
    """A bitmap whose set bits (plus the 4 padding elements) exceed INT_MAX:
    both entry points return TSP_EINVAL with the 64-bit count, before any
    int offset could wrap (and nothing is written to the values)."""
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    hip = tsp.load()[0]
    assert hip.tsp_device_init(0) == 0
    bm, bn, prec = 64, 32, 0                      # 2048 slots = 32 bitmap words per tile
    tilenum = (2 ** 31) // 2048 + 1               # every bit set: 2^31 + 2048 values
    words = tilenum * (bm * bn // 64)
    say(f"pack overflow guard: tilenum={tilenum}, {words * 8 >> 20} MiB of all-ones bitmap")
    d_bmp, d_vp, d_pv = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert hip.tsp_malloc(C.byref(d_bmp), words * 8) == 0
    try:
        assert hip.tsp_memset(d_bmp, 0xFF, words * 8) == 0
        assert hip.tsp_malloc(C.byref(d_vp), 4 * (tilenum + 1)) == 0
        assert hip.tsp_malloc(C.byref(d_pv), 64) == 0
        want = tilenum * bm * bn
        n = C.c_longlong(-1)
        pv, vp = C.c_void_p(), C.c_void_p()
        st = hip.tsp_tiles_pack_device(tilenum, bm, bn, prec, d_bmp, d_bmp, C.byref(n), C.byref(pv), C.byref(vp),
                                       None)
        assert st != 0 and n.value == want and not pv.value and not vp.value
        n.value = -1
        st = hip.tsp_tiles_pack_device_noalloc(tilenum, bm, bn, prec, d_bmp, d_bmp, d_pv, 1 << 40, d_vp,
                                               C.byref(n), None)
        assert st != 0 and n.value == want
        # one tile fewer than the limit needs: both accept the count query
        ok = (2 ** 31 - 1 - 4) // 2048
        n.value = -1
        assert hip.tsp_tiles_pack_device(ok, bm, bn, prec, d_bmp, d_bmp, C.byref(n), None, None, None) == 0
        assert n.value == ok * 2048
    finally:
        for p in (d_bmp, d_vp, d_pv):
            if p.value:
                hip.tsp_free(p)
