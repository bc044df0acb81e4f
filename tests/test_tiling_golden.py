"""The committed tiling fixtures (tests/golden/tiling_golden.json, written by
tests/golden/make_tiling_golden.py from the CPU oracle): row split, tiles,
schedules and the integer-stream C of C1, a 2k Laplacian, a 4k block-sparse
matrix, RMAT scale 12 and dc2 over a gamma x delta grid.

CPU: the product host library reproduces every hash, and so does the oracle
(on the small inputs), so a change to either side shows here.  GPU: the
device tile conversion reproduces the tile hashes, and a full plan (tiles
uploaded, kernels, C downloaded) reproduces C bit for bit."""
import importlib.util
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN

spec = importlib.util.spec_from_file_location("make_tiling_golden", os.path.join(GOLDEN, "make_tiling_golden.py"))
mk = importlib.util.module_from_spec(spec)
spec.loader.exec_module(mk)

FIX = json.load(open(os.path.join(GOLDEN, "tiling_golden.json")))


@pytest.fixture(scope="module")
def structures(tsp, dc2_path):
    A, _, _, _ = tsp.gen_config(1)
    out = {"c1": (A.rows, A.cols, A.rowptr, A.colidx),
           "lap2k": mk.laplacian(45),
           "blk4k": mk.block_sparse(4096, np.random.default_rng(4)),
           "rmat12": mk.rmat(12, 1 << 16, np.random.default_rng(12))}
    m, n, rp, ci, _, _ = tsp.mm_read(dc2_path)
    out["dc2"] = (m, n, rp, ci)
    return out


def case_inputs(tsp, structures, name, prec, seed):
    rows, cols, rp, ci = structures[name]
    rp = np.asarray(rp, dtype=np.int32)
    ci = np.asarray(ci, dtype=np.int32)
    rng = np.random.default_rng(seed)
    bits = mk.int_values(rng, len(ci), prec)
    Bv = (1 + rng.integers(0, 3, (cols, FIX["colB"]))).astype(np.float32)
    store = bits.astype(np.uint16) if prec == 0 else bits.view(np.float32)
    return tsp.Csr(rows, cols, rp, ci, store, prec), bits, Bv


def check_tiles(e, arrays, prec, what):
    assert mk.sha(arrays["tile_ptr"], np.int32) == e["tile_ptr"], f"{what}: tile_ptr"
    assert mk.sha(arrays["tile_colidx"], np.int32) == e["tile_colidx"], f"{what}: tile_colidx"
    assert mk.sha(arrays["tile_nnz"], np.int32) == e["tile_nnz"], f"{what}: tile_nnz"
    assert mk.sha(arrays["bitmap"], np.uint64) == e["bitmap"], f"{what}: bitmap"
    dense = np.ascontiguousarray(arrays["dense"]).view(np.uint16 if prec == 0 else np.uint32)
    assert mk.sha(dense, dense.dtype) == e["dense"], f"{what}: dense values"


def test_fixture_covers_the_listed_inputs():
    names = {c["name"] for c in FIX["cases"]}
    assert names == {"c1", "lap2k", "blk4k", "rmat12", "dc2"}
    dc2 = {(c["gamma"], c["delta"]) for c in FIX["cases"] if c["name"] == "dc2" and c["prec"] == 0}
    assert dc2 == {(g, d) for g in (0.0, 1.0, 2.4, 5.0) for d in (0.0, 1.2, 1.5, 3.0)}
    # every class occurs with tiles somewhere, on both precisions
    for prec in (0, 1):
        for k in range(3):
            assert any(c["classes"][k].get("tilenum", 0) > 0 for c in FIX["cases"] if c["prec"] == prec)


def test_host_library_matches_golden(tsp, structures):
    for c in FIX["cases"]:
        what = f"{c['name']} prec {c['prec']} gamma {c['gamma']} delta {c['delta']}"
        A, _, _ = case_inputs(tsp, structures, c["name"], c["prec"], c["seed"])
        assert mk.sha(np.concatenate([A.rowptr, A.colidx]), np.int32) == c["input"], f"{what}: input"
        assert mk.sha(tsp.split_classes(A, c["gamma"], c["delta"]), np.int32) == c["split"], f"{what}: split"
        subs = tsp.matrix_split(A, c["gamma"], c["delta"])
        for e, s in zip(c["classes"], subs):
            assert s.rows == e["rows"], f"{what}: class {e['bm']} rows"
            if not s.rows:
                continue
            t = tsp.tile_create(s, A.cols, e["bm"], c["prec"])
            assert t.tilenum == e["tilenum"], f"{what}: class {e['bm']} tilenum"
            assert mk.sha(s.orig_row, np.int32) == e["orig_row"]
            check_tiles(e, t.arrays(), c["prec"], f"{what}: class {e['bm']}")
            for th in (8, 32):
                r, cs = tsp.pretreatment(t, th)
                assert mk.sha(np.concatenate([r.view(np.int32), cs]), np.int32) == e[f"sched{th}"]


def test_oracle_matches_golden(orc, tsp, structures):
    """The oracle itself still writes the committed hashes (small inputs)."""
    for c in FIX["cases"]:
        if c["name"] == "dc2":
            continue
        _, bits, _ = case_inputs(tsp, structures, c["name"], c["prec"], c["seed"])
        rows, cols, rp, ci = structures[c["name"]]
        rc = orc.split_classes(rows, cols, rp, ci, c["gamma"], c["delta"])
        assert mk.sha(rc, np.int32) == c["split"]
        for k, e in enumerate(c["classes"]):
            sr, sp, sc, sv, so = orc.sub_csr(rows, rp, ci, bits, rc, k)
            if not sr:
                continue
            o = orc.tile_create(sr, cols, sp, sc, sv, c["prec"], e["bm"], tsp.tile_bn(e["bm"], c["prec"]))
            check_tiles(e, o, c["prec"], f"oracle {c['name']} class {e['bm']}")


@pytest.mark.gpu
def test_device_tiling_matches_golden(tsp, structures):
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    for c in FIX["cases"]:
        if c["name"] == "dc2" and (c["gamma"], c["delta"]) not in ((1.0, 1.2), (2.4, 1.5), (0.0, 0.0), (5.0, 3.0)):
            continue
        what = f"device {c['name']} prec {c['prec']} gamma {c['gamma']} delta {c['delta']}"
        print(what, flush=True)
        A, _, _ = case_inputs(tsp, structures, c["name"], c["prec"], c["seed"])
        subs = tsp.matrix_split(A, c["gamma"], c["delta"])
        for e, s in zip(c["classes"], subs):
            if not s.rows:
                continue
            d = tsp.tile_create_device(s, A.cols, e["bm"], c["prec"])
            check_tiles(e, d, c["prec"], f"{what}: class {e['bm']}")


@pytest.mark.gpu
def test_plan_c_matches_golden(tsp, structures):
    """Host tiles -> plan -> kernels -> C: the fixture's exact integer C."""
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    colB = FIX["colB"]
    for p in FIX["products"]:
        for g, d in ((1.4, 1.4), (0.0, 0.0), (5.0, 3.0)):
            print(f"plan C: {p['name']} prec {p['prec']} gamma {g} delta {d}", flush=True)
            A, _, Bv = case_inputs(tsp, structures, p["name"], p["prec"], p["seed"])
            cbp = tsp.colB_padded(colB)
            B = np.zeros((A.cols, cbp), dtype=np.float32)
            B[:, :colB] = Bv
            if p["prec"] == 0:
                B = B.astype(np.float16).view(np.uint16)
            subs = tsp.matrix_split(A, g, d)
            tiles = [tsp.tile_create(s, A.cols, bm, A.prec) for s, bm in zip(subs, (64, 16, 8))]
            plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, A.prec, B)
            try:
                plan.set_th(8, 8, 8)
                plan.run(zero_c=True)
                Cg = plan.download_c()
            finally:
                plan.close()
            assert mk.sha(np.ascontiguousarray(Cg[:, :colB]), np.float32) == p["C"], (p["name"], p["prec"], g, d)
