"""Writes tests/golden/tiling_golden.json: split, tile and schedule hashes,
and the hash of C for an integer value stream, on small fixed inputs.

Every output comes from the CPU oracle (oracle/: the C restatement of
src/hetero_split.h:144-291, src/csr2tile.h:15-434,724-795, checked against
closed forms and invariants in tests/test_oracle_pins.py).  The inputs:

  c1      configuration 1 in full (4096^2, 8 distinct uniform columns per
          row), from the library's own generator; its input hash is stored,
          so the generator is pinned too
  lap2k   5-point Laplacian on a 45 x 45 grid (2025 rows: a ragged last
          row-block for every class)
  blk4k   4096^2 block-sparse: 2% of the 16 x 16 blocks of a 256 x 256 block
          grid, plus 1e-4 singletons
  rmat12  RMAT scale 12, 2^16 edges, (a, b, c) = (.57, .19, .19), symmetrised
  dc2     the reference's data/dc2.mtx (tests/golden/dc2.mtx.gz) over gamma
          {0, 1.0, 2.4, 5} x delta {0, 1.2, 1.5, 3}

Values are small integers (1 + u, u uniform in {0, 1, 2}) for A and B, so C
is exact in fp32 on every path and its hash can be compared bit for bit.

Run from the repository root:  python tests/golden/make_tiling_golden.py
"""
import gzip
import hashlib
import json
import os
import shutil
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
OUT = os.path.join(ROOT, "tests", "golden", "tiling_golden.json")
COLB = 32
SPLITS = [(0.0, 0.0), (5.0, 0.0), (5.0, 3.0), (1.4, 1.4), (2.4, 1.5)]
DC2_SPLITS = [(g, d) for g in (0.0, 1.0, 2.4, 5.0) for d in (0.0, 1.2, 1.5, 3.0)]


def sha(a, dtype):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=dtype).tobytes()).hexdigest()[:24]


def csr_from_pairs(n_rows, r, c):
    key = np.unique(r.astype(np.int64) * (1 << 32) + c.astype(np.int64))
    r, c = (key >> 32).astype(np.int32), (key & 0xffffffff).astype(np.int32)
    rp = np.zeros(n_rows + 1, dtype=np.int64)
    np.add.at(rp, r + 1, 1)
    return np.cumsum(rp).astype(np.int32), c


def laplacian(nx):
    r, c = [], []
    for y in range(nx):
        for x in range(nx):
            i = y * nx + x
            for dx, dy in ((0, -1), (-1, 0), (0, 0), (1, 0), (0, 1)):
                if 0 <= x + dx < nx and 0 <= y + dy < nx:
                    r.append(i)
                    c.append((y + dy) * nx + x + dx)
    return nx * nx, nx * nx, *csr_from_pairs(nx * nx, np.array(r), np.array(c))


def block_sparse(n, rng):
    nb = n // 16
    blocks = rng.choice(nb * nb, size=round(0.02 * nb * nb), replace=False)
    br, bc = blocks // nb, blocks % nb
    ii, jj = np.meshgrid(np.arange(16), np.arange(16), indexing="ij")
    r = (br[:, None] * 16 + ii.reshape(-1)[None, :]).reshape(-1)
    c = (bc[:, None] * 16 + jj.reshape(-1)[None, :]).reshape(-1)
    k = round(1e-4 * n * n)
    sr, sc = rng.integers(0, n, k), rng.integers(0, n, k)
    return n, n, *csr_from_pairs(n, np.concatenate([r, sr]), np.concatenate([c, sc]))


def rmat(scale, edges, rng, a=0.57, b=0.19, c=0.19):
    n = 1 << scale
    r = np.zeros(edges, dtype=np.int64)
    s = np.zeros(edges, dtype=np.int64)
    for bit in range(scale):
        u = rng.random(edges)
        down = u >= a + b                       # quadrants c, d: lower half
        right = ((u >= a) & (u < a + b)) | (u >= a + b + c)
        r |= down.astype(np.int64) << bit
        s |= right.astype(np.int64) << bit
    return n, n, *csr_from_pairs(n, np.concatenate([r, s]), np.concatenate([s, r]))


def int_values(rng, nnz, prec):
    v = (1 + rng.integers(0, 3, nnz)).astype(np.float32)
    if prec == 0:
        return v.astype(np.float16).view(np.uint16).astype(np.uint32)
    return v.view(np.uint32)


def inputs():
    import oracle
    import tilespmm_amd as tsp
    A, _, _, _ = tsp.gen_config(1)
    yield "c1", A.rows, A.cols, A.rowptr, A.colidx, SPLITS
    yield ("lap2k", *laplacian(45), SPLITS)
    yield ("blk4k", *block_sparse(4096, np.random.default_rng(4)), SPLITS)
    yield ("rmat12", *rmat(12, 1 << 16, np.random.default_rng(12)), SPLITS)
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "dc2.mtx")
        with gzip.open(os.path.join(ROOT, "tests", "golden", "dc2.mtx.gz"), "rb") as fi, open(path, "wb") as fo:
            shutil.copyfileobj(fi, fo)
        m, n, rp, ci, _, _ = oracle.mm_read(path)
    yield "dc2", m, n, rp, ci, DC2_SPLITS


def main():
    import oracle
    oracle.build()
    cases, products = [], []
    for name, rows, cols, rp, ci, splits in inputs():
        rp = np.asarray(rp, dtype=np.int32)
        ci = np.asarray(ci, dtype=np.int32)
        for prec in (0, 1):
            seed = int(hashlib.sha256(f"{name}/{prec}".encode()).hexdigest()[:8], 16)
            rng = np.random.default_rng(seed)
            bits = int_values(rng, len(ci), prec)
            Bv = (1 + rng.integers(0, 3, (cols, COLB))).astype(np.float64)
            a64 = oracle.values_f64(bits.astype(np.uint16) if prec == 0 else bits.view(np.float32), prec)
            Cm = oracle.spmm_f64(rows, rp, ci, a64, Bv, COLB)
            assert np.all(Cm == np.round(Cm)) and np.abs(Cm).max() < 2 ** 24
            products.append({"name": name, "prec": prec, "colB": COLB, "seed": seed,
                             "C": sha(Cm.astype(np.float32), np.float32)})
            for g, d in (splits if prec == 0 or name != "dc2" else splits[::5]):
                rc = oracle.split_classes(rows, cols, rp, ci, g, d)
                cls = []
                for k, bm in enumerate((64, 16, 8)):
                    bn = {(64, 0): 32, (16, 0): 16, (8, 0): 16, (64, 1): 16, (16, 1): 8, (8, 1): 8}[(bm, prec)]
                    sr, sp, sc, sv, so = oracle.sub_csr(rows, rp, ci, bits, rc, k)
                    e = {"bm": bm, "rows": int(sr)}
                    if sr:
                        t = oracle.tile_create(sr, cols, sp, sc, sv, prec, bm, bn)
                        r8, c8 = oracle.pretreatment(t["tile_ptr"], so[::bm], 8)
                        r32, c32 = oracle.pretreatment(t["tile_ptr"], so[::bm], 32)
                        e.update({"orig_row": sha(so, np.int32), "tilenum": int(t["tilenum"]),
                                  "tile_ptr": sha(t["tile_ptr"], np.int32),
                                  "tile_colidx": sha(t["tile_colidx"], np.int32),
                                  "tile_nnz": sha(t["tile_nnz"], np.int32),
                                  "bitmap": sha(t["bitmap"], np.uint64),
                                  "dense": sha(t["dense"], np.uint16 if prec == 0 else np.uint32),
                                  "sched8": sha(np.concatenate([r8.view(np.int32), c8]), np.int32),
                                  "sched32": sha(np.concatenate([r32.view(np.int32), c32]), np.int32)})
                    cls.append(e)
                cases.append({"name": name, "prec": prec, "gamma": g, "delta": d, "rows": int(rows),
                              "cols": int(cols), "nnz": int(len(ci)), "seed": seed,
                              "input": sha(np.concatenate([rp, ci]), np.int32),
                              "split": sha(rc, np.int32), "classes": cls})
        print(name, rows, cols, len(ci), flush=True)
    with open(OUT, "w") as fo:
        json.dump({"source": "oracle/ (CPU restatement); see the docstring of make_tiling_golden.py",
                   "colB": COLB, "cases": cases, "products": products}, fo, indent=0)
    print("wrote", len(cases), "split/tile cases and", len(products), "products")


if __name__ == "__main__":
    main()
