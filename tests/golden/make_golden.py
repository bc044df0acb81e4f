"""Writes the committed golden fixtures of tests/golden/.

  policy_golden.json  (features -> gamma, delta) from the reference's own
                      src/ml_predict.c + src/model.h, compiled from the
                      reference sources into oracle/_ref/model.so by
                      oracle/Makefile (needs the reference checkout).
  rand1325.json       the first draws of glibc rand() after srand(1325), the
                      value stream of the reference CLI (src/main.cu:176-207).

Run from the repository root:  python tests/golden/make_golden.py
"""
import ctypes as C
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
OUT = os.path.join(ROOT, "tests", "golden")


def policy_vectors(rng):
    vecs = []
    caps = [7.0, 7.5, 8.0, 8.6, 8.9, 9.0, 9.5, 10.0, 12.0]
    for _ in range(3000):
        rows = int(10 ** rng.uniform(2, 7.5))
        cols = int(rows * 10 ** rng.uniform(-0.5, 0.5)) + 1
        avg = 10 ** rng.uniform(0, 2.5)
        nnz = int(min(rows * avg, rows * cols))
        mx = int(avg * 10 ** rng.uniform(0, 3)) + 1
        mn = int(rng.integers(0, max(1, int(avg)) + 1))
        cap = float(rng.choice(caps))
        colB = int(rng.choice([32, 64, 96, 128, 256, 512]))
        f = [0.0, 0.0, rows, cols, nnz, 1.0 - nnz / (rows * cols), nnz / rows, mx, mn, cap, colB]
        vecs.append(f)
    # missing values exercise the tree's missing_left_mask branches
    for i in range(200):
        f = list(vecs[i])
        f[2 + (i % 9)] = float("nan")
        vecs.append(f)
    return vecs


def main():
    import oracle
    oracle.build()
    so = os.path.join(oracle.REF_DIR, "model.so")
    lib = C.CDLL(so)
    for name in ("tilespmm_predict_fp16", "tilespmm_predict_tf32"):
        getattr(lib, name).argtypes = [C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_float)]
        getattr(lib, name).restype = None
    rng = np.random.default_rng(20260101)
    rows = []
    for f in policy_vectors(rng):
        a = np.array(f, dtype=np.float64)
        out = {}
        for prec, name in (("fp16", "tilespmm_predict_fp16"), ("tf32", "tilespmm_predict_tf32")):
            g, d = C.c_float(), C.c_float()
            getattr(lib, name)(a.ctypes.data_as(C.c_void_p), C.byref(g), C.byref(d))
            out[prec] = [g.value, d.value]
        rows.append({"f": [None if np.isnan(x) else x for x in f], **out})
    with open(os.path.join(OUT, "policy_golden.json"), "w") as fo:
        json.dump({"source": "reference src/ml_predict.c + src/model.h via oracle/_ref/model.so",
                   "vectors": rows}, fo)
    libc = C.CDLL("libc.so.6")
    libc.srand(1325)
    draws = [libc.rand() for _ in range(8192)]
    with open(os.path.join(OUT, "rand1325.json"), "w") as fo:
        json.dump({"source": "glibc rand() after srand(1325)", "draws": draws}, fo)
    print("wrote", len(rows), "policy vectors and", len(draws), "rand draws")


if __name__ == "__main__":
    main()
