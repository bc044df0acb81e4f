"""Parity checks shared by the GPU tests and their CPU self-tests.

TOL: element-wise tolerances, normalised by the magnitude sum |A|.|B| of the
entry (fp16 path 1e-3, tf32 path 1e-4).
"""
import numpy as np

TOL = {0: 1e-3, 1: 1e-4}


def assert_checksums(orc, A, B, colB, Cg, what=""):
    """Every row and every column of C at O(nnz) cost, for sizes whose full
    fp64 product is too slow: C·1 = A·(B·1) row by row and 1ᵀC = (1ᵀA)·B
    column by column, on the kernel's exact inputs.  Summing the elementwise
    bound |C - Cref| <= tol·Cabs over a row or a column bounds both, so a
    result that passes assert_close passes these; a dropped, doubled or
    misplaced contribution anywhere in C fails them."""
    tf = A.prec == 1
    a = orc.values_f64(A.val, A.prec, tf32_round=tf)
    b = orc.values_f64(B[:, :colB].reshape(-1), A.prec, tf32_round=tf).reshape(B.shape[0], colB)
    rp, ci = A.rowptr, A.colidx
    rows = np.repeat(np.arange(A.rows), np.diff(rp))
    C = Cg[:, :colB].astype(np.float64)
    assert np.isfinite(C).all(), what
    tol = TOL[A.prec]
    ref_r = np.bincount(rows, weights=a * b.sum(axis=1)[ci], minlength=A.rows)
    abs_r = np.bincount(rows, weights=np.abs(a) * np.abs(b).sum(axis=1)[ci], minlength=A.rows)
    err_r = np.abs(C.sum(axis=1) - ref_r)
    bad = err_r > tol * abs_r * (1 + 1e-9) + 1e-30
    assert not bad.any(), f"{what}: {bad.sum()} row sums out of tolerance, first row {np.argmax(bad)}"
    del rows
    u = np.bincount(ci, weights=a, minlength=A.cols)
    uabs = np.bincount(ci, weights=np.abs(a), minlength=A.cols)
    err_c = np.abs(C.sum(axis=0) - u @ b)
    bad = err_c > tol * (uabs @ np.abs(b)) * (1 + 1e-9) + 1e-30
    assert not bad.any(), f"{what}: {bad.sum()} column sums out of tolerance, first column {np.argmax(bad)}"
