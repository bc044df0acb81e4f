"""CPU self-test of the full-size parity identities the GPU tests apply to C
(tests/parity_checks.py): they accept the oracle's own product, rounded to
fp32 as a kernel's output is, and reject it once a mistake is planted in it
(a dropped contribution, two rows swapped, a value moved between columns)."""
import numpy as np
import pytest

from parity_checks import assert_checksums


def small_case(tsp, orc, prec, seed):
    rng = np.random.default_rng(seed)
    rows, cols, colB = 300, 257, 48
    lens = rng.integers(0, 30, rows)
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ci = np.concatenate([rng.choice(cols, size=int(l), replace=False) for l in lens]).astype(np.int32)
    v = rng.uniform(-1, 1, rp[-1]).astype(np.float32)
    val = v.astype(np.float16).view(np.uint16) if prec == 0 else v
    A = tsp.Csr(rows, cols, rp, ci, val, prec)
    cbp = tsp.colB_padded(colB)
    b = np.zeros((cols, cbp), np.float32)
    b[:, :colB] = rng.uniform(-1, 1, (cols, colB))
    B = b.astype(np.float16).view(np.uint16) if prec == 0 else b
    tf = prec == 1
    a64 = orc.values_f64(A.val, prec, tf32_round=tf)
    b64 = orc.values_f64(B[:, :colB].reshape(-1), prec, tf32_round=tf).reshape(cols, colB)
    Cref = orc.spmm_f64(rows, rp, ci, a64, b64, colB)
    C = np.zeros((rows, cbp), np.float32)
    C[:, :colB] = Cref.astype(np.float32)
    return A, B, colB, C, a64, b64


@pytest.mark.parametrize("prec", [0, 1])
def test_checksums_accept_the_oracle_product(tsp, orc, prec):
    A, B, colB, C, _, _ = small_case(tsp, orc, prec, 5 + prec)
    assert_checksums(orc, A, B, colB, C, "oracle product")


@pytest.mark.parametrize("prec", [0, 1])
def test_checksums_reject_planted_mistakes(tsp, orc, prec):
    A, B, colB, C, a64, b64 = small_case(tsp, orc, prec, 9 + prec)
    rp, ci = A.rowptr, A.colidx
    lens = np.diff(rp)
    # one nonzero's contribution dropped from its row
    r = int(np.argmax(lens))
    e = rp[r] + int(np.argmax(np.abs(a64[rp[r]:rp[r + 1]])))
    bad = C.copy()
    bad[r, :colB] -= (a64[e] * b64[ci[e]]).astype(np.float32)
    with pytest.raises(AssertionError, match="row sums"):
        assert_checksums(orc, A, B, colB, bad, "dropped contribution")
    # two rows of C swapped (the column sums stay the same)
    sums = C[:, :colB].astype(np.float64).sum(axis=1)
    r1, r2 = int(np.argmax(sums)), int(np.argmin(sums))
    bad = C.copy()
    bad[[r1, r2]] = bad[[r2, r1]]
    with pytest.raises(AssertionError, match="row sums"):
        assert_checksums(orc, A, B, colB, bad, "rows swapped")
    # a value moved from one column to another inside a row (its row sum stays)
    bad = C.copy()
    x = np.float32(np.abs(C[r, :colB]).max())
    bad[r, 0] += x
    bad[r, 1] -= x
    with pytest.raises(AssertionError, match="column sums"):
        assert_checksums(orc, A, B, colB, bad, "value moved between columns")
