"""Pins the CPU oracle (oracle/oracle.c) against things other than itself:
numpy/scipy, closed forms, hand-computed cases, the reference's own compiled
policy code, and the reference's shipped input (dc2.mtx)."""
import ctypes as C
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN


# --------------------------------------------------------------------------
# binary16 / tf32 conversions
# --------------------------------------------------------------------------
def test_half_to_float_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([orc.half_to_float(int(x)) for x in h], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_matches_numpy(orc):
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 6, 20000),
        # exact ties between adjacent halves, subnormal range, overflow edge
        (np.arange(0, 4096, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10) + 1,
        np.float32(2.0 ** -24) * (np.arange(200, dtype=np.float32) / 4),
        np.array([65504, 65519.99, 65520, 65536, -65520, 1e-8, -0.0, 0.0, np.inf, -np.inf], dtype=np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([orc.float_to_half(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_round_tf32_ties_and_grid(orc):
    # 1 + k*2^-10 are tf32 values; halfway points round to the even neighbour.
    for k in range(0, 64):
        lo = np.float32(1 + k * 2.0 ** -10)
        mid = np.float32(1 + (k + 0.5) * 2.0 ** -10)
        want = lo if k % 2 == 0 else np.float32(1 + (k + 1) * 2.0 ** -10)
        assert orc.round_tf32(float(mid)) == want
        assert orc.round_tf32(float(lo)) == lo
    x = np.float32(1.0) + np.float32(2.0 ** -12)        # below half an ulp -> down
    assert orc.round_tf32(float(x)) == 1.0


# --------------------------------------------------------------------------
# Matrix Market reader
# --------------------------------------------------------------------------
def test_mm_read_dc2_header_facts(orc, dc2_path):
    m, n, rp, ci, v, sym = orc.mm_read(dc2_path)
    # UF/SuiteSparse IBM_EDA/dc2: 116835 x 116835, 766396 entries, general
    assert (m, n, sym) == (116835, 116835, False)
    assert rp[-1] == 766396 and len(ci) == 766396
    lens = np.diff(rp)
    assert lens.min() >= 1 and lens.max() == 114190


def test_mm_read_matches_scipy(orc, dc2_path):
    import scipy.io
    A = scipy.io.mmread(dc2_path).tocoo()
    m, n, rp, ci, v, sym = orc.mm_read(dc2_path)
    rows = np.repeat(np.arange(m), np.diff(rp))
    # same multiset of (row, col, value); file order is kept within rows
    a = np.lexsort((ci, rows))
    b = np.lexsort((A.col, A.row))
    assert np.array_equal(rows[a], A.row[b]) and np.array_equal(ci[a], A.col[b])
    assert np.allclose(v[a], A.data[b], rtol=0, atol=0)


def test_mm_read_symmetric_pattern_known_csr(orc, tmp_path):
    p = tmp_path / "s.mtx"
    p.write_text("%%MatrixMarket matrix coordinate pattern symmetric\n% c\n3 3 4\n1 1\n2 1\n3 2\n3 3\n")
    m, n, rp, ci, v, sym = orc.mm_read(str(p))
    # file order within each row; off-diagonals mirrored, diagonal once
    assert sym and (m, n) == (3, 3)
    assert rp.tolist() == [0, 2, 4, 6]
    assert ci.tolist() == [0, 1, 0, 2, 1, 2]
    assert v.tolist() == [1.0] * 6


def test_mm_read_integer_complex_skew(orc, tmp_path):
    p = tmp_path / "i.mtx"
    p.write_text("%%MatrixMarket matrix coordinate integer general\n2 2 3\n2 2 7\n1 2 -3\n2 1 5\n")
    m, n, rp, ci, v, sym = orc.mm_read(str(p))
    assert rp.tolist() == [0, 1, 3] and ci.tolist() == [1, 1, 0] and v.tolist() == [-3, 7, 5]
    p = tmp_path / "c.mtx"
    p.write_text("%%MatrixMarket matrix coordinate complex general\n1 1 1\n1 1 2.5 -1\n")
    assert orc.mm_read(str(p))[4].tolist() == [2.5]
    p = tmp_path / "k.mtx"
    p.write_text("%%MatrixMarket matrix coordinate real skew-symmetric\n2 2 1\n2 1 4\n")
    m, n, rp, ci, v, sym = orc.mm_read(str(p))
    assert not sym and rp.tolist() == [0, 0, 1]     # skew is not mirrored by mmio_allinone


# --------------------------------------------------------------------------
# matrix_split
# --------------------------------------------------------------------------
def laplacian_structure(nx):
    rows = []
    for y in range(nx):
        for x in range(nx):
            r = y * nx + x
            cs = []
            if y > 0: cs.append(r - nx)
            if x > 0: cs.append(r - 1)
            cs.append(r)
            if x < nx - 1: cs.append(r + 1)
            if y < nx - 1: cs.append(r + nx)
            rows.append(cs)
    rp = np.zeros(nx * nx + 1, dtype=np.int32)
    rp[1:] = np.cumsum([len(c) for c in rows])
    return rp, np.concatenate([np.array(c, dtype=np.int32) for c in rows])


@pytest.fixture(scope="module")
def lap512():
    return laplacian_structure(512)


def test_split_fixed_groups(orc):
    rng = np.random.default_rng(3)
    rows, cols = 100, 50
    rp = np.zeros(rows + 1, dtype=np.int32)
    rp[1:] = np.cumsum(rng.integers(0, 6, rows))
    ci = rng.integers(0, cols, rp[-1]).astype(np.int32)
    assert (orc.split_classes(rows, cols, rp, ci, 0.0, 1.5) == 0).all()
    assert (orc.split_classes(rows, cols, rp, ci, -1.0, 1.5) == 0).all()
    assert (orc.split_classes(rows, cols, rp, ci, 5.0, 0.0) == 1).all()
    assert (orc.split_classes(rows, cols, rp, ci, 5.0, 3.0) == 2).all()


def test_split_laplacian_closed_forms(orc, lap512):
    rp, ci = lap512
    n = 512 * 512
    # 64-row window inside one grid row: N64 = 64+66+64 = 194, four 16-row
    # windows sum to 4*50 = 200 (edges: 193 vs 199, 130 vs 136), so every
    # window is 64-row iff gamma < 199/193.
    assert (orc.split_classes(n, n, rp, ci, 1.02, 3.0) == 0).all()
    # No 64 (gamma >= 4): 16-row window N16 = 16+18+16 = 50, the two 8-row
    # windows sum to 52 (edges 49 vs 51, 34 vs 36): all 16-row at delta = 1.
    assert (orc.split_classes(n, n, rp, ci, 4.0, 1.0) == 1).all()
    # delta = 1.05: interior 52 < 52.5 -> 8-row; first/last grid rows
    # (36 >= 35.7, 35 >= 34.65 at the corner window) stay 16-row.
    cls = orc.split_classes(n, n, rp, ci, 4.0, 1.05)
    y = np.arange(n) // 512
    want = np.where((y == 0) | (y == 511), 1, 2)
    assert np.array_equal(cls, want)


def test_split_hand_example(orc):
    # 24 rows.  Rows 0-7 share columns {0..3}; rows 8-15 each have one
    # private column; rows 16-23 are empty.  gamma = 5 (no 64), delta = 1:
    # window at 0: N16 = 4 + 8 = 12, S8 = 4 < 12, S8 + 8 = 12 >= 12 -> 16-row.
    # window at 16: i + 16 > 24 -> 8-row.
    rows = []
    for r in range(8):
        rows.append([0, 1, 2, 3])
    for r in range(8, 16):
        rows.append([100 + r])
    for r in range(16, 24):
        rows.append([])
    rp = np.zeros(25, dtype=np.int32)
    rp[1:] = np.cumsum([len(c) for c in rows])
    ci = np.array(sum(rows, []), dtype=np.int32)
    cls = orc.split_classes(24, 200, rp, ci, 5.0, 1.0)
    assert cls.tolist() == [1] * 16 + [2] * 8
    # delta = 1.01: 12 >= 12.12 fails -> rows 0-7 8-row; then window at 8:
    # N16 = 8 (rows 16-23 empty), S8 = 8 >= 8.08? no, +0 -> no -> 8-row.
    cls = orc.split_classes(24, 200, rp, ci, 5.0, 1.01)
    assert cls.tolist() == [2] * 24


def test_split_partition_invariant(orc):
    rng = np.random.default_rng(5)
    for trial in range(20):
        rows = int(rng.integers(1, 400))
        cols = int(rng.integers(1, 300))
        rp = np.zeros(rows + 1, dtype=np.int32)
        rp[1:] = np.cumsum(rng.integers(0, 12, rows))
        ci = rng.integers(0, cols, rp[-1]).astype(np.int32)
        g, d = float(rng.uniform(0.5, 4.5)), float(rng.uniform(0.2, 2.5))
        cls = orc.split_classes(rows, cols, rp, ci, g, d)
        # chunks: 64-row runs start at multiples of 8 and are full; 16/8-row
        # runs start at multiples of 8 and only the matrix's last one is short
        i = 0
        while i < rows:
            c = cls[i]
            size = {0: 64, 1: 16, 2: 8}[c]
            assert i % 8 == 0
            end = min(i + size, rows)
            assert (cls[i:end] == c).all()
            if c == 0:
                assert end == i + 64
            i = end


# --------------------------------------------------------------------------
# Tile_create
# --------------------------------------------------------------------------
def expand_tiles(t, bm, bn, prec):
    """Re-expand canonical tiles to {(row, col): value bits}."""
    out = {}
    dense = t["dense"].reshape(-1, bm, bn)
    for b in range(t["tilem"]):
        for tl in range(t["tile_ptr"][b], t["tile_ptr"][b + 1]):
            cols = t["tile_colidx"][tl * bn:(tl + 1) * bn]
            words = t["bitmap"][tl * ((bm * bn + 63) // 64):(tl + 1) * ((bm * bn + 63) // 64)]
            for r in range(bm):
                for s in range(bn):
                    bit = (int(words[(r * bn + s) // 64]) >> ((r * bn + s) % 64)) & 1
                    if bit:
                        out[(b * bm + r, int(cols[s]))] = int(dense[tl, r, s])
                    else:
                        assert dense[tl, r, s] == 0
    return out


@pytest.mark.parametrize("prec,bm,bn", [(0, 64, 32), (0, 16, 16), (0, 8, 16), (1, 64, 16), (1, 16, 8), (1, 8, 8)])
def test_tile_invariants_and_reexpansion(orc, prec, bm, bn):
    rng = np.random.default_rng(7 + bm + prec)
    rows, cols = 203, 157
    dens = []
    rp = [0]
    ci = []
    for r in range(rows):
        k = int(rng.integers(0, 30))
        c = sorted(rng.choice(cols, size=k, replace=False).tolist())
        rng.shuffle(c)                       # CSR order need not be sorted
        ci += c
        rp.append(len(ci))
    rp = np.array(rp, dtype=np.int32)
    ci = np.array(ci, dtype=np.int32)
    vals = rng.uniform(-1, 1, len(ci)).astype(np.float32)
    vb = vals.astype(np.float16).view(np.uint16).astype(np.uint32) if prec == 0 else vals.view(np.uint32)
    t = orc.tile_create(rows, cols, rp, ci, vb, prec, bm, bn)
    # tiles per block = ceil(distinct / BN)
    for b in range(t["tilem"]):
        seg = ci[rp[b * bm]:rp[min(rows, (b + 1) * bm)]]
        d = len(np.unique(seg))
        assert t["tile_ptr"][b + 1] - t["tile_ptr"][b] == (d + bn - 1) // bn
        got = t["tile_colidx"][t["tile_ptr"][b] * bn:t["tile_ptr"][b + 1] * bn]
        u = np.unique(seg)
        assert np.array_equal(got[:d], u)                       # sorted distinct
        assert (got[d:] == (u[-1] if d else 0)).all()            # padded with last
    assert t["tile_nnz"][-1] == len(ci)
    assert (np.diff(t["tile_nnz"]) >= 0).all()
    # re-expansion reproduces the input exactly (no duplicates here)
    want = {(r, int(ci[k])): int(vb[k]) for r in range(rows) for k in range(rp[r], rp[r + 1])}
    assert expand_tiles(t, bm, bn, prec) == want


def test_tile_duplicates_round_per_add(orc):
    # Three entries on one slot: 2048 + 1 + 1 in half precision.  Rounding
    # after every add (2048+1 -> 2048, ties to even) gives 2048, not 2050.
    rp = np.array([0, 3], dtype=np.int32)
    ci = np.array([5, 5, 5], dtype=np.int32)
    vb = np.array([2048, 1, 1], dtype=np.float16).view(np.uint16).astype(np.uint32)
    t = orc.tile_create(1, 10, rp, ci, vb, 0, 8, 16)
    assert t["tilenum"] == 1 and t["tile_nnz"].tolist() == [0, 3]
    assert np.float16(t["dense"].view(np.float16)[0]) == np.float16(2048)
    # tf32 storage keeps fp32 adds: 1 + 2^-24 + 2^-24 -> 1 (each add rounds)
    vb = np.array([1.0, 2.0 ** -24, 2.0 ** -24], dtype=np.float32).view(np.uint32)
    t = orc.tile_create(1, 10, rp, ci, vb, 1, 8, 8)
    assert t["dense"].view(np.float32)[0] == np.float32(1.0)


def test_tile_laplacian_counts(orc, lap512):
    rp, ci = lap512
    n = 512 * 512
    vb = np.zeros(len(ci), dtype=np.uint32)
    t = orc.tile_create(n, n, rp, ci, vb, 0, 64, 32)
    lens = np.diff(t["tile_ptr"])
    y = np.arange(t["tilem"]) // 8
    x = (np.arange(t["tilem"]) % 8) * 64
    # interior 64-row block: 194 distinct -> 7 tiles of 32; y-edge: 130 -> 5;
    # x-edge blocks lose one column: 193 -> 7, (y-edge) 129 -> 5
    want = np.where((y == 0) | (y == 511), 5, 7)
    assert np.array_equal(lens, want)
    t = orc.tile_create(n, n, rp, ci, vb, 0, 16, 16)
    lens = np.diff(t["tile_ptr"])
    y = np.arange(t["tilem"]) // 32
    xi = np.arange(t["tilem"]) % 32
    # 50 distinct -> 4 tiles; y-edge 34 -> 3; x-edge 49 -> 4; corner 33 -> 3
    want = np.where((y == 0) | (y == 511), 3, 4)
    assert np.array_equal(lens, want)
    assert t["tile_nnz"][-1] == len(ci)


# --------------------------------------------------------------------------
# tile_pretreatment
# --------------------------------------------------------------------------
def test_pretreatment_closed_form(orc):
    lens = np.array([0, 1, 7, 8, 9, 16, 17, 100, 33], dtype=np.int32)
    tp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    orow = np.arange(len(lens), dtype=np.int32) * 64
    for th in (8, 16, 32):
        rows, cs = orc.pretreatment(tp, orow, th)
        k = 0
        for b, L in enumerate(lens):
            n = 1 if L <= th else -(-L // th)
            per = -(-L // n) if L else 0
            for p in range(n):
                flag = 0x80000000 if L > th else 0
                assert int(rows[k]) == (int(orow[b]) | flag)
                size = cs[k + 1] - cs[k]
                assert size == (per if p < n - 1 else L - per * (n - 1))
                k += 1
        assert k == len(rows) and cs[0] == 0 and cs[-1] == tp[-1]


# --------------------------------------------------------------------------
# get_optimal_prefetch_th
# --------------------------------------------------------------------------
def params(**kw):
    import oracle
    p = oracle.ThParams(sm_count=10, threads_per_sm=2048, registers_per_sm=65536, blocks_per_sm=32,
                        shared_bytes_per_sm=100 * 1024, l2_bytes=1 << 20, kernel_threads=64,
                        kernel_registers=32, kernel_shared_bytes=4608, iteration_bytes=4096,
                        lambda_atom=0.01)
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_optimal_th_hand_computed(orc):
    # Two row-blocks of 20 tiles, colB 64, BM 16.
    # blk_sm = min(2048/64=32, 65536/(32*64)=32, 102400/4608=22, 32) = 22,
    # cap = 220, lambda_L2 = 4096*220/2^20 = 0.859375, atom_pen = 0.01/32*64
    # = 0.02 (max 20 <= 5*avg 20, no long-tail scaling).
    # TH=8:  blk=3, per=7, total=6 blocks; cost = 6/220*8 + 7 + 2*(2/3)*0.859375 + 0.02*4
    # TH=16: blk=2, per=10; cost = 4/220*16 + 10 + 2*0.5*0.859375 + 0.02*2
    # TH=24: blk=1, per=20; cost = 2/220*24 + 20
    tp = np.array([0, 20, 40], dtype=np.int32)
    n, top4 = orc.optimal_th(16, 64, tp, params())
    c8 = 6 / 220 * 8 + 7 + 2 * (2 / 3) * 0.859375 + 0.08
    c16 = 4 / 220 * 16 + 10 + 0.859375 + 0.04
    c24 = 2 / 220 * 24 + 20
    order = [th for _, th in sorted([(c8, 8), (c16, 16), (c24, 24)])]
    assert n == 3 and top4.tolist() == order + [order[0]]


def test_optimal_th_degenerate(orc):
    n, top4 = orc.optimal_th(8, 64, np.array([0, 0, 0], dtype=np.int32), params())
    assert top4.tolist() == [32, 32, 32, 32]
    n, top4 = orc.optimal_th(8, 64, np.array([0, 3, 5], dtype=np.int32), params())
    assert n == 1 and top4.tolist() == [8, 8, 8, 8]


# --------------------------------------------------------------------------
# features + policy, pinned by the reference's own compiled model.so
# --------------------------------------------------------------------------
def _golden_policy():
    with open(os.path.join(GOLDEN, "policy_golden.json")) as f:
        return json.load(f)["vectors"]


def test_policy_walk_reproduces_reference_model(orc):
    tree = orc.load_ref_policy_tree()
    if tree is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    nodes, cands, r16, r32 = tree
    for v in _golden_policy():
        f = np.array([np.nan if x is None else x for x in v["f"]], dtype=np.float64)
        assert list(orc.policy_select(f, nodes, cands, r16)) == pytest.approx(v["fp16"], abs=0)
        assert list(orc.policy_select(f, nodes, cands, r32)) == pytest.approx(v["tf32"], abs=0)


def test_policy_golden_covers_several_actions():
    acts = {tuple(v["fp16"]) for v in _golden_policy()} | {tuple(v["tf32"]) for v in _golden_policy()}
    assert len(acts) >= 5


def test_features_closed_form(orc):
    rp = np.array([0, 2, 2, 7], dtype=np.int32)
    f = orc.features(3, 10, 7, rp, 9.5, 128)
    assert f.tolist() == [0, 0, 3, 10, 7, 1 - 7 / 30, 7 / 3, 5, 0, 9.5, 128]
    assert orc.features(3, 10, 6, rp, 9.5, 128) is None          # nnz mismatch
    assert orc.features(3, 10, 7, rp, 0.0, 128) is None          # bad capability


# --------------------------------------------------------------------------
# CSR SpMM and the CLI value stream
# --------------------------------------------------------------------------
def test_spmm_f64_matches_dense(orc):
    import scipy.sparse as sp
    rng = np.random.default_rng(11)
    A = sp.random(70, 50, density=0.1, random_state=1, format="csr")
    B = rng.standard_normal((50, 13))
    Cm = orc.spmm_f64(70, A.indptr, A.indices, A.data, B, 13)
    assert np.allclose(Cm, A.toarray() @ B, rtol=1e-13, atol=1e-13)
    Cf, used = orc.spmm_f32_omp(70, A.indptr, A.indices, A.data.astype(np.float32),
                                B.astype(np.float32), 13)
    assert used >= 1 and np.allclose(Cf, Cm, rtol=1e-5, atol=1e-5)


def test_cli_rand_stream_fixture():
    libc = C.CDLL("libc.so.6")
    with open(os.path.join(GOLDEN, "rand1325.json")) as f:
        draws = json.load(f)["draws"]
    libc.srand(1325)
    assert [libc.rand() for _ in range(len(draws))] == draws
    # glibc TYPE_3 additive generator: r[i] = r[i-3] + r[i-31] (mod 2^32),
    # output r >> 1, once the 34 seeding steps and 310 discards are done.
    r = [0] * 34
    r[0] = 1325
    for i in range(1, 31):
        r[i] = (16807 * r[i - 1]) % 2147483647
        if r[i] < 0:
            r[i] += 2147483647
    for i in range(31, 34):
        r[i] = r[i - 31]
    for i in range(34, 344 + len(draws)):
        r.append((r[i - 31] + r[i - 3]) & 0xffffffff)
    assert [x >> 1 for x in r[344:344 + len(draws)]] == draws


def test_round_tf32_array_matches_scalar(orc):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(5000) * 10.0 ** rng.integers(-30, 30, 5000)).astype(np.float32)
    x[:3] = [np.inf, -np.inf, 0.0]
    got = orc.round_tf32_array(x)
    want = np.array([orc.round_tf32(float(v)) for v in x], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_optimal_th_colB32_block_packing(orc):
    # colB 32: 8- and 16-row kernels pack four tasks per block, total_block =
    # ceil(total_chunk / 4); 64-row tiles do not (src/csr2tile.h:592-597).
    # One SM, one resident block: cap = 1, lambda_L2 = 4096/2^20; atom_pen =
    # 0.01/32*32 = 0.01; two row-blocks of 20 tiles (Tmax 24).
    #   TH  8: chunks 6, per 7, atoms 4   BM 8/16: 2 blocks -> 2*8 + 7 = 23.05
    #                                      BM 64:   6 blocks -> 6*8 + 7 = 55.05
    #   TH 16: chunks 4, per 10, atoms 2  BM 8/16: 1 -> 16 + 10 = 26.02; BM 64: 64 + 10 = 74.02
    #   TH 24: chunks 2, per 20            BM 8/16: 1 -> 24 + 20 = 44;    BM 64: 48 + 20 = 68
    p = params(sm_count=1, threads_per_sm=64)
    tp = np.array([0, 20, 40], dtype=np.int32)
    for bm in (8, 16):
        n, top4 = orc.optimal_th(bm, 32, tp, p)
        assert n == 3 and top4.tolist() == [8, 16, 24, 8], bm
    n, top4 = orc.optimal_th(64, 32, tp, p)
    assert n == 3 and top4.tolist() == [8, 24, 16, 8]
    # colB 64 goes through the column-grid branch: same as the 64-row order
    n, top4 = orc.optimal_th(16, 64, tp, p)
    assert n == 3 and top4.tolist() == [8, 24, 16, 8]


def test_optimal_th_long_tail_atomic_discount(orc):
    # Nine row-blocks of 1 tile and one of 100: max 100 > 5 * mean 10.9, so the
    # atomic weight is multiplied by 0.04 (src/csr2tile.h:549).  lambda_atom 2
    # at colB 64: atom_pen = 2/32*64 = 4, discounted 0.16.  22000 resident
    # blocks and 1-byte iterations make the throughput and L2 terms < 0.03, so
    # the cost is max_chunk + atom_pen * (tasks - 1) of the long row-block:
    #   TH:    8     16    24    32    40    56    104   (48, 64-96 repeat a task count)
    #   per:   8     15    20    25    34    50    100
    #   atoms: 12    6     4     3     2     1     0
    # discounted: 9.92 15.96 20.64 25.48 34.32 50.16 100  -> 8, 16, 24, 32
    # full 4:     56   39    36    37    42    54    100  -> 24, 32, 16, 40
    p = params(sm_count=1000, iteration_bytes=1, lambda_atom=2.0)
    tp = np.concatenate([[0], np.cumsum([1] * 9 + [100])]).astype(np.int32)
    n, top4 = orc.optimal_th(16, 64, tp, p)
    assert n == 7 and top4.tolist() == [8, 16, 24, 32]
    # without the long tail (the 100-tile block alone) the full weight applies
    n, top4 = orc.optimal_th(16, 64, np.array([0, 100], dtype=np.int32), p)
    assert top4.tolist() == [24, 32, 16, 40]
