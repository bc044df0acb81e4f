"""Product host library (libtilespmm_host.so) vs the pinned CPU oracle:
split, tiles (bit-exact), schedule, cost model, features, Matrix Market,
plus properties of the synthetic generators.  CPU only."""
import ctypes as C

import numpy as np
import pytest


def random_csr(rng, rows, cols, maxlen, dup=False, sorted_cols=False, empty_frac=0.0):
    rp = [0]
    ci = []
    for r in range(rows):
        if rng.random() < empty_frac:
            rp.append(len(ci))
            continue
        k = int(rng.integers(0, maxlen + 1))
        if dup:
            c = rng.integers(0, cols, k).tolist()
        else:
            c = rng.choice(cols, size=min(k, cols), replace=False).tolist()
        if sorted_cols:
            c.sort()
        ci += c
        rp.append(len(ci))
    return np.array(rp, dtype=np.int32), np.array(ci, dtype=np.int32)


def values_for(rng, n, prec):
    v = rng.uniform(-1, 1, n).astype(np.float32)
    if prec == 0:
        store = v.astype(np.float16).view(np.uint16)
        return store, store.astype(np.uint32)
    return v, v.view(np.uint32)


def make(tsp, rows, cols, rp, ci, val, prec):
    return tsp.Csr(rows, cols, rp, ci, val, prec)


CANDS = [(0.0, 1.5), (5.0, 0.0), (5.0, 3.0), (1.0, 1.0), (1.4, 1.2), (2.0, 1.5), (2.4, 2.0), (3.8, 1.8),
         (4.0, 1.4), (2.5, 1.0), (3.5, 1.0), (1.8, 1.2)]


@pytest.mark.parametrize("seed", range(8))
def test_split_matches_oracle(tsp, orc, seed):
    rng = np.random.default_rng(100 + seed)
    rows = int(rng.integers(1, 700))
    cols = int(rng.integers(1, 400))
    rp, ci = random_csr(rng, rows, cols, int(rng.integers(1, 40)), dup=bool(seed % 2), empty_frac=0.2 * (seed % 3))
    A = make(tsp, rows, cols, rp, ci, None, 0)
    for g, d in CANDS + [(float(rng.uniform(0.5, 4.5)), float(rng.uniform(0.1, 2.5))) for _ in range(6)]:
        a = tsp.split_classes(A, g, d)
        b = orc.split_classes(rows, cols, rp, ci, g, d)
        assert np.array_equal(a, b), (g, d)


def test_split_dc2_matches_oracle(tsp, orc, dc2_path):
    m, n, rp, ci, v, sym = orc.mm_read(dc2_path)
    A = make(tsp, m, n, rp, ci, None, 0)
    for g, d in CANDS:
        assert np.array_equal(tsp.split_classes(A, g, d), orc.split_classes(m, n, rp, ci, g, d)), (g, d)


def compare_tiles(tsp, orc, rows, cols, rp, ci, prec, bm, store, bits):
    bn = tsp.tile_bn(bm, prec)
    sub = tsp.Csr(rows, cols, rp, ci, store, prec)
    sub.orig_row = np.arange(rows, dtype=np.int32)
    t = tsp.tile_create(sub, cols, bm, prec)
    o = orc.tile_create(rows, cols, rp, ci, bits, prec, bm, bn)
    a = t.arrays()
    assert t.tilenum == o["tilenum"] and t.tilem == o["tilem"]
    assert np.array_equal(a["tile_ptr"], o["tile_ptr"])
    assert np.array_equal(a["tile_colidx"], o["tile_colidx"])
    assert np.array_equal(a["tile_nnz"], o["tile_nnz"])
    dense = a["dense"].view(np.uint16 if prec == 0 else np.uint32)
    assert np.array_equal(dense, o["dense"].astype(dense.dtype))
    assert np.array_equal(a["bitmap"], o["bitmap"])
    return t


@pytest.mark.parametrize("prec", [0, 1])
@pytest.mark.parametrize("bm", [64, 16, 8])
@pytest.mark.parametrize("seed", range(3))
def test_tiles_bit_exact(tsp, orc, prec, bm, seed):
    rng = np.random.default_rng(1000 * bm + 10 * seed + prec)
    rows = int(rng.integers(1, 500))           # ragged last row-block
    cols = int(rng.integers(1, 3000))
    rp, ci = random_csr(rng, rows, cols, int(rng.integers(1, 90)), dup=(seed == 2), empty_frac=0.1 * seed)
    store, bits = values_for(rng, len(ci), prec)
    compare_tiles(tsp, orc, rows, cols, rp, ci, prec, bm, store, bits)


@pytest.mark.parametrize("prec", [0, 1])
def test_tiles_duplicates_rounding(tsp, orc, prec):
    # many duplicates on few slots: per-add rounding must match exactly
    rng = np.random.default_rng(77)
    rows, cols = 40, 6
    rp, ci = random_csr(rng, rows, cols, 60, dup=True)
    v = (rng.uniform(-1, 1, len(ci)) * 2.0 ** rng.integers(-12, 12, len(ci))).astype(np.float32)
    if prec == 0:
        store = v.astype(np.float16).view(np.uint16)
        bits = store.astype(np.uint32)
    else:
        store, bits = v, v.view(np.uint32)
    for bm in (64, 16, 8):
        compare_tiles(tsp, orc, rows, cols, rp, ci, prec, bm, store, bits)


def test_tiles_dc2_bit_exact(tsp, orc, dc2_path):
    m, n, rp, ci, v, sym = orc.mm_read(dc2_path)
    store = v.astype(np.float16).view(np.uint16)
    compare_tiles(tsp, orc, m, n, rp, ci, 0, 16, store, store.astype(np.uint32))


def test_split_then_tiles_full_pipeline(tsp, orc):
    """matrix_split -> sub-CSRs -> Tile_create for all three classes equals the
    oracle's split + sub_csr + tile restatement."""
    rng = np.random.default_rng(5)
    rows, cols = 1500, 900
    rp, ci = random_csr(rng, rows, cols, 50, empty_frac=0.1)
    for prec in (0, 1):
        store, bits = values_for(rng, len(ci), prec)
        A = tsp.Csr(rows, cols, rp, ci, store, prec)
        for g, d in [(2.0, 1.5), (1.0, 1.0), (3.0, 2.0), (0.0, 1.5), (5.0, 0.0), (5.0, 3.0)]:
            subs = tsp.matrix_split(A, g, d)
            cls = orc.split_classes(rows, cols, rp, ci, g, d)
            for k, bm in enumerate((64, 16, 8)):
                sr, sp, sc, sv, so = orc.sub_csr(rows, rp, ci, bits, cls, k)
                s = subs[k]
                assert s.rows == sr
                if sr == 0:
                    continue
                assert np.array_equal(s.rowptr, sp) and np.array_equal(s.colidx, sc)
                assert np.array_equal(s.orig_row, so)
                assert np.array_equal(s.val.view(np.uint16 if prec == 0 else np.uint32).astype(np.uint32), sv)
                t = tsp.tile_create(s, cols, bm, prec)
                o = orc.tile_create(sr, cols, sp, sc, sv, prec, bm, tsp.tile_bn(bm, prec))
                a = t.arrays()
                assert np.array_equal(a["tile_ptr"], o["tile_ptr"])
                assert np.array_equal(a["tile_colidx"], o["tile_colidx"])
                assert np.array_equal(a["orig_tile_row_idx"], so[::bm])
                for th in (8, 16, 24, 64):
                    r1, c1 = tsp.pretreatment(t, th)
                    r2, c2 = orc.pretreatment(o["tile_ptr"], so[::bm], th)
                    assert np.array_equal(r1, r2) and np.array_equal(c1, c2)


def ref_geometry_params(tsp, bm, colB, **kw):
    p = tsp.ThParams(sm_count=132, threads_per_sm=2048, registers_per_sm=65536, blocks_per_sm=32,
                     shared_bytes_per_sm=228 * 1024, l2_bytes=50 * 1024 * 1024, kernel_threads=64,
                     kernel_registers=40, kernel_shared_bytes=4608, iteration_bytes=2 * (bm * 16 + 16 * 64),
                     lambda_atom=0.01, lambda_l2_scale=1.0)
    p.tasks_per_block = 4 if (colB == 32 and bm in (8, 16)) else 1
    p.cols_per_task = 32 if colB == 32 else 64
    for k, v in kw.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("colB", [32, 64, 128, 256])
@pytest.mark.parametrize("bm", [64, 16, 8])
def test_cost_model_matches_oracle(tsp, orc, bm, colB):
    rng = np.random.default_rng(bm * 7 + colB)
    for trial in range(6):
        tilem = int(rng.integers(1, 3000))
        lens = rng.integers(0, [5, 40, 200, 2000][trial % 4], tilem)
        if trial == 5:
            lens[:] = 3
        tp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        kw = dict(kernel_threads=int(rng.choice([64, 128, 256])), kernel_registers=int(rng.integers(16, 128)),
                  lambda_atom=float(rng.uniform(0.001, 0.03)))
        p = ref_geometry_params(tsp, bm, colB, **kw)
        import oracle
        q = oracle.ThParams(**{f: getattr(p, f) for f, _ in oracle.ThParams._fields_})
        n1, t1 = tsp.optimal_th(bm, colB, tp, p)
        n2, t2 = orc.optimal_th(bm, colB, tp, q)
        assert n1 == n2 and np.array_equal(t1, t2)


def test_features_match_oracle(tsp, orc):
    rng = np.random.default_rng(9)
    for trial in range(10):
        rows, cols = int(rng.integers(1, 300)), int(rng.integers(1, 300))
        rp, ci = random_csr(rng, rows, cols, 20, empty_frac=0.3)
        A = tsp.Csr(rows, cols, rp, ci, None, 0)
        f1 = tsp.features(A, 9.5, 96)
        f2 = orc.features(rows, cols, len(ci), rp, 9.5, 96)
        assert np.array_equal(f1, f2)


def test_policy_candidates_match_reference_table(tsp, orc):
    tree = orc.load_ref_policy_tree()
    if tree is None:
        pytest.skip("oracle/_ref not built")
    g, d = tsp.policy_candidates()
    cands = tree[1]
    assert len(g) == len(cands) == 66
    assert np.array_equal(g, cands[:, 0]) and np.array_equal(d, cands[:, 1])


def test_predict_returns_a_candidate(tsp):
    g, d = tsp.policy_candidates()
    f = np.array([0, 0, 1e5, 1e5, 1e6, 0.9999, 10, 50, 1, 9.5, 128], dtype=np.float64)
    for prec in (0, 1):
        pg, pd = tsp.predict(f, prec)
        assert any((pg == a and pd == b) for a, b in zip(g, d))


def test_mm_read_matches_oracle(tsp, orc, dc2_path, tmp_path):
    a = tsp.mm_read(dc2_path)
    b = orc.mm_read(dc2_path)
    for x, y in zip(a[:5], b[:5]):
        assert np.array_equal(np.asarray(x), np.asarray(y))
    assert a[5] == b[5]
    p = tmp_path / "s.mtx"
    p.write_text("%%MatrixMarket matrix coordinate real symmetric\n4 4 5\n1 1 1.5\n3 1 2\n4 2 -1\n2 2 3\n4 4 4\n")
    a, b = tsp.mm_read(str(p)), orc.mm_read(str(p))
    for x, y in zip(a[:5], b[:5]):
        assert np.array_equal(np.asarray(x), np.asarray(y))


def test_mm_read_values_correctly_rounded(tsp, tmp_path):
    """Every decimal spelling of a value parses to the correctly rounded
    double (Python's float() is correctly rounded): short decimals, 17
    significant digits, exponents at and beyond the fast-path range, signs,
    leading zeros, integers, and more than 19 digits."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal(4000) * 10.0 ** rng.integers(-30, 30, 4000)
    toks = []
    for i, v in enumerate(x):
        f = ["%.17g", "%.6e", "%.3f", "%+.9E", "%.0f", "%.25f", "%.20e"][i % 7]
        toks.append(f % v)
    toks += ["0", "-0", "+0.0", "000123", "-000.000450", "1e22", "1e23", "9007199254740993", "1.5e-22",
             "4.9e-324", "1.7976931348623157e308", "12345678901234567890123", "0.1", ".5", "5.", "-.25e+2"]
    n = len(toks)
    body = "".join(f"{i + 1} 1 {t}\n" for i, t in enumerate(toks))
    p = tmp_path / "v.mtx"
    p.write_text(f"%%MatrixMarket matrix coordinate real general\n{n} 1 {n}\n" + body)
    m, _, rp, ci, v, _ = tsp.mm_read(str(p))
    want = np.array([float(t) for t in toks])
    assert m == n and np.array_equal(rp, np.arange(n + 1))
    assert np.array_equal(v.view(np.uint64), want.view(np.uint64))


def test_mm_read_parallel_and_fallback(tsp, orc, tmp_path):
    """A multi-chunk file (parsed in parallel) and the same entries spread
    over several lines per entry (parsed by the sequential fallback) give the
    oracle's CSR, for general, symmetric, pattern and integer files."""
    rng = np.random.default_rng(12)
    n, nz = 3000, 120000
    r = rng.integers(1, n + 1, nz)
    c = rng.integers(1, n + 1, nz)
    vals = rng.integers(-50, 50, nz)
    for kind in ("real general", "real symmetric", "pattern general", "integer general"):
        if "pattern" in kind:
            lines = [f"{a} {b}" for a, b in zip(r, c)]
        else:
            lines = [f"{a} {b} {v}" for a, b, v in zip(r, c, vals)]
        if "symmetric" in kind:
            keep = r >= c
            lines = [l for l, k in zip(lines, keep) if k]
        for split in (False, True):
            body = "\n".join(l.replace(" ", "\n") if split else l for l in lines) + "\n"
            p = tmp_path / "p.mtx"
            p.write_text(f"%%MatrixMarket matrix coordinate {kind}\n% comment\n{n} {n} {len(lines)}\n" + body)
            a, b = tsp.mm_read(str(p)), orc.mm_read(str(p))
            for x, y in zip(a[:5], b[:5]):
                assert np.array_equal(np.asarray(x), np.asarray(y)), (kind, split)
            assert a[5] == b[5]


def test_mm_read_errors(tsp, tmp_path):
    with pytest.raises(tsp.TspError):
        tsp.mm_read(str(tmp_path / "missing.mtx"))
    p = tmp_path / "bad.mtx"
    p.write_text("%%MatrixMarket matrix coordinate real general\n3 3 2\n1 1 1.0\n4 1 2.0\n")
    with pytest.raises(tsp.TspError):
        tsp.mm_read(str(p))
    p.write_text("not a matrix market file\n")
    with pytest.raises(tsp.TspError):
        tsp.mm_read(str(p))


# --------------------------------------------------------------------------
# generators
# --------------------------------------------------------------------------
def test_gen_c1(tsp):
    A, B, colB, cbp = tsp.gen_config(1)
    assert (A.rows, A.cols, A.nnz, colB, cbp) == (4096, 4096, 32768, 32, 32)
    assert (np.diff(A.rowptr) == 8).all()
    for r in range(0, 4096, 97):
        row = A.colidx[A.rowptr[r]:A.rowptr[r + 1]]
        assert len(np.unique(row)) == 8 and (np.diff(row) > 0).all()
    v = A.val.view(np.float16).astype(np.float32)
    assert v.min() >= -1 and v.max() <= 1 and abs(v.mean()) < 0.05
    assert B.shape == (4096, 32)
    # determinism
    A2, B2, _, _ = tsp.gen_config(1)
    assert np.array_equal(A.colidx, A2.colidx) and np.array_equal(B, B2)


def test_gen_c2_laplacian(tsp):
    rows, cols, rp, ci = tsp.gen_structure(2)
    assert rows == 262144 and rp[-1] == 1308672
    A, B, colB, cbp = tsp.gen_config(2)
    v = A.val.view(np.float16).astype(np.float32)
    assert set(np.unique(v).tolist()) == {-1.0, 4.0}
    assert B.shape == (262144, 128)


@pytest.mark.slow
def test_gen_c3_powerlaw(tsp):
    rows, cols, rp, ci = tsp.gen_structure(3)
    L = np.diff(rp)
    assert rows == 1 << 20 and abs(L.mean() - 16) <= 0.05
    assert L.min() >= 1 and L.max() <= 10000
    # heavy tail: some rows far above the mean
    assert (L > 1000).sum() > 10


@pytest.mark.slow
def test_gen_c4_blocksparse(tsp):
    rows, cols, rp, ci = tsp.gen_structure(4)
    assert rows == 65536
    nnz = int(rp[-1])
    # singletons that land inside one of the blocks (2% of the area) are dropped
    assert abs(nnz - (335544 * 256 + 429497 * 0.98)) < 1000


def test_split_bf16_bits(tsp):
    """The split form the tf32 tile-pair kernels read B in
    (tsp_split_bf16_bits): the high bf16 half is the value's top 16 bits, the
    low half is the remainder, so hi + lo == x exactly for every tf32 value
    of magnitude at least 2^-116 (the remainder has at most 3 significant
    bits and the sign of x); below that the remainder is an fp32 subnormal,
    truncated to its top 16 bits, and hi + lo is within 2^-126 of x.  Inf
    keeps a zero low half and every NaN becomes a NaN pair.  Checked against
    the definition on random values of every exponent, the extremes and the
    specials."""
    hip = tsp.load()[0]
    rng = np.random.default_rng(5)
    raw = rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32)
    ex = (raw >> 23) & 0xFF
    raw = raw[(ex > 0) & (ex < 255)]                      # normal numbers
    x = np.concatenate([raw, np.array([0x3F800000, 0x7F7FE000, 0xFF7FE000, 0x00800000, 0x80800000, 0, 0x80000000,
                                       0x7F800000, 0xFF800000, 0x7F800001, 0x7FFFFFFF, 0xFFC00000], np.uint32)])
    tf = np.zeros_like(x)
    assert hip.tsp_round_tf32_bits(x.ctypes.data_as(C.c_void_p), tf.ctypes.data_as(C.c_void_p), x.size) == 0
    out = np.zeros_like(tf)
    assert hip.tsp_split_bf16_bits(tf.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), tf.size) == 0
    hi_bits = out & np.uint32(0xFFFF0000)
    lo_bits = (out << np.uint32(16)).astype(np.uint32)
    hi, lo = hi_bits.view(np.float32), lo_bits.view(np.float32)
    f = tf.view(np.float32)
    fin = np.isfinite(f)
    assert np.array_equal(hi_bits[fin], tf[fin] & np.uint32(0xFFFF0000))
    with np.errstate(invalid="ignore"):
        err = np.abs(hi.astype(np.float64) + lo.astype(np.float64) - f.astype(np.float64))
    big = fin & (((tf >> np.uint32(23)) & np.uint32(0xFF)) >= 11)       # |x| >= 2^-116
    assert big.sum() > 190000
    assert (err[big] == 0).all()
    assert (err[fin & ~big] < 2.0 ** -126).all()
    nz = big & (lo != 0)
    assert np.array_equal(np.signbit(lo[nz]), np.signbit(f[nz]))
    # at most 3 significant bits below the high half's 8
    assert ((lo_bits[nz] & np.uint32(0x001F0000)) == 0).all()
    inf = np.isinf(f)
    assert np.array_equal(hi_bits[inf], tf[inf]) and (lo_bits[inf] == 0).all()
    nan = np.isnan(f)
    assert nan.sum() == 3 and (out[nan] == np.uint32(0x7FC07FC0)).all()


def test_pack_3byte_bits(tsp):
    """The 3-byte form of B (tsp_pack_3byte_bits, the function the device
    packing calls): value i occupies bytes 3i .. 3i+2, little-endian, and
    holds bits 8-31 of its fp32 word, so widening (bytes as bits 8-31, zero
    low byte) gives back every tf32 value exactly -- every sign, exponent
    and mantissa, zeros, subnormals and Inf; a NaN stays a NaN (one whose
    payload lies only in the dropped byte gets the quiet bit); n must be a
    multiple of 4."""
    hip = tsp.load()[0]
    rng = np.random.default_rng(6)
    raw = rng.integers(0, 1 << 32, 100000, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([raw, np.array([0x3F800000, 0x7F7FFFFF, 0x00000001, 0x00800000, 0x80000000, 0,
                                       0x7F800000, 0xFF800000, 0x7F800001, 0xFF8000FF, 0x7FC00000, 0x7F800100],
                                      np.uint32)])
    x = x[: x.size // 4 * 4]
    tf = np.zeros_like(x)
    assert hip.tsp_round_tf32_bits(x.ctypes.data_as(C.c_void_p), tf.ctypes.data_as(C.c_void_p), x.size) == 0
    out = np.zeros(3 * tf.size, np.uint8)
    assert hip.tsp_pack_3byte_bits(tf.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), tf.size) == 0
    b = out.reshape(-1, 3).astype(np.uint32)
    wide = (b[:, 0] << np.uint32(8)) | (b[:, 1] << np.uint32(16)) | (b[:, 2] << np.uint32(24))
    f, g = tf.view(np.float32), wide.view(np.float32)
    nan = np.isnan(f)
    assert nan.sum() >= 3
    # tf32 values have a zero low byte: the form is the identity on them
    assert ((tf[~nan] & np.uint32(0xFF)) == 0).all()
    assert np.array_equal(wide[~nan], tf[~nan])
    assert np.isnan(g[nan]).all() and np.array_equal(np.signbit(g[nan]), np.signbit(f[nan]))
    assert np.array_equal(wide[nan] & np.uint32(0xFF800000), tf[nan] & np.uint32(0xFF800000))
    # a NaN whose payload is all in the low byte keeps being a NaN, quiet
    lowpay = nan & ((tf & np.uint32(0x007FFF00)) == 0)
    assert lowpay.sum() >= 2 and ((wide[lowpay] & np.uint32(0x00400000)) != 0).all()
    # four values per 12 bytes, n a multiple of 4
    assert hip.tsp_pack_3byte_bits(tf.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), 6) == 1001


def test_round_tf32_bits_special_values(tsp, orc):
    """The kernels' tf32 operand rounding (tsp_round_tf32_bits, the same
    function the device code calls) equals the oracle's nearest-even rounding
    on finite values and passes Inf and every NaN through unchanged (a bias
    added to a NaN would carry into the exponent or sign: 0x7f800001 -> Inf,
    0x7fffffff -> -0)."""
    import ctypes as C
    hip = tsp.load()[0]
    special = np.array([0x00000000, 0x80000000, 0x00000001, 0x00001000, 0x00003000, 0x00002fff, 0x3f801000,
                        0x3f803000, 0x7f7fe000, 0x7f7fefff, 0x7f7ff000, 0x7f7fffff, 0xff7fffff, 0x7f800000,
                        0xff800000, 0x7f800001, 0x7f801000, 0x7fc00000, 0x7fffe000, 0x7ffff000, 0x7fffffff,
                        0xffffffff, 0xff800001, 0xffc00001], dtype=np.uint32)
    rnd = np.random.default_rng(3).integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([special, rnd])
    out = np.zeros_like(x)
    assert hip.tsp_round_tf32_bits(x.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), x.size) == 0
    exp_all_ones = (x & 0x7F800000) == 0x7F800000
    want = orc.round_tf32_array(x.view(np.float32)).view(np.uint32)
    assert np.array_equal(out[~exp_all_ones], want[~exp_all_ones])
    assert np.array_equal(out[exp_all_ones], x[exp_all_ones])          # Inf and NaN unchanged
    f = out.view(np.float32)
    assert np.isnan(f[np.isnan(x.view(np.float32))]).all()
    # hand values: ties to even, the largest finite value rounds to Inf
    hand = dict(zip(special.tolist(), out[: special.size].tolist()))
    assert hand[0x00001000] == 0x00000000 and hand[0x00003000] == 0x00004000
    assert hand[0x3f801000] == 0x3f800000 and hand[0x3f803000] == 0x3f804000
    assert hand[0x7f7fffff] == 0x7f800000 and hand[0xff7fffff] == 0xff800000
    assert hand[0x7f7fefff] == 0x7f7fe000 and hand[0x7f7ff000] == 0x7f800000
