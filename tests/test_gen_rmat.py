"""Configuration 5's RMAT generator (tsp_gen_rmat, host/gen.cpp) at scale 12,
against an independent numpy restatement of its random streams -- xoshiro256**
seeded through splitmix64, one stream per chunk of 1/1024 of the edges, one
uniform draw per level deciding the quadrant (a, b, c, d) = (.57, .19, .19,
.05) -- and against the properties configuration 5 states: symmetric, no
duplicate (row, column), self-loops kept, columns ascending, values
1/deg(row) rounded to the value type (exact in tf32 / fp16)."""
import numpy as np
import pytest

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def u64(v):
    return np.uint64(v)


def splitmix64(x):
    """(new state, output) of SplitMix64 on a uint64 array (wrapping arithmetic)."""
    x = x + u64(0x9E3779B97F4A7C15)
    z = x
    z = (z ^ (z >> u64(30))) * u64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> u64(27))) * u64(0x94D049BB133111EB)
    return x, z ^ (z >> u64(31))


def rotl(v, k):
    return (v << u64(k)) | (v >> u64(64 - k))


def stream_seed(seed, tag, chunks):
    x = np.full(chunks.shape, u64(seed), dtype=np.uint64) ^ (u64(tag) * u64(0xD1B54A32D192ED03))
    _, a = splitmix64(x)
    x = a ^ (chunks * u64(0x9E3779B97F4A7C15))
    _, out = splitmix64(x)
    return out


def xoshiro_states(seeds):
    s = []
    x = seeds.copy()
    for _ in range(4):
        x, z = splitmix64(x)
        s.append(z)
    return s


def xoshiro_next(s):
    r = rotl(s[1] * u64(5), 7) * u64(9)
    t = s[1] << u64(17)
    s[2] ^= s[0]
    s[3] ^= s[1]
    s[1] ^= s[2]
    s[0] ^= s[3]
    s[2] ^= t
    s[3] = rotl(s[3], 45)
    return r


def rmat_restated(scale, edges, seed):
    chunks = 1024
    per = (edges + chunks - 1) // chunks
    s = xoshiro_states(stream_seed(seed, 1, np.arange(chunks, dtype=np.uint64)))
    u = np.zeros((chunks, per), dtype=np.int64)
    v = np.zeros((chunks, per), dtype=np.int64)
    for e in range(per):
        for _ in range(scale):
            p = (xoshiro_next(s) >> u64(11)).astype(np.float64) * 2.0 ** -53
            bu = p >= 0.76
            bv = ((p >= 0.57) & (p < 0.76)) | (p >= 0.95)
            u[:, e] = (u[:, e] << 1) | bu
            v[:, e] = (v[:, e] << 1) | bv
    u, v = u.reshape(-1)[:edges], v.reshape(-1)[:edges]     # chunk c holds edges c*per .. c*per+per-1
    n = 1 << scale
    key = np.unique(np.concatenate([u * n + v, v * n + u]))
    r, c = key // n, key % n
    rp = np.concatenate([[0], np.cumsum(np.bincount(r, minlength=n))])
    return rp.astype(np.int32), c.astype(np.int32)


def test_splitmix64_published_value():
    # SplitMix64 from state 0: first output 0xE220A8397B1DCDAF (Vigna's reference generator)
    _, z = splitmix64(np.zeros(1, dtype=np.uint64))
    assert int(z[0]) == 0xE220A8397B1DCDAF


@pytest.mark.parametrize("prec", [0, 1])
def test_rmat_scale12_matches_restatement(tsp, orc, prec):
    scale, edges, seed = 12, 16 << 12, 20260005
    A = tsp.gen_rmat(scale, edges, seed, prec)
    rp, ci = rmat_restated(scale, edges, seed)
    assert A.rows == A.cols == 1 << scale
    assert np.array_equal(A.rowptr, rp) and np.array_equal(A.colidx, ci)
    n = A.rows
    r = np.repeat(np.arange(n), np.diff(A.rowptr))
    # columns strictly ascending within each row: sorted, no duplicates
    same_row = r[1:] == r[:-1]
    assert (A.colidx[1:][same_row] > A.colidx[:-1][same_row]).all()
    # symmetric: the transposed pattern is the same set
    fwd = r.astype(np.int64) * n + A.colidx
    bwd = A.colidx.astype(np.int64) * n + r
    assert np.array_equal(np.sort(fwd), np.sort(bwd))
    # self-loops kept (vertex 0 draws quadrant a at every level often enough)
    assert (A.colidx == r).sum() > 0
    # dedup removed something: fewer entries than the 2 * edges directed pairs
    assert A.nnz < 2 * edges
    # values: 1/deg(row) in fp32, rounded to the value type
    deg = np.diff(A.rowptr)[r].astype(np.float32)
    q = np.float32(1.0) / deg
    if prec == 1:
        want = orc.round_tf32_array(q)
        got = A.val.view(np.float32) if A.val.dtype == np.uint32 else A.val.astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert (got.view(np.uint32) & 0x1FFF == 0).all()          # exact in tf32
    else:
        want = q.astype(np.float16)
        assert np.array_equal(A.val.view(np.uint16), want.view(np.uint16))
