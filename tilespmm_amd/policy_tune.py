"""Retrain the (gamma, delta) split policy for MI355X by exhaustive tuning.

The reference ships a decision tree trained on NVIDIA GPUs
(src/model.h:14-3499); its training code is not part of the reference.  This
tool rebuilds the policy for gfx950:

  sweep  -- for each matrix of a corpus and each colB / precision, time the
            full tiled SpMM (split + tiles + cost-model thresholds + runtime
            threshold tuning, then 200 timed steps) for every one of the 66
            (gamma, delta) candidates; candidates that give the same row split
            share one measurement.  One JSON line per (matrix, colB, prec).
  fit    -- fit a regret-minimising decision tree on the sweep results: every
            leaf holds the candidate with the lowest mean normalised time
            (time / best time of that matrix) over its training matrices.  The
            tree is written as tilespmm_amd/host/model.h in the format of
            the reference's src/model.h (tilespmm_policy_node table,
            candidates, tilespmm_policy_select, predictparams_*; binary
            nodes: left_feature = right_feature = -1), so the reference's
            src/ml_predict.c builds against it into a drop-in lib/model.so.
  export -- rewrite model.h (or --out FILE) from the tree the last fit
            stored beside it (model_tree.json), without refitting.
  check  -- report, per swept matrix, the policy's pick vs the exhaustive
            optimum (the "checked against exhaustive tuning" figure).
  thsweep -- per matrix / precision / colB and active row class, the class
            kernel's time at every split threshold TH = 8..128 (distinct task
            counts only) plus the class's tile-length histogram and probed
            resources.
  thfit  -- fit the threshold cost model's weights (lambda_atom, and the
            weight of the L2 re-read term) so that the model's top-4
            thresholds, which the runtime tuning times, contain a near-best
            one; writes tilespmm_amd/host/th_calibration.h.

  python -m tilespmm_amd.policy_tune sweep --corpus small --out sweeps/policy.jsonl
  python -m tilespmm_amd.policy_tune fit --inp sweeps/policy.jsonl
  python -m tilespmm_amd.policy_tune check --inp sweeps/policy.jsonl
  python -m tilespmm_amd.policy_tune thsweep --configs 1 2 3 4 --corpus small --out sweeps/th.jsonl
  python -m tilespmm_amd.policy_tune thfit --inp sweeps/th.jsonl --header tilespmm_amd/host/th_calibration.h
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import tilespmm_amd as tsp  # noqa: E402

FEATURE_NAMES = ["rows", "cols", "nnz", "sparsity", "avg_row_nnz", "max_row_nnz", "min_row_nnz",
                 "capability", "colB"]


# ---------------------------------------------------------------------------
# corpus: seeded synthetic structures of several families
# ---------------------------------------------------------------------------
def _csr_from_rows(n_rows, n_cols, rows_cols):
    lens = np.array([len(c) for c in rows_cols], dtype=np.int64)
    rp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ci = np.concatenate([np.sort(np.asarray(c, dtype=np.int64)) for c in rows_cols]).astype(np.int32) \
        if lens.sum() else np.zeros(0, np.int32)
    return n_rows, n_cols, rp, ci


def _coo_to_csr(n_rows, n_cols, r, c):
    key = np.unique(r.astype(np.int64) * n_cols + c.astype(np.int64))
    r, c = (key // n_cols).astype(np.int32), (key % n_cols).astype(np.int32)
    rp = np.zeros(n_rows + 1, dtype=np.int64)
    np.add.at(rp, r + 1, 1)
    return n_rows, n_cols, np.cumsum(rp).astype(np.int32), c


def gen_uniform(rng, n, k):
    r = np.repeat(np.arange(n), k)
    c = rng.integers(0, n, n * k)
    return _coo_to_csr(n, n, r, c)


def gen_stencil2d(nx, nine=False):
    y, x = np.divmod(np.arange(nx * nx), nx)
    rs, cs = [], []
    offs = [(dy, dx) for dy in (-1, 0, 1) for dx in (-1, 0, 1) if nine or abs(dy) + abs(dx) <= 1]
    for dy, dx in offs:
        ok = (y + dy >= 0) & (y + dy < nx) & (x + dx >= 0) & (x + dx < nx)
        rs.append(np.nonzero(ok)[0])
        cs.append((y[ok] + dy) * nx + x[ok] + dx)
    return _coo_to_csr(nx * nx, nx * nx, np.concatenate(rs), np.concatenate(cs))


def gen_stencil3d(n):
    z, rem = np.divmod(np.arange(n ** 3), n * n)
    y, x = np.divmod(rem, n)
    rs, cs = [], []
    for dz, dy, dx in [(0, 0, 0), (-1, 0, 0), (1, 0, 0), (0, -1, 0), (0, 1, 0), (0, 0, -1), (0, 0, 1)]:
        ok = (z + dz >= 0) & (z + dz < n) & (y + dy >= 0) & (y + dy < n) & (x + dx >= 0) & (x + dx < n)
        rs.append(np.nonzero(ok)[0])
        cs.append(((z[ok] + dz) * n + y[ok] + dy) * n + x[ok] + dx)
    return _coo_to_csr(n ** 3, n ** 3, np.concatenate(rs), np.concatenate(cs))


def gen_blocks(rng, n, bs, density, singles=0.0):
    nb = n // bs
    nblk = int(density * nb * nb)
    ids = np.unique(rng.integers(0, nb * nb, nblk))
    br, bc = ids // nb, ids % nb
    ii, jj = np.meshgrid(np.arange(bs), np.arange(bs), indexing="ij")
    r = (br[:, None] * bs + ii.reshape(1, -1)).reshape(-1)
    c = (bc[:, None] * bs + jj.reshape(1, -1)).reshape(-1)
    ns = int(singles * n * n)
    if ns:
        r = np.concatenate([r, rng.integers(0, n, ns)])
        c = np.concatenate([c, rng.integers(0, n, ns)])
    return _coo_to_csr(n, n, r, c)


def gen_banded(rng, n, bw, k):
    r = np.repeat(np.arange(n), k)
    c = np.clip(r + rng.integers(-bw, bw + 1, n * k), 0, n - 1)
    return _coo_to_csr(n, n, r, c)


def gen_powerlaw(rng, n, mean, alpha):
    u = rng.random(n) + 1e-12
    lo, hi = 0.05, float(mean)
    for _ in range(50):
        xm = 0.5 * (lo + hi)
        L = np.clip(np.round(xm * u ** (-1.0 / (alpha - 1.0))), 1, min(n, 10000))
        if L.mean() < mean:
            lo = xm
        else:
            hi = xm
    L = L.astype(np.int64)
    r = np.repeat(np.arange(n), L)
    c = rng.integers(0, n, L.sum())
    return _coo_to_csr(n, n, r, c)


def gen_rmat(rng, scale, ef, a=0.57, b=0.19, c=0.19):
    n = 1 << scale
    m = n * ef
    u = np.zeros(m, dtype=np.int64)
    v = np.zeros(m, dtype=np.int64)
    for _ in range(scale):
        p = rng.random(m)
        bu = (p >= a + b).astype(np.int64)
        bv = (((p >= a) & (p < a + b)) | (p >= a + b + c)).astype(np.int64)
        u = (u << 1) | bu
        v = (v << 1) | bv
    return _coo_to_csr(n, n, np.concatenate([u, v]), np.concatenate([v, u]))


def corpus(which):
    rng = np.random.default_rng(20260777)
    items = []

    # the extra corpora: each matrix draws from its own generator, seeded
    # from its name, so any subset (--only) generates the same instances
    def seeded(name, make):
        return name, lambda: make(np.random.default_rng(int(hashlib.sha1(name.encode()).hexdigest()[:8], 16)))

    if which in ("small", "full"):
        items += [
            ("uniform_2^16_k4", lambda: gen_uniform(rng, 1 << 16, 4)),
            ("uniform_2^16_k32", lambda: gen_uniform(rng, 1 << 16, 32)),
            ("uniform_2^18_k16", lambda: gen_uniform(rng, 1 << 18, 16)),
            ("lap2d_512", lambda: gen_stencil2d(512)),
            ("lap2d9_384", lambda: gen_stencil2d(384, nine=True)),
            ("lap3d_48", lambda: gen_stencil3d(48)),
            ("blocks16_2^15_d2", lambda: gen_blocks(rng, 1 << 15, 16, 0.02, 1e-4)),
            ("blocks8_2^15_d1", lambda: gen_blocks(rng, 1 << 15, 8, 0.01)),
            ("blocks32_2^14_d4", lambda: gen_blocks(rng, 1 << 14, 32, 0.04)),
            ("blocks4_2^16_d05", lambda: gen_blocks(rng, 1 << 16, 4, 0.005)),
            ("banded_2^18_bw64_k8", lambda: gen_banded(rng, 1 << 18, 64, 8)),
            ("banded_2^17_bw512_k24", lambda: gen_banded(rng, 1 << 17, 512, 24)),
            ("powerlaw_2^18_m16_a2.1", lambda: gen_powerlaw(rng, 1 << 18, 16, 2.1)),
            ("powerlaw_2^18_m8_a1.8", lambda: gen_powerlaw(rng, 1 << 18, 8, 1.8)),
            ("rmat_16_ef16", lambda: gen_rmat(rng, 16, 16)),
            ("rmat_18_ef8", lambda: gen_rmat(rng, 18, 8)),
            ("rmat_18_ef16_skew", lambda: gen_rmat(rng, 18, 16, 0.45, 0.15, 0.15)),
        ]
    if which == "full":
        items += [
            ("uniform_2^20_k8", lambda: gen_uniform(rng, 1 << 20, 8)),
            ("lap2d_1024", lambda: gen_stencil2d(1024)),
            ("blocks16_2^16_d1", lambda: gen_blocks(rng, 1 << 16, 16, 0.01)),
            ("powerlaw_2^20_m16_a2.5", lambda: gen_powerlaw(rng, 1 << 20, 16, 2.5)),
            ("rmat_20_ef16", lambda: gen_rmat(rng, 20, 16)),
        ]
    if which == "extra":
        # neighbours of the matrices a leave-one-matrix-out refit served worst
        # (block-sparse families, small uniform matrices), more RMAT scales and
        # power-law exponents, and other band widths
        extra = [
            ("blocks32_2^15_d2", lambda rng: gen_blocks(rng, 1 << 15, 32, 0.02)),
            ("blocks32_2^13_d8", lambda rng: gen_blocks(rng, 1 << 13, 32, 0.08)),
            ("blocks16_2^14_d4", lambda rng: gen_blocks(rng, 1 << 14, 16, 0.04)),
            ("blocks64_2^14_d2", lambda rng: gen_blocks(rng, 1 << 14, 64, 0.02)),
            ("blocks8_2^14_d2", lambda rng: gen_blocks(rng, 1 << 14, 8, 0.02)),
            ("blocks8_2^16_d05", lambda rng: gen_blocks(rng, 1 << 16, 8, 0.005, 1e-5)),
            ("uniform_2^13_k8", lambda rng: gen_uniform(rng, 1 << 13, 8)),
            ("uniform_2^12_k16", lambda rng: gen_uniform(rng, 1 << 12, 16)),
            ("uniform_2^15_k32", lambda rng: gen_uniform(rng, 1 << 15, 32)),
            ("uniform_2^17_k24", lambda rng: gen_uniform(rng, 1 << 17, 24)),
            ("rmat_17_ef16", lambda rng: gen_rmat(rng, 17, 16)),
            ("rmat_19_ef8", lambda rng: gen_rmat(rng, 19, 8)),
            ("powerlaw_2^19_m12_a2.1", lambda rng: gen_powerlaw(rng, 1 << 19, 12, 2.1)),
            ("banded_2^16_bw128_k16", lambda rng: gen_banded(rng, 1 << 16, 128, 16)),
            ("blocks64_2^15_d1", lambda rng: gen_blocks(rng, 1 << 15, 64, 0.01)),
            ("blocks64_2^13_d4", lambda rng: gen_blocks(rng, 1 << 13, 64, 0.04, 1e-4)),
            ("blocks48_2^14_d2", lambda rng: gen_blocks(rng, 3 << 13, 48, 0.02)),
        ]
        items += [seeded(n, mk) for n, mk in extra]
    if which == "extra2":
        # small matrices beside the ones a depth-3 leave-one-matrix-out refit
        # served worst (small uniform and 8-row-block matrices, whose steps of
        # a few microseconds pay for every extra class launch)
        extra2 = [
            ("uniform_2^12_k8", lambda rng: gen_uniform(rng, 1 << 12, 8)),
            ("uniform_2^12_k32", lambda rng: gen_uniform(rng, 1 << 12, 32)),
            ("uniform_2^13_k16", lambda rng: gen_uniform(rng, 1 << 13, 16)),
            ("uniform_2^14_k16", lambda rng: gen_uniform(rng, 1 << 14, 16)),
            ("uniform_2^16_k16", lambda rng: gen_uniform(rng, 1 << 16, 16)),
            ("blocks8_2^13_d2", lambda rng: gen_blocks(rng, 1 << 13, 8, 0.02)),
            ("blocks8_2^14_d4", lambda rng: gen_blocks(rng, 1 << 14, 8, 0.04)),
            ("blocks8_2^15_d2", lambda rng: gen_blocks(rng, 1 << 15, 8, 0.02)),
        ]
        items += [seeded(n, mk) for n, mk in extra2]
    if which == "extra3":
        # neighbours of the one matrix a depth-4 leave-one-matrix-out refit
        # served worst (64-row dense blocks with scattered single entries,
        # unlike any other matrix of the corpora above), and the small
        # 4-per-row uniform matrices next in that ranking
        extra3 = [
            ("blocks64_2^12_d8_s", lambda rng: gen_blocks(rng, 1 << 12, 64, 0.08, 1e-4)),
            ("blocks64_2^13_d2_s", lambda rng: gen_blocks(rng, 1 << 13, 64, 0.02, 1e-4)),
            ("blocks64_2^14_d2_s", lambda rng: gen_blocks(rng, 1 << 14, 64, 0.02, 1e-4)),
            ("blocks64_2^14_d4_s", lambda rng: gen_blocks(rng, 1 << 14, 64, 0.04, 1e-4)),
            ("blocks32_2^13_d4_s", lambda rng: gen_blocks(rng, 1 << 13, 32, 0.04, 1e-4)),
            ("blocks48_2^13_d4_s", lambda rng: gen_blocks(rng, 3 << 12, 48, 0.04, 1e-4)),
            ("uniform_2^15_k4", lambda rng: gen_uniform(rng, 1 << 15, 4)),
            ("uniform_2^17_k4", lambda rng: gen_uniform(rng, 1 << 17, 4)),
        ]
        items += [seeded(n, mk) for n, mk in extra3]
    if which == "extra4":
        # neighbours of the block-sparse matrices a depth-4 leave-one-matrix-out
        # refit of all earlier sweeps served worst (16-row blocks at 2^16,
        # 8-row blocks at 2^14-2^15)
        extra4 = [
            ("blocks16_2^16_d05", lambda rng: gen_blocks(rng, 1 << 16, 16, 0.005)),
            ("blocks16_2^15_d1", lambda rng: gen_blocks(rng, 1 << 15, 16, 0.01)),
            ("blocks16_2^14_d2", lambda rng: gen_blocks(rng, 1 << 14, 16, 0.02)),
            ("blocks16_2^15_d05", lambda rng: gen_blocks(rng, 1 << 15, 16, 0.005)),
            ("blocks8_2^14_d8", lambda rng: gen_blocks(rng, 1 << 14, 8, 0.08)),
            ("blocks8_2^13_d4", lambda rng: gen_blocks(rng, 1 << 13, 8, 0.04)),
            ("blocks8_2^15_d4", lambda rng: gen_blocks(rng, 1 << 15, 8, 0.04)),
            ("blocks8_2^16_d1", lambda rng: gen_blocks(rng, 1 << 16, 8, 0.01)),
        ]
        items += [seeded(n, mk) for n, mk in extra4]
    if which == "extra5":
        # neighbours of the banded matrix a depth-4 leave-one-matrix-out refit
        # of all earlier sweeps served worst (the only banded matrix at 2^16
        # rows: band widths 64-256, 8-32 entries per row, 2^15-2^17 rows)
        extra5 = [
            ("banded_2^16_bw64_k16", lambda rng: gen_banded(rng, 1 << 16, 64, 16)),
            ("banded_2^16_bw256_k16", lambda rng: gen_banded(rng, 1 << 16, 256, 16)),
            ("banded_2^15_bw128_k16", lambda rng: gen_banded(rng, 1 << 15, 128, 16)),
            ("banded_2^17_bw128_k16", lambda rng: gen_banded(rng, 1 << 17, 128, 16)),
            ("banded_2^16_bw128_k8", lambda rng: gen_banded(rng, 1 << 16, 128, 8)),
            ("banded_2^16_bw128_k32", lambda rng: gen_banded(rng, 1 << 16, 128, 32)),
        ]
        items += [seeded(n, mk) for n, mk in extra5]
    return items


# ---------------------------------------------------------------------------
# sweep
# ---------------------------------------------------------------------------
def time_candidate(A, B, colB, cbp, g, d, reps, tune):
    """Split + tiles + thresholds (cost-model top-1, or runtime-tuned) and the
    mean time of `reps` full SpMM steps."""
    subs = tsp.matrix_split(A, g, d)
    plan = tsp.Plan.from_csr(subs, A.rows, A.cols, cbp, A.prec, B)     # tiles built on the GPU
    try:
        th, _, _ = plan.tune(tune)
        plan.warmup(5)
        ms = plan.time(reps)
        tilenum = [tsp.load()[1].tsp_plan_tilenum(plan.p, bm) for bm in (64, 16, 8)]
    finally:
        plan.close()
    return ms, th, tilenum


def sweep_matrix(name, A, colB, reps, out, tune=False):
    cbp = tsp.colB_padded(colB)
    rng = np.random.default_rng(7)
    b = np.zeros((A.cols, cbp), dtype=np.float32)
    b[:, :colB] = rng.uniform(-1, 1, (A.cols, colB))
    B = b.astype(np.float16).view(np.uint16) if A.prec == 0 else b
    f = tsp.features(A, 9.5, colB)
    gs, ds = tsp.policy_candidates()
    seen = {}
    times = []
    for g, d in zip(gs.tolist(), ds.tolist()):
        cls = tsp.split_classes(A, g, d)
        sig = hashlib.sha1(cls.tobytes()).hexdigest()
        if sig not in seen:
            seen[sig] = time_candidate(A, B, colB, cbp, g, d, reps, tune)
            print(f"   ({g:.2f},{d:.2f}): {seen[sig][0]:.4f} ms, tiles {seen[sig][2]}", flush=True)
        times.append(seen[sig][0])
    best = int(np.argmin(times))
    rec = {"matrix": name, "prec": A.prec, "colB": colB, "features": f.tolist(), "times_ms": times,
           "best": best, "best_ms": times[best], "distinct_splits": len(seen),
           "pred_default": tsp.predict(f, A.prec)}
    out.write(json.dumps(rec) + "\n")
    out.flush()
    print(f"{name} prec={A.prec} colB={colB}: best cand {best} ({gs[best]:.2f},{ds[best]:.2f}) "
          f"{times[best]:.4f} ms, worst {max(times):.4f} ms, {len(seen)} distinct splits", flush=True)


def with_values(rows, cols, rp, ci, prec, seed):
    n = len(ci)
    v = np.random.default_rng(seed).uniform(-1, 1, n).astype(np.float32)
    val = v.astype(np.float16).view(np.uint16) if prec == 0 else v
    return tsp.Csr(rows, cols, rp, ci, val, prec)


def cmd_sweep(args):
    tsp.load()
    if not tsp.device_available():
        raise SystemExit("policy_tune sweep needs a gfx950 device")
    with open(args.out, "a") as out:
        mats = []
        for cfg in args.configs:
            mats.append((f"config{cfg}", lambda cfg=cfg: tsp.gen_structure(cfg)))
        if args.corpus:
            mats += corpus(args.corpus)
        if args.only:
            mats = [m for m in mats if any(o in m[0] for o in args.only)]
        for name, make in mats:
            t0 = time.time()
            rows, cols, rp, ci = make()
            print(f"-- {name}: {rows} rows, {int(rp[-1])} nnz ({time.time() - t0:.1f}s)", flush=True)
            for prec in args.precs:
                A = with_values(rows, cols, rp, ci, prec, 11)
                for colB in args.colBs:
                    sweep_matrix(name, A, colB, args.reps, out, args.tune)


# ---------------------------------------------------------------------------
# fit + export
# ---------------------------------------------------------------------------
def load_results(paths):
    """Sweep records from one file or several."""
    recs = []
    for path in ([paths] if isinstance(paths, str) else paths):
        recs += [json.loads(l) for l in open(path) if l.strip()]
    return [r for r in recs if "times_ms" in r]


def fit_tree(recs, max_depth, min_leaf, worst_weight=0.0):
    """Greedy binary tree over features; leaf = candidate with the lowest
    summed normalised time (time / best time of the case) over its cases,
    plus worst_weight x cases x the worst of them (a robust leaf: a case
    that is far off in a leaf counts beyond its share); splits maximise the
    drop in that cost."""
    X = np.array([[r["features"][i + 2] for i in range(9)] for r in recs], dtype=np.float64)
    T = np.array([np.array(r["times_ms"]) / r["best_ms"] for r in recs], dtype=np.float64)

    def leaf_cost(idx):
        c = T[idx].sum(axis=0) + worst_weight * len(idx) * T[idx].max(axis=0)
        a = int(np.argmin(c))
        return a, float(c[a])

    nodes = []

    def build(idx, depth):
        a, cost = leaf_cost(idx)
        if depth >= max_depth or len(idx) < 2 * min_leaf:
            return -1 - a
        best = None
        for f in range(X.shape[1]):
            vals = np.unique(X[idx, f])
            for lo, hi in zip(vals[:-1], vals[1:]):
                cut = np.float32((lo + hi) / 2)
                left = idx[X[idx, f].astype(np.float32) < cut]
                right = idx[X[idx, f].astype(np.float32) >= cut]
                if len(left) < min_leaf or len(right) < min_leaf:
                    continue
                c = leaf_cost(left)[1] + leaf_cost(right)[1]
                if best is None or c < best[0] - 1e-9:
                    best = (c, f, float(cut), left, right)
        if best is None or best[0] >= cost - 1e-6:
            return -1 - a
        me = len(nodes)
        nodes.append(None)
        l_child = build(best[3], depth + 1)
        r_child = build(best[4], depth + 1)
        nodes[me] = {"feature": best[1], "cut": best[2], "left": l_child, "right": r_child}
        return me

    root = build(np.arange(len(recs)), 0)
    return root, nodes


def policy_candidates_f32():
    """The 66 (gamma, delta) actions in the reference's order
    (src/model.h:14-38): three fixed-group actions, ten gammas x six deltas,
    and three extra pairs -- built by rule, as float32."""
    c = [(0.0, 1.5), (5.0, 0.0), (5.0, 3.0)]
    c += [(g, d) for g in (1.0, 1.4, 1.8, 2.0, 2.4, 2.8, 3.0, 3.4, 3.8, 4.0) for d in (1.0, 1.2, 1.4, 1.5, 1.8, 2.0)]
    c += [(2.5, 1.0), (2.5, 1.2), (3.5, 1.0)]
    return [(np.float32(g), np.float32(d)) for g, d in c]


def _cf(x):
    """A float32 as a C literal that reads back to the same float."""
    return f"{np.float32(x).item()!r}f"


# The walk over the 4-way node format (one node may test two adjacent
# levels: child0/child1 under the left branch, child2/child3 under the
# right; a branch with feature -1 goes straight to child0 / child2), as the
# reference's policy ABI defines it; NaN features follow missing_left_mask.
_WALK = """static inline void tilespmm_policy_select(const double *features, float *gamma, float *delta, int index)
{
    while (index >= 0) {
        const tilespmm_policy_node *n = &tilespmm_shared_nodes[index];
        float v = (float)features[n->feature + 2];
        const int go_left = isnan(v) ? (n->missing_left_mask & 1) != 0 : v < n->cut;
        const int sub = go_left ? n->left_feature : n->right_feature;
        const float sub_cut = go_left ? n->left_cut : n->right_cut;
        const int lo = go_left ? n->child0 : n->child2;
        const int hi = go_left ? n->child1 : n->child3;
        if (sub < 0) {
            index = lo;
        } else {
            v = (float)features[sub + 2];
            const int bit = go_left ? 2 : 4;
            index = (isnan(v) ? (n->missing_left_mask & bit) != 0 : v < sub_cut) ? lo : hi;
        }
    }
    const int action = -1 - index;
    *gamma = tilespmm_model_candidates[action][0];
    *delta = tilespmm_model_candidates[action][1];
}"""


def export_header(path, roots, nodes_all, note):
    """Writes the policy table in the reference's model.h format (type
    tilespmm_policy_node, tables tilespmm_model_candidates and
    tilespmm_shared_nodes, tilespmm_policy_select, predictparams_fp16/_tf32;
    src/model.h:1-40,3463-3499), so the reference's own src/ml_predict.c
    builds against it unchanged and lib/model.so stays a drop-in."""
    lines = [
        "/* model.h -- (gamma, delta) split policy retrained on MI355X (gfx950).",
        " *",
        f" * GENERATED by tilespmm_amd/policy_tune.py fit ({note}).",
        " *",
        " * Same layout as the policy table the reference's src/ml_predict.c",
        " * includes: 11 input features [0, 0, rows, cols, nnz, sparsity,",
        " * avg_row_nnz, max_row_nnz, min_row_nnz, capability, colB], nodes that",
        " * compare (float)features[feature + 2] < cut, leaves -1 - action, and",
        " * 66 actions.  Binary nodes here: left_feature = right_feature = -1. */",
        "#ifndef TILESPMM_MODEL_H",
        "#define TILESPMM_MODEL_H",
        "#include <math.h>",
        "#define TILESPMM_MODEL_FEATURE_COUNT 11",
        "typedef struct {",
        "    int feature, left_feature, right_feature;",
        "    int child0, child1, child2, child3, missing_left_mask;",
        "    float cut, left_cut, right_cut;",
        "} tilespmm_policy_node;",
        "static const float tilespmm_model_candidates[66][2] = {",
    ]
    for g, d in policy_candidates_f32():
        lines.append(f"    {{{_cf(g)}, {_cf(d)}}},")
    lines += ["};", "static const tilespmm_policy_node tilespmm_shared_nodes[] = {"]
    for n in nodes_all:
        lines.append(f"    {{{n['feature']}, -1, -1, {n['left']}, -1, {n['right']}, -1, 1, "
                     f"{_cf(n['cut'])}, 0.0f, 0.0f}},")
    if not nodes_all:
        lines.append("    {4, -1, -1, -1, -1, -1, -1, 0, 0.0f, 0.0f, 0.0f},")
    lines += ["};", _WALK,
              "static inline void predictparams_fp16(const double *features, float *gamma, float *delta)",
              "{", f"    tilespmm_policy_select(features, gamma, delta, {roots[0]});", "}",
              "static inline void predictparams_tf32(const double *features, float *gamma, float *delta)",
              "{", f"    tilespmm_policy_select(features, gamma, delta, {roots[1]});", "}",
              "#endif /* TILESPMM_MODEL_H */", ""]
    open(path, "w").write("\n".join(lines))
    # the tree beside it, so `export` can rewrite the table without refitting
    with open(os.path.splitext(path)[0] + "_tree.json", "w") as fh:
        json.dump({"roots": roots, "nodes": nodes_all, "note": note}, fh, indent=1)


def cmd_export(args):
    """Rewrites the header from the tree the last fit stored beside it."""
    tree = json.load(open(os.path.splitext(args.header)[0] + "_tree.json"))
    export_header(args.out or args.header, tree["roots"], tree["nodes"], tree["note"])
    print(f"wrote {args.out or args.header}: {len(tree['nodes'])} nodes, roots {tree['roots']}")


def cmd_fit(args):
    recs = load_results(args.inp)
    roots, allnodes = [], []
    for prec in (0, 1):
        rs = [r for r in recs if r["prec"] == prec] or recs
        root, nodes = fit_tree(rs, args.depth, args.min_leaf, args.worst_weight)
        off = len(allnodes)

        def shift(x):
            return x + off if x >= 0 else x
        for n in nodes:
            allnodes.append({"feature": n["feature"], "cut": n["cut"], "left": shift(n["left"]),
                             "right": shift(n["right"])})
        roots.append(shift(root))
    note = (f"{len(recs)} swept (matrix, colB, precision) cases, depth <= {args.depth}, at least {args.min_leaf} "
            f"cases per leaf, worst-case weight {args.worst_weight}")
    if args.lomo:
        # leave one matrix out: refit without it, score its cases
        def walk(root, nodes, f):
            x = root
            while x >= 0:
                n = nodes[x]
                x = n["left"] if np.float32(f[n["feature"] + 2]) < np.float32(n["cut"]) else n["right"]
            return -1 - x
        reg, insample = [], []
        for prec in (0, 1):
            rs = [r for r in recs if r["prec"] == prec]
            root, nodes = fit_tree(rs, args.depth, args.min_leaf, args.worst_weight)
            insample += [r["times_ms"][walk(root, nodes, r["features"])] / r["best_ms"] for r in rs]
            for m in sorted(set(r["matrix"] for r in rs)):
                root, nodes = fit_tree([r for r in rs if r["matrix"] != m], args.depth, args.min_leaf,
                                       args.worst_weight)
                reg += [r["times_ms"][walk(root, nodes, r["features"])] / r["best_ms"]
                        for r in rs if r["matrix"] == m]
        note += (f"; in-sample mean x{np.mean(insample):.3f} worst x{np.max(insample):.3f}, "
                 f"leave-one-matrix-out mean x{np.mean(reg):.3f} worst x{np.max(reg):.3f}")
        print(note)
    export_header(args.header, roots, allnodes, note)
    print(f"wrote {args.header}: {len(allnodes)} nodes, roots {roots}")


def cmd_check(args):
    recs = load_results(args.inp)
    tsp.load()
    tot = []
    for r in recs:
        g, d = tsp.predict(np.array(r["features"]), r["prec"])
        gs, ds = tsp.policy_candidates()
        a = [i for i in range(len(gs)) if gs[i] == np.float32(g) and ds[i] == np.float32(d)][0]
        slow = r["times_ms"][a] / r["best_ms"]
        tot.append(slow)
        print(f"{r['matrix']:28s} prec={r['prec']} colB={r['colB']:4d} policy ({g:.2f},{d:.2f}) "
              f"{r['times_ms'][a]:.4f} ms vs best {r['best_ms']:.4f} ms -> x{slow:.3f}")
    if tot:
        print(f"mean slowdown vs exhaustive optimum: x{np.mean(tot):.3f}, worst x{np.max(tot):.3f}")


# ---------------------------------------------------------------------------
# threshold (TH) cost model calibration
# ---------------------------------------------------------------------------
def cmd_thsweep(args):
    """Per matrix / colB / precision and per active class: the time of the
    class kernel at every threshold TH = 8..128 (distinct task counts only),
    plus the class's tile-length histogram and the probed resources, so the
    cost model can be re-evaluated offline for any lambda."""
    tsp.load()
    if not tsp.device_available():
        raise SystemExit("policy_tune thsweep needs a gfx950 device")
    mats = [(f"config{cfg}", lambda cfg=cfg: tsp.gen_structure(cfg)) for cfg in args.configs]
    if args.corpus:
        mats += corpus(args.corpus)
    if args.only:
        mats = [m for m in mats if any(o in m[0] for o in args.only)]
    with open(args.out, "a") as out:
        for name, make in mats:
            rows, cols, rp, ci = make()
            for prec in args.precs:
                A = with_values(rows, cols, rp, ci, prec, 11)
                for colB in args.colBs:
                    cbp = tsp.colB_padded(colB)
                    b = np.zeros((A.cols, cbp), dtype=np.float32)
                    b[:, :colB] = np.random.default_rng(7).uniform(-1, 1, (A.cols, colB))
                    B = b.astype(np.float16).view(np.uint16) if prec == 0 else b
                    g, d = tsp.predict(tsp.features(A, 9.5, colB), prec)
                    subs = tsp.matrix_split(A, g, d)
                    tiles = [tsp.tile_create(s, A.cols, bm, prec) for s, bm in zip(subs, (64, 16, 8))]
                    plan = tsp.Plan(tiles[0], tiles[1], tiles[2], A.rows, A.cols, cbp, prec, B)
                    try:
                        for t, bm in zip(tiles, (64, 16, 8)):
                            if t.tilenum == 0:
                                continue
                            lens = np.diff(t.arrays()["tile_ptr"])
                            maxlen = int(lens.max())
                            ths, times, seen = [], [], set()
                            for th in range(8, min(128, (maxlen + 7) // 8 * 8) + 1, 8):
                                nt = int(np.where(lens <= th, 1, -(-lens // th)).sum())
                                if nt in seen:
                                    continue
                                seen.add(nt)
                                plan.set_th(th if bm == 64 else 0, th if bm == 16 else 0, th if bm == 8 else 0)
                                plan.time_class(bm, 3)
                                ths.append(th)
                                times.append(plan.time_class(bm, args.reps))
                            u, c = np.unique(lens[lens > 0], return_counts=True)
                            prm = tsp.ThParams()
                            hip, host = tsp.load()
                            host.tsp_th_params_probe(0, bm, prec, cbp, C_byref(prm))
                            rec = {"matrix": name, "prec": prec, "colB": colB, "colB_p": cbp, "bm": bm,
                                   "tilem": int(len(lens)), "hist_len": u.tolist(), "hist_cnt": c.tolist(),
                                   "th": ths, "ms": times,
                                   "params": {f: getattr(prm, f) for f, _ in tsp.ThParams._fields_}}
                            out.write(json.dumps(rec) + "\n")
                            out.flush()
                            best = ths[int(np.argmin(times))]
                            print(f"{name} prec={prec} colB={colB} bm={bm}: best TH {best}, "
                                  f"{min(times):.4f} ms ({len(ths)} THs)", flush=True)
                    finally:
                        plan.close()


def C_byref(x):
    import ctypes
    return ctypes.byref(x)


def model_top4(rec, lam, l2s=None):
    """The product cost model (tsp_optimal_th) on a recorded histogram with
    lambda_atom = lam (and lambda_l2_scale = l2s when given): its four best
    thresholds, best first."""
    prm = tsp.ThParams(**{k: v for k, v in rec["params"].items() if k in dict(tsp.ThParams._fields_)})
    prm.lambda_atom = lam
    prm.lambda_l2_scale = rec["params"].get("lambda_l2_scale", 1.0) if l2s is None else l2s
    lens = np.repeat(np.array(rec["hist_len"], dtype=np.int64), rec["hist_cnt"])
    tp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _, top4 = tsp.optimal_th(rec["bm"], rec["colB_p"], tp, prm)
    return [int(x) for x in top4 if int(x) > 0]


def th_regret(r, lam, l2s, top):
    """Measured time of the best of the model's top-`top` thresholds over the
    best measured time of any threshold."""
    t = dict(zip(r["th"], r["ms"]))
    # a TH not timed has the task count of the next smaller timed TH
    ths = model_top4(r, lam, l2s)[:top]
    cands = [max([x for x in r["th"] if x <= th] or [r["th"][0]]) for th in ths]
    return min(t[c] for c in cands) / min(r["ms"])


TH_LAMS = [0.0005, 0.001, 0.002, 0.004, 0.008, 0.015, 0.03, 0.08]
TH_L2S = [0.0, 0.0001, 0.0003, 0.001, 0.003, 0.01, 0.03, 0.1, 0.3, 1.0]


def export_th_header(path, table, note):
    lines = [
        "// th_calibration.h -- MI355X weights of the split-threshold cost model:",
        "// lambda_atom and lambda_l2_scale per (row class, precision, width class",
        "// colB_p == 32 or >= 64), chosen to minimise the measured regret of the",
        "// model's top-4 thresholds over an exhaustive per-threshold sweep.",
        "//",
        f"// GENERATED by tilespmm_amd/policy_tune.py thfit ({note}).",
        "#pragma once",
        "",
        "struct tsp_th_weight {",
        "    int bm, prec, wide;",
        "    float lambda_atom, lambda_l2_scale;",
        "};",
        "",
        "static const tsp_th_weight tsp_th_weight_table[] = {",
    ]
    for (bm, prec, wide), (lam, l2s) in sorted(table.items()):
        lines.append(f"    {{{bm}, {prec}, {wide}, {float(lam)!r}f, {float(l2s)!r}f}},")
    lines += ["};", ""]
    open(path, "w").write("\n".join(lines))


def fit_th_pair(recs, top):
    """(lambda_atom, lambda_l2_scale) minimising the mean top-k regret over
    recs; ties -> the larger weights (closer to the reference's model)."""
    res = []
    for l2s in TH_L2S:
        for lam in TH_LAMS:
            reg = [th_regret(r, lam, l2s, top) for r in recs]
            res.append((round(float(np.mean(reg)), 4), -l2s, -lam))
    best = min(res)
    return -best[2], -best[1]


def cmd_thfit(args):
    """Fits the cost model's (lambda_atom, lambda_l2_scale) on a thsweep file:
    one pair for all classes by default (per-class fits overfit the small
    64-row groups), per (class, precision, width) group with --per-group.
    Reports the top-4 regret in-sample and leave-one-matrix-out; with
    --header writes the generated calibration table."""
    tsp.load()
    recs = [json.loads(l) for l in open(args.inp) if l.strip()]
    keyf = lambda r: (r["bm"], r["prec"], 0 if r["colB_p"] == 32 else 1)
    groups = {}
    for r in recs:
        groups.setdefault(keyf(r), []).append(r)

    def fit(rs):
        if not args.per_group:
            pair = fit_th_pair(rs, args.top)
            return {k: pair for k in groups}
        return {k: fit_th_pair([r for r in rs if keyf(r) == k] or rs, args.top) for k in groups}

    table = fit(recs)
    new = [th_regret(r, *table[keyf(r)], args.top) for r in recs]
    cur = [th_regret(r, r["params"]["lambda_atom"], None, args.top) for r in recs]
    lomo = []
    for m in sorted(set(r["matrix"] for r in recs)):
        t = fit([r for r in recs if r["matrix"] != m])
        lomo += [th_regret(r, *t[keyf(r)], args.top) for r in recs if r["matrix"] == m]
    for key, rs in sorted(groups.items()):
        g = [th_regret(r, *table[key], args.top) for r in rs]
        print(f"class bm={key[0]} prec={key[1]} width={'32' if key[2] == 0 else '>=64'}: {len(rs)} cases; "
              f"lambda_atom {table[key][0]} l2_scale {table[key][1]}: mean x{np.mean(g):.3f} "
              f"worst x{np.max(g):.3f}")
    note = (f"{len(recs)} class sweeps, {'per-group' if args.per_group else 'pooled'} fit, top-{args.top} "
            f"regret mean x{np.mean(new):.3f} worst x{np.max(new):.3f}, leave-one-matrix-out mean "
            f"x{np.mean(lomo):.3f} worst x{np.max(lomo):.3f}; as recorded mean x{np.mean(cur):.3f} "
            f"worst x{np.max(cur):.3f}")
    print(note)
    if args.header:
        export_th_header(args.header, table, note)
        print("wrote", args.header)


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("thsweep")
    t.add_argument("--configs", type=int, nargs="*", default=[])
    t.add_argument("--corpus", choices=["small", "full"], default=None)
    t.add_argument("--precs", type=int, nargs="*", default=[0, 1])
    t.add_argument("--colBs", type=int, nargs="*", default=[32, 128])
    t.add_argument("--reps", type=int, default=20)
    t.add_argument("--only", nargs="*", default=None)
    t.add_argument("--out", required=True)
    tf = sub.add_parser("thfit")
    tf.add_argument("--top", type=int, default=4,
                    help="regret of the best measured among the model's top-k (the plan tunes k=4)")
    tf.add_argument("--inp", required=True)
    tf.add_argument("--header", default=None, help="write the calibration table (host/th_calibration.h)")
    tf.add_argument("--per-group", action="store_true", help="one weight pair per (class, prec, width)")
    s = sub.add_parser("sweep")
    s.add_argument("--configs", type=int, nargs="*", default=[])
    s.add_argument("--corpus", choices=["small", "full", "extra", "extra2", "extra3", "extra4", "extra5"], default=None)
    s.add_argument("--precs", type=int, nargs="*", default=[0, 1])
    s.add_argument("--colBs", type=int, nargs="*", default=[32, 128])
    s.add_argument("--reps", type=int, default=30)
    s.add_argument("--tune", action="store_true", help="runtime-tune thresholds for every candidate")
    s.add_argument("--only", nargs="*", default=None, help="substrings of matrix names to keep")
    s.add_argument("--out", required=True)
    f = sub.add_parser("fit")
    f.add_argument("--inp", required=True, nargs="+")
    f.add_argument("--header", default=os.path.join(HERE, "host", "model.h"))
    f.add_argument("--depth", type=int, default=4)
    f.add_argument("--min-leaf", type=int, default=3)
    f.add_argument("--worst-weight", type=float, default=0.0,
                   help="leaf cost = summed regret + this x cases x worst regret (robust leaves)")
    f.add_argument("--lomo", action="store_true", help="also report leave-one-matrix-out regret")
    c = sub.add_parser("check")
    c.add_argument("--inp", required=True, nargs="+")
    e = sub.add_parser("export")
    e.add_argument("--header", default=os.path.join(HERE, "host", "model.h"),
                   help="the fitted table whose model_tree.json is read")
    e.add_argument("--out", default=None, help="write here instead (e.g. a reference checkout's src/model.h)")
    e.add_argument("--reference", action="store_true",
                   help="the reference's src/model.h format (the only format this build writes)")
    args = ap.parse_args()
    {"sweep": cmd_sweep, "fit": cmd_fit, "check": cmd_check, "thsweep": cmd_thsweep,
     "thfit": cmd_thfit, "export": cmd_export}[args.cmd](args)


if __name__ == "__main__":
    main()
