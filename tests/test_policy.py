"""The MI355X (gamma, delta) policy: its tree walk matches the oracle's
restatement of the reference walk, and its picks are checked against the
exhaustive tuning sweep it was trained on (tilespmm_amd/policy_data)."""
import json
import os
import re

import numpy as np
import pytest

from conftest import ROOT

DATA = os.path.join(ROOT, "tilespmm_amd", "policy_data", "mi355x_sweep.jsonl")
HEADER = os.path.join(ROOT, "tilespmm_amd", "host", "model.h")


def header_tree(orc):
    text = open(HEADER).read()
    rows = re.findall(r"\{\s*(-?\d+),\s*(-?\d+),\s*(-?\d+),\s*(-?\d+),\s*(-?\d+),\s*(-?\d+),\s*(-?\d+),\s*(-?\d+),"
                      r"\s*([-0-9.e]+)f,\s*([-0-9.e]+)f,\s*([-0-9.e]+)f\s*\}", text)
    nodes = (orc.PolicyNode * len(rows))()
    for i, r in enumerate(rows):
        for j, name in enumerate(["feature", "left_feature", "right_feature", "child0", "child1", "child2",
                                  "child3", "missing_left_mask"]):
            setattr(nodes[i], name, int(r[j]))
        nodes[i].cut, nodes[i].left_cut, nodes[i].right_cut = float(r[8]), float(r[9]), float(r[10])
    r16 = int(re.search(r"predictparams_fp16\(.*?tilespmm_policy_select\(features, gamma, delta, (-?\d+)\)",
                        text, re.S).group(1))
    r32 = int(re.search(r"predictparams_tf32\(.*?tilespmm_policy_select\(features, gamma, delta, (-?\d+)\)",
                        text, re.S).group(1))
    return nodes, r16, r32


def records():
    return [json.loads(l) for l in open(DATA) if l.strip()]


def test_product_walk_matches_oracle_walk(tsp, orc):
    nodes, r16, r32 = header_tree(orc)
    g, d = tsp.policy_candidates()
    cands = np.stack([g, d], axis=1).astype(np.float32)
    rng = np.random.default_rng(3)
    feats = [np.array(r["features"]) for r in records()]
    for _ in range(300):
        f = feats[rng.integers(len(feats))].copy()
        f[2 + rng.integers(9)] *= rng.uniform(0.5, 2.0)
        feats.append(f)
    for f in feats:
        assert tsp.predict(f, 0) == orc.policy_select(f, nodes, cands, r16)
        assert tsp.predict(f, 1) == orc.policy_select(f, nodes, cands, r32)


def _predictor(path):
    import ctypes as C
    lib = C.CDLL(path)
    for name in ("tilespmm_predict_fp16", "tilespmm_predict_tf32"):
        fn = getattr(lib, name)
        fn.restype = None
        fn.argtypes = [C.POINTER(C.c_double), C.POINTER(C.c_float), C.POINTER(C.c_float)]

    def predict(f, prec):
        f = np.ascontiguousarray(f, dtype=np.float64)
        g, d = C.c_float(), C.c_float()
        fn = lib.tilespmm_predict_fp16 if prec == 0 else lib.tilespmm_predict_tf32
        fn(f.ctypes.data_as(C.POINTER(C.c_double)), C.byref(g), C.byref(d))
        return np.float32(g.value), np.float32(d.value)
    return predict


REF_SRC = "/root/reference/src"


def test_table_is_a_model_so_drop_in(tsp):
    """The retrained table is written in the reference's model.h format: the
    reference's own src/ml_predict.c, built against it (oracle/Makefile,
    target _ref/model_mi355x.so), predicts exactly what this build's
    CPU-only lib/model.so and the host library predict -- on the reference's
    golden feature vectors, the sweep's features and perturbed ones, NaN
    features included.  The reference's own table picks differently, so the
    build really used the retrained one."""
    import subprocess
    if not os.path.exists(os.path.join(REF_SRC, "ml_predict.c")):
        pytest.skip("reference checkout not mounted: src/ml_predict.c is needed to build the drop-in check")
    r = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "_ref/model_mi355x.so", "_ref/model.so"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    ref_built = _predictor(os.path.join(ROOT, "oracle", "_ref", "model_mi355x.so"))
    ours = _predictor(os.path.join(ROOT, "tilespmm_amd", "lib", "model.so"))
    ref_table = _predictor(os.path.join(ROOT, "oracle", "_ref", "model.so"))
    gold = json.load(open(os.path.join(ROOT, "tests", "golden", "policy_golden.json")))["vectors"]
    feats = [np.array(v["f"], dtype=np.float64) for v in gold] + [np.array(r["features"]) for r in records()]
    rng = np.random.default_rng(5)
    for f in list(feats[:400]):
        g = f.copy()
        g[2 + rng.integers(9)] *= rng.uniform(0.3, 3.0)
        feats.append(g)
        h = f.copy()
        h[2 + rng.integers(9)] = np.nan
        feats.append(h)
    differs = 0
    for f in feats:
        for prec in (0, 1):
            a = ref_built(f, prec)
            assert a == ours(f, prec) == tsp.predict(f, prec), (f, prec)
            differs += a != ref_table(f, prec)
    assert differs > 0


EXTRA = os.path.join(ROOT, "tilespmm_amd", "policy_data", "mi355x_sweep_extra.jsonl")
EXTRA2 = os.path.join(ROOT, "tilespmm_amd", "policy_data", "mi355x_sweep_extra2.jsonl")
EXTRA3 = os.path.join(ROOT, "tilespmm_amd", "policy_data", "mi355x_sweep_extra3.jsonl")
EXTRA4 = os.path.join(ROOT, "tilespmm_amd", "policy_data", "mi355x_sweep_extra4.jsonl")
EXTRA5 = os.path.join(ROOT, "tilespmm_amd", "policy_data", "mi355x_sweep_extra5.jsonl")


def all_records():
    return records() + [json.loads(l) for f in (EXTRA, EXTRA2, EXTRA3, EXTRA4, EXTRA5) for l in open(f) if l.strip()]


def test_policy_against_exhaustive_tuning(tsp):
    """On its training sweeps (584 cases, 73 matrices) the shipped tree is
    x1.010 of the exhaustive optimum on average and x1.27 at worst; the
    provisional single-leaf table (candidate 24) is x1.15 (worst x3.32)."""
    g, d = tsp.policy_candidates()
    slow = []
    recs = all_records()
    assert len(recs) == 584 and len({r["matrix"] for r in recs}) == 73
    for r in recs:
        pg, pd = tsp.predict(np.array(r["features"]), r["prec"])
        a = [i for i in range(len(g)) if g[i] == np.float32(pg) and d[i] == np.float32(pd)]
        assert a, (pg, pd)
        slow.append(r["times_ms"][a[0]] / r["best_ms"])
    assert np.mean(slow) <= 1.011 and max(slow) <= 1.28, (np.mean(slow), max(slow))
    prov = [r["times_ms"][24] / r["best_ms"] for r in recs]
    assert np.mean(slow) < np.mean(prov)


def test_policy_leave_one_matrix_out():
    """The fit generalises to matrices it has not seen: refitting without
    each matrix in turn (policy_tune's fit as shipped: depth 4, at least 4
    cases per leaf, worst-case weight 0.3) and scoring the held-out matrix's
    cases gives x1.032 on average, with 83% of the cases within x1.05.  The
    worst held-out cases (x1.69 and x1.64 for small 64-row-block matrices
    with scattered entries, x1.64 for a banded matrix) are matrices of a few
    microseconds per step whose best split the 11 policy features cannot
    tell from their neighbours' (banded matrices that differ only in band
    width have the same features)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("policy_tune", os.path.join(ROOT, "tilespmm_amd", "policy_tune.py"))
    pt = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(pt)
    recs = all_records()

    def walk(root, nodes, f):
        x = root
        while x >= 0:
            n = nodes[x]
            x = n["left"] if np.float32(f[n["feature"] + 2]) < np.float32(n["cut"]) else n["right"]
        return -1 - x
    held = []
    for prec in (0, 1):
        rs = [r for r in recs if r["prec"] == prec]
        for m in sorted({r["matrix"] for r in rs}):
            root, nodes = pt.fit_tree([r for r in rs if r["matrix"] != m], 4, 4, 0.3)
            held += [r["times_ms"][walk(root, nodes, r["features"])] / r["best_ms"] for r in rs if r["matrix"] == m]
    held = np.array(held)
    assert held.size == 584
    assert held.mean() <= 1.033 and (held <= 1.05).mean() >= 0.82 and held.max() <= 1.69, \
        (held.mean(), (held <= 1.05).mean(), held.max())


HELDOUT = os.path.join(ROOT, "tilespmm_amd", "policy_data", "mi355x_heldout_config5.jsonl")


def test_policy_on_held_out_config5(tsp):
    """Configuration 5 (RMAT scale 22) is not in the training sweep.  Its
    exhaustive sweep with the full shipped path (runtime tuning of every
    candidate) puts the policy's pick within a few percent of the best
    candidate: fp16 x1.000 (colB 64) and x1.038 (colB 128), tf32 x1.002 and
    x1.000."""
    g, d = tsp.policy_candidates()
    recs = [json.loads(l) for l in open(HELDOUT) if l.strip()]
    assert {(r["prec"], r["colB"]) for r in recs} == {(0, 64), (0, 128), (1, 64), (1, 128)}
    slow = []
    for r in recs:
        pg, pd = tsp.predict(np.array(r["features"]), r["prec"])
        a = [i for i in range(len(g)) if g[i] == np.float32(pg) and d[i] == np.float32(pd)]
        assert a, (pg, pd)
        slow.append(r["times_ms"][a[0]] / r["best_ms"])
    assert max(slow) <= 1.05 and np.mean(slow) <= 1.02, slow


TH_DATA = os.path.join(ROOT, "tilespmm_amd", "policy_data", "mi355x_thsweep.jsonl")


def th_regret(tsp, r, lam, l2s):
    """Measured time of the best of the cost model's top-4 thresholds (what
    the runtime tuning times) over the best threshold of the sweep."""
    p = tsp.ThParams(**{k: v for k, v in r["params"].items() if k in dict(tsp.ThParams._fields_)})
    p.lambda_atom, p.lambda_l2_scale = lam, l2s
    lens = np.repeat(np.array(r["hist_len"], dtype=np.int64), r["hist_cnt"])
    tp = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _, top4 = tsp.optimal_th(r["bm"], r["colB_p"], tp, p)
    t = dict(zip(r["th"], r["ms"]))
    # a threshold that was not timed has the task count of the next smaller timed one
    cands = [max([x for x in r["th"] if x <= th] or [r["th"][0]]) for th in top4]
    return min(t[c] for c in cands) / min(r["ms"])


def test_threshold_weights_against_exhaustive_sweep(tsp):
    """The MI355X cost-model weights (tsp_th_weights) put a threshold within a
    few percent of the best measured one into the top 4 on every class sweep;
    the reference's weights (L2 scale 1, per-class lambda_atom table) do not."""
    recs = [json.loads(l) for l in open(TH_DATA) if l.strip()]
    assert len(recs) >= 60
    new, ref = [], []
    for r in recs:
        lam, l2s = tsp.th_weights(r["bm"], r["prec"], r["colB_p"])
        new.append(th_regret(tsp, r, lam, l2s))
        ref.append(th_regret(tsp, r, r["params"]["lambda_atom"], 1.0))
    # on the recorded sweep (the current kernels) the worst case costs x1.10;
    # on the sweep the weights were fitted to, one outlier (config 4, colB
    # 128, 16-row tiles of dense 16x16 blocks: no split was best and the top
    # 4 stop at 64) cost x1.29 and every other case was within x1.09
    assert np.mean(new) <= 1.01 and max(new) <= 1.30, (np.mean(new), max(new))
    assert sorted(new)[-2] <= 1.10
    assert np.mean(ref) > 1.10 and np.mean(new) < np.mean(ref)
