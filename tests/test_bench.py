"""bench.py's one-line JSON contract: the fields the driver reads, their
types and the relations between them (value from ms_per_step, roofline.frac
from achieved / peak), and the refusal of more than one GPU."""
import json
import os
import subprocess
import sys

import pytest

from conftest import ROOT

BENCH = os.path.join(ROOT, "bench.py")


def test_alg_bytes_formula():
    """The roofline's unit of work: configuration 5 (RMAT scale 22, tf32,
    colB 64; nnz as the generator makes it) moves 3190.7 MB."""
    sys.path.insert(0, ROOT)
    import bench
    m = 1 << 22
    assert bench.alg_bytes(m, 128305642, 4, m, 64, 4) == 4 * (m + 1) + 128305642 * 8 + 2 * m * 64 * 4
    assert round(bench.alg_bytes(m, 128305642, 4, m, 64, 4) / 1e6, 1) == 3190.7


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.gpu
def test_bench_json_line(tsp):
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    print("bench.py --config 1 --targets 1 --steps 20 --warmup 5", flush=True)
    r = subprocess.run([sys.executable, "-u", BENCH, "--config", "1", "--targets", "1", "--steps", "20",
                        "--warmup", "5", "--class-reps", "10", "--cold-reps", "3"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if l.strip()]
    assert len(lines) == 1, r.stdout
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 20 and d["warmup"] == 5
    assert d["unit"] == "TFLOPS" and d["higher_is_better"] is True and d["vs_baseline"] is None
    assert d["dtype"] == "fp16" and d["data"] == "synthetic" and "workload" in d["config"]
    cfg = d["config"]
    assert cfg["nnz"] == 32768 and cfg["colB"] == 32
    # value is 2 nnz colB / step time
    assert d["ms_per_step"] > 0
    assert d["value"] == pytest.approx(2 * cfg["nnz"] * cfg["colB"] / (d["ms_per_step"] * 1e-3) / 1e12, rel=2e-3)
    roof = d["roofline"]
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in roof, k
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"], rel=1e-2, abs=1e-4)
    # algorithmic bytes: CSR A, all K rows of B once, C once in fp32
    # (4(M+1) + nnz(4+s) + K*N*s + M*N*4 at M = K = 4096, nnz 32768, N 32, fp16)
    assert roof["step_alg_bytes"] == 4 * 4097 + 32768 * 6 + 4096 * 32 * 2 + 4096 * 32 * 4
    assert roof["alg_bytes_touched_per_launch"] <= roof["alg_bytes_per_launch"]
    # the same achieved rate against the copy bandwidth measured in the run
    assert 1000 < roof["copy_peak_gbs"] < roof["peak"]
    assert roof["frac_of_copy"] == pytest.approx(roof["achieved"] / roof["copy_peak_gbs"], rel=1e-2, abs=1e-4)
    cpu = d["cpu_baseline"]
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in cpu, k
    assert cpu["kind"] in ("port", "reference") and cpu["value"] > 0 and cpu["cores"] >= 1
    assert "whole matrix" in cpu["sample"]
    cold = d["cold_cache"]
    assert cold["reps"] == 3 and cold["ms_per_step"] > 0 and cold["copy_cold_ms"] > 0
    # the HIP graph leg: the same steps replayed from a graph
    gr = d["graph"]
    assert gr["steps_per_graph"] >= 10 and gr["replays"] >= 3 and gr["ms_per_step"] > 0
    assert gr["tflops"] == pytest.approx(2 * 32768 * 32 / (gr["ms_per_step"] * 1e-3) / 1e12, rel=2e-3)
    # the roofline's kernel runs inside the step: its time cannot exceed the
    # step's (C1's 4-microsecond steps are launch-bound and excepted)
    if d["ms_per_step"] > 0.05:
        assert roof["kernel_ms"] <= d["ms_per_step"] * 1.05
    assert d["warmup_clock"]["steps"] >= 1 and d["long_window"]["steps"] >= 20
    assert d["gather"]["ceiling_glines_per_s"] > 0
    # the floor of the headline's own B-row gathers, beside its step
    fl = d["gather_floor"]
    assert fl["row_bytes"] == 64 and fl["indices"] >= 32768 and fl["floor_ms"] > 0
    assert fl["floor_over_step"] == pytest.approx(fl["floor_ms"] / d["ms_per_step"], rel=1e-2, abs=1e-3)
    # the fp16 / colB 128 target record of the same run
    t = d["targets"]["C1"]
    assert "fp16, colB 128" in t["workload"] and t["tflops"] > 0
    assert t["tflops"] == pytest.approx(2 * 32768 * 128 / (t["ms_per_step"] * 1e-3) / 1e12, rel=2e-3)
    assert t["frac"] > 0 and t["kernel"].startswith("spmm_kernel<")
    assert t["cold_cache"]["reps"] == 3 and t["cold_cache"]["ms_per_step"] > 0
    assert d["replay"].startswith("--no-tune --th ")


@pytest.mark.gpu
def test_bench_hub_split(tsp):
    """bench.py --hub-split: the whole matrix, its hub part and its cold part
    as three tuned plans; one line per plan, then the summary."""
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    print("bench.py --config 1 --hub-split 256 --steps 10", flush=True)
    r = subprocess.run([sys.executable, "-u", BENCH, "--config", "1", "--hub-split", "256", "--steps", "10"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [json.loads(l) for l in r.stdout.splitlines() if l.strip()]
    assert [l.get("hub_split", "summary").split()[0] for l in lines] == ["whole", "hub", "cold", "summary"]
    s = lines[-1]
    assert s["hub_split_summary"] == 256 and 0 < s["hub_share_of_nnz"] < 1
    assert lines[1]["nnz"] + lines[2]["nnz"] == lines[0]["nnz"] == 32768
    assert s["hub_plus_cold_ms"] == pytest.approx(s["hub_ms"] + s["cold_ms"], abs=2e-5)


@pytest.mark.gpu
def test_bench_gather_stream(tsp):
    """bench.py --gather-stream: the workload's own B-row index stream (every
    class's tile column indices) gathered alone, in place and with the hot
    rows, beside the tuned step; on configuration 1 (fp16, colB 32: 64-byte
    rows) every index is a gather of 4096 rows."""
    if not tsp.device_available():
        pytest.fail("no gfx950 device: GPU tests need an MI355X")
    print("bench.py --config 1 --gather-stream --steps 20", flush=True)
    r = subprocess.run([sys.executable, "-u", BENCH, "--config", "1", "--gather-stream", "--steps", "20"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    j = json.loads(r.stdout.strip().splitlines()[-1])
    assert j["row_bytes"] == 64 and j["indices"] % 16 == 0 and j["indices"] >= 32768
    for k in ("canonical", "hot_rows"):
        assert j[k]["ms"] > 0 and j[k]["g_rows_per_s"] > 0
    assert 0 <= j["hot_share_of_gathers"] <= 1 and j["tuned_step_ms"] > 0
