"""Host preprocessing under AddressSanitizer and UndefinedBehaviorSanitizer.

Builds tests/sanitize_host.cpp together with the host library's sources
(Matrix Market reader, row split, tile conversion, schedule, cost model,
policy, generators) with -fsanitize=address,undefined, on the CPU, and runs
it: a sanitizer report (out-of-bounds access, use after free, leak, signed
overflow, misaligned access ...) fails the test.
"""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT

HOST = os.path.join(ROOT, "tilespmm_amd", "host")
SOURCES = ["mmio.cpp", "split.cpp", "tiles.cpp", "cost_model.cpp", "policy.cpp", "gen.cpp"]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_preprocessing_under_asan_ubsan(tmp_path):
    exe = tmp_path / "sanitize_host"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fopenmp", "-mf16c",
           "-fsanitize=address,undefined", "-static-libasan", "-fno-sanitize-recover=undefined", "-I", os.path.join(ROOT, "include"),
           "-o", str(exe), os.path.join(ROOT, "tests", "sanitize_host.cpp")] + [os.path.join(HOST, s) for s in SOURCES]
    build = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert build.returncode == 0, build.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="4")
    run = subprocess.run([str(exe), str(tmp_path)], capture_output=True, text=True, timeout=600, env=env)
    assert run.returncode == 0, (run.stdout[-2000:], run.stderr[-6000:])
    assert "sanitize_host: ok" in run.stdout
