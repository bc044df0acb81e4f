"""The C-ABI libraries load and export every function include/*.h declares
(no compute calls: this runs without a GPU)."""
import ctypes as C
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADERS = ["include/tilespmm_hip.h", "include/tilespmm.h"]


def declared(header):
    text = open(os.path.join(ROOT, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "defined")))


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if l.strip()}


def test_headers_declare_expected_entry_points():
    hip = declared(HEADERS[0])
    host = declared(HEADERS[1])
    for n in ("tsp_spmm_launch", "tsp_switch_v64", "tsp_switch_v16", "tsp_switch_v8", "tsp_device_init"):
        assert n in hip
    for n in ("tsp_matrix_split", "tsp_tile_create", "tsp_tile_pretreatment", "tsp_optimal_th",
              "tilespmm_predict_fp16", "tilespmm_predict_tf32", "tsp_call_tilespmm"):
        assert n in host


def test_libraries_export_every_declared_symbol(tsp):
    libdir = os.path.join(ROOT, "tilespmm_amd", "lib")
    hip_syms = exported(os.path.join(libdir, "libtilespmm_hip.so"))
    host_syms = exported(os.path.join(libdir, "libtilespmm_host.so"))
    missing = [n for n in declared(HEADERS[0]) if n not in hip_syms]
    missing += [n for n in declared(HEADERS[1]) if n not in host_syms]
    assert not missing, missing


def test_python_binding_covers_headers(tsp):
    bound = set(tsp.HIP_SYMBOLS) | set(tsp.HOST_SYMBOLS)
    missing = [n for h in HEADERS for n in declared(h) if n not in bound]
    assert not missing, missing


def test_kernels_built_for_gfx950():
    lib = os.path.join(ROOT, "tilespmm_amd", "lib", "libtilespmm_hip.so")
    # the embedded offload bundle names its target triple
    data = open(lib, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_error_strings_and_arg_checks(tsp):
    hip, _ = tsp.load()
    assert b"gfx950" in hip.tsp_hip_version()
    assert hip.tsp_hip_error_string(1001)
    # invalid class / width are rejected on the host before any launch
    assert hip.tsp_spmm_launch(32, 0, 1, 128, None, None, None, None, None, None, 0, None) == 1001
    assert hip.tsp_spmm_launch(16, 0, 1, 96, None, None, None, None, None, None, 0, None) == 1001
    assert hip.tsp_spmm_launch(16, 2, 1, 128, None, None, None, None, None, None, 0, None) == 1001
    assert hip.tsp_spmm_launch(16, 0, 1, 128, None, None, None, None, None, None, 0, None) == 1001
    assert hip.tsp_spmm_launch(16, 0, 0, 128, None, None, None, None, None, None, 0, None) == 0
    # XCD placement: only contiguous (0) and interleaved (1); packed needs
    # the value offsets and is 8-/16-row only
    placed = lambda bm, bmp, vptr, place: hip.tsp_spmm_launch_placed(
        bm, 0, 1, 128, None, bmp, vptr, None, None, None, None, None, 0, None, 0, 0, 0, 0, place)
    for place in (-1, 2, 7):
        assert placed(16, None, None, place) == 1001
    assert placed(16, None, None, 0) == 1001 and placed(16, None, None, 1) == 1001   # null buffers
    dummy = C.c_void_p(1)
    assert placed(64, dummy, dummy, 0) == 1001 and placed(8, dummy, None, 0) == 1001
    # panel-synchronised sweep: contiguous or interleaved placement, panels a
    # power of two of at least 64 rows, B rows and a counter buffer given;
    # these refusals come before any device call
    panels = lambda place, b_rows, panel_rows, sync, ints, ntasks=1, lag=2: hip.tsp_spmm_launch_panels(
        16, 0, ntasks, 128, dummy, None, None, dummy, dummy, dummy, dummy, dummy, 0, None, 0, 0, 0, 0, place, 0,
        b_rows, panel_rows, lag, sync, ints)
    assert panels(2, 1000, 256, dummy, 1024) == 1001                # chunk per XCD group
    for pr in (0, 32, 96, 1000):
        assert panels(0, 1000, pr, dummy, 1024) == 1001             # bad panel size
    assert panels(0, 0, 256, dummy, 1024) == 1001                   # no B rows
    assert panels(0, 1000, 256, None, 1024) == 1001                 # no counters
    assert panels(0, 1000, 256, dummy, 0) == 1001
    assert panels(0, 1000, 256, dummy, 1024, lag=0) == 1001          # a lead of at least one panel
    assert panels(1, 1000, 256, dummy, 1024, ntasks=0) == 0          # nothing to do
    # HIP graphs: the null stream cannot be captured, a null graph is neither
    # launched nor an error to free, and a null plan is refused; all before
    # any device call
    assert hip.tsp_stream_begin_capture(None) == 1001
    assert hip.tsp_stream_end_capture(None, None) == 1001
    assert hip.tsp_graph_launch(None, None) == 1001
    assert hip.tsp_graph_destroy(None) == 0
    _, host = tsp.load()
    # tile pairs: fp16 8- and 16-row tiles at 64- or 128-column chunks only
    assert [hip.tsp_pairs_supported(bm, pr, w) for bm, pr, w in
            ((16, 0, 64), (8, 0, 128), (8, 1, 64), (16, 1, 64), (8, 1, 128), (64, 0, 64), (8, 0, 32),
             (16, 0, 256))] == [1, 1, 1, 0, 0, 0, 0, 0]
    assert hip.tsp_split_bf16_bits(None, None, 1) == hip.tsp_split_bf16_device(None, None, 1, None) == 1001
    assert host.tsp_plan_set_pairs(None, 16, 1) == 1001 and host.tsp_plan_get_pairs(None, 16) == -1
    # 3-byte B: tf32 operands only (OPERANDS_TF32 set), no tile pairs; refused
    # before any device call
    b3 = lambda prec, flags: hip.tsp_spmm_launch_ex(8, prec, 1, 64, dummy, None, None, dummy, dummy, dummy, dummy,
                                                    dummy, 0, None, 64, 1, 0, 0, 0, flags)
    assert b3(0, 1 | 32) == 1001 and b3(1, 32) == 1001 and b3(1, 1 | 8 | 32) == 1001
    assert hip.tsp_pack_3byte_bits(None, None, 4) == hip.tsp_pack_3byte_device(None, None, 4, None) == 1001
    assert hip.tsp_pack_3byte_device(dummy, C.c_void_p(1 << 20), 6, None) == 1001   # n a multiple of 4
    assert hip.tsp_pack_3byte_device(C.c_void_p(1 << 20), C.c_void_p((1 << 20) + 8), 16, None) == 1001  # overlap
    assert host.tsp_plan_set_b_3byte(None, 8, 1) == 1001 and host.tsp_plan_get_b_3byte(None, 8) == -1
    assert host.tsp_plan_graph_capture(None, 1) == 1001
    assert host.tsp_plan_graph_run(None, 1) == 1001
    assert host.tsp_plan_graph_time(None, 1, None) == 1001
    assert host.tsp_plan_graph_free(None) == 1001


def test_cli_usage_and_errors(tmp_path):
    exe = os.path.join(ROOT, "tilespmm_amd", "bin", "tilespmm_fp16")
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 1 and "Usage" in r.stdout
    r = subprocess.run([exe, "-d", "0", str(tmp_path / "nope.mtx"), "32"], capture_output=True, text=True)
    assert r.returncode == 1
    p = tmp_path / "a.mtx"
    p.write_text("%%MatrixMarket matrix coordinate pattern general\n2 2 1\n1 1\n")
    r = subprocess.run([exe, "-d", "0", str(p), "0"], capture_output=True, text=True)
    assert r.returncode == 1 and "colB" in r.stderr


def test_cli_rejects_malformed_and_oversized_inputs(tmp_path, tsp):
    """Fail-fast paths the reference leaves undefined (it ignores
    mmio_allinone's status): every bad input ends with exit status 1 and a
    message, never a signal.  The oversized header runs under a 2 GB address
    space limit, so the reader's allocation fails instead of the machine
    swapping."""
    import resource
    exe = os.path.join(ROOT, "tilespmm_amd", "bin", "tilespmm_fp16")
    files = {
        "truncated": "%%MatrixMarket matrix coordinate real general\n3 3 2\n1 1 1.0\n",
        "no_header": "garbage\n1 2 3\n",
        "out_of_range": "%%MatrixMarket matrix coordinate real general\n3 3 2\n1 1 1.0\n9 1 2.0\n",
        "bad_number": "%%MatrixMarket matrix coordinate real general\n3 3 1\n1 x 1.0\n",
        "huge": "%%MatrixMarket matrix coordinate real general\n300000000 300000000 900000000\n1 1 1.0\n",
    }
    limit = lambda: resource.setrlimit(resource.RLIMIT_AS, (2 << 30, 2 << 30))
    for name, text in files.items():
        p = tmp_path / f"{name}.mtx"
        p.write_text(text)
        r = subprocess.run([exe, "-d", "0", str(p), "32"], capture_output=True, text=True, timeout=120,
                           preexec_fn=limit if name == "huge" else None)
        assert r.returncode == 1, (name, r.returncode, r.stderr[-500:])
        assert "Cannot read Matrix Market file" in r.stderr, (name, r.stderr[-500:])
    if not tsp.device_available():
        p = tmp_path / "ok.mtx"
        p.write_text("%%MatrixMarket matrix coordinate real general\n4 4 2\n1 1 1.0\n2 3 2.0\n")
        r = subprocess.run([exe, "-d", "0", str(p), "32"], capture_output=True, text=True, timeout=120)
        assert r.returncode == 1 and "not a usable gfx950" in r.stderr, r.stderr[-500:]
