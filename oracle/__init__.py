"""CPU oracle for the TileSpMM hot path -- TEST INFRASTRUCTURE ONLY.

ctypes access to ``oracle/liboracle.so`` (built from ``oracle/oracle.c`` by
``oracle/Makefile``), a naive C restatement of the reference's host
algorithms.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
reported CPU baseline -- never as the computation under test.

Parity status of each function (what pins it) is documented in the header
of oracle.c; the pinning tests are tests/test_oracle_*.py.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

PREC_FP16 = 0
PREC_TF32 = 1

_lib = None
_P = C.c_void_p
_IP = C.POINTER(C.c_int)


class ThParams(C.Structure):
    _fields_ = [
        ("sm_count", C.c_int), ("threads_per_sm", C.c_int), ("registers_per_sm", C.c_int),
        ("blocks_per_sm", C.c_int), ("shared_bytes_per_sm", C.c_longlong), ("l2_bytes", C.c_longlong),
        ("kernel_threads", C.c_int), ("kernel_registers", C.c_int), ("kernel_shared_bytes", C.c_longlong),
        ("iteration_bytes", C.c_int), ("lambda_atom", C.c_float),
    ]


class PolicyNode(C.Structure):
    _fields_ = [
        ("feature", C.c_int), ("left_feature", C.c_int), ("right_feature", C.c_int),
        ("child0", C.c_int), ("child1", C.c_int), ("child2", C.c_int), ("child3", C.c_int),
        ("missing_left_mask", C.c_int), ("cut", C.c_float), ("left_cut", C.c_float),
        ("right_cut", C.c_float),
    ]


def build(force: bool = False) -> None:
    """Compile liboracle.so (and oracle/_ref when the reference is mounted)."""
    if force or not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(os.path.join(HERE, "oracle.c")):
        subprocess.run(["make", "-C", HERE, "-B", "liboracle.so"], check=True, capture_output=True)
    if os.path.isdir("/root/reference/src"):
        subprocess.run(["make", "-C", HERE, "ref"], check=True, capture_output=True)
        subprocess.run([os.path.join(REF_DIR, "policy_dump"), os.path.join(REF_DIR, "policy_tree.bin")],
                       check=True, capture_output=True)


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = C.CDLL(LIB)
        sig = {
            "orc_free": (None, [_P]),
            "orc_half_to_float": (C.c_float, [C.c_uint16]),
            "orc_float_to_half": (C.c_uint16, [C.c_float]),
            "orc_round_tf32": (C.c_float, [C.c_float]),
            "orc_mm_read": (C.c_int, [C.c_char_p, _IP, _IP, C.POINTER(C.c_longlong), _IP, C.POINTER(_IP),
                                      C.POINTER(_IP), C.POINTER(C.POINTER(C.c_double))]),
            "orc_matrix_split": (C.c_int, [C.c_int, C.c_int, _P, _P, C.c_float, C.c_float, _P]),
            "orc_sub_csr": (None, [C.c_int, _P, _P, _P, _P, C.c_int, _IP, C.POINTER(C.c_longlong), _P, _P, _P,
                                   _P]),
            "orc_tile_count": (C.c_int, [C.c_int, C.c_int, _P, _P, C.c_int, C.c_int, _P]),
            "orc_tile_fill": (C.c_int, [C.c_int, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P,
                                        _P]),
            "orc_tile_pretreatment": (C.c_int, [C.c_int, _P, _P, C.c_int, _P, _P]),
            "orc_optimal_th": (C.c_int, [C.c_int, C.c_int, C.c_int, _P, C.POINTER(ThParams), _P]),
            "orc_features_from_csr": (C.c_int, [C.c_int, C.c_int, C.c_longlong, _P, C.c_double, C.c_int, _P]),
            "orc_policy_select": (None, [_P, _P, _P, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
            "orc_spmm_f64": (None, [C.c_int, _P, _P, _P, C.c_int, _P, C.c_longlong, _P, C.c_longlong]),
            "orc_spmm_f32_omp": (C.c_int, [C.c_int, _P, _P, _P, C.c_int, _P, C.c_longlong, _P, C.c_longlong]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _take(ptr, n, dtype):
    lib = load()
    addr = C.cast(ptr, C.c_void_p).value
    if not addr:
        return np.zeros(0, dtype=dtype)
    out = np.frombuffer((C.c_char * max(1, n * np.dtype(dtype).itemsize)).from_address(addr), dtype=dtype)[:n].copy()
    lib.orc_free(C.c_void_p(addr))
    return out


def half_to_float(h: int) -> float:
    return load().orc_half_to_float(h)


def float_to_half(f: float) -> int:
    return load().orc_float_to_half(f)


def round_tf32(f: float) -> float:
    return load().orc_round_tf32(f)


def mm_read(path: str):
    lib = load()
    m, n, sym = C.c_int(), C.c_int(), C.c_int()
    nnz = C.c_longlong()
    rp, ci = _IP(), _IP()
    vv = C.POINTER(C.c_double)()
    st = lib.orc_mm_read(path.encode(), C.byref(m), C.byref(n), C.byref(nnz), C.byref(sym), C.byref(rp),
                         C.byref(ci), C.byref(vv))
    if st != 0:
        raise IOError(f"orc_mm_read({path}) -> {st}")
    return (m.value, n.value, _take(rp, m.value + 1, np.int32), _take(ci, nnz.value, np.int32),
            _take(vv, nnz.value, np.float64), bool(sym.value))


def split_classes(rows, cols, rowptr, colidx, gamma, delta):
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colidx = np.ascontiguousarray(colidx, dtype=np.int32)
    out = np.zeros(max(rows, 1), dtype=np.int32)
    st = load().orc_matrix_split(rows, cols, _p(rowptr), _p(colidx), gamma, delta, _p(out))
    assert st == 0
    return out[:rows]


def sub_csr(rows, rowptr, colidx, valbits_u32, row_class, cls):
    """Rows of one class in ascending order -> (rows, rowptr, colidx, valbits, orig_row)."""
    lib = load()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colidx = np.ascontiguousarray(colidx, dtype=np.int32)
    vb = np.ascontiguousarray(valbits_u32, dtype=np.uint32)
    rc = np.ascontiguousarray(row_class, dtype=np.int32)
    sr, snz = C.c_int(), C.c_longlong()
    lib.orc_sub_csr(rows, _p(rowptr), _p(colidx), _p(vb), _p(rc), cls, C.byref(sr), C.byref(snz), None, None,
                    None, None)
    p = np.zeros(sr.value + 1, dtype=np.int32)
    c = np.zeros(max(snz.value, 1), dtype=np.int32)
    v = np.zeros(max(snz.value, 1), dtype=np.uint32)
    o = np.zeros(max(sr.value, 1), dtype=np.int32)
    lib.orc_sub_csr(rows, _p(rowptr), _p(colidx), _p(vb), _p(rc), cls, C.byref(sr), C.byref(snz), _p(p), _p(c),
                    _p(v), _p(o))
    return sr.value, p, c[:snz.value], v[:snz.value], o[:sr.value]


def tile_create(rows, cols, rowptr, colidx, valbits_u32, prec, bm, bn):
    """-> dict(tilem, tilenum, tile_ptr, tile_colidx, tile_nnz, dense, bitmap, overflow)."""
    lib = load()
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colidx = np.ascontiguousarray(colidx, dtype=np.int32)
    vb = np.ascontiguousarray(valbits_u32, dtype=np.uint32)
    tilem = (rows + bm - 1) // bm
    tp = np.zeros(tilem + 1, dtype=np.int32)
    tilenum = lib.orc_tile_count(rows, cols, _p(rowptr), _p(colidx), bm, bn, _p(tp))
    words = (bm * bn + 63) // 64
    ci = np.zeros(max(tilenum * bn, 1), dtype=np.int32)
    tn = np.zeros(tilenum + 1, dtype=np.int32)
    dt = np.uint16 if prec == PREC_FP16 else np.uint32
    dense = np.zeros(max(tilenum * bm * bn, 1), dtype=dt)
    bmap = np.zeros(max(tilenum * words, 1), dtype=np.uint64)
    ov = lib.orc_tile_fill(rows, cols, _p(rowptr), _p(colidx), _p(vb), prec, bm, bn, _p(tp), _p(ci), _p(tn),
                           _p(dense), _p(bmap))
    return {
        "tilem": tilem, "tilenum": tilenum, "tile_ptr": tp, "tile_colidx": ci[:tilenum * bn],
        "tile_nnz": tn, "dense": dense[:tilenum * bm * bn], "bitmap": bmap[:tilenum * words],
        "overflow": ov,
    }


def pretreatment(tile_ptr, orig_tile_row, th):
    lib = load()
    tp = np.ascontiguousarray(tile_ptr, dtype=np.int32)
    orow = np.ascontiguousarray(orig_tile_row, dtype=np.int32)
    tilem = len(tp) - 1
    n = lib.orc_tile_pretreatment(tilem, _p(tp), _p(orow), th, None, None)
    rows = np.zeros(max(n, 1), dtype=np.uint32)
    cs = np.zeros(n + 1, dtype=np.int32)
    lib.orc_tile_pretreatment(tilem, _p(tp), _p(orow), th, _p(rows), _p(cs))
    return rows[:n], cs


def optimal_th(bm, colB, tile_ptr, params: ThParams):
    tp = np.ascontiguousarray(tile_ptr, dtype=np.int32)
    top4 = np.zeros(4, dtype=np.int32)
    n = load().orc_optimal_th(bm, colB, len(tp) - 1, _p(tp), C.byref(params), _p(top4))
    return n, top4


def features(rows, cols, nnz, rowptr, capability, colB):
    rp = np.ascontiguousarray(rowptr, dtype=np.int32)
    f = np.zeros(11, dtype=np.float64)
    ok = load().orc_features_from_csr(rows, cols, nnz, _p(rp), capability, colB, _p(f))
    return f if ok else None


def policy_select(f, nodes, cands, root):
    f = np.ascontiguousarray(f, dtype=np.float64)
    g, d = C.c_float(), C.c_float()
    load().orc_policy_select(_p(f), C.cast(nodes, C.c_void_p), _p(np.ascontiguousarray(cands, dtype=np.float32)),
                             root, C.byref(g), C.byref(d))
    return g.value, d.value


def load_ref_policy_tree():
    """(nodes ctypes array, candidates [n,2] float32, root_fp16, root_tf32) from
    oracle/_ref/policy_tree.bin (the reference's own table, dumped by
    oracle/policy_dump.c), or None when the reference was not available."""
    path = os.path.join(REF_DIR, "policy_tree.bin")
    if not os.path.exists(path):
        return None
    raw = open(path, "rb").read()
    hdr = np.frombuffer(raw[:16], dtype=np.int32)
    nn, nc, r16, r32 = (int(x) for x in hdr)
    nodes = (PolicyNode * nn).from_buffer_copy(raw[16:16 + nn * C.sizeof(PolicyNode)])
    off = 16 + nn * C.sizeof(PolicyNode)
    cands = np.frombuffer(raw[off:off + nc * 8], dtype=np.float32).reshape(nc, 2).copy()
    return nodes, cands, r16, r32


def spmm_f64(rows, rowptr, colidx, val_f64, B_f64, n):
    rp = np.ascontiguousarray(rowptr, dtype=np.int32)
    ci = np.ascontiguousarray(colidx, dtype=np.int32)
    v = np.ascontiguousarray(val_f64, dtype=np.float64)
    B = np.ascontiguousarray(B_f64, dtype=np.float64)
    Cm = np.zeros((rows, n), dtype=np.float64)
    load().orc_spmm_f64(rows, _p(rp), _p(ci), _p(v), n, _p(B), B.shape[1], _p(Cm), n)
    return Cm


def spmm_f32_omp(rows, rowptr, colidx, val_f32, B_f32, n, C_out=None):
    rp = np.ascontiguousarray(rowptr, dtype=np.int32)
    ci = np.ascontiguousarray(colidx, dtype=np.int32)
    v = np.ascontiguousarray(val_f32, dtype=np.float32)
    B = np.ascontiguousarray(B_f32, dtype=np.float32)
    Cm = np.zeros((rows, n), dtype=np.float32) if C_out is None else C_out
    used = load().orc_spmm_f32_omp(rows, _p(rp), _p(ci), _p(v), n, _p(B), B.shape[1], _p(Cm), n)
    return Cm, used


def round_tf32_array(x):
    """Vectorised nearest-even rounding of float32 values to tf32 (same rule as
    orc_round_tf32; tests/test_oracle_pins.py checks the two agree)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    fin = (b & 0x7f800000) != 0x7f800000
    r = ((b + 0xfff + ((b >> 13) & 1)) & 0xffffe000) & 0xffffffff
    return np.where(fin, r, b).astype(np.uint32).view(np.float32)


def values_f64(val, prec, tf32_round=False):
    """Stored values (half bits or float32) -> float64, optionally tf32-rounded."""
    v = np.asarray(val)
    if prec == PREC_FP16:
        return v.view(np.float16).astype(np.float64)
    f = v.view(np.float32) if v.dtype == np.uint32 else v.astype(np.float32)
    return (round_tf32_array(f) if tf32_round else f).astype(np.float64)
