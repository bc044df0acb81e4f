"""tilespmm_amd -- Python access to the MI355X TileSpMM libraries.

The product is the pair of in-tree shared libraries built by
``tilespmm_amd/Makefile``:

* ``lib/libtilespmm_hip.so``  -- gfx950 HIP kernels and the device C ABI
  (``include/tilespmm_hip.h``);
* ``lib/libtilespmm_host.so`` -- the C++ host library (Matrix Market reader,
  matrix_split, csr2tile tiles, task schedule, threshold model, policy,
  synthetic inputs, device plan; ``include/tilespmm.h``).

This module only binds them with ctypes; no computation happens in Python and
there is no CPU fallback: if the libraries are missing, ``load()`` raises.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

__all__ = [
    "PREC_FP16", "PREC_TF32", "load", "TspError", "Csr", "TileMatrix", "SubCsr",
    "gen_config", "gen_structure", "matrix_split", "split_classes", "tile_create",
    "tile_bn", "colB_padded", "pretreatment", "optimal_th", "ThParams", "features",
    "predict", "policy_candidates", "mm_read", "Plan", "device_available",
]

PREC_FP16 = 0
PREC_TF32 = 1

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
BIN_DIR = os.path.join(_HERE, "bin")

_hip = None
_host = None


class TspError(RuntimeError):
    """Non-zero status from the C ABI."""

    def __init__(self, what: str, status: int):
        msg = f"{what} failed with status {status}"
        if _hip is not None:
            try:
                msg += ": " + _hip.tsp_hip_error_string(status).decode()
            except Exception:  # pragma: no cover - best effort text
                pass
        super().__init__(msg)
        self.status = status


def _check(what: str, st: int) -> None:
    if st != 0:
        raise TspError(what, st)


class Tile_matrix(C.Structure):
    """Mirror of Tile_matrix in include/tilespmm.h."""

    _fields_ = [
        ("tilem", C.c_int), ("tilen", C.c_int), ("tilenum", C.c_int),
        ("tile_ptr", C.POINTER(C.c_int)), ("tile_nnz", C.POINTER(C.c_int)),
        ("tile_colidx", C.POINTER(C.c_int)), ("Blockdense_Val", C.c_void_p),
        ("dnssize", C.c_size_t), ("rowblkblock", C.c_int),
        ("blkcoostylerowidx", C.POINTER(C.c_uint)),
        ("blkcoostylerowidx_colstart", C.POINTER(C.c_int)),
        ("orig_tile_row_idx", C.POINTER(C.c_int)),
        ("bm", C.c_int), ("bn", C.c_int), ("prec", C.c_int),
        ("bitmap_words", C.c_int), ("tile_bitmap", C.POINTER(C.c_uint64)),
    ]


class tsp_sub_csr(C.Structure):
    _fields_ = [
        ("rows", C.c_int), ("nnz", C.c_longlong), ("ptr", C.POINTER(C.c_int)),
        ("idx", C.POINTER(C.c_int)), ("val", C.c_void_p), ("orig_row", C.POINTER(C.c_int)),
    ]


class ThParams(C.Structure):
    """Mirror of tsp_th_params (threshold cost-model resources)."""

    _fields_ = [
        ("sm_count", C.c_int), ("threads_per_sm", C.c_int), ("registers_per_sm", C.c_int),
        ("blocks_per_sm", C.c_int), ("shared_bytes_per_sm", C.c_longlong),
        ("l2_bytes", C.c_longlong), ("kernel_threads", C.c_int), ("kernel_registers", C.c_int),
        ("kernel_shared_bytes", C.c_longlong), ("iteration_bytes", C.c_int),
        ("lambda_atom", C.c_float), ("tasks_per_block", C.c_int), ("cols_per_task", C.c_int),
        ("lambda_l2_scale", C.c_float),
    ]


class DeviceInfo(C.Structure):
    _fields_ = [
        ("cu_count", C.c_int), ("max_threads_per_cu", C.c_int), ("regs_per_cu", C.c_int),
        ("max_blocks_per_cu", C.c_int), ("lds_bytes_per_cu", C.c_longlong),
        ("l2_bytes", C.c_longlong), ("wavefront_size", C.c_int), ("clock_khz", C.c_int),
        ("memory_clock_khz", C.c_int), ("memory_bus_width", C.c_int),
        ("name", C.c_char * 256), ("gcn_arch", C.c_char * 64),
    ]


class KernelInfo(C.Structure):
    _fields_ = [
        ("threads", C.c_int), ("tasks_per_block", C.c_int), ("registers_per_thread", C.c_int),
        ("shared_bytes", C.c_longlong), ("iteration_bytes", C.c_int), ("cols_per_task", C.c_int),
    ]


class DevTiles(C.Structure):
    """tsp_dev_tiles: device tile arrays made by tsp_tile_create_device."""
    _fields_ = [("tilem", C.c_int), ("tilenum", C.c_int), ("bm", C.c_int), ("bn", C.c_int),
                ("prec", C.c_int), ("bitmap_words", C.c_int), ("d_tile_ptr", C.c_void_p),
                ("d_tile_nnz", C.c_void_p), ("d_tile_colidx", C.c_void_p), ("d_val", C.c_void_p),
                ("d_bitmap", C.c_void_p)]


class RunResult(C.Structure):
    _fields_ = [
        ("th64", C.c_int), ("th16", C.c_int), ("th8", C.c_int), ("pre_time_ms", C.c_double),
        ("time_ms", C.c_double), ("tflops", C.c_double), ("model_ms", C.c_double),
        ("tune_ms", C.c_double), ("warmup_iters", C.c_int), ("clock_mhz", C.c_uint),
    ]


# Every symbol include/tilespmm_hip.h and include/tilespmm.h declare, with
# (restype, argtypes).  Tests check that the built libraries export them all.
_P = C.c_void_p
_IP = C.POINTER(C.c_int)
HIP_SYMBOLS = {
    "tsp_hip_version": (C.c_char_p, []),
    "tsp_hip_error_string": (C.c_char_p, [C.c_int]),
    "tsp_device_init": (C.c_int, [C.c_int]),
    "tsp_device_probe": (C.c_int, [C.c_int, C.POINTER(DeviceInfo)]),
    "tsp_kernel_probe": (C.c_int, [C.c_int, C.c_int, C.c_int, C.POINTER(KernelInfo)]),
    "tsp_gpu_clock_mhz": (C.c_int, [C.c_int, C.POINTER(C.c_uint), C.POINTER(C.c_uint)]),
    "tsp_malloc": (C.c_int, [C.POINTER(C.c_void_p), C.c_size_t]),
    "tsp_free": (C.c_int, [_P]),
    "tsp_memcpy_h2d": (C.c_int, [_P, _P, C.c_size_t]),
    "tsp_memcpy_d2h": (C.c_int, [_P, _P, C.c_size_t]),
    "tsp_memcpy_h2d_async": (C.c_int, [_P, _P, C.c_size_t, _P]),
    "tsp_memset": (C.c_int, [_P, C.c_int, C.c_size_t]),
    "tsp_memset_async": (C.c_int, [_P, C.c_int, C.c_size_t, _P]),
    "tsp_stream_create": (C.c_int, [C.POINTER(C.c_void_p)]),
    "tsp_stream_destroy": (C.c_int, [_P]),
    "tsp_stream_sync": (C.c_int, [_P]),
    "tsp_device_sync": (C.c_int, []),
    "tsp_event_create": (C.c_int, [C.POINTER(C.c_void_p)]),
    "tsp_event_destroy": (C.c_int, [_P]),
    "tsp_event_record": (C.c_int, [_P, _P]),
    "tsp_event_sync": (C.c_int, [_P]),
    "tsp_event_elapsed_ms": (C.c_int, [C.POINTER(C.c_float), _P, _P]),
    "tsp_stream_create_nonblocking": (C.c_int, [C.POINTER(C.c_void_p)]),
    "tsp_stream_wait_event": (C.c_int, [_P, _P]),
    "tsp_stream_begin_capture": (C.c_int, [_P]),
    "tsp_stream_end_capture": (C.c_int, [_P, C.POINTER(_P)]),
    "tsp_graph_launch": (C.c_int, [_P, _P]),
    "tsp_graph_destroy": (C.c_int, [_P]),
    "tsp_spmm_launch": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P,
                                  C.c_int, _P]),
    "tsp_spmm_launch_variant": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P,
                                          C.c_int, _P, C.c_int, C.c_int, C.c_int, C.c_int]),
    "tsp_spmm_launch_packed": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P, _P, _P,
                                         C.c_int, _P, C.c_int, C.c_int, C.c_int, C.c_int]),
    "tsp_spmm_launch_placed": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P, _P, _P,
                                         C.c_int, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "tsp_spmm_launch_ex": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P, _P, _P,
                                     C.c_int, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "tsp_spmm_launch_panels": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P, _P, _P,
                                         C.c_int, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                         C.c_int, C.c_int, C.c_int, _P, C.c_longlong]),
    "tsp_pairs_supported": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "tsp_split_bf16_bits": (C.c_int, [_P, _P, C.c_size_t]),
    "tsp_split_bf16_device": (C.c_int, [_P, _P, C.c_size_t, _P]),
    "tsp_pack_3byte_bits": (C.c_int, [_P, _P, C.c_size_t]),
    "tsp_pack_3byte_device": (C.c_int, [_P, _P, C.c_size_t, _P]),
    "tsp_switch_v64": (C.c_int, [C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P, C.c_int, _P]),
    "tsp_switch_v16": (C.c_int, [C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P, C.c_int, _P]),
    "tsp_switch_v8": (C.c_int, [C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P, C.c_int, _P]),
    "tsp_vendor_spmm": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_longlong, _P, _P, _P, C.c_int,
                                  C.c_int, _P, _P, C.c_int, C.c_int, C.POINTER(C.c_double),
                                  C.POINTER(C.c_double)]),
    "tsp_round_tf32_bits": (C.c_int, [_P, _P, C.c_size_t]),
    "tsp_round_tf32_device": (C.c_int, [_P, C.c_size_t, _P]),
    "tsp_copy_kernel": (C.c_int, [_P, _P, C.c_size_t, _P]),
    "tsp_gather_kernel": (C.c_int, [_P, C.c_size_t, C.c_int, C.c_int, C.c_uint, _P, _P]),
    "tsp_gather_index_stream": (C.c_int, [_P, C.c_longlong, C.c_int, _P, C.c_longlong, _P, _P]),
    "tsp_colidx_count": (C.c_int, [_P, C.c_longlong, C.c_int, _P, C.c_int, _P, _P]),
    "tsp_colidx_remap": (C.c_int, [_P, C.c_longlong, C.c_int, _P, C.c_int, _P, _P]),
    "tsp_hot_rows_gather": (C.c_int, [_P, C.c_int, C.c_longlong, _P, C.c_int, _P]),
    "tsp_tile_create_device": (C.c_int, [C.POINTER(DevTiles), C.c_int, C.c_int, C.c_longlong, _P, _P, _P,
                                         C.c_int, C.c_int, C.c_int, _P]),
    "tsp_dev_tiles_free": (C.c_int, [C.POINTER(DevTiles)]),
    "tsp_tiles_pack_device": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, C.POINTER(C.c_longlong),
                                        C.POINTER(C.c_void_p), C.POINTER(C.c_void_p), _P]),
    "tsp_tiles_pack_device_noalloc": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, C.c_longlong, _P,
                                                C.POINTER(C.c_longlong), _P]),
}
HOST_SYMBOLS = {
    "tsp_mm_read": (C.c_int, [C.c_char_p, _IP, _IP, C.POINTER(C.c_longlong), _IP,
                              C.POINTER(_IP), C.POINTER(_IP), C.POINTER(C.POINTER(C.c_double))]),
    "tsp_free_host": (None, [_P]),
    "tsp_matrix_split": (C.c_int, [C.c_int, C.c_int, C.c_longlong, _P, _P, _P, C.c_int, C.c_float,
                                   C.c_float, C.POINTER(tsp_sub_csr), C.POINTER(tsp_sub_csr),
                                   C.POINTER(tsp_sub_csr)]),
    "tsp_split_classes": (C.c_int, [C.c_int, C.c_int, _P, _P, C.c_float, C.c_float, _P]),
    "tsp_sub_csr_free": (None, [C.POINTER(tsp_sub_csr)]),
    "tsp_tile_create": (C.c_int, [C.POINTER(Tile_matrix), C.c_int, C.c_int, C.c_longlong, _P, _P,
                                  _P, _P, C.c_int, C.c_int, C.c_int]),
    "tsp_tile_destroy": (None, [C.POINTER(Tile_matrix)]),
    "tsp_tile_bn": (C.c_int, [C.c_int, C.c_int]),
    "tsp_tile_pretreatment": (C.c_int, [C.POINTER(Tile_matrix), C.c_int, _IP,
                                        C.POINTER(C.POINTER(C.c_uint)), C.POINTER(_IP)]),
    "tsp_th_params_probe": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(ThParams)]),
    "tsp_th_weights": (C.c_int, [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    "tsp_optimal_th": (C.c_int, [C.c_int, C.c_int, C.c_int, _P, C.POINTER(ThParams), _P]),
    "tsp_features_from_csr": (C.c_int, [C.c_int, C.c_int, C.c_longlong, _P, C.c_double, C.c_int,
                                        _P]),
    "tilespmm_predict_fp16": (None, [_P, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    "tilespmm_predict_tf32": (None, [_P, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    "tsp_gen_config": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_ulonglong, _IP, _IP,
                                 C.POINTER(C.c_longlong), C.POINTER(_IP), C.POINTER(_IP),
                                 C.POINTER(C.c_void_p), _IP, C.POINTER(C.c_void_p)]),
    "tsp_gen_structure": (C.c_int, [C.c_int, C.c_ulonglong, _IP, _IP, C.POINTER(C.c_longlong),
                                    C.POINTER(_IP), C.POINTER(_IP)]),
    "tsp_gen_rmat": (C.c_int, [C.c_int, C.c_longlong, C.c_ulonglong, C.c_int, _IP, C.POINTER(C.c_longlong),
                               C.POINTER(_IP), C.POINTER(_IP), C.POINTER(C.c_void_p)]),
    "tsp_gen_values": (C.c_int, [C.c_int, C.c_int, C.c_ulonglong, C.c_size_t, _P]),
    "tsp_colB_padded": (C.c_int, [C.c_int]),
    "tsp_plan_create": (C.c_int, [C.POINTER(C.c_void_p), C.c_int, C.POINTER(Tile_matrix),
                                  C.POINTER(Tile_matrix), C.POINTER(Tile_matrix), C.c_int, C.c_int,
                                  C.c_int, C.c_int, _P]),
    "tsp_plan_create_csr": (C.c_int, [C.POINTER(C.c_void_p), C.c_int, C.POINTER(tsp_sub_csr),
                                      C.POINTER(tsp_sub_csr), C.POINTER(tsp_sub_csr), C.c_int, C.c_int,
                                      C.c_int, C.c_int, _P, C.POINTER(C.c_double)]),
    "tsp_plan_set_th": (C.c_int, [_P, C.c_int, C.c_int, C.c_int]),
    "tsp_plan_tune": (C.c_int, [_P, C.c_int, _P, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "tsp_plan_set_variant": (C.c_int, [_P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "tsp_plan_set_format": (C.c_int, [_P, C.c_int, C.c_int]),
    "tsp_plan_get_format": (C.c_int, [_P, C.c_int]),
    "tsp_plan_get_variant": (C.c_int, [_P, C.c_int, _IP, _IP, _IP, _IP]),
    "tsp_plan_set_placement": (C.c_int, [_P, C.c_int, C.c_int]),
    "tsp_plan_set_lane_indices": (C.c_int, [_P, C.c_int, C.c_int]),
    "tsp_plan_get_lane_indices": (C.c_int, [_P, C.c_int]),
    "tsp_plan_set_pairs": (C.c_int, [_P, C.c_int, C.c_int]),
    "tsp_plan_get_pairs": (C.c_int, [_P, C.c_int]),
    "tsp_plan_set_b_3byte": (C.c_int, [_P, C.c_int, C.c_int]),
    "tsp_plan_get_b_3byte": (C.c_int, [_P, C.c_int]),
    "tsp_plan_get_placement": (C.c_int, [_P, C.c_int]),
    "tsp_plan_set_panels": (C.c_int, [_P, C.c_int, C.c_int, C.c_int]),
    "tsp_plan_get_panels": (C.c_int, [_P, C.c_int, _IP, _IP]),
    "tsp_plan_set_hot_rows": (C.c_int, [_P, C.c_longlong]),
    "tsp_plan_set_tune_mode": (C.c_int, [_P, C.c_int]),
    "tsp_plan_get_tune_mode": (C.c_int, [_P]),
    "tsp_plan_get_hot_rows": (C.c_int, [_P, _IP, C.POINTER(C.c_longlong)]),
    "tsp_plan_run": (C.c_int, [_P, C.c_int]),
    "tsp_plan_warmup": (C.c_int, [_P, C.c_int]),
    "tsp_plan_warmup_clock": (C.c_int, [_P, C.c_int, _IP, C.POINTER(C.c_uint)]),
    "tsp_plan_time": (C.c_int, [_P, C.c_int, C.POINTER(C.c_double)]),
    "tsp_plan_time_ex": (C.c_int, [_P, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "tsp_plan_graph_capture": (C.c_int, [_P, C.c_int]),
    "tsp_plan_graph_run": (C.c_int, [_P, C.c_int]),
    "tsp_plan_graph_time": (C.c_int, [_P, C.c_int, C.POINTER(C.c_double)]),
    "tsp_plan_graph_free": (C.c_int, [_P]),
    "tsp_plan_time_class": (C.c_int, [_P, C.c_int, C.c_int, C.POINTER(C.c_double)]),
    "tsp_plan_download_c": (C.c_int, [_P, _P]),
    "tsp_plan_device_c": (C.c_int, [_P, C.POINTER(C.c_void_p)]),
    "tsp_plan_destroy": (C.c_int, [_P]),
    "tsp_call_tilespmm": (C.c_int, [C.c_int, C.POINTER(Tile_matrix), C.POINTER(Tile_matrix),
                                    C.POINTER(Tile_matrix), C.c_int, C.c_int, C.c_int,
                                    C.c_longlong, C.c_int, _P, _P, C.c_double, C.c_int, C.c_int,
                                    C.c_int, _P, C.POINTER(RunResult)]),
    "tsp_plan_execute": (C.c_int, [_P, C.c_longlong, _P, C.c_double, C.c_int, C.c_int, C.c_int, _P,
                                   C.POINTER(RunResult)]),
    "tsp_plan_tilenum": (C.c_int, [_P, C.c_int]),
    "tsp_policy_candidates": (C.c_int, [_P, _P]),
}


def _bind(lib, table):
    for name, (res, args) in table.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def load():
    """Load (once) and return (hip_lib, host_lib).  Raises if not built."""
    global _hip, _host
    if _host is None:
        hip_path = os.path.join(LIB_DIR, "libtilespmm_hip.so")
        host_path = os.path.join(LIB_DIR, "libtilespmm_host.so")
        for p in (hip_path, host_path):
            if not os.path.exists(p):
                raise ImportError(f"{p} is not built; run __graft_entry__.build() or make -C tilespmm_amd")
        hip = C.CDLL(hip_path, mode=C.RTLD_GLOBAL)
        host = C.CDLL(host_path, mode=C.RTLD_GLOBAL)
        _bind(hip, HIP_SYMBOLS)
        _bind(host, HOST_SYMBOLS)
        _hip, _host = hip, host
    return _hip, _host


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _vdtype(prec: int):
    return np.uint16 if prec == PREC_FP16 else np.float32


def _take(ptr, n, dtype):
    """Copy n elements from a malloc'd C pointer into numpy, then free it."""
    _, host = load()
    if n == 0 or not ptr:
        if ptr:
            host.tsp_free_host(C.cast(ptr, C.c_void_p))
        return np.zeros(0, dtype=dtype)
    addr = C.cast(ptr, C.c_void_p).value
    out = np.frombuffer((C.c_char * (n * np.dtype(dtype).itemsize)).from_address(addr), dtype=dtype).copy()
    host.tsp_free_host(C.c_void_p(addr))
    return out


def _view(ptr, n, dtype):
    if n == 0 or not ptr:
        return np.zeros(0, dtype=dtype)
    addr = C.cast(ptr, C.c_void_p).value
    return np.frombuffer((C.c_char * (n * np.dtype(dtype).itemsize)).from_address(addr), dtype=dtype).copy()


def tile_bn(bm: int, prec: int) -> int:
    return load()[1].tsp_tile_bn(bm, prec)


def colB_padded(colB: int) -> int:
    return load()[1].tsp_colB_padded(colB)


def device_available() -> bool:
    """True when a gfx950 device can be initialised (initialises HIP)."""
    hip, _ = load()
    return hip.tsp_device_init(0) == 0


class Csr:
    """Host CSR matrix (numpy arrays, int32 indices, values in prec storage)."""

    def __init__(self, rows, cols, rowptr, colidx, val, prec):
        self.rows, self.cols = int(rows), int(cols)
        self.rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
        self.colidx = np.ascontiguousarray(colidx, dtype=np.int32)
        self.prec = prec
        self.val = None if val is None else np.ascontiguousarray(val, dtype=_vdtype(prec))

    @property
    def nnz(self) -> int:
        return int(self.rowptr[-1]) if self.rows else 0

    def values_f64(self) -> np.ndarray:
        if self.prec == PREC_FP16:
            return self.val.view(np.float16).astype(np.float64)
        return self.val.astype(np.float64)


def gen_config(config: int, prec: int = -1, colB: int = -1, seed: int = 0):
    """Synthetic benchmark input: returns (Csr A, B ndarray [cols, colB_p], colB, colB_p)."""
    _, host = load()
    rows, cols, cbp = C.c_int(), C.c_int(), C.c_int()
    nnz = C.c_longlong()
    rp, ci = _IP(), _IP()
    v, b = C.c_void_p(), C.c_void_p()
    _check("tsp_gen_config", host.tsp_gen_config(config, prec, colB, seed, C.byref(rows), C.byref(cols),
                                                 C.byref(nnz), C.byref(rp), C.byref(ci), C.byref(v),
                                                 C.byref(cbp), C.byref(b)))
    if prec < 0:
        prec = {1: 0, 2: 0, 3: 1, 4: 0, 5: 1}[config]
    if colB <= 0:
        colB = {1: 32, 2: 128, 3: 128, 4: 256, 5: 64}[config]
    dt = _vdtype(prec)
    A = Csr(rows.value, cols.value, _take(rp, rows.value + 1, np.int32), _take(ci, nnz.value, np.int32),
            _take(v, nnz.value, dt), prec)
    B = _take(b, cols.value * cbp.value, dt).reshape(cols.value, cbp.value)
    return A, B, colB, cbp.value


def gen_rmat(scale: int, edges: int, seed: int, prec: int):
    """RMAT graph of the configuration-5 generator at any scale (Csr, values 1/deg)."""
    _, host = load()
    rows, nnz = C.c_int(), C.c_longlong()
    rp, ci, v = _IP(), _IP(), C.c_void_p()
    _check("tsp_gen_rmat", host.tsp_gen_rmat(scale, edges, seed, prec, C.byref(rows), C.byref(nnz), C.byref(rp),
                                             C.byref(ci), C.byref(v)))
    return Csr(rows.value, rows.value, _take(rp, rows.value + 1, np.int32), _take(ci, nnz.value, np.int32),
               _take(v, nnz.value, _vdtype(prec)), prec)


def gen_structure(config: int, seed: int = 0):
    _, host = load()
    rows, cols = C.c_int(), C.c_int()
    nnz = C.c_longlong()
    rp, ci = _IP(), _IP()
    _check("tsp_gen_structure", host.tsp_gen_structure(config, seed, C.byref(rows), C.byref(cols),
                                                       C.byref(nnz), C.byref(rp), C.byref(ci)))
    return (rows.value, cols.value, _take(rp, rows.value + 1, np.int32), _take(ci, nnz.value, np.int32))


def mm_read(path: str):
    """Matrix Market -> (rows, cols, rowptr, colidx, values float64, is_symmetric)."""
    _, host = load()
    rows, cols, sym = C.c_int(), C.c_int(), C.c_int()
    nnz = C.c_longlong()
    rp, ci = _IP(), _IP()
    vv = C.POINTER(C.c_double)()
    _check("tsp_mm_read", host.tsp_mm_read(path.encode(), C.byref(rows), C.byref(cols), C.byref(nnz),
                                           C.byref(sym), C.byref(rp), C.byref(ci), C.byref(vv)))
    return (rows.value, cols.value, _take(rp, rows.value + 1, np.int32), _take(ci, nnz.value, np.int32),
            _take(vv, nnz.value, np.float64), bool(sym.value))


def split_classes(A: Csr, gamma: float, delta: float) -> np.ndarray:
    _, host = load()
    out = np.zeros(max(A.rows, 1), dtype=np.int32)
    _check("tsp_split_classes", host.tsp_split_classes(A.rows, A.cols, _ptr(A.rowptr), _ptr(A.colidx),
                                                       gamma, delta, _ptr(out)))
    return out[:A.rows]


class SubCsr:
    def __init__(self, s: tsp_sub_csr, prec: int, cols: int):
        self.rows = s.rows
        self.nnz = s.nnz
        self.prec = prec
        self.cols = cols
        self.rowptr = _view(s.ptr, s.rows + 1 if s.rows else 0, np.int32)
        self.colidx = _view(s.idx, s.nnz, np.int32)
        self.val = _view(s.val, s.nnz, _vdtype(prec))
        self.orig_row = _view(s.orig_row, s.rows, np.int32)


def matrix_split(A: Csr, gamma: float, delta: float):
    """matrix_split -> (sub64, sub16, sub8) as SubCsr (copies)."""
    _, host = load()
    subs = [tsp_sub_csr(), tsp_sub_csr(), tsp_sub_csr()]
    _check("tsp_matrix_split", host.tsp_matrix_split(A.rows, A.cols, A.nnz, _ptr(A.rowptr), _ptr(A.colidx),
                                                     _ptr(A.val), A.prec, gamma, delta, C.byref(subs[0]),
                                                     C.byref(subs[1]), C.byref(subs[2])))
    out = [SubCsr(s, A.prec, A.cols) for s in subs]
    for s in subs:
        host.tsp_sub_csr_free(C.byref(s))
    return tuple(out)


class TileMatrix:
    """Owns a C Tile_matrix; exposes numpy copies of its arrays."""

    def __init__(self):
        self.m = Tile_matrix()

    def __del__(self):
        if _host is not None:
            _host.tsp_tile_destroy(C.byref(self.m))

    @property
    def tilem(self):
        return self.m.tilem

    @property
    def tilenum(self):
        return self.m.tilenum

    @property
    def bm(self):
        return self.m.bm

    @property
    def bn(self):
        return self.m.bn

    def arrays(self):
        m = self.m
        dt = _vdtype(m.prec)
        return {
            "tile_ptr": _view(m.tile_ptr, m.tilem + 1, np.int32),
            "tile_nnz": _view(m.tile_nnz, m.tilenum + 1, np.int32),
            "tile_colidx": _view(m.tile_colidx, m.tilenum * m.bn, np.int32),
            "dense": _view(m.Blockdense_Val, m.tilenum * m.bm * m.bn, dt),
            "bitmap": _view(m.tile_bitmap, m.tilenum * m.bitmap_words, np.uint64),
            "orig_tile_row_idx": _view(m.orig_tile_row_idx, m.tilem, np.int32),
        }


def tile_create(sub, colA: int, bm: int, prec: int, bn: Optional[int] = None) -> TileMatrix:
    _, host = load()
    bn = tile_bn(bm, prec) if bn is None else bn
    t = TileMatrix()
    if sub.rows == 0:
        t.m.bm, t.m.bn, t.m.prec = bm, bn, prec
        return t
    _check("tsp_tile_create", host.tsp_tile_create(C.byref(t.m), sub.rows, colA, sub.nnz, _ptr(sub.rowptr),
                                                   _ptr(sub.colidx), _ptr(sub.val), _ptr(sub.orig_row), bm,
                                                   bn, prec))
    return t


class _DevBuf:
    """A device buffer holding a copy of a host numpy array."""

    def __init__(self, a: np.ndarray):
        hip, _ = load()
        a = np.ascontiguousarray(a)
        self.p = C.c_void_p()
        _check("tsp_malloc", hip.tsp_malloc(C.byref(self.p), max(a.nbytes, 16)))
        if a.nbytes:
            _check("tsp_memcpy_h2d", hip.tsp_memcpy_h2d(self.p, _ptr(a), a.nbytes))

    def free(self):
        if self.p:
            load()[0].tsp_free(self.p)
            self.p = C.c_void_p()


def _d2h(ptr, n, dtype) -> np.ndarray:
    out = np.zeros(n, dtype=dtype)
    if n:
        _check("tsp_memcpy_d2h", load()[0].tsp_memcpy_d2h(_ptr(out), ptr, out.nbytes))
    return out


def tile_create_device(sub, colA: int, bm: int, prec: int, bn: Optional[int] = None) -> dict:
    """Builds the tiles of one class sub-CSR on the GPU (tsp_tile_create_device)
    and returns host copies of the arrays, keyed like TileMatrix.arrays()
    (without orig_tile_row_idx)."""
    hip, _ = load()
    bn = tile_bn(bm, prec) if bn is None else bn
    bufs = [_DevBuf(np.asarray(sub.rowptr, dtype=np.int32)), _DevBuf(np.asarray(sub.colidx, dtype=np.int32)),
            _DevBuf(np.asarray(sub.val))]
    t = DevTiles()
    try:
        _check("tsp_tile_create_device",
               hip.tsp_tile_create_device(C.byref(t), sub.rows, colA, sub.nnz, bufs[0].p, bufs[1].p, bufs[2].p,
                                          bm, bn, prec, None))
        try:
            return {
                "tile_ptr": _d2h(t.d_tile_ptr, t.tilem + 1, np.int32),
                "tile_nnz": _d2h(t.d_tile_nnz, t.tilenum + 1, np.int32),
                "tile_colidx": _d2h(t.d_tile_colidx, t.tilenum * bn, np.int32),
                "dense": _d2h(t.d_val, t.tilenum * bm * bn, _vdtype(prec)),
                "bitmap": _d2h(t.d_bitmap, t.tilenum * t.bitmap_words, np.uint64),
            }
        finally:
            hip.tsp_dev_tiles_free(C.byref(t))
    finally:
        for b in bufs:
            b.free()


def pretreatment(t: TileMatrix, th: int):
    _, host = load()
    n = C.c_int()
    rows = C.POINTER(C.c_uint)()
    cs = _IP()
    _check("tsp_tile_pretreatment", host.tsp_tile_pretreatment(C.byref(t.m), th, C.byref(n), C.byref(rows),
                                                               C.byref(cs)))
    return _take(rows, n.value, np.uint32), _take(cs, n.value + 1, np.int32)


def optimal_th(bm: int, colB: int, tile_ptr: np.ndarray, params: ThParams):
    _, host = load()
    tp = np.ascontiguousarray(tile_ptr, dtype=np.int32)
    top4 = np.zeros(4, dtype=np.int32)
    n = host.tsp_optimal_th(bm, colB, len(tp) - 1, _ptr(tp), C.byref(params), _ptr(top4))
    return n, top4


def th_weights(bm: int, prec: int, colB_p: int):
    """(lambda_atom, lambda_l2_scale) of the MI355X threshold calibration."""
    _, host = load()
    lam, l2s = C.c_float(), C.c_float()
    _check("tsp_th_weights", host.tsp_th_weights(bm, prec, colB_p, C.byref(lam), C.byref(l2s)))
    return lam.value, l2s.value


def features(A: Csr, capability: float, colB: int) -> np.ndarray:
    _, host = load()
    f = np.zeros(11, dtype=np.float64)
    ok = host.tsp_features_from_csr(A.rows, A.cols, A.nnz, _ptr(A.rowptr), capability, colB, _ptr(f))
    if not ok:
        raise TspError("tsp_features_from_csr", -1)
    return f


def predict(f: np.ndarray, prec: int):
    _, host = load()
    f = np.ascontiguousarray(f, dtype=np.float64)
    g, d = C.c_float(), C.c_float()
    fn = host.tilespmm_predict_fp16 if prec == PREC_FP16 else host.tilespmm_predict_tf32
    fn(_ptr(f), C.byref(g), C.byref(d))
    return g.value, d.value


def policy_candidates():
    _, host = load()
    g = np.zeros(128, dtype=np.float32)
    d = np.zeros(128, dtype=np.float32)
    n = host.tsp_policy_candidates(_ptr(g), _ptr(d))
    return g[:n], d[:n]


class Plan:
    """Device plan: the three classes + B + C resident in HBM (tsp_plan_*)."""

    def __init__(self, t64: TileMatrix, t16: TileMatrix, t8: TileMatrix, rowA: int, colA: int,
                 colB_p: int, prec: int, B: np.ndarray, device: int = 0):
        _, host = load()
        self._keep = (t64, t16, t8)
        self.rowA, self.colB_p = rowA, colB_p
        self.p = C.c_void_p()
        B = np.ascontiguousarray(B)
        _check("tsp_plan_create", host.tsp_plan_create(C.byref(self.p), device, C.byref(t64.m), C.byref(t16.m),
                                                       C.byref(t8.m), rowA, colA, colB_p, prec, _ptr(B)))

    @classmethod
    def from_csr(cls, subs, rowA: int, colA: int, colB_p: int, prec: int, B: np.ndarray, device: int = 0):
        """Plan whose tiles are built on the device from the class sub-CSRs
        (tsp_plan_create_csr); .tile_ms = upload + device conversion time."""
        _, host = load()
        self = cls.__new__(cls)
        self.rowA, self.colB_p = rowA, colB_p
        self.p = C.c_void_p()
        B = np.ascontiguousarray(B)
        keep, structs = [], []
        for s in subs:
            rp, ci, v, orow = (np.ascontiguousarray(a) for a in (s.rowptr, s.colidx, s.val, s.orig_row))
            keep.append((rp, ci, v, orow))
            structs.append(tsp_sub_csr(s.rows, s.nnz, rp.ctypes.data_as(_IP), ci.ctypes.data_as(_IP),
                                       v.ctypes.data_as(C.c_void_p), orow.ctypes.data_as(_IP)))
        self._keep = (keep, structs)
        ms = C.c_double()
        _check("tsp_plan_create_csr",
               host.tsp_plan_create_csr(C.byref(self.p), device, C.byref(structs[0]), C.byref(structs[1]),
                                        C.byref(structs[2]), rowA, colA, colB_p, prec, _ptr(B), C.byref(ms)))
        self.tile_ms = ms.value
        return self

    def close(self):
        if self.p and _host is not None:
            _host.tsp_plan_destroy(self.p)
            self.p = C.c_void_p()

    def __del__(self):
        self.close()

    def tilenum(self, bm: int) -> int:
        """Tiles of one class (0 when the class is empty)."""
        return load()[1].tsp_plan_tilenum(self.p, bm)

    def set_th(self, th64: int, th16: int, th8: int):
        _check("tsp_plan_set_th", load()[1].tsp_plan_set_th(self.p, th64, th16, th8))

    def tune(self, tune: bool = True):
        th = np.zeros(3, dtype=np.int32)
        mm, tm = C.c_double(), C.c_double()
        _check("tsp_plan_tune", load()[1].tsp_plan_tune(self.p, int(tune), _ptr(th), C.byref(mm), C.byref(tm)))
        return tuple(int(x) for x in th), mm.value, tm.value

    def set_variant(self, bm: int, w: int = 0, stages: int = 0, tasks_per_wave: int = 0, order: int = 0):
        _check("tsp_plan_set_variant", load()[1].tsp_plan_set_variant(self.p, bm, w, stages, tasks_per_wave,
                                                                      order))

    def set_format(self, bm: int, fmt: int):
        """1 = dense tiles, 2 = bitmap-packed (8-/16-row classes)."""
        _check("tsp_plan_set_format", load()[1].tsp_plan_set_format(self.p, bm, fmt))

    def get_format(self, bm: int) -> int:
        return load()[1].tsp_plan_get_format(self.p, bm)

    def get_variant(self, bm: int):
        """(w, stages, tasks_per_wave, order) the class is pinned to (0 = default)."""
        v = [C.c_int() for _ in range(4)]
        _check("tsp_plan_get_variant", load()[1].tsp_plan_get_variant(self.p, bm, *[C.byref(x) for x in v]))
        return tuple(x.value for x in v)

    def set_lane_indices(self, bm: int, on: bool):
        """Packed format: lane-loaded column indices (True) or scalar ones."""
        _check("tsp_plan_set_lane_indices", load()[1].tsp_plan_set_lane_indices(self.p, bm, int(on)))

    def get_lane_indices(self, bm: int) -> int:
        return load()[1].tsp_plan_get_lane_indices(self.p, bm)

    def set_pairs(self, bm: int, on: bool):
        """Tile pairs (two tiles per K = 32 MFMA; fp16 8-/16-row classes,
        tf32 8-row classes)."""
        _check("tsp_plan_set_pairs", load()[1].tsp_plan_set_pairs(self.p, bm, int(on)))

    def get_pairs(self, bm: int) -> int:
        return load()[1].tsp_plan_get_pairs(self.p, bm)

    def set_b_3byte(self, bm: int, on: bool):
        """B in the 3-byte form for a class of a tf32 plan (single tiles,
        no panel sweep): same result, a quarter fewer bytes per gathered B
        row."""
        _check("tsp_plan_set_b_3byte", load()[1].tsp_plan_set_b_3byte(self.p, bm, int(on)))

    def get_b_3byte(self, bm: int) -> int:
        """Whether the class's launches read B in the 3-byte form."""
        return load()[1].tsp_plan_get_b_3byte(self.p, bm)

    def set_placement(self, bm: int, placement: int):
        """XCD placement: 0 = contiguous eighths, 1 = runs dealt round-robin."""
        _check("tsp_plan_set_placement", load()[1].tsp_plan_set_placement(self.p, bm, placement))

    def get_placement(self, bm: int) -> int:
        return load()[1].tsp_plan_get_placement(self.p, bm)

    def set_panels(self, bm: int, panel_rows: int, lag: int = 2):
        """Panel-synchronised sweep with panel_rows B rows per panel and a
        lead of at most `lag` panels (dense format; panel_rows 0 = off)."""
        _check("tsp_plan_set_panels", load()[1].tsp_plan_set_panels(self.p, bm, int(panel_rows), int(lag)))

    def get_panels(self, bm: int):
        """(panel rows, lag) of the class's panel sweep (0 rows = off)."""
        r, g = C.c_int(), C.c_int()
        _check("tsp_plan_get_panels", load()[1].tsp_plan_get_panels(self.p, bm, C.byref(r), C.byref(g)))
        return r.value, g.value

    def set_tune_mode(self, cold: bool):
        """Tune for single steps from a cold cache (True) or back-to-back steps."""
        _check("tsp_plan_set_tune_mode", load()[1].tsp_plan_set_tune_mode(self.p, 1 if cold else 0))

    def get_tune_mode(self) -> int:
        return load()[1].tsp_plan_get_tune_mode(self.p)

    def set_hot_rows(self, budget_bytes: int):
        """Copy the most-gathered B rows (at most budget_bytes) into spare rows
        of B before every step; 0 restores the canonical column indices."""
        _check("tsp_plan_set_hot_rows", load()[1].tsp_plan_set_hot_rows(self.p, int(budget_bytes)))

    def get_hot_rows(self):
        """(hot slots, bytes) currently copied per step."""
        n, b = C.c_int(), C.c_longlong()
        _check("tsp_plan_get_hot_rows", load()[1].tsp_plan_get_hot_rows(self.p, C.byref(n), C.byref(b)))
        return n.value, b.value

    def run(self, zero_c: bool = True):
        _check("tsp_plan_run", load()[1].tsp_plan_run(self.p, int(zero_c)))

    def warmup(self, iters: int):
        """Clock-stable warm-up of at most `iters` steps; returns (steps run,
        last GFX clock reading in MHz, 0 when unreadable)."""
        n, mhz = C.c_int(), C.c_uint()
        _check("tsp_plan_warmup_clock", load()[1].tsp_plan_warmup_clock(self.p, iters, C.byref(n), C.byref(mhz)))
        return n.value, mhz.value

    def time(self, reps: int) -> float:
        ms = C.c_double()
        _check("tsp_plan_time", load()[1].tsp_plan_time(self.p, reps, C.byref(ms)))
        return ms.value

    def time_ex(self, reps: int):
        """(ms per step from events, host ms per step to submit the steps)."""
        ms, sub = C.c_double(), C.c_double()
        _check("tsp_plan_time_ex", load()[1].tsp_plan_time_ex(self.p, reps, C.byref(ms), C.byref(sub)))
        return ms.value, sub.value

    def graph_capture(self, steps: int) -> None:
        """Capture `steps` steps into a HIP graph (tsp_plan_graph_capture)."""
        _check("tsp_plan_graph_capture", load()[1].tsp_plan_graph_capture(self.p, steps))

    def graph_run(self, replays: int = 1) -> None:
        _check("tsp_plan_graph_run", load()[1].tsp_plan_graph_run(self.p, replays))

    def graph_time(self, replays: int) -> float:
        """Milliseconds per step over `replays` replays of the captured graph."""
        ms = C.c_double()
        _check("tsp_plan_graph_time", load()[1].tsp_plan_graph_time(self.p, replays, C.byref(ms)))
        return ms.value

    def graph_free(self) -> None:
        _check("tsp_plan_graph_free", load()[1].tsp_plan_graph_free(self.p))

    def time_class(self, bm: int, reps: int) -> float:
        ms = C.c_double()
        _check("tsp_plan_time_class", load()[1].tsp_plan_time_class(self.p, bm, reps, C.byref(ms)))
        return ms.value

    def download_c(self) -> np.ndarray:
        out = np.zeros((self.rowA, self.colB_p), dtype=np.float32)
        _check("tsp_plan_download_c", load()[1].tsp_plan_download_c(self.p, _ptr(out)))
        return out
