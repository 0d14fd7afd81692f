"""ctypes binding of libmpserve_amd.so (the C ABI declared in include/mpserve_amd.h).

The library is required: importing a function from here on a machine where it
has not been built raises ImportError naming the build command. There is no
CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmpserve_amd.so")

MPS_OK = 0
MPS_ERR_INVALID_ARGUMENT = -1
MPS_ERR_RUNTIME = -2
MPS_ERR_HIP = -3
MPS_ERR_NO_MEMORY = -4

MPS_STATUS_BAD_BUCKET = 0x1
MPS_STATUS_BAD_ROW = 0x2
MPS_STATUS_BAD_TABLE = 0x4
MPS_STATUS_DESYNC = 0x8

_p = ctypes.c_void_p
_i64 = ctypes.c_int64


class MpsFp8Tensor(ctypes.Structure):
    """mps_fp8_tensor: one FP8 tensor + sidecar, device pointers."""

    _fields_ = [
        ("fp8", _p), ("bitstream", _p), ("bitstream_words", _i64),
        ("decode_syms", _p), ("decode_lens", _p), ("num_tables", _i64),
        ("bucket_table", _p), ("bucket_col_start", _p), ("bucket_col_len", _p),
        ("bucket_row_offsets", _p), ("row_indices", _p), ("num_row_indices", _i64),
        ("bucket_thread_startbit", _p), ("bucket_bit_base", _p), ("num_buckets", _i64),
        ("k", _i64), ("n", _i64), ("m", _i64), ("out", _p),
    ]


class MpsFp8EncodeIn(ctypes.Structure):
    """mps_fp8_encode_in: device inputs of the GPU sidecar builder."""

    _fields_ = [
        ("bf16", _p), ("fp8", _p), ("scales", _p), ("numel", _i64),
        ("ndim", ctypes.c_int32), ("scale_ndim", ctypes.c_int32),
        ("dims", _i64 * 8), ("scale_dims", _i64 * 8), ("scale_numel", _i64),
        ("max_len", _i64), ("threads_per_block", _i64),
    ]


class MpsAwqTensor(ctypes.Structure):
    """mps_awq_tensor: one AWQ int4 tensor + sidecar (row or by-scale layout), device pointers."""

    _fields_ = [
        ("int4", _p), ("bitstream", _p), ("bitstream_words", _i64),
        ("decode_syms", _p), ("decode_lens", _p), ("num_tables", _i64),
        ("bucket_table", _p), ("bucket_col_start", _p), ("bucket_col_len", _p),
        ("bucket_row_offsets", _p), ("row_indices", _p), ("num_row_indices", _i64),
        ("group_col_start", _p), ("group_size", _i64),
        ("bucket_thread_startbit", _p), ("bucket_bit_base", _p), ("num_buckets", _i64),
        ("k", _i64), ("n", _i64), ("m", _i64), ("out", _p),
    ]


class MpsAwqEncodeIn(ctypes.Structure):
    """mps_awq_encode_in: device inputs of the AWQ int4 sidecar builders."""

    _fields_ = [
        ("bf16", _p), ("int4", _p), ("scales", _p), ("n", _i64), ("m", _i64),
        ("scale_ndim", ctypes.c_int32), ("by_scale", ctypes.c_int32),
        ("scale_dims", _i64 * 2), ("scale_numel", _i64),
        ("max_len", _i64), ("threads_per_block", _i64), ("group_cap", _i64),
    ]


_lib = None


def lib():
    """The loaded library; raises ImportError if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"mpserve_amd native library missing at {LIB_PATH}; build it with "
            "`python -m mpserve_amd.build` (hipcc, gfx950)")
    L = ctypes.CDLL(LIB_PATH)
    L.mps_last_error.restype = ctypes.c_char_p
    L.mps_clock_rate_khz.argtypes = [ctypes.c_int, ctypes.POINTER(_i64)]
    L.mps_fp8_decode.argtypes = [ctypes.POINTER(MpsFp8Tensor), _i64, _p]
    L.mps_fp8_plan_create.argtypes = [ctypes.POINTER(MpsFp8Tensor), _i64, _p, ctypes.POINTER(_p)]
    L.mps_fp8_plan_decode.argtypes = [_p, _p]
    L.mps_fp8_plan_decode_into.argtypes = [_p, _p, _p]
    L.mps_fp8_plan_info.argtypes = [_p, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]
    L.mps_fp8_plan_read_status.argtypes = [_p, _p, ctypes.POINTER(ctypes.c_uint32)]
    L.mps_fp8_plan_destroy.argtypes = [_p]
    L.mps_fp8_read_status.argtypes = [ctypes.c_int, _p, ctypes.POINTER(ctypes.c_uint32)]
    L.mps_fp8_decode_batch_noalloc.argtypes = [ctypes.POINTER(MpsFp8Tensor), _i64, _i64, _p]
    L.mps_stream_capture_id.argtypes = [_p, ctypes.POINTER(ctypes.c_uint64)]
    if hasattr(L, "mps_fp8_encode"):
        L.mps_fp8_encode.argtypes = [ctypes.POINTER(MpsFp8EncodeIn), _p, ctypes.POINTER(_p)]
        L.mps_fp8_sidecar_sizes.argtypes = [_p, ctypes.POINTER(_i64)]
        L.mps_fp8_sidecar_copy.argtypes = [_p, ctypes.POINTER(_p), _p]
        L.mps_fp8_sidecar_free.argtypes = [_p]
        L.mps_fp8_sidecar_stats.argtypes = [_p, ctypes.POINTER(_i64)]
    L.mps_awq_decode.argtypes = [ctypes.POINTER(MpsAwqTensor), _i64, _p]
    L.mps_awq_encode.argtypes = [ctypes.POINTER(MpsAwqEncodeIn), _p, ctypes.POINTER(_p)]
    L.mps_awq_plan_create.argtypes = [ctypes.POINTER(MpsAwqTensor), _i64, _p, ctypes.POINTER(_p)]
    L.mps_awq_plan_decode.argtypes = [_p, _p]
    L.mps_awq_plan_decode_into.argtypes = [_p, _p, _p]
    L.mps_awq_plan_info.argtypes = [_p, ctypes.POINTER(_i64)]
    L.mps_awq_plan_read_status.argtypes = [_p, _p, ctypes.POINTER(ctypes.c_uint32)]
    L.mps_awq_plan_destroy.argtypes = [_p]
    for name in ("mps_clock_rate_khz", "mps_fp8_decode", "mps_fp8_plan_create", "mps_fp8_plan_decode",
                 "mps_fp8_plan_decode_into", "mps_fp8_plan_info", "mps_fp8_plan_read_status",
                 "mps_fp8_plan_destroy", "mps_fp8_read_status", "mps_fp8_decode_batch_noalloc", "mps_stream_capture_id",
                 "mps_awq_decode", "mps_awq_encode",
                 "mps_awq_plan_create", "mps_awq_plan_decode", "mps_awq_plan_decode_into", "mps_awq_plan_info", "mps_awq_plan_read_status",
                 "mps_awq_plan_destroy"):
        getattr(L, name).restype = ctypes.c_int
    _lib = L
    return L


def check(rc: int) -> None:
    """Raise the Python exception matching an MPS_ERR_* code."""
    if rc == MPS_OK:
        return
    msg = lib().mps_last_error().decode(errors="replace")
    if rc == MPS_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    if rc == MPS_ERR_NO_MEMORY:
        raise MemoryError(msg)
    raise RuntimeError(msg)
