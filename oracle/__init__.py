"""CPU parity oracle for the FP8 + Huffman-sidecar path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for
``cpu_baseline``, as the timed host decoder of the same sidecar format). The
product package ``mpserve_amd`` never imports it.

The C restatement lives in ``fp8_huffman_oracle.c`` (``liboracle.so``, built by
``oracle/Makefile``). Each function cites the reference lines it follows.

How each part is pinned (the reference ships no tests, golden vectors or
fixtures, and its encoder cannot be built in this image, so ``oracle/_ref`` is
empty; see the Makefile):

* ``package_merge`` (build_huffman.cu:46-118): brute-force optimality over every
  length vector with Kraft sum <= 1 on small alphabets, equality with textbook
  Huffman cost when the limit does not bind, Kraft equality, monotonicity
  (heavier symbol never longer), plus hand-traced vectors of the reference's
  tie rule (leaf before package on equal weight) and a second, independent
  formulation (leaf counts of selected prefixes) that must agree exactly.
* histogram, key order, bucketing, bucket_table/U/uniq/uidx: closed forms
  recomputed with numpy in the tests (np.unique / lexsort), not retyped C.
* canonical codes + LUT fill: prefix-freeness, Kraft equality, LUT coverage
  (every entry decodes the code that prefixes it), and the (count asc, sym asc)
  hand-out order checked on hand-traced vectors.
* bitstream + starts: round trip decode(encode(x)) == x bit-exact, per-bucket
  bit length == starts[k_eff], 64-bit aligned bases, monotone starts, and an
  independent numpy re-packing of the per-element code words.
* ESC path: forced >2^L-symbol keys round-trip; esc_sym is the smallest u16
  outside the kept set (checked against a brute-force scan).

Parity unpinned (no reference run possible, no golden vectors exist): the
exact choice among equal-cost length vectors is pinned only by the hand traces
of the reference's merge order, not by a reference execution.

The AWQ int4 bucket builders and decoders (``awq_huffman_oracle.c``,
``awq_encode`` / ``awq_decode`` below) share package-merge with the FP8 oracle
and are pinned in tests/test_awq_oracle.py:
- round trips for both layouts, every scale mode, and k below and above the
  column count;
- numpy closed forms of the keys, ``bucket_table``, row order and group
  order/chunking;
- Kraft sums, LUT coverage and the single nibble-15 ESC entry;
- brute-force scans of both ESC symbol rules;
- the hand-out order of both ESC lists, (count asc, sym asc) for row buckets
  against (count desc, sym asc) with ESC last by scale.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Dict

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

ORC_OK = 0
ORC_INVALID_ARGUMENT = 1
ORC_RUNTIME_ERROR = 2

MODE_LOSSLESS = 0
MODE_REFERENCE_KERNEL = 1

_i64 = ctypes.c_int64
_p = ctypes.c_void_p


class _Sidecar(ctypes.Structure):
    _fields_ = [
        ("G", _i64), ("table_size", _i64), ("packed_len_size", _i64),
        ("decode_syms", _p), ("decode_lens", _p), ("table_scale", _p), ("table_fp8", _p),
        ("B", _i64), ("bucket_scale", _p), ("bucket_row_offsets", _p), ("R", _i64),
        ("row_indices", _p), ("bucket_table", _p), ("bucket_col_start", _p), ("bucket_col_len", _p),
        ("k", _i64), ("bucket_thread_startbit", _p), ("bucket_bit_base", _p), ("W", _i64),
        ("bitstream", _p), ("shape_nmk", _i64 * 3), ("bucket_U", _p), ("bucket_unique_gid", _p),
        ("bucket_fp8_uidx", _p), ("esc_keys", _i64), ("esc_collisions", _i64), ("esc_elements", _i64),
    ]


class _AwqSidecar(ctypes.Structure):
    _fields_ = [
        ("G", _i64), ("table_size", _i64), ("packed_len_size", _i64),
        ("decode_syms", _p), ("decode_lens", _p), ("table_scale", _p), ("table_qv", _p),
        ("B", _i64), ("bucket_scale", _p), ("row_offsets", _p), ("R", _i64), ("row_indices", _p),
        ("col_start", _p), ("col_len", _p), ("bucket_table", _p), ("k", _i64), ("startbit", _p),
        ("bit_base", _p), ("W", _i64), ("bitstream", _p), ("shape", _i64 * 4), ("group_size", _i64),
        ("esc_keys", _i64), ("esc_collisions", _i64), ("esc_elements", _i64),
    ]


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (``force``: always, even
    when the library is newer than its sources)."""
    if force or not os.path.exists(_LIB_PATH) or any(
        os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, src))
        for src in ("fp8_huffman_oracle.c", "awq_huffman_oracle.c")
    ):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []) + ["liboracle.so"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.orc_last_error.restype = ctypes.c_char_p
    lib.orc_encode.restype = ctypes.c_int
    lib.orc_encode.argtypes = [_p, _p, _i64, ctypes.c_int, _p, _p, _i64, ctypes.c_int, _p, _i64, _i64,
                               ctypes.POINTER(ctypes.POINTER(_Sidecar))]
    lib.orc_free.argtypes = [ctypes.POINTER(_Sidecar)]
    lib.orc_decode.restype = ctypes.c_int
    lib.orc_decode.argtypes = [_p, _p, _i64, _p, _p, _i64, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64,
                               _i64, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _p]
    lib.orc_package_merge.restype = ctypes.c_int
    lib.orc_package_merge.argtypes = [_p, ctypes.c_int, ctypes.c_int, _p]
    lib.orc_awq_last_error.restype = ctypes.c_char_p
    lib.orc_awq_encode.restype = ctypes.c_int
    lib.orc_awq_encode.argtypes = [_p, _p, _i64, _i64, _p, _i64, ctypes.c_int, _p, _i64, _i64, _i64, ctypes.c_int,
                                   ctypes.POINTER(ctypes.POINTER(_AwqSidecar))]
    lib.orc_awq_free.argtypes = [ctypes.POINTER(_AwqSidecar)]
    lib.orc_awq_decode.restype = ctypes.c_int
    lib.orc_awq_decode.argtypes = [_p, _p, _i64, _p, _p, _i64, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64, _p,
                                   _i64, _i64, _i64, ctypes.c_int, _p]
    _lib = lib
    return lib


def _raise(rc: int):
    msg = _load().orc_last_error().decode()
    if rc == ORC_INVALID_ARGUMENT:
        raise ValueError(msg)
    raise RuntimeError(msg)


def _copy(ptr, count, dtype, shape=None):
    count = int(count)
    a = np.empty(count, dtype=dtype)
    if count:
        ctypes.memmove(a.ctypes.data, ptr, count * a.itemsize)
    return a.reshape(shape) if shape is not None else a


def package_merge(weights, max_len: int):
    """Code lengths for ascending ``weights`` (build_huffman.cu:46-118)."""
    w = np.ascontiguousarray(np.asarray(weights, dtype=np.int64).astype(np.int32))
    out = np.zeros(max(1, w.size), dtype=np.int32)
    rc = _load().orc_package_merge(w.ctypes.data, int(w.size), int(max_len), out.ctypes.data)
    if rc != ORC_OK:
        _raise(rc)
    return [int(x) for x in out[: w.size]]


def encode(bf16_bits: np.ndarray, fp8_u8: np.ndarray, scales_u16: np.ndarray,
           max_len: int = 7, threads_per_block: int = 1024, with_stats: bool = False):
    """Sidecar of ``bf16_bits`` (u16 BF16 patterns) given FP8 bytes and u16 scale keys.

    Mirrors huffman_build_fp8_decode_tables_entry (build_huffman.cu:292-969):
    returns the 17 arrays under the reference's dict keys (wrapper.cpp:429-446).
    """
    bf = np.ascontiguousarray(bf16_bits, dtype=np.uint16)
    q = np.ascontiguousarray(fp8_u8, dtype=np.uint8)
    sc = np.ascontiguousarray(scales_u16, dtype=np.uint16)
    if q.size != bf.size:
        raise ValueError("bf16_params and fp8_params must have same numel")
    dims = np.array(bf.shape if bf.ndim else (), dtype=np.int64)
    sdims = np.array(sc.shape if sc.ndim else (), dtype=np.int64)
    out = ctypes.POINTER(_Sidecar)()
    lib = _load()
    rc = lib.orc_encode(bf.ctypes.data, q.ctypes.data, int(bf.size), int(bf.ndim),
                        dims.ctypes.data if dims.size else None,
                        sc.ctypes.data, int(sc.size), int(sc.ndim), sdims.ctypes.data if sdims.size else None,
                        int(max_len), int(threads_per_block), ctypes.byref(out))
    if rc != ORC_OK:
        _raise(rc)
    s = out.contents
    try:
        G, T, P, B, R, k, W = s.G, s.table_size, s.packed_len_size, s.B, s.R, s.k, s.W
        d = {
            "decode_syms_u16": _copy(s.decode_syms, G * T, np.uint16, (G, T)),
            "decode_lens_u8": _copy(s.decode_lens, G * P, np.uint8, (G, P)),
            "table_scale_u16": _copy(s.table_scale, G, np.uint16),
            "table_fp8_u16": _copy(s.table_fp8, G, np.uint16),
            "bucket_scale_u16": _copy(s.bucket_scale, B, np.uint16),
            "bucket_row_offsets_i32": _copy(s.bucket_row_offsets, B + 1, np.int32),
            "row_indices_i32": _copy(s.row_indices, R, np.int32),
            "bucket_table_i32": _copy(s.bucket_table, B * 256, np.int32, (B, 256)),
            "bucket_col_start_i32": _copy(s.bucket_col_start, B, np.int32),
            "bucket_col_len_i32": _copy(s.bucket_col_len, B, np.int32),
            "bucket_thread_startbit_u32": _copy(s.bucket_thread_startbit, B * (k + 1), np.uint32, (B, k + 1)),
            "bucket_bit_base_i64": _copy(s.bucket_bit_base, B + 1, np.int64),
            "bitstream_u64": _copy(s.bitstream, W, np.uint64),
            "shape_nmk_i64": np.array(list(s.shape_nmk), dtype=np.int64),
            "bucket_U_i32": _copy(s.bucket_U, B, np.int32),
            "bucket_unique_gid_i32": _copy(s.bucket_unique_gid, B * 256, np.int32, (B, 256)),
            "bucket_fp8_uidx_i16": _copy(s.bucket_fp8_uidx, B * 256, np.int16, (B, 256)),
        }
        stats = {"esc_keys": int(s.esc_keys), "esc_collisions": int(s.esc_collisions),
                 "esc_elements": int(s.esc_elements)}
    finally:
        lib.orc_free(out)
    return (d, stats) if with_stats else d


def decode(sc: Dict[str, np.ndarray], fp8_u8: np.ndarray, n: int, m: int, max_len: int = 7,
           mode: int = MODE_LOSSLESS, nthreads: int = 1, out: np.ndarray | None = None) -> np.ndarray:
    """BF16 bit patterns [n, m] rebuilt from FP8 bytes + sidecar (decode_huffman.cu:188-372 semantics).

    ``mode=MODE_LOSSLESS`` reads the raw 16 bits after ESC codes and walks columns
    as e % col_len; ``MODE_REFERENCE_KERNEL`` reproduces the reference kernel.
    Elements no lane writes keep the contents of ``out`` (zeros if not given).
    """
    arrs = {
        "q": np.ascontiguousarray(fp8_u8, dtype=np.uint8),
        "bs": np.ascontiguousarray(sc["bitstream_u64"]).view(np.uint64),
        "syms": np.ascontiguousarray(sc["decode_syms_u16"]).view(np.uint16),
        "lens": np.ascontiguousarray(sc["decode_lens_u8"], dtype=np.uint8),
        "bt": np.ascontiguousarray(sc["bucket_table_i32"], dtype=np.int32),
        "cs": np.ascontiguousarray(sc["bucket_col_start_i32"], dtype=np.int32),
        "cl": np.ascontiguousarray(sc["bucket_col_len_i32"], dtype=np.int32),
        "ro": np.ascontiguousarray(sc["bucket_row_offsets_i32"], dtype=np.int32),
        "ri": np.ascontiguousarray(sc["row_indices_i32"], dtype=np.int32),
        "sb": np.ascontiguousarray(sc["bucket_thread_startbit_u32"]).view(np.uint32),
        "bb": np.ascontiguousarray(sc["bucket_bit_base_i64"], dtype=np.int64),
    }
    if out is None:
        out = np.zeros((n, m), dtype=np.uint16)
    assert out.dtype == np.uint16 and out.flags.c_contiguous and out.size == n * m
    if arrs["q"].size != n * m:
        raise ValueError("fp8_params_u8 numel must equal n*m")
    B = arrs["bt"].shape[0]
    k = arrs["sb"].shape[1] - 1
    G = arrs["syms"].shape[0]
    rc = _load().orc_decode(arrs["q"].ctypes.data, arrs["bs"].ctypes.data, int(arrs["bs"].size),
                            arrs["syms"].ctypes.data, arrs["lens"].ctypes.data, int(G),
                            arrs["bt"].ctypes.data, arrs["cs"].ctypes.data, arrs["cl"].ctypes.data,
                            arrs["ro"].ctypes.data, arrs["ri"].ctypes.data, int(arrs["ri"].size),
                            arrs["sb"].ctypes.data, int(k), arrs["bb"].ctypes.data, int(B),
                            int(n), int(m), int(max_len), int(mode), int(nthreads), out.ctypes.data)
    if rc != ORC_OK:
        _raise(rc)
    return out


# --------------------------------------------------------------------------
# AWQ int4 bucket variants (awq_huffman_oracle.c)
# --------------------------------------------------------------------------
def _awq_raise(rc: int):
    msg = _load().orc_awq_last_error().decode()
    if rc == ORC_INVALID_ARGUMENT:
        raise ValueError(msg)
    raise RuntimeError(msg)


def awq_encode(bf16_bits: np.ndarray, int4_u8: np.ndarray, scales_u16: np.ndarray, max_len: int = 11,
               threads: int = 256, group_cap: int = 1024, by_scale: bool = False, with_stats: bool = False):
    """AWQ int4 sidecar under the reference's dict keys.

    ``by_scale=False`` mirrors huffman_build_awq_int4_bucket_decode_tables_entry
    (build_huffman.cu:1583-2126, 14 keys, wrapper.cpp:268-281); ``by_scale=True``
    mirrors ..._by_scale_entry (build_huffman.cu:1075-1580, 13 keys, wrapper.cpp:301-313).
    """
    bf = np.ascontiguousarray(bf16_bits, dtype=np.uint16)
    q = np.ascontiguousarray(int4_u8, dtype=np.uint8)
    sc = np.ascontiguousarray(scales_u16, dtype=np.uint16)
    if bf.ndim != 2:
        raise ValueError("bf16_params must be 2D [n,m]")
    if q.shape != bf.shape:
        raise ValueError("int4_values_u8 shape must match bf16_params")
    n, m = bf.shape
    sdims = np.array(sc.shape if sc.ndim else (), dtype=np.int64)
    out = ctypes.POINTER(_AwqSidecar)()
    lib = _load()
    rc = lib.orc_awq_encode(bf.ctypes.data, q.ctypes.data, int(n), int(m), sc.ctypes.data, int(sc.size),
                            int(sc.ndim), sdims.ctypes.data if sdims.size else None, int(max_len), int(threads),
                            int(group_cap), int(bool(by_scale)), ctypes.byref(out))
    if rc != ORC_OK:
        _awq_raise(rc)
    s = out.contents
    try:
        G, T, P, B, R, k, W = s.G, s.table_size, s.packed_len_size, s.B, s.R, s.k, s.W
        head = {
            "decode_syms_u16": _copy(s.decode_syms, G * T, np.uint16, (G, T)),
            "decode_lens_u8": _copy(s.decode_lens, G * P, np.uint8, (G, P)),
            "table_scale_u16": _copy(s.table_scale, G, np.uint16),
            "table_qv_u16": _copy(s.table_qv, G, np.uint16),
            "bucket_scale_u16": _copy(s.bucket_scale, B, np.uint16),
        }
        tail = {
            "bucket_thread_startbit_u32": _copy(s.startbit, B * (k + 1), np.uint32, (B, k + 1)),
            "bucket_bit_base_i64": _copy(s.bit_base, B + 1, np.int64),
            "bitstream_u64": _copy(s.bitstream, W, np.uint64),
        }
        table = _copy(s.bucket_table, B * 16, np.int32, (B, 16))
        if by_scale:
            d = dict(head)
            d["bucket_group_offsets_i32"] = _copy(s.row_offsets, B + 1, np.int32)
            d["group_rows_i32"] = _copy(s.row_indices, R, np.int32)
            d["group_col_start_i32"] = _copy(s.col_start, R, np.int32)
            d["bucket_table_i32"] = table
            d.update(tail)
            d["shape_nmkg_i64"] = np.array(list(s.shape), dtype=np.int64)
        else:
            d = dict(head)
            d["bucket_row_offsets_i32"] = _copy(s.row_offsets, B + 1, np.int32)
            d["row_indices_i32"] = _copy(s.row_indices, R, np.int32)
            d["bucket_table_i32"] = table
            d["bucket_col_start_i32"] = _copy(s.col_start, B, np.int32)
            d["bucket_col_len_i32"] = _copy(s.col_len, B, np.int32)
            d.update(tail)
            d["shape_nmk_i64"] = np.array(list(s.shape)[:3], dtype=np.int64)
        stats = {"esc_keys": int(s.esc_keys), "esc_collisions": int(s.esc_collisions),
                 "esc_elements": int(s.esc_elements)}
    finally:
        lib.orc_awq_free(out)
    return (d, stats) if with_stats else d


def awq_decode(sc: Dict[str, np.ndarray], int4_u8: np.ndarray, n: int, m: int, group_size: int | None = None,
               nthreads: int = 1, out: np.ndarray | None = None) -> np.ndarray:
    """BF16 bit patterns [n, m] from int4 values + an AWQ sidecar of either layout
    (decode_huffman.cu:378-589 semantics, columns walked as e % col_len)."""
    by_scale = "bucket_group_offsets_i32" in sc
    q = np.ascontiguousarray(int4_u8, dtype=np.uint8)
    bs = np.ascontiguousarray(sc["bitstream_u64"]).view(np.uint64)
    syms = np.ascontiguousarray(sc["decode_syms_u16"]).view(np.uint16)
    lens = np.ascontiguousarray(sc["decode_lens_u8"], dtype=np.uint8)
    bt = np.ascontiguousarray(sc["bucket_table_i32"], dtype=np.int32)
    sb = np.ascontiguousarray(sc["bucket_thread_startbit_u32"]).view(np.uint32)
    bb = np.ascontiguousarray(sc["bucket_bit_base_i64"], dtype=np.int64)
    if by_scale:
        ro = np.ascontiguousarray(sc["bucket_group_offsets_i32"], dtype=np.int32)
        ri = np.ascontiguousarray(sc["group_rows_i32"], dtype=np.int32)
        gc = np.ascontiguousarray(sc["group_col_start_i32"], dtype=np.int32)
        gs = int(group_size if group_size is not None else sc["shape_nmkg_i64"][3])
        cs = cl = None
    else:
        ro = np.ascontiguousarray(sc["bucket_row_offsets_i32"], dtype=np.int32)
        ri = np.ascontiguousarray(sc["row_indices_i32"], dtype=np.int32)
        cs = np.ascontiguousarray(sc["bucket_col_start_i32"], dtype=np.int32)
        cl = np.ascontiguousarray(sc["bucket_col_len_i32"], dtype=np.int32)
        gc, gs = None, 0
    if out is None:
        out = np.zeros((n, m), dtype=np.uint16)
    assert out.dtype == np.uint16 and out.flags.c_contiguous and out.size == n * m
    if q.size != n * m:
        raise ValueError("int4_values_u8 numel must equal n*m")
    ptr = lambda a: a.ctypes.data if a is not None else None  # noqa: E731
    rc = _load().orc_awq_decode(q.ctypes.data, bs.ctypes.data, int(bs.size), syms.ctypes.data, lens.ctypes.data,
                                int(syms.shape[0]), bt.ctypes.data, ptr(cs), ptr(cl), ro.ctypes.data, ri.ctypes.data,
                                int(ri.size), ptr(gc), int(gs), sb.ctypes.data, int(sb.shape[1] - 1), bb.ctypes.data,
                                int(bt.shape[0]), int(n), int(m), int(nthreads), out.ctypes.data)
    if rc != ORC_OK:
        _awq_raise(rc)
    return out
