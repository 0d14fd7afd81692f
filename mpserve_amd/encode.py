"""GPU sidecar builder behind MPServe_cuda.huffman_build_fp8_decode_tables.

Argument checks follow the reference entry (kernel/build_huffman.cu:298-366) in
order and wording; the work itself runs in libmpserve_amd.so (mps_fp8_encode).
"""
from __future__ import annotations

import ctypes
from typing import Dict

import torch

from . import _native

# (key, dtype) of the 17 outputs in the reference's order (kernel/wrapper.cpp:429-446)
_OUTPUTS = (
    ("decode_syms_u16", torch.uint16), ("decode_lens_u8", torch.uint8), ("table_scale_u16", torch.uint16),
    ("table_fp8_u16", torch.uint16), ("bucket_scale_u16", torch.uint16), ("bucket_row_offsets_i32", torch.int32),
    ("row_indices_i32", torch.int32), ("bucket_table_i32", torch.int32), ("bucket_col_start_i32", torch.int32),
    ("bucket_col_len_i32", torch.int32), ("bucket_thread_startbit_u32", torch.uint32),
    ("bucket_bit_base_i64", torch.int64), ("bitstream_u64", torch.uint64), ("shape_nmk_i64", torch.int64),
    ("bucket_U_i32", torch.int32), ("bucket_unique_gid_i32", torch.int32), ("bucket_fp8_uidx_i16", torch.int16),
)


def _shapes(G: int, B: int, k: int, L: int, sizes) -> list:
    table = 1 << L
    packed = max(1, table // 2)
    return [(G, table), (G, packed), (G,), (G,), (B,), (B + 1,), (int(sizes[6]),), (B, 256), (B,), (B,),
            (B, k + 1), (B + 1,), (int(sizes[12]),), (3,), (B,), (B, 256), (B, 256)]


def build_fp8_sidecar(bf16_params: torch.Tensor, fp8_params: torch.Tensor, scales: torch.Tensor,
                      max_len: int = 12, threads_per_block: int = 256, *, with_stats: bool = False):
    """The 17-key sidecar dict of one weight, built on the GPU (see module doc)."""
    if bf16_params is None or fp8_params is None or scales is None:
        raise ValueError("inputs must be defined")
    if bf16_params.dtype != torch.bfloat16:
        raise ValueError("bf16_params must be torch.bfloat16")
    if fp8_params.dtype != torch.uint8:
        raise ValueError("fp8_params must be torch.uint8")
    if max_len <= 0 or max_len > 15:
        raise ValueError("max_len must be in [1, 15]")
    if threads_per_block <= 0 or threads_per_block > 1024:
        raise ValueError("threads_per_block must be in [1, 1024]")
    if fp8_params.numel() != bf16_params.numel():
        raise ValueError("bf16_params and fp8_params must have same numel")
    if scales.dtype not in (torch.uint16, torch.bfloat16):
        raise ValueError("scales must be torch.uint16 or torch.bfloat16")
    if not torch.cuda.is_available():
        raise RuntimeError("huffman_build_fp8_decode_tables runs on the GPU in this build; no GPU is visible")
    on_host = not bf16_params.is_cuda
    dev = bf16_params.device if bf16_params.is_cuda else torch.device("cuda", torch.cuda.current_device())
    bf = bf16_params.contiguous().to(dev).view(torch.uint16)
    q = fp8_params.contiguous().to(dev)
    sc = scales.contiguous().to(dev).view(torch.uint16)
    if bf.dim() > 8 or sc.dim() > 8:
        raise ValueError("too many dimensions")

    a = _native.MpsFp8EncodeIn()
    a.bf16 = bf.data_ptr()
    a.fp8 = q.data_ptr()
    a.scales = sc.data_ptr()
    a.numel = bf.numel()
    a.ndim = bf.dim()
    a.scale_ndim = sc.dim()
    for i, d in enumerate(bf.shape):
        a.dims[i] = d
    for i, d in enumerate(sc.shape):
        a.scale_dims[i] = d
    a.scale_numel = sc.numel()
    a.max_len = int(max_len)
    a.threads_per_block = int(threads_per_block)
    lib = _native.lib()
    handle = ctypes.c_void_p()
    with torch.cuda.device(dev):
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _native.check(lib.mps_fp8_encode(ctypes.byref(a), stream, ctypes.byref(handle)))
        try:
            sizes = (ctypes.c_int64 * 17)()
            _native.check(lib.mps_fp8_sidecar_sizes(handle, sizes))
            stats = (ctypes.c_int64 * 4)()
            _native.check(lib.mps_fp8_sidecar_stats(handle, stats))
            G = int(sizes[2])
            B = int(sizes[4])
            shapes = _shapes(G, B, int(threads_per_block), int(max_len), sizes)
            out: Dict[str, torch.Tensor] = {}
            ptrs = (ctypes.c_void_p * 17)()
            for i, ((key, dt), shp) in enumerate(zip(_OUTPUTS, shapes)):
                t = torch.empty(shp, dtype=dt, device="cpu" if on_host else dev)
                out[key] = t
                ptrs[i] = t.data_ptr() if t.numel() else None
            _native.check(lib.mps_fp8_sidecar_copy(handle, ptrs, stream))
        finally:
            lib.mps_fp8_sidecar_free(handle)
    if with_stats:
        return out, {"esc_keys": int(stats[0]), "esc_collisions": int(stats[1]), "distinct_pairs": int(stats[2]),
                     "hash_slots": int(stats[3])}
    return out
