"""AWQ int4 + Huffman-sidecar ops of ``MPServe_cuda``, served by HIP kernels on MI355X.

The reference binds two builders and two decoders for AWQ int4 weights
(kernel/wrapper.cpp:258-416):

* ``huffman_build_awq_int4_bucket_decode_tables`` (row buckets,
  build_huffman.cu:1583-2126) and ``huffman_decode_awq_int4_bucket``
  (decode_huffman.cu:877-1018 with the kernel at :378-475);
* ``huffman_build_awq_int4_bucket_decode_tables_by_scale`` (buckets of
  quantisation groups that share one exact scale, build_huffman.cu:1075-1580)
  and ``huffman_decode_awq_int4_bucket_by_scale`` (decode_huffman.cu:760-875,
  kernel :477-589).

Same op and argument names, defaults, dict keys, argument checks in order and
wording. The builders run on the GPU (libmpserve_amd.so, mps_awq_encode) and
give the reference builders' bytes; CPU inputs come back as CPU tensors. The
decoders run on the current stream of the int4 tensor's device (mps_awq_decode).
"""
from __future__ import annotations

import ctypes
from typing import Dict

import torch

from . import _native
from ._common import _check_cuda_contig, _maybe_check_status, _stream_handle

# Dict keys in the reference's order (wrapper.cpp:268-281, :301-313) and the
# builder-handle slot each comes from.
BUCKET_KEYS = (
    ("decode_syms_u16", 0, torch.uint16), ("decode_lens_u8", 1, torch.uint8), ("table_scale_u16", 2, torch.uint16),
    ("table_qv_u16", 3, torch.uint16), ("bucket_scale_u16", 4, torch.uint16),
    ("bucket_row_offsets_i32", 5, torch.int32), ("row_indices_i32", 6, torch.int32),
    ("bucket_table_i32", 7, torch.int32), ("bucket_col_start_i32", 8, torch.int32),
    ("bucket_col_len_i32", 9, torch.int32), ("bucket_thread_startbit_u32", 10, torch.uint32),
    ("bucket_bit_base_i64", 11, torch.int64), ("bitstream_u64", 12, torch.uint64), ("shape_nmk_i64", 13, torch.int64),
)
BY_SCALE_KEYS = (
    ("decode_syms_u16", 0, torch.uint16), ("decode_lens_u8", 1, torch.uint8), ("table_scale_u16", 2, torch.uint16),
    ("table_qv_u16", 3, torch.uint16), ("bucket_scale_u16", 4, torch.uint16),
    ("bucket_group_offsets_i32", 5, torch.int32), ("group_rows_i32", 6, torch.int32),
    ("group_col_start_i32", 8, torch.int32), ("bucket_table_i32", 7, torch.int32),
    ("bucket_thread_startbit_u32", 10, torch.uint32), ("bucket_bit_base_i64", 11, torch.int64),
    ("bitstream_u64", 12, torch.uint64), ("shape_nmkg_i64", 13, torch.int64),
)


def build_awq_sidecar(bf16, int4, scales, max_len: int = 11, threads: int = 256, group_cap: int = 1024,
                      by_scale: bool = False, *, with_stats: bool = False):
    """Either AWQ int4 sidecar dict; with ``with_stats`` also {esc_keys, esc_collisions}:
    keys coded with an ESC symbol, and elements whose symbol equals their key's
    ESC symbol without being kept (the row-bucket builder can pick such a
    symbol; those elements are written as a bare ESC code, which decodes to
    16 bits read from the next codes, in the reference as here)."""
    return _build(bf16, int4, scales, int(max_len), int(threads), int(group_cap), bool(by_scale), with_stats)


def _build(bf16, int4, scales, max_len, threads, group_cap, by_scale: bool, with_stats: bool = False):
    # build_huffman.cu:1082-1123 (by scale) / :1589-1623, in order
    if bf16 is None or int4 is None or scales is None:
        raise ValueError("inputs must be defined")
    if bf16.dtype != torch.bfloat16:
        raise ValueError("bf16_params must be torch.bfloat16")
    if int4.dtype != torch.uint8:
        raise ValueError("int4_values_u8 must be torch.uint8")
    if scales.dtype != torch.uint16:
        raise ValueError("scales_u16 must be torch.uint16 (bf16 raw bits)")
    if max_len <= 0 or max_len > 15:
        raise ValueError("max_len must be in (0,15]")
    if threads <= 0 or threads > 1024:
        raise ValueError("threads_per_block must be in [1,1024]")
    if by_scale and group_cap <= 0:
        raise ValueError("group_cap must be > 0")
    if bf16.dim() != 2:
        raise ValueError("bf16_params must be 2D [n,m]")
    if int4.shape != bf16.shape:
        raise ValueError("int4_values_u8 shape must match bf16_params")
    n, m = int(bf16.shape[0]), int(bf16.shape[1])
    if n <= 0 or m <= 0:
        raise ValueError("bf16_params shape must be non-empty")
    if scales.dim() > 2:
        raise ValueError("unsupported scales_u16 shape: use scalar, per-row (n,), or 2D block-wise [n/bs0,m/bs1]")
    if not torch.cuda.is_available():
        raise RuntimeError("the AWQ int4 builders run on the GPU in this build; no GPU is visible")
    on_host = not bf16.is_cuda
    dev = bf16.device if bf16.is_cuda else torch.device("cuda", torch.cuda.current_device())
    bf = bf16.contiguous().to(dev).view(torch.uint16)
    q = int4.contiguous().to(dev)
    sc = scales.contiguous().to(dev)
    a = _native.MpsAwqEncodeIn()
    a.bf16, a.int4, a.scales = bf.data_ptr(), q.data_ptr(), sc.data_ptr()
    a.n, a.m = n, m
    a.scale_ndim = sc.dim()
    for i, d in enumerate(sc.shape):
        a.scale_dims[i] = d
    a.scale_numel = sc.numel()
    a.by_scale = int(by_scale)
    a.max_len, a.threads_per_block, a.group_cap = int(max_len), int(threads), int(group_cap)
    lib = _native.lib()
    handle = ctypes.c_void_p()
    keys = BY_SCALE_KEYS if by_scale else BUCKET_KEYS
    with torch.cuda.device(dev):
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _native.check(lib.mps_awq_encode(ctypes.byref(a), stream, ctypes.byref(handle)))
        try:
            sizes = (ctypes.c_int64 * 17)()
            _native.check(lib.mps_fp8_sidecar_sizes(handle, sizes))
            G, B, L = int(sizes[2]), int(sizes[4]), int(max_len)
            shape = {0: (G, 1 << L), 1: (G, max(1, (1 << L) // 2)), 7: (B, 16), 10: (B, int(threads) + 1)}
            ptrs = (ctypes.c_void_p * 17)()
            out: Dict[str, torch.Tensor] = {}
            for key, slot, dt in keys:
                t = torch.empty(shape.get(slot, (int(sizes[slot]),)), dtype=dt, device="cpu" if on_host else dev)
                out[key] = t
                ptrs[slot] = t.data_ptr() if t.numel() else None
            _native.check(lib.mps_fp8_sidecar_copy(handle, ptrs, stream))
            stats = (ctypes.c_int64 * 4)()
            _native.check(lib.mps_fp8_sidecar_stats(handle, stats))
        finally:
            lib.mps_fp8_sidecar_free(handle)
    if with_stats:
        return out, {"esc_keys": int(stats[0]), "esc_collisions": int(stats[1])}
    return out


def huffman_build_awq_int4_bucket_decode_tables(bf16_params: torch.Tensor, int4_values_u8: torch.Tensor,
                                                scales_u16: torch.Tensor, max_len: int = 11,
                                                threads_per_block: int = 256) -> Dict[str, torch.Tensor]:
    """Row-bucket AWQ int4 sidecar, 14 keys (build_huffman.cu:1583-2126, wrapper.cpp:258-288)."""
    return _build(bf16_params, int4_values_u8, scales_u16, int(max_len), int(threads_per_block), 1, False)


def huffman_build_awq_int4_bucket_decode_tables_by_scale(bf16_values: torch.Tensor, int4_values: torch.Tensor,
                                                         scales_u16: torch.Tensor, max_len: int = 11,
                                                         threads: int = 256,
                                                         group_cap: int = 1024) -> Dict[str, torch.Tensor]:
    """By-scale AWQ int4 sidecar, 13 keys (build_huffman.cu:1075-1580, wrapper.cpp:290-321)."""
    return _build(bf16_values, int4_values, scales_u16, int(max_len), int(threads), int(group_cap), True)


def _dt(t: torch.Tensor, dtype, dim: int | None, msg: str) -> None:
    if t.dtype != dtype or (dim is not None and t.dim() != dim):
        raise ValueError(msg)


class _AwqTensorPlan:
    """A device plan of one AWQ tensor that holds no reference to its tensors (the
    cache entry that owns it checks they are alive before every use)."""

    def __init__(self, desc: "_native.MpsAwqTensor", stream: int):
        arr = (_native.MpsAwqTensor * 1)(desc)
        self.handle = ctypes.c_void_p()
        _native.check(_native.lib().mps_awq_plan_create(arr, 1, ctypes.c_void_p(stream), ctypes.byref(self.handle)))

    def decode_into(self, out: torch.Tensor, stream: int) -> None:
        _native.check(_native.lib().mps_awq_plan_decode_into(self.handle, ctypes.c_void_p(out.data_ptr()),
                                                             ctypes.c_void_p(stream)))

    def close(self) -> None:
        if self.handle:
            _native.lib().mps_awq_plan_destroy(self.handle)
            self.handle = ctypes.c_void_p()


_AWQ_PLANS = None


def _plan_cache():
    """The AWQ decoders' per-sidecar plan cache (the FP8 op's rules: a plan from the
    second call on a sidecar, dropped when a tensor is freed or written through torch;
    MPSERVE_DECODE_PLANS=0 turns it off; clear_decode_plans() empties it)."""
    global _AWQ_PLANS
    if _AWQ_PLANS is None:
        from .mpserve_cuda import _SidecarPlans

        _AWQ_PLANS = _SidecarPlans(factory=_AwqTensorPlan)
    return _AWQ_PLANS


def _launch(int4, bitstream, syms, lens, table, col_start, col_len, offsets, rows, group_col, group_size,
            startbit, bit_base, n, m, max_len, out) -> torch.Tensor:
    dev = int4.device
    if out is None:
        out = torch.empty((n, m), dtype=torch.bfloat16, device=dev)
    elif out.dtype != torch.bfloat16 or out.device != dev or not out.is_contiguous() or out.numel() != n * m:
        raise ValueError("out must be a contiguous bfloat16 tensor of n*m elements on the int4 device")
    d = _native.MpsAwqTensor()
    d.int4 = int4.data_ptr()
    d.bitstream, d.bitstream_words = bitstream.data_ptr(), bitstream.numel()
    d.decode_syms, d.decode_lens, d.num_tables = syms.data_ptr(), lens.data_ptr(), syms.size(0)
    d.bucket_table = table.data_ptr()
    d.bucket_col_start = col_start.data_ptr() if col_start is not None else None
    d.bucket_col_len = col_len.data_ptr() if col_len is not None else None
    d.bucket_row_offsets = offsets.data_ptr()
    d.row_indices, d.num_row_indices = rows.data_ptr(), rows.numel()
    d.group_col_start = group_col.data_ptr() if group_col is not None else None
    d.group_size = int(group_size)
    d.bucket_thread_startbit, d.bucket_bit_base = startbit.data_ptr(), bit_base.data_ptr()
    d.num_buckets, d.k = table.size(0), startbit.size(1) - 1
    d.n, d.m, d.out = n, m, out.data_ptr()
    if n * m >= (1 << 31):
        raise ValueError("tensor too large for the AWQ decode kernel (n*m >= 2^31)")
    # From its second call on a sidecar that the slab path can take (k = 1024: by-scale
    # with 128-column groups, or row buckets; k = 256 or 512: by-scale with 128-column
    # groups, or row buckets when m is a multiple of 4k, whose buckets the plan splits
    # into ranges decoded side by side) the op launches the sidecar's cached plan; other
    # sidecars (whose plans would take the per-lane path, slower than this kernel's two
    # workgroups per bucket when a tensor has fewer buckets than CUs) and the first call
    # decode over whole buckets, as the reference does.
    key_tensors = tuple(t for t in (int4, bitstream, syms, lens, table, col_start, col_len, offsets, rows, group_col,
                                    startbit, bit_base) if t is not None)
    k = startbit.size(1) - 1
    if group_col is None:
        slab = k == 1024 or (k in (256, 512) and m % (4 * k) == 0)
    else:
        slab = k in (256, 512, 1024) and int(group_size) == 128
    with torch.cuda.device(dev):
        stream = _stream_handle(dev)
        plan = None
        if slab and table.size(0) > 0 and out.data_ptr() % 8 == 0:
            plan = _plan_cache().get(key_tensors, n, m, d, dev, stream, extra=(int(group_size),))
        if plan is not None:
            plan.decode_into(out, stream)
        else:
            _native.check(_native.lib().mps_awq_decode(ctypes.byref(d), int(max_len), ctypes.c_void_p(stream)))
    _maybe_check_status(dev, "AWQ int4 decode")
    return out


def huffman_decode_awq_int4_bucket(int4_values_u8: torch.Tensor, bitstream_u64: torch.Tensor,
                                   decode_syms_u16: torch.Tensor, decode_lens_u8: torch.Tensor,
                                   bucket_table_i32: torch.Tensor, bucket_col_start_i32: torch.Tensor,
                                   bucket_col_len_i32: torch.Tensor, bucket_row_offsets_i32: torch.Tensor,
                                   row_indices_i32: torch.Tensor, bucket_thread_startbit_u32: torch.Tensor,
                                   bucket_bit_base_i64: torch.Tensor, n: int, m: int, max_len: int = 11, *,
                                   out: torch.Tensor | None = None) -> torch.Tensor:
    """BF16 ``[n, m]`` from int4 values + row-bucket sidecar (decode_huffman.cu:877-1018)."""
    n, m, max_len = int(n), int(m), int(max_len)
    dev = int4_values_u8.device if isinstance(int4_values_u8, torch.Tensor) else None
    for t, name in ((int4_values_u8, "int4_values_u8"), (bitstream_u64, "bitstream_u64"),
                    (decode_syms_u16, "decode_syms_u16"), (decode_lens_u8, "decode_lens_u8"),
                    (bucket_table_i32, "bucket_table_i32"), (bucket_col_start_i32, "bucket_col_start_i32"),
                    (bucket_col_len_i32, "bucket_col_len_i32"), (bucket_row_offsets_i32, "bucket_row_offsets_i32"),
                    (row_indices_i32, "row_indices_i32"), (bucket_thread_startbit_u32, "bucket_thread_startbit_u32"),
                    (bucket_bit_base_i64, "bucket_bit_base_i64")):
        _check_cuda_contig(t, name, dev)
    _dt(int4_values_u8, torch.uint8, None, "int4_values_u8 must be uint8 CUDA")
    _dt(bitstream_u64, torch.uint64, 1, "bitstream_u64 must be uint64 1D CUDA")
    _dt(decode_syms_u16, torch.uint16, 2, "decode_syms_u16 must be uint16 2D CUDA [G, 2^L]")
    _dt(decode_lens_u8, torch.uint8, 2, "decode_lens_u8 must be uint8 2D CUDA [G, 2^(L-1)]")
    if bucket_table_i32.dtype != torch.int32 or bucket_table_i32.dim() != 2 or bucket_table_i32.size(1) != 16:
        raise ValueError("bucket_table_i32 must be int32 CUDA [B,16]")
    _dt(bucket_col_start_i32, torch.int32, 1, "bucket_col_start_i32 must be int32 1D CUDA [B]")
    _dt(bucket_col_len_i32, torch.int32, 1, "bucket_col_len_i32 must be int32 1D CUDA [B]")
    _dt(bucket_row_offsets_i32, torch.int32, 1, "bucket_row_offsets_i32 must be int32 1D CUDA [B+1]")
    _dt(row_indices_i32, torch.int32, 1, "row_indices_i32 must be int32 1D CUDA")
    _dt(bucket_thread_startbit_u32, torch.uint32, 2, "bucket_thread_startbit_u32 must be uint32 2D CUDA [B,k+1]")
    _dt(bucket_bit_base_i64, torch.int64, 1, "bucket_bit_base_i64 must be int64 1D CUDA [B+1]")
    if max_len <= 0 or max_len > 15:
        raise ValueError("max_len must be in [1,15]")
    if max_len != 11:
        raise ValueError("AWQ bucket decode kernel is specialized: max_len must be 11")
    if n <= 0 or m <= 0:
        raise ValueError("n,m must be > 0")
    if int4_values_u8.numel() != n * m:
        raise ValueError("int4_values_u8 numel must equal n*m")
    B = bucket_table_i32.size(0)
    if bucket_col_start_i32.numel() != B:
        raise ValueError("bucket_col_start_i32 length must be B")
    if bucket_col_len_i32.numel() != B:
        raise ValueError("bucket_col_len_i32 length must be B")
    if bucket_row_offsets_i32.numel() != B + 1:
        raise ValueError("bucket_row_offsets_i32 length must be B+1")
    if bucket_thread_startbit_u32.size(0) != B:
        raise ValueError("bucket_thread_startbit_u32 first dim must be B")
    if bucket_bit_base_i64.numel() != B + 1:
        raise ValueError("bucket_bit_base_i64 length must be B+1")
    _tables_and_k(decode_syms_u16, decode_lens_u8, bucket_thread_startbit_u32)
    return _launch(int4_values_u8, bitstream_u64, decode_syms_u16, decode_lens_u8, bucket_table_i32,
                   bucket_col_start_i32, bucket_col_len_i32, bucket_row_offsets_i32, row_indices_i32, None, 0,
                   bucket_thread_startbit_u32, bucket_bit_base_i64, n, m, max_len, out)


def _tables_and_k(syms: torch.Tensor, lens: torch.Tensor, startbit: torch.Tensor) -> None:
    if syms.size(1) != 2048:
        raise ValueError("decode_syms_u16 second dim must be 2^max_len")
    if lens.size(1) != 1024:
        raise ValueError("decode_lens_u8 second dim must be 2^(max_len-1)")
    if syms.size(0) != lens.size(0):
        raise ValueError("decode_syms_u16 and decode_lens_u8 first dim must match")
    k = startbit.size(1) - 1
    if k <= 0 or k > 1024:
        raise ValueError("bucket_thread_startbit_u32 has invalid k (must be 1..1024)")


def huffman_decode_awq_int4_bucket_by_scale(int4_values_u8: torch.Tensor, bitstream_u64: torch.Tensor,
                                            decode_syms_u16: torch.Tensor, decode_lens_u8: torch.Tensor,
                                            bucket_table_i32: torch.Tensor, bucket_group_offsets_i32: torch.Tensor,
                                            group_rows_i32: torch.Tensor, group_col_start_i32: torch.Tensor,
                                            bucket_thread_startbit_u32: torch.Tensor,
                                            bucket_bit_base_i64: torch.Tensor, n: int, m: int, max_len: int,
                                            group_size: int, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """BF16 ``[n, m]`` from int4 values + by-scale sidecar (decode_huffman.cu:760-875)."""
    n, m, max_len, group_size = int(n), int(m), int(max_len), int(group_size)
    dev = int4_values_u8.device if isinstance(int4_values_u8, torch.Tensor) else None
    for t, name in ((int4_values_u8, "int4_values_u8"), (bitstream_u64, "bitstream_u64"),
                    (decode_syms_u16, "decode_syms_u16"), (decode_lens_u8, "decode_lens_u8"),
                    (bucket_table_i32, "bucket_table_i32"), (bucket_group_offsets_i32, "bucket_group_offsets_i32"),
                    (group_rows_i32, "group_rows_i32"), (group_col_start_i32, "group_col_start_i32"),
                    (bucket_thread_startbit_u32, "bucket_thread_startbit_u32"),
                    (bucket_bit_base_i64, "bucket_bit_base_i64")):
        _check_cuda_contig(t, name, dev)
    _dt(int4_values_u8, torch.uint8, 2, "int4_values_u8 must be uint8 2D CUDA [n,m]")
    _dt(bitstream_u64, torch.uint64, 1, "bitstream_u64 must be uint64 1D CUDA")
    _dt(decode_syms_u16, torch.uint16, 2, "decode_syms_u16 must be uint16 2D CUDA [G,2^L]")
    _dt(decode_lens_u8, torch.uint8, 2, "decode_lens_u8 must be uint8 2D CUDA [G,2^(L-1)]")
    if bucket_table_i32.dtype != torch.int32 or bucket_table_i32.dim() != 2 or bucket_table_i32.size(1) != 16:
        raise ValueError("bucket_table_i32 must be int32 2D CUDA [B,16]")
    _dt(bucket_group_offsets_i32, torch.int32, 1, "bucket_group_offsets_i32 must be int32 1D CUDA [B+1]")
    _dt(group_rows_i32, torch.int32, 1, "group_rows_i32 must be int32 1D CUDA")
    _dt(group_col_start_i32, torch.int32, 1, "group_col_start_i32 must be int32 1D CUDA")
    _dt(bucket_thread_startbit_u32, torch.uint32, 2, "bucket_thread_startbit_u32 must be uint32 2D CUDA [B,k+1]")
    _dt(bucket_bit_base_i64, torch.int64, 1, "bucket_bit_base_i64 must be int64 1D CUDA [B+1]")
    if max_len <= 0 or max_len > 15:
        raise ValueError("max_len must be in [1,15]")
    if max_len != 11:
        raise ValueError("AWQ ragged bucket decode kernel is specialized: max_len must be 11")
    if n <= 0 or m <= 0:
        raise ValueError("n,m must be > 0")
    if group_size <= 0 or group_size > m:
        raise ValueError("group_size must be in (0,m]")
    if int4_values_u8.numel() != n * m:
        raise ValueError("int4_values_u8 numel must equal n*m")
    B = bucket_table_i32.size(0)
    if bucket_group_offsets_i32.numel() != B + 1:
        raise ValueError("bucket_group_offsets_i32 length must be B+1")
    if bucket_thread_startbit_u32.size(0) != B:
        raise ValueError("bucket_thread_startbit_u32 first dim must be B")
    if bucket_bit_base_i64.numel() != B + 1:
        raise ValueError("bucket_bit_base_i64 length must be B+1")
    if group_rows_i32.numel() != group_col_start_i32.numel():
        raise ValueError("group_rows_i32 and group_col_start_i32 length must match")
    _tables_and_k(decode_syms_u16, decode_lens_u8, bucket_thread_startbit_u32)
    return _launch(int4_values_u8, bitstream_u64, decode_syms_u16, decode_lens_u8, bucket_table_i32, None, None,
                   bucket_group_offsets_i32, group_rows_i32, group_col_start_i32, group_size,
                   bucket_thread_startbit_u32, bucket_bit_base_i64, n, m, max_len, out)


def _sidecar_descriptor(int4: torch.Tensor, sc, out: torch.Tensor) -> "_native.MpsAwqTensor":
    """Descriptor of one tensor for a plan: either layout's dict (as the
    builders return it, on the int4 tensor's device) and a contiguous BF16 out."""
    by_scale = "bucket_group_offsets_i32" in sc
    n, m = int(int4.shape[0]), int(int4.shape[1])
    dev = int4.device
    names = ["bitstream_u64", "decode_syms_u16", "decode_lens_u8", "bucket_table_i32",
             "bucket_thread_startbit_u32", "bucket_bit_base_i64"]
    names += (["bucket_group_offsets_i32", "group_rows_i32", "group_col_start_i32"] if by_scale else
              ["bucket_col_start_i32", "bucket_col_len_i32", "bucket_row_offsets_i32", "row_indices_i32"])
    _check_cuda_contig(int4, "int4_values_u8", dev)
    for key in names:
        _check_cuda_contig(sc[key], key, dev)
    if int4.dtype != torch.uint8 or int4.dim() != 2:
        raise ValueError("int4_values_u8 must be uint8 2D CUDA [n,m]")
    if sc["decode_syms_u16"].shape[1:] != (2048,) or sc["decode_lens_u8"].shape[1:] != (1024,) \
            or sc["bucket_table_i32"].dim() != 2 or sc["bucket_table_i32"].shape[1] != 16:
        raise ValueError("not an AWQ int4 sidecar with max_len 11")
    B = sc["bucket_table_i32"].shape[0]
    offs = sc["bucket_group_offsets_i32" if by_scale else "bucket_row_offsets_i32"]
    if offs.numel() != B + 1 or sc["bucket_thread_startbit_u32"].shape[0] != B or \
            sc["bucket_bit_base_i64"].numel() != B + 1:
        raise ValueError("inconsistent bucket counts in the sidecar")
    if out.dtype != torch.bfloat16 or out.device != dev or not out.is_contiguous() or out.numel() != n * m:
        raise ValueError("out must be a contiguous bfloat16 tensor of n*m elements on the int4 device")
    if n * m >= (1 << 31):
        raise ValueError("tensor too large for the AWQ decode kernel (n*m >= 2^31)")
    d = _native.MpsAwqTensor()
    d.int4 = int4.data_ptr()
    d.bitstream, d.bitstream_words = sc["bitstream_u64"].data_ptr(), sc["bitstream_u64"].numel()
    d.decode_syms, d.decode_lens = sc["decode_syms_u16"].data_ptr(), sc["decode_lens_u8"].data_ptr()
    d.num_tables = sc["decode_syms_u16"].shape[0]
    d.bucket_table = sc["bucket_table_i32"].data_ptr()
    if by_scale:
        d.bucket_row_offsets = sc["bucket_group_offsets_i32"].data_ptr()
        d.row_indices, d.num_row_indices = sc["group_rows_i32"].data_ptr(), sc["group_rows_i32"].numel()
        if sc["group_col_start_i32"].numel() != sc["group_rows_i32"].numel():
            raise ValueError("group_rows_i32 and group_col_start_i32 length must match")
        d.group_col_start = sc["group_col_start_i32"].data_ptr() if B else None
        d.group_size = int(sc["shape_nmkg_i64"][3])
    else:
        if sc["bucket_col_start_i32"].numel() != B or sc["bucket_col_len_i32"].numel() != B:
            raise ValueError("inconsistent bucket counts in the sidecar")
        d.bucket_col_start, d.bucket_col_len = sc["bucket_col_start_i32"].data_ptr(), sc["bucket_col_len_i32"].data_ptr()
        d.bucket_row_offsets = sc["bucket_row_offsets_i32"].data_ptr()
        d.row_indices, d.num_row_indices = sc["row_indices_i32"].data_ptr(), sc["row_indices_i32"].numel()
    d.bucket_thread_startbit, d.bucket_bit_base = (sc["bucket_thread_startbit_u32"].data_ptr(),
                                                   sc["bucket_bit_base_i64"].data_ptr())
    d.num_buckets, d.k = B, sc["bucket_thread_startbit_u32"].shape[1] - 1
    d.n, d.m, d.out = n, m, out.data_ptr()
    return d


class AwqDecodePlan:
    """Decode a fixed list of AWQ int4 tensors (either sidecar layout) in one launch.

    ``items``: (int4_u8 [n, m] uint8, sidecar dict as the AWQ builders return it,
    out contiguous bfloat16 of n*m elements), all on one device. The reference
    launches once per tensor (decode_huffman.cu:857, :998); a plan's launch runs
    one workgroup per CU, which take the plan's work records (buckets, runs of
    buckets, row ranges) from a queue, largest first. Launches on different
    streams may overlap: each stream gets a queue of its own. The plan keeps
    references to every tensor it points at.
    """

    def __init__(self, items):
        self._keep = []
        descs = []
        self.device = None
        for int4, sc, out in items:
            if self.device is None:
                self.device = int4.device
            elif int4.device != self.device:
                raise ValueError("all tensors of an AwqDecodePlan must be on one device")
            descs.append(_sidecar_descriptor(int4, sc, out))
            self._keep.append((int4, sc, out))
        self.outputs = [o for _, _, o in self._keep]
        arr = (_native.MpsAwqTensor * max(1, len(descs)))(*descs)
        self._plan = ctypes.c_void_p()
        if self.device is not None:
            # creation waits for the current stream, which may still be writing the sidecars
            with torch.cuda.device(self.device):
                _native.check(_native.lib().mps_awq_plan_create(arr, len(descs),
                                                                ctypes.c_void_p(_stream_handle(self.device)),
                                                                ctypes.byref(self._plan)))

    def decode(self, stream: torch.cuda.Stream | None = None):
        """Enqueue the decode on ``stream`` (default: the current stream); returns the outputs."""
        if self.device is None:
            return self.outputs
        h = stream.cuda_stream if stream is not None else _stream_handle(self.device)
        with torch.cuda.device(self.device):
            _native.check(_native.lib().mps_awq_plan_decode(self._plan, ctypes.c_void_p(h)))
        return self.outputs

    def info(self) -> Dict[str, int]:
        """Work items (buckets) of a launch."""
        wi = ctypes.c_int64(0)
        if self._plan:
            _native.check(_native.lib().mps_awq_plan_info(self._plan, ctypes.byref(wi)))
        return {"work_items": int(wi.value)}

    def read_status(self, stream: torch.cuda.Stream | None = None) -> int:
        """MPS_STATUS_* flags this plan's decodes recorded since the last read (synchronises)."""
        v = ctypes.c_uint32(0)
        if self._plan:
            h = stream.cuda_stream if stream is not None else _stream_handle(self.device)
            _native.check(_native.lib().mps_awq_plan_read_status(self._plan, ctypes.c_void_p(h), ctypes.byref(v)))
        return int(v.value)

    def close(self) -> None:
        if getattr(self, "_plan", None):
            _native.lib().mps_awq_plan_destroy(self._plan)
            self._plan = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
