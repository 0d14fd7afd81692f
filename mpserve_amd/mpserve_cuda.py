"""The ``MPServe_cuda`` op surface, served by HIP kernels on MI355X.

Same op names, argument names, defaults, dict keys and error types as the
reference's pybind11 module (kernel/wrapper.cpp:132-504); the repository root
module ``MPServe_cuda`` re-exports this one so ``import MPServe_cuda`` keeps
working. Tensors cross into libmpserve_amd.so as raw device pointers.

Every op runs on the GPU. There is no CPU fallback: without the native
library the ops raise ImportError, and without a GPU they raise RuntimeError.
"""
from __future__ import annotations

import collections
import ctypes
import os
import threading
import weakref
from typing import Dict, Optional, Sequence

import torch

from . import _native
from ._common import _check_cuda_contig, _maybe_check_status, _stream_handle, read_status  # noqa: F401

__all__ = [
    "huffman_build_fp8_decode_tables",
    "huffman_decode_fp8",
    "cuda_clock_rate_khz",
    "clear_decode_plans",
    "SIDECAR_KEYS",
]

# Output keys of the build op, in the reference's tuple order (wrapper.cpp:429-446).
SIDECAR_KEYS = (
    "decode_syms_u16", "decode_lens_u8", "table_scale_u16", "table_fp8_u16",
    "bucket_scale_u16", "bucket_row_offsets_i32", "row_indices_i32", "bucket_table_i32",
    "bucket_col_start_i32", "bucket_col_len_i32", "bucket_thread_startbit_u32",
    "bucket_bit_base_i64", "bitstream_u64", "shape_nmk_i64", "bucket_U_i32",
    "bucket_unique_gid_i32", "bucket_fp8_uidx_i16",
)


def cuda_clock_rate_khz() -> int:
    """Clock rate (kHz) of the current device (wrapper.cpp:133-141)."""
    if not torch.cuda.is_available():
        raise RuntimeError("cudaGetDevice failed: no GPU device is visible")
    v = ctypes.c_int64(0)
    _native.check(_native.lib().mps_clock_rate_khz(torch.cuda.current_device(), ctypes.byref(v)))
    return int(v.value)


def _descriptor(fp8_u8, bitstream_u64, decode_syms_u16, decode_lens_u8, bucket_table_i32,
                bucket_col_start_i32, bucket_col_len_i32, bucket_row_offsets_i32, row_indices_i32,
                bucket_thread_startbit_u32, bucket_bit_base_i64, n: int, m: int,
                out: torch.Tensor) -> _native.MpsFp8Tensor:
    d = _native.MpsFp8Tensor()
    d.fp8 = fp8_u8.data_ptr()
    d.bitstream = bitstream_u64.data_ptr()
    d.bitstream_words = bitstream_u64.numel()
    d.decode_syms = decode_syms_u16.data_ptr()
    d.decode_lens = decode_lens_u8.data_ptr()
    d.num_tables = decode_syms_u16.size(0)
    d.bucket_table = bucket_table_i32.data_ptr()
    d.bucket_col_start = bucket_col_start_i32.data_ptr()
    d.bucket_col_len = bucket_col_len_i32.data_ptr()
    d.bucket_row_offsets = bucket_row_offsets_i32.data_ptr()
    d.row_indices = row_indices_i32.data_ptr()
    d.num_row_indices = row_indices_i32.numel()
    d.bucket_thread_startbit = bucket_thread_startbit_u32.data_ptr()
    d.bucket_bit_base = bucket_bit_base_i64.data_ptr()
    d.num_buckets = bucket_table_i32.size(0)
    d.k = bucket_thread_startbit_u32.size(1) - 1
    d.n = int(n)
    d.m = int(m)
    d.out = out.data_ptr()
    return d


def validate_decode_args(fp8_params_u8, bitstream_u64, decode_syms_u16, decode_lens_u8, bucket_table_i32,
                         bucket_col_start_i32, bucket_col_len_i32, bucket_row_offsets_i32, row_indices_i32,
                         bucket_thread_startbit_u32, bucket_bit_base_i64, n, m, max_len) -> None:
    """The argument checks of huffman_decode_fp8_entry (decode_huffman.cu:606-697), same messages."""
    dev = fp8_params_u8.device if isinstance(fp8_params_u8, torch.Tensor) else None
    named = (
        (fp8_params_u8, "fp8_params_u8"), (bitstream_u64, "bitstream_u64"), (decode_syms_u16, "decode_syms_u16"),
        (decode_lens_u8, "decode_lens_u8"), (bucket_table_i32, "bucket_table_i32"),
        (bucket_col_start_i32, "bucket_col_start_i32"), (bucket_col_len_i32, "bucket_col_len_i32"),
        (bucket_row_offsets_i32, "bucket_row_offsets_i32"), (row_indices_i32, "row_indices_i32"),
        (bucket_thread_startbit_u32, "bucket_thread_startbit_u32"), (bucket_bit_base_i64, "bucket_bit_base_i64"),
    )
    for t, name in named:
        _check_cuda_contig(t, name, dev)
    if fp8_params_u8.dtype != torch.uint8:
        raise ValueError("fp8_params_u8 must be uint8 CUDA")
    if bitstream_u64.dtype != torch.uint64 or bitstream_u64.dim() != 1:
        raise ValueError("bitstream_u64 must be uint64 1D CUDA")
    if decode_syms_u16.dtype != torch.uint16 or decode_syms_u16.dim() != 2:
        raise ValueError("decode_syms_u16 must be uint16 2D CUDA [G, 2^L]")
    if decode_lens_u8.dtype != torch.uint8 or decode_lens_u8.dim() != 2:
        raise ValueError("decode_lens_u8 must be uint8 2D CUDA [G, 2^(L-1)]")
    if bucket_table_i32.dtype != torch.int32 or bucket_table_i32.dim() != 2 or bucket_table_i32.size(1) != 256:
        raise ValueError("bucket_table_i32 must be int32 CUDA [B,256]")
    if bucket_col_start_i32.dtype != torch.int32 or bucket_col_start_i32.dim() != 1:
        raise ValueError("bucket_col_start_i32 must be int32 1D CUDA [B]")
    if bucket_col_len_i32.dtype != torch.int32 or bucket_col_len_i32.dim() != 1:
        raise ValueError("bucket_col_len_i32 must be int32 1D CUDA [B]")
    if bucket_row_offsets_i32.dtype != torch.int32 or bucket_row_offsets_i32.dim() != 1:
        raise ValueError("bucket_row_offsets_i32 must be int32 1D CUDA [B+1]")
    if row_indices_i32.dtype != torch.int32 or row_indices_i32.dim() != 1:
        raise ValueError("row_indices_i32 must be int32 1D CUDA")
    if bucket_thread_startbit_u32.dtype != torch.uint32 or bucket_thread_startbit_u32.dim() != 2:
        raise ValueError("bucket_thread_startbit_u32 must be uint32 2D CUDA [B,k+1]")
    if bucket_bit_base_i64.dtype != torch.int64 or bucket_bit_base_i64.dim() != 1:
        raise ValueError("bucket_bit_base_i64 must be int64 1D CUDA [B+1]")
    if max_len <= 0 or max_len > 15:
        raise ValueError("max_len must be in [1,15]")
    if max_len != 7:
        raise ValueError("decode kernel is specialized: max_len must be 7")
    if n <= 0 or m <= 0:
        raise ValueError("n,m must be > 0")
    if fp8_params_u8.numel() != n * m:
        raise ValueError("fp8_params_u8 numel must equal n*m")
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
    if decode_syms_u16.size(1) != 128:
        raise ValueError("decode_syms_u16 second dim must be 2^max_len")
    if decode_lens_u8.size(1) != 64:
        raise ValueError("decode_lens_u8 second dim must be 2^(max_len-1)")
    if decode_syms_u16.size(0) != decode_lens_u8.size(0):
        raise ValueError("decode_syms_u16 and decode_lens_u8 first dim must match")
    k = bucket_thread_startbit_u32.size(1) - 1
    if k <= 0 or k > 1024:
        raise ValueError("bucket_thread_startbit_u32 has invalid k (must be 1..1024)")


class _TensorPlan:
    """A device plan of one tensor that holds no reference to its tensors (the
    cache entry that owns it checks they are alive before every use)."""

    def __init__(self, desc: _native.MpsFp8Tensor, stream: int):
        arr = (_native.MpsFp8Tensor * 1)(desc)
        self.handle = ctypes.c_void_p()
        _native.check(_native.lib().mps_fp8_plan_create(arr, 1, ctypes.c_void_p(stream), ctypes.byref(self.handle)))

    def decode_into(self, out: torch.Tensor, stream: int) -> None:
        _native.check(_native.lib().mps_fp8_plan_decode_into(self.handle, ctypes.c_void_p(out.data_ptr()),
                                                             ctypes.c_void_p(stream)))

    def close(self) -> None:
        if self.handle:
            _native.lib().mps_fp8_plan_destroy(self.handle)
            self.handle = ctypes.c_void_p()


_CACHES: list = []  # every per-sidecar plan cache, for clear_decode_plans()


class _CacheEntry:
    """One sidecar's slot in a _SidecarPlans: weak references to its tensors'
    storages and their versions, its plan once built, and whether a graph
    captured a launch of that plan."""

    __slots__ = ("refs", "versions", "plan", "pinned")

    def __init__(self, tensors: Sequence[torch.Tensor]):
        self.refs = [weakref.ref(t.untyped_storage()) for t in tensors]
        self.versions = [t._version for t in tensors]
        self.plan = None
        self.pinned = False

    def valid(self, tensors: Sequence[torch.Tensor]) -> bool:
        for r, v, t in zip(self.refs, self.versions, tensors):
            if r() is not t.untyped_storage() or t._version != v:
                return False
        return True


class _SidecarPlans:
    """Single-tensor decode plans behind huffman_decode_fp8, one per sidecar.

    The reference decodes every call over whole buckets, one workgroup each
    (decode_huffman.cu:699-739), so a tensor with few buckets for the CUs (a
    70B k_proj has 8 for 256 CUs) runs on few CUs. A plan splits large buckets
    into row ranges that start from lane checkpoints, but computing those
    walks every substream once and synchronises. So the op decodes a sidecar's
    first call over whole buckets, builds its plan on the second call, and
    launches the plan from then on, on any stream: a plan gives each stream
    that launches it a work queue of its own.

    Invalidation rule. An entry is keyed by the device addresses of the FP8
    tensor and the ten sidecar arrays, with n and m. For each of the eleven
    tensors it keeps a weak reference to the tensor's storage and the tensor's
    version counter (dtype views such as int64 -> uint64 share both with the
    tensor they view). It is used only while every storage is alive and no
    version has changed, so a sidecar that was freed (another may now sit at
    the same addresses) or rewritten in place through torch gets a new plan.
    A writer that bypasses torch's version counters (another library writing
    through the raw pointers) must call clear_decode_plans(). At most
    ``capacity`` entries are kept, least recently used first out;
    MPSERVE_DECODE_PLANS=0 turns the cache off.

    Graph capture. No plan is built while the current stream captures
    (building synchronises and allocates); built plans launch there like any
    kernel. A plan launched during a capture is pinned: a replay of that graph
    may launch it at any later time, so when its entry is evicted or
    invalidated the plan is kept alive until clear_decode_plans(). No plan is
    freed while the stream captures (hipFree there would break the capture):
    such plans are freed on the next call made outside a capture.
    """

    def __init__(self, capacity: int = 256, factory=None):
        self.capacity = capacity
        self.factory = factory if factory is not None else _TensorPlan  # (descriptor, stream) -> plan
        self._entries: "collections.OrderedDict[tuple, _CacheEntry]" = collections.OrderedDict()
        self._kept: list = []      # plans of dropped entries that a captured graph may still launch
        self._deferred: list = []  # plans dropped during a capture, to free outside it
        self._lock = threading.Lock()
        _CACHES.append(self)

    def get(self, tensors: Sequence[torch.Tensor], n: int, m: int, desc, device: torch.device, stream: int,
            extra: tuple = ()) -> Optional[_TensorPlan]:
        """The sidecar's plan, building it on its second sighting; None: decode over whole buckets.
        ``extra``: further key parts (an AWQ group size)."""
        if self.capacity <= 0 or os.environ.get("MPSERVE_DECODE_PLANS", "1") == "0":
            return None
        capturing = torch.cuda.is_current_stream_capturing()
        key = (device.index, n, m) + tuple(extra) + tuple(t.data_ptr() for t in tensors)
        dropped = []
        try:
            with self._lock:
                entry = self._entries.get(key)
                if entry is not None and not entry.valid(tensors):
                    dropped.append(self._entries.pop(key))
                    entry = None
                if entry is None:
                    self._entries[key] = _CacheEntry(tensors)
                    while len(self._entries) > self.capacity:
                        dropped.append(self._entries.popitem(last=False)[1])
                    return None
                self._entries.move_to_end(key)
                if entry.plan is None:
                    if capturing:
                        return None
                    entry.plan = self.factory(desc, stream)
                if capturing:
                    entry.pinned = True
                return entry.plan
        finally:
            self._release(dropped, capturing)

    def _release(self, dropped, capturing: bool) -> None:
        """Free the plans of dropped entries, keeping those a captured graph may
        launch and deferring every free while the stream captures."""
        free = []
        with self._lock:
            for e in dropped:
                if e.plan is None:
                    continue
                if e.pinned:
                    self._kept.append(e.plan)
                elif capturing:
                    self._deferred.append(e.plan)
                else:
                    free.append(e.plan)
            if not capturing:
                free += self._deferred
                self._deferred = []
        for p in free:
            p.close()

    def clear(self) -> None:
        """Drop every entry and free every plan, pinned ones included: call it
        when no captured graph that launched them will replay again."""
        capturing = torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
        with self._lock:
            plans = [e.plan for e in self._entries.values() if e.plan is not None] + self._kept + self._deferred
            self._entries.clear()
            self._kept = []
            self._deferred = []
            if capturing:
                self._deferred = plans
                plans = []
        for p in plans:
            p.close()

    def __len__(self) -> int:
        return len(self._entries)


_PLANS = _SidecarPlans()


def clear_decode_plans() -> None:
    """Drop every cached per-sidecar plan of the decode ops (huffman_decode_fp8 and the
    AWQ int4 decoders; see _SidecarPlans)."""
    for c in list(_CACHES):
        c.clear()


def huffman_decode_fp8(fp8_params_u8: torch.Tensor, bitstream_u64: torch.Tensor, decode_syms_u16: torch.Tensor,
                       decode_lens_u8: torch.Tensor, bucket_table_i32: torch.Tensor,
                       bucket_col_start_i32: torch.Tensor, bucket_col_len_i32: torch.Tensor,
                       bucket_row_offsets_i32: torch.Tensor, row_indices_i32: torch.Tensor,
                       bucket_thread_startbit_u32: torch.Tensor, bucket_bit_base_i64: torch.Tensor,
                       n: int, m: int, max_len: int = 12, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """BF16 ``[n, m]`` rebuilt from FP8 bytes + Huffman sidecar (wrapper.cpp:456-503).

    Runs on the current stream of the FP8 tensor's device. ``out`` (keyword
    only, not in the reference) decodes into a caller-owned contiguous BF16
    buffer of n*m elements, e.g. a preallocated scratch weight. From its
    second call on a sidecar the op launches a cached plan of that sidecar on
    whatever stream is current (_SidecarPlans); the second call synchronises
    the stream once.
    """
    n = int(n)
    m = int(m)
    max_len = int(max_len)
    tensors = (fp8_params_u8, bitstream_u64, decode_syms_u16, decode_lens_u8, bucket_table_i32,
               bucket_col_start_i32, bucket_col_len_i32, bucket_row_offsets_i32, row_indices_i32,
               bucket_thread_startbit_u32, bucket_bit_base_i64)
    validate_decode_args(*tensors, n, m, max_len)
    dev = fp8_params_u8.device
    if out is None:
        out = torch.empty((n, m), dtype=torch.bfloat16, device=dev)
    else:
        if out.dtype != torch.bfloat16 or out.device != dev or not out.is_contiguous() or out.numel() != n * m:
            raise ValueError("out must be a contiguous bfloat16 tensor of n*m elements on the fp8 device")
    d = _descriptor(*tensors, n, m, out)
    with torch.cuda.device(dev):
        stream = _stream_handle(dev)
        plan = _PLANS.get(tensors, n, m, d, dev, stream) if bucket_table_i32.size(0) > 0 else None
        if plan is not None:
            plan.decode_into(out, stream)
        else:
            _native.check(_native.lib().mps_fp8_decode(ctypes.byref(d), max_len, ctypes.c_void_p(stream)))
    _maybe_check_status(dev)
    return out


def huffman_build_fp8_decode_tables(bf16_params: torch.Tensor, fp8_params: torch.Tensor, scales: torch.Tensor,
                                    max_len: int = 12, threads_per_block: int = 256) -> Dict[str, torch.Tensor]:
    """Build the Huffman sidecar on the GPU (build_huffman.cu:292-969, bound at wrapper.cpp:418-454).

    Returns the reference's 17-key dict, byte-identical to its builder. CPU
    inputs (the reference's contract) are copied to the current GPU and the
    outputs come back as CPU tensors; CUDA inputs give CUDA outputs.
    """
    from .encode import build_fp8_sidecar

    return build_fp8_sidecar(bf16_params, fp8_params, scales, int(max_len), int(threads_per_block))


def _not_in_scope(name: str):
    def f(*args, **kwargs):
        raise NotImplementedError(f"MPServe_cuda.{name} is not provided by the MI355X build "
                                  "(the FP8 and AWQ int4 bucket Huffman paths are)")
    f.__name__ = name
    return f


# Names the reference module binds (wrapper.cpp:142-179, :180-416) outside the FP8 path.
for _name in ("init_cuda", "cleanup_cuda", "build_trie_AWQ", "build_trie", "query_trie", "free_trie",
              "get_trie_count", "get_tot_path_length", "save_trie_collection", "load_trie_collection",
              "save_trie_collection_awq", "load_trie_collection_awq", "load_bf16_from_int8", "dequantize_awq",
              "build_trie_AWQ_to_FP8", "save_trie_collection_awq_to_fp8", "load_trie_collection_awq_to_fp8",
              "huffman_build_awq_decode_tables", "huffman_decode_awq_shared_table"):
    globals()[_name] = _not_in_scope(_name)

# AWQ int4 bucket builders and decoders (wrapper.cpp:258-416).
from .awq import (huffman_build_awq_int4_bucket_decode_tables,  # noqa: E402
                  huffman_build_awq_int4_bucket_decode_tables_by_scale, huffman_decode_awq_int4_bucket,
                  huffman_decode_awq_int4_bucket_by_scale)

__all__ += ["huffman_build_awq_int4_bucket_decode_tables", "huffman_build_awq_int4_bucket_decode_tables_by_scale",
            "huffman_decode_awq_int4_bucket", "huffman_decode_awq_int4_bucket_by_scale"]
