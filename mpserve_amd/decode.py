"""Batched decode: one HIP launch rebuilds many BF16 weights (a layer, a model).

A ``DecodePlan`` holds the device descriptors of a fixed list of
(FP8 bytes, sidecar, output) triples and replays the decode on any stream.
The reference decodes tensor by tensor (kernel/decode_huffman.cu:739, called
per linear from scripts/mpserve_vllm_fp8_huffman.py:474-489); the plan keeps
that op's semantics per tensor and removes the per-tensor launch and
allocation cost.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Iterable, Mapping, Sequence, Tuple

import torch

from . import _native
from .mpserve_cuda import _descriptor, _stream_handle, validate_decode_args

# sidecar keys as the build op names them, and the names the compress script
# stores them under (with "huff_" prefix and signed dtypes)
_VIEW_AS = {
    "bitstream_u64": torch.uint64,
    "decode_syms_u16": torch.uint16,
    "bucket_thread_startbit_u32": torch.uint32,
}


def normalize_sidecar(sc: Mapping[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """Accept build-op keys or compress-script keys (``huff_*``, signed dtypes); return
    build-op keys with the decode op's dtypes (same views as
    scripts/mpserve_vllm_fp8_huffman.py:457-472)."""
    out: Dict[str, torch.Tensor] = {}
    for k, v in sc.items():
        key = k.split(".")[-1]
        if key.startswith("huff_"):
            key = key[len("huff_"):]
        out[key] = v
    for key, dt in _VIEW_AS.items():
        if key in out and out[key].dtype != dt:
            out[key] = out[key].view(dt)
    return out


def sidecar_decode_args(fp8_u8: torch.Tensor, sc: Mapping[str, torch.Tensor], max_len: int = 7) -> Tuple:
    """Positional arguments of huffman_decode_fp8 for one tensor."""
    s = normalize_sidecar(sc)
    n, m = int(fp8_u8.shape[0]), int(fp8_u8.shape[1])
    return (fp8_u8, s["bitstream_u64"], s["decode_syms_u16"], s["decode_lens_u8"], s["bucket_table_i32"],
            s["bucket_col_start_i32"], s["bucket_col_len_i32"], s["bucket_row_offsets_i32"],
            s["row_indices_i32"], s["bucket_thread_startbit_u32"], s["bucket_bit_base_i64"], n, m, max_len)


class DecodePlan:
    """Decode a fixed list of tensors in one launch.

    ``items``: (fp8_u8 [n, m] uint8, sidecar mapping, out) with ``out`` a
    contiguous bfloat16 tensor of n*m elements; all on one device. The plan
    keeps references to every tensor it points at. Creation synchronises
    ``stream`` (default: the current stream), which may still be writing the
    sidecars, and reads their bucket metadata; it allocates the plan's device
    memory. Decodes allocate nothing and flag into the plan's own status word.
    A decode hands the work items out through a queue in the plan's memory, so
    two decodes of one plan must not overlap: launch them on one stream (or
    order their streams), and give each concurrent stream a plan of its own.
    """

    def __init__(self, items: Iterable[Tuple[torch.Tensor, Mapping[str, torch.Tensor], torch.Tensor]],
                 stream: torch.cuda.Stream | None = None):
        self._keep = []
        descs = []
        device = None
        for fp8_u8, sc, out in items:
            args = sidecar_decode_args(fp8_u8, sc)
            validate_decode_args(*args)
            n, m = args[11], args[12]
            if out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() != n * m \
                    or out.device != fp8_u8.device:
                raise ValueError("out must be a contiguous bfloat16 tensor of n*m elements on the fp8 device")
            if device is None:
                device = fp8_u8.device
            elif fp8_u8.device != device:
                raise ValueError("all tensors of a DecodePlan must be on one device")
            descs.append(_descriptor(*args[:11], n, m, out))
            self._keep.append((args, out))
        self.device = device
        self.count = len(descs)
        arr = (_native.MpsFp8Tensor * max(1, self.count))(*descs)
        self._plan = ctypes.c_void_p()
        if device is not None:
            h = stream.cuda_stream if stream is not None else _stream_handle(device)
            with torch.cuda.device(device):
                _native.check(_native.lib().mps_fp8_plan_create(arr, self.count, ctypes.c_void_p(h),
                                                                ctypes.byref(self._plan)))
        self.outputs = [o for _, o in self._keep]
        self.bytes_out = sum(o.numel() * 2 for o in self.outputs)

    def decode(self, stream: torch.cuda.Stream | None = None) -> Sequence[torch.Tensor]:
        """Enqueue the decode on ``stream`` (default: the current stream); returns the outputs."""
        if self.device is None:
            return self.outputs
        h = stream.cuda_stream if stream is not None else _stream_handle(self.device)
        with torch.cuda.device(self.device):
            _native.check(_native.lib().mps_fp8_plan_decode(self._plan, ctypes.c_void_p(h)))
        return self.outputs

    def decode_into(self, out: torch.Tensor, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """Decode into ``out`` instead of the outputs given at creation: ``out`` is a
        contiguous bfloat16 buffer laid out like them, every tensor's output moving by
        the offset of ``out`` from the first one (a single tensor, or row slices of
        one weight). Flags go to the device status word, as the op's do."""
        first = self.outputs[0] if self.outputs else None
        if first is not None:
            lo = min(o.data_ptr() for o in self.outputs)
            span = max(o.data_ptr() + 2 * o.numel() for o in self.outputs) - lo
            if lo != first.data_ptr():
                raise ValueError("decode_into needs the plan's first output to be its lowest")
            if out.dtype != torch.bfloat16 or not out.is_contiguous() or out.device != self.device \
                    or 2 * out.numel() < span:
                raise ValueError("out must be a contiguous bfloat16 buffer on the plan's device covering its outputs")
            h = stream.cuda_stream if stream is not None else _stream_handle(self.device)
            with torch.cuda.device(self.device):
                _native.check(_native.lib().mps_fp8_plan_decode_into(self._plan, ctypes.c_void_p(out.data_ptr()),
                                                                     ctypes.c_void_p(h)))
        return out

    def read_status(self, stream: torch.cuda.Stream | None = None) -> int:
        """MPS_STATUS_* flags this plan's decodes recorded since the last read (synchronises)."""
        v = ctypes.c_uint32(0)
        if self._plan:
            h = stream.cuda_stream if stream is not None else _stream_handle(self.device)
            _native.check(_native.lib().mps_fp8_plan_read_status(self._plan, ctypes.c_void_p(h), ctypes.byref(v)))
        return int(v.value)

    def info(self) -> Dict[str, int]:
        """Work items of a launch (buckets, or row ranges of buckets the plan split)
        and bytes of LDS per workgroup."""
        wi, lds = ctypes.c_int64(0), ctypes.c_int64(0)
        if self._plan:
            _native.check(_native.lib().mps_fp8_plan_info(self._plan, ctypes.byref(wi), ctypes.byref(lds)))
        return {"work_items": int(wi.value), "lds_bytes": int(lds.value)}

    def close(self) -> None:
        if getattr(self, "_plan", None):
            _native.lib().mps_fp8_plan_destroy(self._plan)
            self._plan = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
