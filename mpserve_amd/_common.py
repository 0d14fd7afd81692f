"""Helpers shared by the op modules: the current stream's handle, the reference's
contiguity check (decode_huffman.cu:59-63) and the device integrity word."""
from __future__ import annotations

import ctypes
import os

import torch

from . import _native


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_cuda_contig(t: torch.Tensor, name: str, device: torch.device | None) -> None:
    # decode_huffman.cu:59-63
    if t is None:
        raise ValueError(f"{name} must be defined")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if device is not None and t.device != device:
        raise ValueError(f"{name} must be on {device}, got {t.device}")


def read_status(device: torch.device | None = None) -> int:
    """MPS_STATUS_* flags recorded by decodes on ``device`` since the last read (synchronises)."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    v = ctypes.c_uint32(0)
    _native.check(_native.lib().mps_fp8_read_status(device.index or 0, ctypes.c_void_p(_stream_handle(device)),
                                                    ctypes.byref(v)))
    return int(v.value)


def _maybe_check_status(device: torch.device, op: str = "huffman_decode_fp8") -> None:
    """With MPSERVE_DECODE_CHECK=1: synchronise and raise if the decode flagged the sidecar."""
    if os.environ.get("MPSERVE_DECODE_CHECK", "0") == "1":
        st = read_status(device)
        if st:
            raise RuntimeError(f"{op}: sidecar integrity flags 0x{st:x} "
                               "(1=bucket range, 2=row index, 4=table id, 8=lane bit desync)")
