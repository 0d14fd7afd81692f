"""Shared test helpers: synthetic inputs, oracle sidecars, device transfer."""
from __future__ import annotations

import numpy as np
import torch

from mpserve_amd.synthetic import make_weight

# numpy dtype of each sidecar key as the build op returns it
NP_DTYPES = {
    "decode_syms_u16": np.uint16, "decode_lens_u8": np.uint8, "table_scale_u16": np.uint16,
    "table_fp8_u16": np.uint16, "bucket_scale_u16": np.uint16, "bucket_row_offsets_i32": np.int32,
    "row_indices_i32": np.int32, "bucket_table_i32": np.int32, "bucket_col_start_i32": np.int32,
    "bucket_col_len_i32": np.int32, "bucket_thread_startbit_u32": np.uint32, "bucket_bit_base_i64": np.int64,
    "bitstream_u64": np.uint64, "shape_nmk_i64": np.int64, "bucket_U_i32": np.int32,
    "bucket_unique_gid_i32": np.int32, "bucket_fp8_uidx_i16": np.int16,
}
TORCH_DTYPES = {
    np.uint16: torch.uint16, np.uint8: torch.uint8, np.int32: torch.int32, np.uint32: torch.uint32,
    np.int64: torch.int64, np.uint64: torch.uint64, np.int16: torch.int16,
}


def synth(n, m, sigma=0.02, seed=0, outlier_p=0.0):
    """(bf16 bits u16 [n,m], fp8 u8 [n,m], scale key u16 [n]) as numpy arrays."""
    w = make_weight(n, m, sigma=sigma, seed=seed, outlier_p=outlier_p)
    return w.bf16.view(torch.uint16).numpy(), w.fp8_u8.numpy(), w.scale_u16.numpy()


def to_torch(sc: dict, device) -> dict:
    """numpy sidecar dict -> torch tensors of the reference's dtypes on ``device``."""
    out = {}
    for k, v in sc.items():
        a = np.ascontiguousarray(v)
        t = torch.from_numpy(a.view(a.dtype.newbyteorder("=")) if a.dtype.byteorder == ">" else a)
        out[k] = t.to(device)
    return out


def decode_args(sc_t: dict, fp8_t: torch.Tensor):
    """Positional arguments of MPServe_cuda.huffman_decode_fp8 from a torch sidecar."""
    n, m = fp8_t.shape
    return (fp8_t, sc_t["bitstream_u64"], sc_t["decode_syms_u16"], sc_t["decode_lens_u8"],
            sc_t["bucket_table_i32"], sc_t["bucket_col_start_i32"], sc_t["bucket_col_len_i32"],
            sc_t["bucket_row_offsets_i32"], sc_t["row_indices_i32"], sc_t["bucket_thread_startbit_u32"],
            sc_t["bucket_bit_base_i64"], n, m, 7)
