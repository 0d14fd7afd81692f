"""Argument checks of the drop-in ops: same exception types and messages as the
reference's entry points (decode_huffman.cu:606-697, build_huffman.cu:298-366)."""
import inspect

import numpy as np
import pytest
import torch

import MPServe_cuda
import oracle
from tests.helpers import decode_args, synth, to_torch


def _cpu_args():
    bf, q, sc = synth(16, 64, seed=1)
    s = to_torch(oracle.encode(bf, q, sc, 7, 32), "cpu")
    return list(decode_args(s, torch.from_numpy(q)))


def test_decode_rejects_cpu_tensors():
    with pytest.raises(ValueError, match="fp8_params_u8 must be a CUDA tensor"):
        MPServe_cuda.huffman_decode_fp8(*_cpu_args())


def test_decode_default_max_len_is_12_and_rejected(monkeypatch):
    # the reference binds max_len=12 by default (wrapper.cpp:502) and the kernel rejects it
    import inspect

    assert inspect.signature(MPServe_cuda.huffman_decode_fp8).parameters["max_len"].default == 12
    assert inspect.signature(MPServe_cuda.huffman_build_fp8_decode_tables).parameters["max_len"].default == 12
    assert inspect.signature(MPServe_cuda.huffman_build_fp8_decode_tables).parameters[
        "threads_per_block"].default == 256


def test_sidecar_keys_match_reference_order():
    assert MPServe_cuda.SIDECAR_KEYS == (
        "decode_syms_u16", "decode_lens_u8", "table_scale_u16", "table_fp8_u16", "bucket_scale_u16",
        "bucket_row_offsets_i32", "row_indices_i32", "bucket_table_i32", "bucket_col_start_i32",
        "bucket_col_len_i32", "bucket_thread_startbit_u32", "bucket_bit_base_i64", "bitstream_u64",
        "shape_nmk_i64", "bucket_U_i32", "bucket_unique_gid_i32", "bucket_fp8_uidx_i16")


def test_out_of_scope_ops_raise_not_implemented():
    for name in ("dequantize_awq", "huffman_decode_awq_shared_table", "build_trie"):
        with pytest.raises(NotImplementedError):
            getattr(MPServe_cuda, name)()


def test_awq_int4_op_signatures_match_reference():
    """Argument names and defaults of wrapper.cpp:258-416."""
    sig = inspect.signature
    p = sig(MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables).parameters
    assert list(p)[:5] == ["bf16_params", "int4_values_u8", "scales_u16", "max_len", "threads_per_block"]
    assert (p["max_len"].default, p["threads_per_block"].default) == (11, 256)
    p = sig(MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables_by_scale).parameters
    assert list(p)[:6] == ["bf16_values", "int4_values", "scales_u16", "max_len", "threads", "group_cap"]
    assert (p["max_len"].default, p["threads"].default, p["group_cap"].default) == (11, 256, 1024)
    p = sig(MPServe_cuda.huffman_decode_awq_int4_bucket).parameters
    assert list(p)[:14] == ["int4_values_u8", "bitstream_u64", "decode_syms_u16", "decode_lens_u8",
                            "bucket_table_i32", "bucket_col_start_i32", "bucket_col_len_i32",
                            "bucket_row_offsets_i32", "row_indices_i32", "bucket_thread_startbit_u32",
                            "bucket_bit_base_i64", "n", "m", "max_len"]
    assert p["max_len"].default == 11
    p = sig(MPServe_cuda.huffman_decode_awq_int4_bucket_by_scale).parameters
    assert list(p)[:14] == ["int4_values_u8", "bitstream_u64", "decode_syms_u16", "decode_lens_u8",
                            "bucket_table_i32", "bucket_group_offsets_i32", "group_rows_i32",
                            "group_col_start_i32", "bucket_thread_startbit_u32", "bucket_bit_base_i64", "n", "m",
                            "max_len", "group_size"]
    assert p["max_len"].default is inspect.Parameter.empty and p["group_size"].default is inspect.Parameter.empty


def test_awq_build_argument_messages():
    """build_huffman.cu:1082-1123 / :1589-1623, checked before any GPU work."""
    bf = torch.zeros(4, 8, dtype=torch.bfloat16)
    q = torch.zeros(4, 8, dtype=torch.uint8)
    sc = torch.zeros(4, dtype=torch.uint16)
    b, bs = MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables, \
        MPServe_cuda.huffman_build_awq_int4_bucket_decode_tables_by_scale
    for args, msg in (((bf.float(), q, sc), "bf16_params must be torch.bfloat16"),
                      ((bf, q.int(), sc), "int4_values_u8 must be torch.uint8"),
                      ((bf, q, sc.int()), r"scales_u16 must be torch.uint16 \(bf16 raw bits\)"),
                      ((bf, q, sc, 0), r"max_len must be in \(0,15\]"),
                      ((bf, q, sc, 11, 1025), r"threads_per_block must be in \[1,1024\]"),
                      ((bf.reshape(-1), q.reshape(-1), sc), r"bf16_params must be 2D \[n,m\]"),
                      ((bf, q[:, :4], sc), "int4_values_u8 shape must match bf16_params")):
        with pytest.raises(ValueError, match=msg):
            b(*args)
    with pytest.raises(ValueError, match="group_cap must be > 0"):
        bs(bf, q, sc, 11, 256, 0)


def test_decode_validation_messages_via_meta_checks(monkeypatch):
    """Run the checks past the device test by faking is_cuda, to pin each message."""
    from mpserve_amd import mpserve_cuda as mc

    monkeypatch.setattr(mc, "_check_cuda_contig", lambda t, name, dev: None)
    args = _cpu_args()
    cases = [
        (0, args[0].to(torch.int8), "fp8_params_u8 must be uint8 CUDA"),
        (1, args[1].view(torch.int64), "bitstream_u64 must be uint64 1D CUDA"),
        (2, args[2].view(torch.int16), r"decode_syms_u16 must be uint16 2D CUDA \[G, 2\^L\]"),
        (4, args[4][:, :255].contiguous(), r"bucket_table_i32 must be int32 CUDA \[B,256\]"),
        (9, args[9].view(torch.int32), r"bucket_thread_startbit_u32 must be uint32 2D CUDA \[B,k\+1\]"),
        (13, 12, "decode kernel is specialized: max_len must be 7"),
        (13, 0, r"max_len must be in \[1,15\]"),
        (11, 0, "n,m must be > 0"),
        (12, 63, "fp8_params_u8 numel must equal n\\*m"),
        (5, args[5][:-1], "bucket_col_start_i32 length must be B"),
        (7, args[7][:-1], r"bucket_row_offsets_i32 length must be B\+1"),
    ]
    for i, val, msg in cases:
        a = list(args)
        a[i] = val
        with pytest.raises(ValueError, match=msg):
            mc.validate_decode_args(*a)
    mc.validate_decode_args(*args)


def test_build_dtype_checks_run_before_any_gpu_work():
    bf = torch.zeros((4, 8), dtype=torch.bfloat16)
    q = torch.zeros((4, 8), dtype=torch.uint8)
    sc = torch.zeros(4, dtype=torch.uint16)
    with pytest.raises(ValueError, match="bf16_params must be torch.bfloat16"):
        MPServe_cuda.huffman_build_fp8_decode_tables(bf.float(), q, sc, 7, 16)
    with pytest.raises(ValueError, match="fp8_params must be torch.uint8"):
        MPServe_cuda.huffman_build_fp8_decode_tables(bf, q.to(torch.int8), sc, 7, 16)
    with pytest.raises(ValueError, match=r"max_len must be in \[1, 15\]"):
        MPServe_cuda.huffman_build_fp8_decode_tables(bf, q, sc, 16, 16)
    with pytest.raises(ValueError, match=r"threads_per_block must be in \[1, 1024\]"):
        MPServe_cuda.huffman_build_fp8_decode_tables(bf, q, sc, 7, 0)
    with pytest.raises(ValueError, match="bf16_params and fp8_params must have same numel"):
        MPServe_cuda.huffman_build_fp8_decode_tables(bf, q[:2], sc, 7, 16)
    with pytest.raises(ValueError, match="scales must be torch.uint16 or torch.bfloat16"):
        MPServe_cuda.huffman_build_fp8_decode_tables(bf, q, sc.to(torch.int32), 7, 16)
