"""Offline compressor (mpserve_amd.compress): a tiny BF16 + FP8 checkpoint pair in
safetensors -> FP8 + Huffman sidecar model.

The CPU tests exercise the compressor's I/O: index and config rewrite, key names,
stored dtypes, scale normalisation, shards, include/exclude, overrides. In them
the CPU oracle stands in for the GPU builder, so the written sidecar can be
decoded back (bit-exact) on the CPU; the GPU test runs the real builder.
"""
import json
import os
from types import SimpleNamespace

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

import oracle
from mpserve_amd import compress as cz
from mpserve_amd.synthetic import make_weight

LAYERS = {"model.layers.0.self_attn.q_proj": (64, 256), "model.layers.0.mlp.down_proj": (48, 320)}


def _model_pair(tmp_path, scale_style="inv_f32_col"):
    """BF16 and FP8 checkpoints (two shards each) with an index and config.json."""
    bf_dir, f8_dir = tmp_path / "bf16", tmp_path / "fp8"
    bf_dir.mkdir()
    f8_dir.mkdir()
    bf_t, f8_t, ref = {}, {}, {}
    for i, (prefix, (n, m)) in enumerate(LAYERS.items()):
        w = make_weight(n, m, seed=300 + i)
        bf_t[prefix + ".weight"] = w.bf16
        f8_t[prefix + ".weight"] = w.fp8_u8.view(torch.float8_e4m3fn)
        if scale_style == "inv_f32_col":
            f8_t[prefix + ".weight_scale_inv"] = w.scale_f32              # [n, 1] fp32
        else:
            f8_t[prefix + ".weight_scale"] = w.scale_f32.reshape(-1).to(torch.float16)  # [n] fp16
        ref[prefix] = (w.bf16.view(torch.uint16).numpy(), w.fp8_u8.numpy(), w.scale_u16.numpy())
    bf_t["model.norm.weight"] = torch.ones(64, dtype=torch.bfloat16)        # 1-D: skipped
    bf_t["model.embed_tokens.weight"] = torch.randn(16, 64).to(torch.bfloat16)
    f8_t["model.embed_tokens.weight"] = torch.zeros(16, 64, dtype=torch.bfloat16)
    for d, tensors in ((bf_dir, bf_t), (f8_dir, f8_t)):
        keys = sorted(tensors)
        half = len(keys) // 2
        wm = {}
        for j, part in enumerate((keys[:half], keys[half:])):
            name = f"model-0000{j + 1}-of-00002.safetensors"
            save_file({k: tensors[k] for k in part}, str(d / name))
            wm.update({k: name for k in part})
        (d / cz.INDEX).write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    (f8_dir / "config.json").write_text(json.dumps({"model_type": "llama", "quantization_config": {"quant_method": "fp8"}}))
    (f8_dir / "tokenizer.json").write_text("{}")
    return bf_dir, f8_dir, ref


def _args(bf_dir, f8_dir, out_dir, **kw):
    a = cz.parse_args(["--bf16_model", str(bf_dir), "--fp8_model", str(f8_dir), "--out_dir", str(out_dir)])
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _oracle_builder(bf16, fp8_u8, scales, max_len, threads):
    sc = scales.numpy() if scales.dtype == torch.uint16 else scales.view(torch.uint16).numpy()
    d = oracle.encode(bf16.view(torch.uint16).numpy(), fp8_u8.numpy(), sc, max_len, threads)
    return {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in d.items()}


def _read_sidecar(out_dir, prefix):
    idx = json.loads((out_dir / cz.INDEX).read_text())["weight_map"]
    got = {}
    for k, f in idx.items():
        if k.startswith(prefix + ".huff_"):
            with safe_open(str(out_dir / f), framework="pt") as h:
                got[k[len(prefix) + 1:]] = h.get_tensor(k)
    return got


def _decode_numpy(side, fp8, n, m):
    d = {k[len("huff_"):]: v.numpy() for k, v in side.items()}
    d["bitstream_u64"] = d["bitstream_u64"].view(np.uint64)
    d["decode_syms_u16"] = d["decode_syms_u16"].view(np.uint16)
    d["bucket_thread_startbit_u32"] = d["bucket_thread_startbit_u32"].view(np.uint32)
    return oracle.decode(d, fp8, n, m, 7)


@pytest.mark.parametrize("scale_style", ["inv_f32_col", "fp16_row"])
def test_compress_writes_reference_layout(tmp_path, scale_style):
    bf_dir, f8_dir, ref = _model_pair(tmp_path, scale_style)
    out = tmp_path / "out"
    summary = cz.compress(_args(bf_dir, f8_dir, out, threads=64), builder=_oracle_builder)
    assert summary["modules"] == 2 and summary["files"] == ["huffman_fp8.safetensors"]
    idx = json.loads((out / cz.INDEX).read_text())["weight_map"]
    cfg = json.loads((out / "config.json").read_text())
    assert cfg["quantization_config"]["quant_method"] == "fp8_huffman" and cfg["quantization_config"]["max_len"] == 7
    assert (out / "tokenizer.json").exists()
    for prefix, (n, m) in LAYERS.items():
        side = _read_sidecar(out, prefix)
        assert set(side) == {"huff_fp8_u8", "huff_bitstream_u64", "huff_decode_syms_u16", "huff_decode_lens_u8",
                             "huff_bucket_table_i32", "huff_bucket_col_start_i32", "huff_bucket_col_len_i32",
                             "huff_bucket_row_offsets_i32", "huff_row_indices_i32", "huff_bucket_thread_startbit_u32",
                             "huff_bucket_bit_base_i64", "huff_2d_nb1_i32", "huff_attn_block_row_start_i32",
                             "huff_attn_block_row_len_i32", "huff_attn_block_col_start_i32",
                             "huff_attn_block_col_len_i32"}
        assert side["huff_bitstream_u64"].dtype == torch.int64 and side["huff_decode_syms_u16"].dtype == torch.int16
        assert side["huff_bucket_thread_startbit_u32"].dtype == torch.int32
        assert side["huff_2d_nb1_i32"].tolist() == [1] and side["huff_attn_block_col_len_i32"].numel() == 0
        bf, q, key = ref[prefix]
        assert np.array_equal(side["huff_fp8_u8"].numpy(), q)
        # the stored arrays are the builder's (bit-preserving signed views) for the per-row u16 keys
        want = oracle.encode(bf, q, key, 7, 64)
        assert np.array_equal(side["huff_bitstream_u64"].numpy().view(np.uint64), want["bitstream_u64"])
        assert np.array_equal(side["huff_decode_syms_u16"].numpy().view(np.uint16), want["decode_syms_u16"])
        assert np.array_equal(_decode_numpy({k: v for k, v in side.items() if k != "huff_fp8_u8"}, q, n, m), bf)
        assert idx[prefix + ".huff_bitstream_u64"] == "huffman_fp8.safetensors"
        assert idx[prefix + ".weight"].startswith("model-")  # FP8 weight entries are kept
    assert "model.norm.weight.huff_fp8_u8" not in idx


def test_compress_shards_filters_and_overrides(tmp_path):
    bf_dir, f8_dir, _ = _model_pair(tmp_path)
    out = tmp_path / "out"
    summary = cz.compress(_args(bf_dir, f8_dir, out, threads=64, max_shard_gb=1e-9, exclude=r"down_proj",
                                store_fp8_u8=False, override_common_from_bf16=True), builder=_oracle_builder)
    assert summary["modules"] == 1 and summary["files"] == ["huffman_fp8-00001.safetensors"]
    idx = json.loads((out / cz.INDEX).read_text())["weight_map"]
    assert "model.layers.0.mlp.down_proj.huff_bitstream_u64" not in idx
    assert idx["model.embed_tokens.weight"] == "overrides_from_bf16.safetensors"
    side = _read_sidecar(out, "model.layers.0.self_attn.q_proj")
    assert tuple(side["huff_fp8_u8"].shape) == (0, 0)


def test_compress_rejects_bad_max_len_and_no_match(tmp_path):
    bf_dir, f8_dir, _ = _model_pair(tmp_path)
    with pytest.raises(SystemExit, match="only reads max_len 7"):
        cz.compress(_args(bf_dir, f8_dir, tmp_path / "o1", max_len=6), builder=_oracle_builder)
    with pytest.raises(SystemExit, match="no module to build"):
        cz.compress(_args(bf_dir, f8_dir, tmp_path / "o2", include=r"nothing"), builder=_oracle_builder)


def test_scale_normalisation_matches_reference_rules():
    """compress_llm_fp8_huffman.py:71-140: the dtype and layout rules, case by case."""
    n, m = 256, 512
    s = torch.arange(4, dtype=torch.float32)
    assert cz.scale_rows(torch.tensor([3.0]), n, m).numel() == 1
    assert cz.scale_rows(torch.ones(n, 1), n, m).shape == (n,)
    assert cz.scale_rows(s, n, m).tolist() == sum([[float(i)] * 64 for i in range(4)], [])
    assert cz.scale_rows(s.reshape(4, 1), n, m).shape == (n,)
    grid = torch.arange(8, dtype=torch.float32).reshape(2, 4)  # [n/128, m/128] blocks: first column block per row block
    assert cz.scale_rows(grid, n, m).tolist() == [0.0] * 128 + [4.0] * 128
    odd = torch.ones(3)  # 3 does not divide 256: left for the builder to reject
    assert cz.scale_rows(odd, n, m) is odd
    assert cz.scale_rows(torch.ones(2, 2, 2), n, m).shape == (2, 2, 2)
    assert cz.scale_keys(torch.tensor([1.0])).dtype == torch.uint16
    assert cz.scale_keys(torch.tensor([1.0])).view(torch.float16).item() == 1.0
    assert cz.scale_keys(torch.tensor([1.0], dtype=torch.float16)).view(torch.float16).item() == 1.0
    assert cz.scale_keys(torch.tensor([2], dtype=torch.int32)).dtype == torch.bfloat16
    b = torch.tensor([1.5], dtype=torch.bfloat16)
    assert cz.scale_keys(b) is b
    assert cz.fp8_bytes(torch.zeros(2, 3, dtype=torch.float8_e4m3fn), 2, 3).dtype == torch.uint8
    # 16-bit stores keep their bytes; float32 stores are rounded to bf16 byte pairs first
    h = torch.tensor([[0x1234, 0xABCD]], dtype=torch.int32).to(torch.uint16).view(torch.bfloat16)
    assert cz.fp8_bytes(h, 1, 4).tolist() == [[0x34, 0x12, 0xCD, 0xAB]]
    f = torch.tensor([[1.0, -2.0]], dtype=torch.float32)
    assert cz.fp8_bytes(f, 1, 4).tolist() == [[0x80, 0x3F, 0x00, 0xC0]]
    with pytest.raises(ValueError, match="needs 6"):
        cz.fp8_bytes(torch.zeros(5, dtype=torch.uint8), 2, 3)


@pytest.mark.gpu
def test_compress_with_gpu_builder_roundtrips(tmp_path):
    import MPServe_cuda
    from mpserve_amd.decode import sidecar_decode_args

    bf_dir, f8_dir, ref = _model_pair(tmp_path)
    out = tmp_path / "out"
    cz.compress(_args(bf_dir, f8_dir, out))  # the default builder: the HIP sidecar builder, k = 1024
    for prefix, (n, m) in LAYERS.items():
        side = _read_sidecar(out, prefix)
        bf, q, key = ref[prefix]
        want = oracle.encode(bf, q, key, 7, 1024)
        assert np.array_equal(side["huff_bitstream_u64"].numpy().view(np.uint64), want["bitstream_u64"])
        assert np.array_equal(side["huff_bucket_thread_startbit_u32"].numpy().view(np.uint32),
                              want["bucket_thread_startbit_u32"])
        dev = {k: v.to("cuda:0") for k, v in side.items()}
        got = MPServe_cuda.huffman_decode_fp8(*sidecar_decode_args(dev["huff_fp8_u8"], dev))
        torch.cuda.synchronize()
        assert np.array_equal(got.view(torch.uint16).cpu().numpy(), bf)
