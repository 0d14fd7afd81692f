"""Offline compressor: FP8 checkpoint + BF16 checkpoint -> FP8 + Huffman sidecar model.

Drop-in for the reference's scripts/compress_llm_fp8_huffman.py (same command
line, same sidecar keys and dtypes, same index.json / config.json rewrite),
with the sidecars built on the GPU by the HIP builder
(MPServe_cuda.huffman_build_fp8_decode_tables, byte-identical to the
reference's host builder)::

    python -m mpserve_amd.compress --bf16_model <bf16 dir> --fp8_model <fp8 dir> --out_dir <out dir>

Steps (reference line numbers in scripts/compress_llm_fp8_huffman.py):
  1. out_dir gets the base model tree (default: the FP8 model), files
     hard-linked where possible; model.safetensors.index.json and config.json
     are copied, since they are rewritten (:143-160).
  2. Every BF16 ``*.weight`` key accepted by --include / --exclude whose FP8
     checkpoint has the same key and a ``weight_scale_inv`` or ``weight_scale``
     is one module (:232-253); 2-D BF16 weights only (:255-258).
  3. FP8 bytes, scale dtype and scale shape are normalised as the reference
     does (:71-140), then the sidecar is built on the GPU.
  4. Sidecar tensors are stored under ``<module>.huff_*`` with the reference's
     signed dtypes (:284-306) into --sidecar_name (one shard, as the reference
     writes it; --max_shard_gb splits it into several shards named
     ``<stem>-NNNNN.safetensors``, all listed in the index).
  5. The index maps every sidecar key to its shard; with
     --override_common_from_bf16, keys in both checkpoints that match
     --override_allow_regex come from the BF16 checkpoint (:330-344).
     config.json gets quantization_config.quant_method = "fp8_huffman" and
     max_len (:350-362).

Host memory: the reference keeps every sidecar tensor of the model in one dict
until the end. Here a shard is written as soon as it reaches --max_shard_gb
(0, the default, keeps the reference's single shard).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import shutil
import sys
import time
from pathlib import Path
from typing import Callable, Dict, List, Optional, Tuple

import torch

INDEX = "model.safetensors.index.json"
# builder outputs that the sidecar does not store (they are returned by the build op only)
_NOT_STORED = ("table_scale_u16", "table_fp8_u16", "bucket_scale_u16", "shape_nmk_i64", "bucket_U_i32",
               "bucket_unique_gid_i32", "bucket_fp8_uidx_i16")
# build-op key -> (sidecar suffix, stored dtype): safetensors has no u16/u32/u64
_STORED = (
    ("bitstream_u64", "huff_bitstream_u64", torch.int64),
    ("decode_syms_u16", "huff_decode_syms_u16", torch.int16),
    ("decode_lens_u8", "huff_decode_lens_u8", torch.uint8),
    ("bucket_table_i32", "huff_bucket_table_i32", torch.int32),
    ("bucket_col_start_i32", "huff_bucket_col_start_i32", torch.int32),
    ("bucket_col_len_i32", "huff_bucket_col_len_i32", torch.int32),
    ("bucket_row_offsets_i32", "huff_bucket_row_offsets_i32", torch.int32),
    ("row_indices_i32", "huff_row_indices_i32", torch.int32),
    ("bucket_thread_startbit_u32", "huff_bucket_thread_startbit_u32", torch.int32),
    ("bucket_bit_base_i64", "huff_bucket_bit_base_i64", torch.int64),
)


def log(msg: str) -> None:
    print(f"[{time.strftime('%Y-%m-%d %H:%M:%S')}] {msg}", flush=True)


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--bf16_model", type=str, required=True, help="Path to BF16 model dir (safetensors)")
    p.add_argument("--fp8_model", type=str, required=True, help="Path to FP8 model dir (safetensors)")
    p.add_argument("--out_dir", type=str, required=True, help="Output model dir (FP8 + Huffman sidecar)")
    p.add_argument("--base_model", type=str, default=None,
                   help="Directory tree to copy/link into out_dir before adding sidecar (default: fp8_model)")
    p.add_argument("--include", type=str, default=None, help="Regex to include BF16 weight keys")
    p.add_argument("--exclude", type=str, default=None, help="Regex to exclude BF16 weight keys")
    p.add_argument("--max_len", type=int, default=7, help="Max Huffman code length (must be 7)")
    p.add_argument("--threads", type=int, default=1024, help="threads_per_block used for bucket metadata")
    p.add_argument("--sidecar_name", type=str, default="huffman_fp8.safetensors", help="Sidecar shard filename")
    p.add_argument("--store_fp8_u8", action="store_true", default=True, help="Store huff_fp8_u8 tensors")
    p.add_argument("--no_store_fp8_u8", action="store_false", dest="store_fp8_u8")
    p.add_argument("--override_common_from_bf16", action="store_true",
                   help="Write a small overrides shard for keys that exist in both BF16 and FP8 checkpoints")
    p.add_argument("--override_allow_regex", type=str, default=r"^(?:model\.embed_tokens\.weight|lm_head\.weight)$",
                   help="Regex filter for override keys (when --override_common_from_bf16 is set)")
    p.add_argument("--max_shard_gb", type=float, default=0.0,
                   help="Split the sidecar into shards of about this size (0: one shard, as the reference)")
    return p.parse_args(argv)


# --- checkpoint access ----------------------------------------------------------
def weight_map(model_dir: Path) -> Dict[str, str]:
    """The ``weight_map`` of a model's safetensors index (compress:45-54)."""
    path = model_dir / INDEX
    if not path.exists():
        raise FileNotFoundError(f"Missing safetensors index: {path}")
    with open(path, "r", encoding="utf-8") as f:
        wm = json.load(f).get("weight_map")
    if not isinstance(wm, dict):
        raise ValueError(f"Invalid weight_map in {path}")
    return wm


def load_tensor(model_dir: Path, wm: Dict[str, str], key: str) -> torch.Tensor:
    """One tensor from the shard the index names for it (compress:57-68)."""
    shard = wm.get(key)
    if not isinstance(shard, str):
        raise KeyError(f"Key not in safetensors index: {key}")
    path = model_dir / shard
    if not path.exists():
        raise FileNotFoundError(f"Missing safetensors shard for {key}: {path}")
    from safetensors import safe_open

    with safe_open(str(path), framework="pt", device="cpu") as f:
        return f.get_tensor(key)


# --- normalisation of the FP8 checkpoint's tensors ------------------------------------
def fp8_bytes(t: torch.Tensor, shape: Tuple[int, int]) -> torch.Tensor:
    """The stored FP8 weight as uint8 [n, m] (compress:71-93): uint8 as is, float8
    and 16-bit dtypes by their bytes, float32 through a bf16 cast."""
    if t.dtype == torch.uint8 or str(t.dtype).startswith("torch.float8"):
        u = t.view(torch.uint8)
    elif t.dtype in (torch.bfloat16, torch.float16):
        u = t.view(torch.uint16).view(torch.uint8)
    elif t.dtype == torch.float32:
        u = t.to(torch.bfloat16).view(torch.uint16).view(torch.uint8)
    else:
        u = t.view(torch.uint8)
    n, m = shape
    if int(u.numel()) != n * m:
        raise ValueError(f"FP8 numel mismatch: got {int(u.numel())} expected {n * m}")
    return u.reshape(n, m)


def scale_keys(scales: torch.Tensor) -> torch.Tensor:
    """Scales in a dtype the build op accepts (compress:96-104): u16 bits and bf16
    as they are, fp16 by its bits, fp32 rounded to fp16 bits, others to bf16."""
    if scales.dtype in (torch.uint16, torch.bfloat16):
        return scales
    if scales.dtype == torch.float16:
        return scales.view(torch.uint16)
    if scales.dtype == torch.float32:
        return scales.to(torch.float16).view(torch.uint16)
    return scales.to(torch.bfloat16)


def scale_shape(scales: torch.Tensor, n: int, m: int) -> torch.Tensor:
    """Scale layouts reduced to what the builder keys rows by (compress:107-140):
    scalar and [n] stay; [n, 1] -> [n]; [n / g] and [n / g, 1] repeat each entry
    g times; a block grid [n / bn, m / bm] keeps its first column block, repeated
    bn times. Anything else is passed through (the build op then rejects it)."""
    total = int(scales.numel())
    if total == 1:
        return scales
    if scales.dim() == 2 and int(scales.size(0)) == n and int(scales.size(1)) == 1:
        scales = scales.squeeze(1)
    if scales.dim() == 1 and total == n:
        return scales
    if scales.dim() == 1 and total > 0 and n % total == 0:
        return scales.repeat_interleave(n // total)
    if scales.dim() == 2 and int(scales.size(1)) == 1 and int(scales.size(0)) > 0 and n % int(scales.size(0)) == 0:
        return scales.squeeze(1).repeat_interleave(n // int(scales.size(0)))
    if scales.dim() == 2 and int(scales.size(0)) > 0 and int(scales.size(1)) > 0:
        if n % int(scales.size(0)) == 0 and m % int(scales.size(1)) == 0:
            return scales[:, 0].repeat_interleave(n // int(scales.size(0)))
    return scales


def sidecar_entries(prefix: str, built: Dict[str, torch.Tensor], fp8_u8: torch.Tensor,
                    store_fp8: bool) -> Dict[str, torch.Tensor]:
    """The ``<prefix>.huff_*`` tensors of one module, as the reference stores them
    (compress:284-306): the FP8 copy (or an empty [0, 0] one), the ten decode
    arrays with signed dtypes, and the five packed-mode fields left at their
    defaults."""
    out = {f"{prefix}.huff_fp8_u8": fp8_u8.contiguous() if store_fp8 else torch.empty((0, 0), dtype=torch.uint8)}
    for key, suffix, dtype in _STORED:
        t = built[key].cpu()
        # bit-preserving for the unsigned -> signed views (u64/u16/u32 do not exist in safetensors)
        out[f"{prefix}.{suffix}"] = (t.view(dtype) if t.element_size() == torch.empty(0, dtype=dtype).element_size()
                                     else t.to(dtype)).contiguous()
    out[f"{prefix}.huff_2d_nb1_i32"] = torch.tensor([1], dtype=torch.int32)
    for f in ("row_start", "row_len", "col_start", "col_len"):
        out[f"{prefix}.huff_attn_block_{f}_i32"] = torch.empty((0,), dtype=torch.int32)
    return out


def link_or_copy_tree(src: Path, dst: Path) -> None:
    """Mirror src into dst: hard links where possible, copies otherwise; the
    index and config.json are always copied (they are rewritten); existing files
    are kept (compress:143-160)."""
    dst.mkdir(parents=True, exist_ok=True)
    for root, dirs, files in os.walk(src):
        rel = Path(root).relative_to(src)
        (dst / rel).mkdir(parents=True, exist_ok=True)
        for d in dirs:
            (dst / rel / d).mkdir(parents=True, exist_ok=True)
        for fn in files:
            sp, dp = Path(root) / fn, dst / rel / fn
            if dp.exists():
                continue
            if fn in (INDEX, "config.json"):
                shutil.copy2(sp, dp)
                continue
            try:
                os.link(sp, dp)
            except OSError:
                shutil.copy2(sp, dp)


def default_builder(bf16: torch.Tensor, fp8_u8: torch.Tensor, scales: torch.Tensor, max_len: int,
                    threads: int) -> Dict[str, torch.Tensor]:
    """The GPU sidecar builder through the MPServe_cuda op surface."""
    from mpserve_amd import mpserve_cuda

    return mpserve_cuda.huffman_build_fp8_decode_tables(bf16, fp8_u8, scales, max_len=max_len,
                                                        threads_per_block=threads)


class ShardWriter:
    """Sidecar shards: one file, or files of about ``max_bytes`` each."""

    def __init__(self, out_dir: Path, name: str, max_bytes: int):
        self.out_dir, self.name, self.max_bytes = out_dir, name, max_bytes
        self.pending: Dict[str, torch.Tensor] = {}
        self.pending_bytes = 0
        self.files: List[str] = []
        self.key_file: Dict[str, str] = {}

    def _shard_name(self, i: int) -> str:
        stem, ext = os.path.splitext(self.name)
        return f"{stem}-{i + 1:05d}{ext}"

    def add(self, tensors: Dict[str, torch.Tensor]) -> None:
        self.pending.update(tensors)
        self.pending_bytes += sum(t.numel() * t.element_size() for t in tensors.values())
        if self.max_bytes > 0 and self.pending_bytes >= self.max_bytes:
            self._flush(self._shard_name(len(self.files)))

    def _flush(self, fname: str) -> None:
        from safetensors.torch import save_file

        log(f"Writing sidecar shard: {self.out_dir / fname} (tensors={len(self.pending)})")
        save_file(self.pending, str(self.out_dir / fname))
        for k in self.pending:
            self.key_file[k] = fname
        self.files.append(fname)
        self.pending, self.pending_bytes = {}, 0

    def close(self) -> None:
        if self.pending:
            self._flush(self.name if self.max_bytes <= 0 else self._shard_name(len(self.files)))


def compress(args: argparse.Namespace, builder: Callable = default_builder) -> Dict[str, object]:
    """Run the compressor; returns a summary (modules built, keys added, shard files)."""
    if int(args.max_len) != 7:
        raise SystemExit("--max_len must be 7 for the FP8 Huffman decode kernel")
    bf16_dir, fp8_dir, out_dir = Path(args.bf16_model), Path(args.fp8_model), Path(args.out_dir)
    base_dir = Path(args.base_model) if args.base_model else fp8_dir
    if not bf16_dir.is_dir():
        raise SystemExit(f"--bf16_model must be a directory: {bf16_dir}")
    if not fp8_dir.is_dir():
        raise SystemExit(f"--fp8_model must be a directory: {fp8_dir}")
    include = re.compile(args.include) if args.include else None
    exclude = re.compile(args.exclude) if args.exclude else None

    def selected(key: str) -> bool:
        return (include is None or include.search(key) is not None) and \
               (exclude is None or exclude.search(key) is None)

    log(f"Start FP8 Huffman sidecar build: bf16_model={bf16_dir} fp8_model={fp8_dir} out_dir={out_dir} "
        f"max_len={args.max_len} threads={args.threads}")
    t0 = time.time()
    link_or_copy_tree(base_dir, out_dir)
    log(f"Prepared out_dir (copy/link): elapsed={time.time() - t0:.2f}s")
    wm_b, wm_f = weight_map(bf16_dir), weight_map(fp8_dir)
    candidates = [k for k in wm_b if k.endswith(".weight")]
    log(f"Loaded safetensors index: bf16_keys={len(wm_b)} fp8_keys={len(wm_f)}; BF16 .weight candidates: "
        f"{len(candidates)}")

    writer = ShardWriter(out_dir, str(args.sidecar_name), int(args.max_shard_gb * 1e9))
    built = missing = not_2d = 0
    for key in candidates:
        if not selected(key):
            continue
        prefix = key[: -len(".weight")]
        scales_key = next((c for c in (f"{prefix}.weight_scale_inv", f"{prefix}.weight_scale") if c in wm_f), None)
        if key not in wm_f or scales_key is None:
            missing += 1
            continue
        bf16 = load_tensor(bf16_dir, wm_b, key).contiguous()
        if bf16.dtype != torch.bfloat16 or bf16.dim() != 2:
            not_2d += 1
            continue
        n, m = int(bf16.shape[0]), int(bf16.shape[1])
        q = fp8_bytes(load_tensor(fp8_dir, wm_f, key).contiguous(), (n, m)).contiguous()
        scales = scale_shape(scale_keys(load_tensor(fp8_dir, wm_f, scales_key).contiguous()), n, m).contiguous()
        log(f"Building artifact '{prefix}'")
        out = builder(bf16, q, scales, int(args.max_len), int(args.threads))
        writer.add(sidecar_entries(prefix, out, q, bool(args.store_fp8_u8)))
        built += 1
        if built % 16 == 0:
            log(f"Built {built} modules...")
    if built == 0:
        raise SystemExit(f"No modules matched. skipped_missing_fp8={missing} skipped_non_bf16_2d={not_2d}")
    writer.close()

    index_path = out_dir / INDEX
    with open(index_path, "r", encoding="utf-8") as f:
        idx = json.load(f)
    wm = idx.get("weight_map")
    if not isinstance(wm, dict):
        raise ValueError(f"Invalid weight_map in {index_path}")
    wm.update(writer.key_file)
    if args.override_common_from_bf16:
        allow = re.compile(args.override_allow_regex) if args.override_allow_regex else None
        common = sorted(set(wm_b) & set(wm_f))
        keys = [k for k in common if allow is None or allow.search(k) is not None]
        log(f"Overriding common keys from BF16: common={len(common)} selected={len(keys)}")
        overrides = {k: load_tensor(bf16_dir, wm_b, k) for k in keys}
        if overrides:
            from safetensors.torch import save_file

            name = "overrides_from_bf16.safetensors"
            log(f"Writing override shard: {out_dir / name} (tensors={len(overrides)})")
            save_file(overrides, str(out_dir / name))
            for k in keys:
                wm[k] = name
    idx["weight_map"] = wm
    with open(index_path, "w", encoding="utf-8") as f:
        json.dump(idx, f, indent=2, sort_keys=True)

    cfg_path = out_dir / "config.json"
    if cfg_path.exists():
        try:
            cfg = json.loads(cfg_path.read_text(encoding="utf-8"))
            qc = cfg.get("quantization_config")
            qc = qc if isinstance(qc, dict) else {}
            qc["quant_method"] = "fp8_huffman"
            qc.setdefault("max_len", int(args.max_len))
            cfg["quantization_config"] = qc
            cfg_path.write_text(json.dumps(cfg, indent=2, sort_keys=True), encoding="utf-8")
        except (ValueError, OSError):
            # the reference also leaves an unreadable config.json as it is
            pass
    for f in writer.files:
        print(f"Wrote sidecar shard: {out_dir / f}")
    print(f"Updated index: {index_path}")
    print(f"Added keys: {len(writer.key_file)}")
    return {"modules": built, "keys": len(writer.key_file), "files": list(writer.files)}


def main(argv=None) -> int:
    compress(parse_args(argv))
    return 0


if __name__ == "__main__":
    sys.exit(main())
