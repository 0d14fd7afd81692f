"""Offline compressor: a BF16 checkpoint and its FP8 checkpoint -> an FP8 model
with a Huffman sidecar per linear weight, built on the GPU.

    python -m mpserve_amd.compress --bf16_model <dir> --fp8_model <dir> --out_dir <dir> [options]

It takes the command line of the reference's offline compressor
(scripts/compress_llm_fp8_huffman.py:164-198) and writes the same files: the
output directory mirrors the base model (the FP8 model unless --base_model is
given), gains ``<sidecar_name>`` with 16 ``<module>.huff_*`` tensors per module
(names and stored dtypes of compress:284-306), and its safetensors index and
config.json are rewritten (compress:318-367). The sidecars come from the GPU
builder behind ``MPServe_cuda.huffman_build_fp8_decode_tables``, whose output
is byte-identical to the reference's host builder.

The work is split into four passes:
  1. ``mirror_tree``: link (or copy) the base model into the output directory.
  2. ``select_modules``: pair each BF16 ``*.weight`` with the FP8 weight of the
     same name and its scale, using only the safetensors headers.
  3. ``build_sidecars``: per module, read the three tensors, bring the FP8
     bytes and the scales into the builder's input forms (``fp8_bytes``,
     ``scale_keys``, ``scale_rows``), build, and hand the stored tensors to a
     ``SidecarStore`` (one shard, as the reference writes, or shards of about
     --max_shard_gb, written as they fill so the host never holds the whole
     model's sidecar).
  4. ``finish``: index, optional BF16 overrides, config.json.
"""
from __future__ import annotations

import argparse
import collections
import json
import os
import re
import shutil
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Dict, List, Optional, Tuple

import torch

INDEX = "model.safetensors.index.json"
OVERRIDES = "overrides_from_bf16.safetensors"

# (build-op key, stored suffix, stored dtype): safetensors has no u16/u32/u64,
# so those arrays are stored as the signed type of the same width (bit for bit)
STORED = (
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
# fields of the packed-layer modes (one layer's linears packed into one weight):
# a plain sidecar stores them at their neutral values
PACK_FIELDS = {"huff_2d_nb1_i32": (1,), "huff_attn_block_row_start_i32": (), "huff_attn_block_row_len_i32": (),
               "huff_attn_block_col_start_i32": (), "huff_attn_block_col_len_i32": ()}


def say(msg: str) -> None:
    print(f"compress [{time.strftime('%H:%M:%S')}] {msg}", flush=True)


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description="Add a Huffman sidecar to an FP8 checkpoint (GPU builder).")
    p.add_argument("--bf16_model", type=str, required=True, help="directory of the BF16 safetensors model")
    p.add_argument("--fp8_model", type=str, required=True, help="directory of the FP8 safetensors model")
    p.add_argument("--out_dir", type=str, required=True, help="where the FP8 + sidecar model is written")
    p.add_argument("--base_model", type=str, default=None,
                   help="model tree mirrored into out_dir first (default: the FP8 model)")
    p.add_argument("--include", type=str, default=None, help="only BF16 weight keys matching this regex")
    p.add_argument("--exclude", type=str, default=None, help="skip BF16 weight keys matching this regex")
    p.add_argument("--max_len", type=int, default=7, help="longest Huffman code (the decoder requires 7)")
    p.add_argument("--threads", type=int, default=1024, help="substreams per bucket (threads_per_block)")
    p.add_argument("--sidecar_name", type=str, default="huffman_fp8.safetensors", help="file name of the sidecar")
    p.add_argument("--store_fp8_u8", action="store_true", default=True,
                   help="store each module's FP8 bytes in the sidecar as huff_fp8_u8 (default)")
    p.add_argument("--no_store_fp8_u8", action="store_false", dest="store_fp8_u8",
                   help="store an empty huff_fp8_u8 instead")
    p.add_argument("--override_common_from_bf16", action="store_true",
                   help="serve keys present in both checkpoints (filtered by --override_allow_regex) from BF16")
    p.add_argument("--override_allow_regex", type=str, default=r"^(?:model\.embed_tokens\.weight|lm_head\.weight)$",
                   help="which common keys --override_common_from_bf16 takes from BF16")
    p.add_argument("--max_shard_gb", type=float, default=0.0,
                   help="split the sidecar into shards of about this many GB (0: a single file)")
    return p.parse_args(argv)


# --------------------------------------------------------------------------- checkpoints
class Checkpoint:
    """A safetensors model directory read through its index; shards are opened
    once and tensors read on demand."""

    def __init__(self, root: Path):
        self.root = Path(root)
        path = self.root / INDEX
        if not path.is_file():
            raise FileNotFoundError(f"{path}: no safetensors index")
        with open(path, "r", encoding="utf-8") as f:
            wm = json.load(f).get("weight_map")
        if not isinstance(wm, dict):
            raise ValueError(f"{path}: weight_map is missing or not an object")
        self.index: Dict[str, str] = wm
        self._open: Dict[str, object] = {}

    def __contains__(self, key: str) -> bool:
        return key in self.index

    def _shard(self, key: str):
        name = self.index.get(key)
        if not isinstance(name, str):
            raise KeyError(f"{key}: not in the index of {self.root}")
        h = self._open.get(name)
        if h is None:
            path = self.root / name
            if not path.is_file():
                raise FileNotFoundError(f"{path}: shard of {key} not found")
            from safetensors import safe_open

            h = safe_open(str(path), framework="pt", device="cpu")
            self._open[name] = h
        return h

    def header(self, key: str) -> Tuple[str, List[int]]:
        """(safetensors dtype name, shape) of a tensor, without reading it."""
        s = self._shard(key).get_slice(key)
        return s.get_dtype(), list(s.get_shape())

    def tensor(self, key: str) -> torch.Tensor:
        return self._shard(key).get_tensor(key)


# --------------------------------------------------------------------------- module selection
@dataclass
class Module:
    prefix: str        # "model.layers.0.self_attn.q_proj"
    weight_key: str    # prefix + ".weight" (BF16 and FP8 checkpoints)
    scale_key: str     # prefix + ".weight_scale_inv" or ".weight_scale" (FP8 checkpoint)


@dataclass
class Selection:
    modules: List[Module] = field(default_factory=list)
    skipped: collections.Counter = field(default_factory=collections.Counter)


def select_modules(bf16: Checkpoint, fp8: Checkpoint, include: Optional[str], exclude: Optional[str]) -> Selection:
    """Modules to build, in the BF16 index's order: a BF16 ``*.weight`` that the
    filters accept, that is a 2-D bfloat16 tensor, and whose FP8 checkpoint has
    the same key and a scale (``weight_scale_inv`` preferred to ``weight_scale``)."""
    inc = re.compile(include) if include else None
    exc = re.compile(exclude) if exclude else None
    sel = Selection()
    for key in bf16.index:
        if not key.endswith(".weight"):
            continue
        if (inc is not None and not inc.search(key)) or (exc is not None and exc.search(key)):
            continue
        prefix = key[: -len(".weight")]
        scale = next((s for s in (prefix + ".weight_scale_inv", prefix + ".weight_scale") if s in fp8), None)
        if key not in fp8 or scale is None:
            sel.skipped["no FP8 weight or scale"] += 1
            continue
        dtype, shape = bf16.header(key)
        if dtype != "BF16" or len(shape) != 2:
            sel.skipped["not a 2-D BF16 weight"] += 1
            continue
        sel.modules.append(Module(prefix, key, scale))
    return sel


# --------------------------------------------------------------------------- builder inputs
def fp8_bytes(t: torch.Tensor, n: int, m: int) -> torch.Tensor:
    """The FP8 checkpoint's weight as the builder's uint8 [n, m].

    Whatever the stored dtype, the weight's bytes are taken as they lie, with one
    exception: a float32 store is rounded to bfloat16 first, since such files
    carry byte pairs widened to float (compress:71-93). A byte count other than
    n*m is an error.
    """
    if t.dtype == torch.float32:
        t = t.to(torch.bfloat16)
    raw = t.contiguous().view(torch.uint8) if t.dim() > 0 else t.reshape(1).view(torch.uint8)
    if raw.numel() != n * m:
        raise ValueError(f"FP8 weight has {raw.numel()} bytes, the BF16 weight {n}x{m} needs {n * m}")
    return raw.reshape(n, m)


# stored scale dtype -> the 16-bit key the builder groups rows by (compress:96-104)
_SCALE_KEY = {
    torch.uint16: lambda s: s,
    torch.bfloat16: lambda s: s,
    torch.float16: lambda s: s.view(torch.uint16),
    torch.float32: lambda s: s.to(torch.float16).view(torch.uint16),
}


def scale_keys(s: torch.Tensor) -> torch.Tensor:
    """Scales in a dtype the builder takes: u16 bits or bf16 as stored, fp16 by its
    bits, fp32 rounded to fp16 bits; any other dtype is cast to bf16."""
    return _SCALE_KEY.get(s.dtype, lambda x: x.to(torch.bfloat16))(s)


def scale_rows(s: torch.Tensor, n: int, m: int) -> torch.Tensor:
    """Scales in a layout the builder keys rows by (compress:107-140).

    * one value: unchanged;
    * a column of L values ([L] or [L, 1]) with L dividing n: each value covers
      n / L consecutive rows (L = n: one per row);
    * a block grid [R, C] with R | n and C | m: each row block takes the scale
      of its first column block;
    * anything else: unchanged (the builder then rejects it).
    """
    if s.numel() == 1:
        return s
    column = s.dim() == 1 or (s.dim() == 2 and s.shape[1] == 1)
    rows = int(s.shape[0]) if s.dim() >= 1 else 0
    if column and rows > 0 and n % rows == 0:
        return s.reshape(rows).repeat_interleave(n // rows)
    if s.dim() == 2 and rows > 0 and s.shape[1] > 0 and n % rows == 0 and m % int(s.shape[1]) == 0:
        return s[:, 0].repeat_interleave(n // rows)
    return s


def stored_tensors(prefix: str, built: Dict[str, torch.Tensor], fp8_u8: torch.Tensor,
                   keep_fp8: bool) -> Dict[str, torch.Tensor]:
    """The 16 tensors stored for one module: its FP8 bytes (or an empty [0, 0]),
    the ten decode arrays in their stored dtypes, and the packed-mode fields."""
    out = {f"{prefix}.huff_fp8_u8": fp8_u8 if keep_fp8 else torch.empty((0, 0), dtype=torch.uint8)}
    for key, suffix, dtype in STORED:
        t = built[key].cpu().contiguous()
        out[f"{prefix}.{suffix}"] = t if t.dtype == dtype else t.view(dtype)
    for name, value in PACK_FIELDS.items():
        out[f"{prefix}.{name}"] = torch.tensor(list(value), dtype=torch.int32)
    return out


def gpu_builder(bf16: torch.Tensor, fp8_u8: torch.Tensor, scales: torch.Tensor, max_len: int,
                threads: int) -> Dict[str, torch.Tensor]:
    """The GPU sidecar builder, through the MPServe_cuda op."""
    from mpserve_amd import mpserve_cuda

    return mpserve_cuda.huffman_build_fp8_decode_tables(bf16, fp8_u8, scales, max_len=max_len,
                                                        threads_per_block=threads)


# --------------------------------------------------------------------------- output
def mirror_tree(src: Path, dst: Path) -> int:
    """Give dst every file of src that it lacks: a hard link where the file system
    allows one, else a copy; the index and config.json are always copies, since
    they are rewritten. Returns the number of files added."""
    added = 0
    for here, _dirs, files in os.walk(src):
        target = dst / Path(here).relative_to(src)
        target.mkdir(parents=True, exist_ok=True)
        for name in files:
            a, b = Path(here) / name, target / name
            if b.exists():
                continue
            linked = False
            if name not in (INDEX, "config.json"):
                try:
                    os.link(a, b)
                    linked = True
                except OSError:
                    pass
            if not linked:
                shutil.copy2(a, b)
            added += 1
    for here, dirs, _files in os.walk(src):  # empty directories too
        for d in dirs:
            (dst / Path(here).relative_to(src) / d).mkdir(parents=True, exist_ok=True)
    return added


class SidecarStore:
    """Collects modules' stored tensors and writes them as one file, or as files
    of about ``shard_bytes`` each (``<stem>-00001.safetensors`` ...) written as
    soon as they fill."""

    def __init__(self, out_dir: Path, name: str, shard_bytes: int):
        self.out_dir, self.name, self.shard_bytes = out_dir, name, shard_bytes
        self._held: Dict[str, torch.Tensor] = {}
        self._held_bytes = 0
        self.files: List[str] = []
        self.where: Dict[str, str] = {}  # tensor key -> file

    def _next_name(self) -> str:
        stem, ext = os.path.splitext(self.name)
        return f"{stem}-{len(self.files) + 1:05d}{ext}"

    def _write(self, fname: str) -> None:
        from safetensors.torch import save_file

        save_file(self._held, str(self.out_dir / fname))
        say(f"wrote {fname}: {len(self._held)} tensors, {self._held_bytes / 1e6:.1f} MB")
        self.where.update(dict.fromkeys(self._held, fname))
        self.files.append(fname)
        self._held, self._held_bytes = {}, 0

    def add(self, tensors: Dict[str, torch.Tensor]) -> None:
        self._held.update(tensors)
        self._held_bytes += sum(t.numel() * t.element_size() for t in tensors.values())
        if 0 < self.shard_bytes <= self._held_bytes:
            self._write(self._next_name())

    def close(self) -> None:
        if self._held:
            self._write(self.name if self.shard_bytes <= 0 else self._next_name())


def build_sidecars(mods: List[Module], bf16: Checkpoint, fp8: Checkpoint, store: SidecarStore, args,
                   builder: Callable) -> int:
    for i, mod in enumerate(mods, 1):
        w = bf16.tensor(mod.weight_key).contiguous()
        n, m = int(w.shape[0]), int(w.shape[1])
        q = fp8_bytes(fp8.tensor(mod.weight_key), n, m).contiguous()
        s = scale_rows(scale_keys(fp8.tensor(mod.scale_key).contiguous()), n, m).contiguous()
        t0 = time.time()
        built = builder(w, q, s, int(args.max_len), int(args.threads))
        store.add(stored_tensors(mod.prefix, built, q, bool(args.store_fp8_u8)))
        say(f"[{i}/{len(mods)}] {mod.prefix} {n}x{m}: {int(built['bucket_table_i32'].shape[0])} buckets, "
            f"{int(built['decode_syms_u16'].shape[0])} tables ({time.time() - t0:.2f} s)")
    return len(mods)


def finish(out_dir: Path, bf16: Checkpoint, fp8: Checkpoint, store: SidecarStore, args) -> Path:
    """Point the index at the sidecar (and at the BF16 overrides), and mark
    config.json's quantization method. JSON is written as the reference writes
    it (2-space indent, sorted keys, no trailing newline)."""
    path = out_dir / INDEX
    with open(path, "r", encoding="utf-8") as f:
        idx = json.load(f)
    wm = idx.get("weight_map")
    if not isinstance(wm, dict):
        raise ValueError(f"{path}: weight_map is missing or not an object")
    wm.update(store.where)
    if args.override_common_from_bf16:
        allow = re.compile(args.override_allow_regex) if args.override_allow_regex else None
        both = sorted(set(bf16.index) & set(fp8.index))
        chosen = [k for k in both if allow is None or allow.search(k)]
        say(f"BF16 overrides: {len(chosen)} of the {len(both)} keys both checkpoints hold")
        if chosen:
            from safetensors.torch import save_file

            save_file({k: bf16.tensor(k) for k in chosen}, str(out_dir / OVERRIDES))
            wm.update(dict.fromkeys(chosen, OVERRIDES))
    idx["weight_map"] = wm
    with open(path, "w", encoding="utf-8") as f:
        json.dump(idx, f, indent=2, sort_keys=True)
    cfg = out_dir / "config.json"
    if cfg.exists():
        try:
            c = json.loads(cfg.read_text(encoding="utf-8"))
        except ValueError:
            c = None  # an unreadable config.json is left as it is
        if isinstance(c, dict):
            qc = c.get("quantization_config")
            qc = qc if isinstance(qc, dict) else {}
            qc["quant_method"] = "fp8_huffman"
            qc.setdefault("max_len", int(args.max_len))
            c["quantization_config"] = qc
            try:
                cfg.write_text(json.dumps(c, indent=2, sort_keys=True), encoding="utf-8")
            except OSError:
                say(f"{cfg}: could not be rewritten; left as it was")
    return path


def compress(args: argparse.Namespace, builder: Callable = gpu_builder) -> Dict[str, object]:
    """Run the four passes; returns {"modules", "keys", "files"}."""
    if int(args.max_len) != 7:
        raise SystemExit(f"--max_len {args.max_len}: the FP8 decode kernel only reads max_len 7 sidecars")
    for flag in ("bf16_model", "fp8_model"):
        if not Path(getattr(args, flag)).is_dir():
            raise SystemExit(f"--{flag} {getattr(args, flag)}: not a directory")
    out_dir = Path(args.out_dir)
    t0 = time.time()
    added = mirror_tree(Path(args.base_model or args.fp8_model), out_dir)
    say(f"mirrored the base model into {out_dir} ({added} files, {time.time() - t0:.1f} s)")
    bf16, fp8 = Checkpoint(Path(args.bf16_model)), Checkpoint(Path(args.fp8_model))
    sel = select_modules(bf16, fp8, args.include, args.exclude)
    say(f"{len(sel.modules)} modules to build; skipped: {dict(sel.skipped) or 'none'}")
    if not sel.modules:
        raise SystemExit("no module to build: " + ", ".join(f"{v} {k}" for k, v in sel.skipped.items()))
    store = SidecarStore(out_dir, str(args.sidecar_name), int(args.max_shard_gb * 1e9))
    build_sidecars(sel.modules, bf16, fp8, store, args, builder)
    store.close()
    index = finish(out_dir, bf16, fp8, store, args)
    say(f"done: {len(store.where)} sidecar tensors in {', '.join(store.files)}; index {index}")
    return {"modules": len(sel.modules), "keys": len(store.where), "files": list(store.files)}


def main(argv=None) -> int:
    compress(parse_args(argv))
    return 0


if __name__ == "__main__":
    sys.exit(main())
