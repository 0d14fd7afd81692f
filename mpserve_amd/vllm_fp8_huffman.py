"""vLLM quantization method ``fp8_huffman`` on ROCm / MI355X.

Keeps the reference plugin's surface (scripts/mpserve_vllm_fp8_huffman.py):
the registration name ``"fp8_huffman"`` (:95), ``FP8HuffmanConfig`` with its
``max_len`` / ``include_regex`` / ``ignore_regex`` keys and the
``MPSERVE_ENABLE_FP8_HUFFMAN=1`` gate (:98-148), and
``FP8HuffmanLinearMethod`` with the same thirteen ``huff_*`` parameters, the
discarded ``weight`` / ``weight_scale_inv`` / ``weight_scale`` parameters, the
three buffers and the shard-aware loaders (:155-360).

``apply()`` keeps the reference's result (BF16 weight rebuilt from FP8 bytes +
sidecar, then ``x @ W.T`` plus bias, :389-665) and changes how it gets there:

* every shard of a merged layer (qkv, gate_up) decodes straight into its row
  slice of one BF16 scratch weight, all shards in one launch of a
  ``DecodePlan`` (the reference decodes shard by shard into fresh tensors and
  concatenates them, :526-543);
* the scratch is a per-device pool keyed by weight size, shared by every layer
  of that size (two slots, so a prefetch of the next layer can overlap the
  current GEMM) instead of a fresh allocation per call;
* ``prefetch(layer)`` enqueues a layer's decode on a side stream; ``apply()``
  then waits on its event instead of decoding. Setting
  ``MPSERVE_FP8_HUFFMAN_CACHE=1`` keeps each layer's decoded weight resident
  (decode once, memory of a BF16 model).

Importing this module requires vLLM (as the reference's does); it registers
the method as a side effect.
"""
from __future__ import annotations

import os
import re
import weakref
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple, cast

import torch

from vllm.model_executor.layers.linear import LinearBase, LinearMethodBase  # noqa: E402
from vllm.model_executor.layers.linear import UnquantizedLinearMethod  # noqa: E402
from vllm.model_executor.layers.quantization import register_quantization_config  # noqa: E402
from vllm.model_executor.layers.quantization.base_config import (  # noqa: E402
    QuantizationConfig,
    QuantizeMethodBase,
)
from vllm.model_executor.parameter import BasevLLMParameter  # noqa: E402

# prefix -> layer, for the layer-pack path (a shard of a leader's packed weight)
_PREFIX_TO_LAYER: "weakref.WeakValueDictionary[str, torch.nn.Module]" = weakref.WeakValueDictionary()

# Parameters the compress script writes per module, with their stored dtypes
# (scripts/compress_llm_fp8_huffman.py:284-306; safetensors has no unsigned
# 16/32/64-bit types, so those are stored signed and viewed back at decode).
HUFF_PARAMS: Tuple[Tuple[str, torch.dtype], ...] = (
    ("huff_fp8_u8", torch.uint8),
    ("huff_bitstream_u64", torch.int64),
    ("huff_decode_syms_u16", torch.int16),
    ("huff_decode_lens_u8", torch.uint8),
    ("huff_bucket_table_i32", torch.int32),
    ("huff_bucket_col_start_i32", torch.int32),
    ("huff_bucket_col_len_i32", torch.int32),
    ("huff_bucket_row_offsets_i32", torch.int32),
    ("huff_row_indices_i32", torch.int32),
    ("huff_bucket_thread_startbit_u32", torch.int32),
    ("huff_bucket_bit_base_i64", torch.int64),
)
_PACK_PARAMS = ("huff_attn_block_row_start_i32", "huff_attn_block_row_len_i32")
# shard id -> row-block index of a merged layer (reference :176-184)
SHARD_INDEX: Dict[object, int] = {0: 0, 1: 1, "q": 0, "k": 1, "v": 2, "gate": 0, "up": 1}
DEFAULT_IGNORE = r"(^lm_head$|^model\.visual\.|.*\.mlp\.gate$|.*\.mlp\.shared_expert_gate$)"


@dataclass(frozen=True)
class FP8HuffmanParams:
    max_len: int = 7


@register_quantization_config("fp8_huffman")
class FP8HuffmanConfig(QuantizationConfig):
    """Config of the ``fp8_huffman`` method (reference :95-148)."""

    def __init__(self, *, max_len: int = 7, include_regex: str | None = None,
                 ignore_regex: str | None = DEFAULT_IGNORE) -> None:
        super().__init__()
        if int(max_len) != 7:
            raise ValueError("fp8_huffman currently requires max_len=7")
        self.params = FP8HuffmanParams(max_len=int(max_len))
        self.include_regex = include_regex
        self._include_re = re.compile(include_regex) if include_regex else None
        self.ignore_regex = ignore_regex
        self._ignore_re = re.compile(ignore_regex) if ignore_regex else None
        self._enabled = os.environ.get("MPSERVE_ENABLE_FP8_HUFFMAN", "0") == "1"

    def get_name(self) -> str:
        return "fp8_huffman"

    def get_supported_act_dtypes(self) -> List[torch.dtype]:
        return [torch.half, torch.bfloat16]

    @classmethod
    def get_min_capability(cls) -> int:
        # The reference asks for 90 (H100). ROCm reports gfx942 as 94 and gfx950 as 95.
        return 90

    @staticmethod
    def get_config_filenames() -> List[str]:
        return []

    @classmethod
    def from_config(cls, config: dict) -> "FP8HuffmanConfig":
        return cls(max_len=int(config.get("max_len", 7)), include_regex=config.get("include_regex", None),
                   ignore_regex=config.get("ignore_regex", None))

    def get_quant_method(self, layer: torch.nn.Module, prefix: str) -> Optional[QuantizeMethodBase]:
        if not self._enabled:
            return UnquantizedLinearMethod()
        if isinstance(layer, LinearBase):
            if self._ignore_re is not None and self._ignore_re.search(prefix) is not None:
                return UnquantizedLinearMethod()
            if self._include_re is None or self._include_re.search(prefix) is not None:
                return FP8HuffmanLinearMethod(self.params)
            return UnquantizedLinearMethod()
        return None


class _ScratchPool:
    """BF16 scratch weights per (device, numel, slot), reused by every layer of that size."""

    def __init__(self) -> None:
        self._bufs: Dict[Tuple[int, int, int], torch.Tensor] = {}

    def get(self, device: torch.device, numel: int, slot: int) -> torch.Tensor:
        key = (device.index if device.index is not None else torch.cuda.current_device(), int(numel), int(slot))
        buf = self._bufs.get(key)
        if buf is None:
            buf = torch.empty(int(numel), dtype=torch.bfloat16, device=device)
            self._bufs[key] = buf
        return buf

    def clear(self) -> None:
        self._bufs.clear()


SCRATCH = _ScratchPool()


def _as_tensor(x: Any) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x
    return cast(torch.Tensor, cast(Any, x)[:])


class FP8HuffmanLinearMethod(LinearMethodBase):
    """Linear method that rebuilds BF16 weights from FP8 + Huffman sidecar (reference :151-665)."""

    def __init__(self, params: FP8HuffmanParams):
        self.params = params

    # ------------------------------------------------------------------ weights
    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: List[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs) -> None:
        tp_rank = getattr(layer, "tp_rank", 0)
        tp_size = getattr(layer, "tp_size", 1)
        if int(tp_rank) != 0 or int(tp_size) != 1:
            raise NotImplementedError("fp8_huffman MVP only supports tp_size=1")
        num_shards = int(len(output_partition_sizes))
        device = torch.device("cuda" if torch.cuda.is_available() else "cpu")

        def _discard_loader(param: torch.Tensor, loaded_weight: torch.Tensor, *args, **kwargs) -> None:
            return

        def _make_loader(attr_name: str):
            def _loader(param: torch.Tensor, loaded_weight: torch.Tensor, shard_id: object | None = None,
                        *args, **kwargs) -> None:
                tgt = _as_tensor(loaded_weight).to(device=param.device).contiguous()
                if num_shards <= 1 or shard_id is None:
                    if int(tgt.numel()) >= int(param.data.numel()):
                        param.data = tgt
                    return
                idx = SHARD_INDEX.get(shard_id, None)
                if idx is None:
                    raise ValueError(f"Unknown shard_id for fp8_huffman: {shard_id!r}")
                shards = getattr(layer, f"_{attr_name}_shards", None)
                if shards is None:
                    shards = {}
                    setattr(layer, f"_{attr_name}_shards", shards)
                shards[int(idx)] = tgt
            return _loader

        for name, dtype in HUFF_PARAMS:
            layer.register_parameter(name, BasevLLMParameter(data=torch.empty((1,), dtype=dtype, device=device),
                                                             weight_loader=_make_loader(name)))
        for name in _PACK_PARAMS:
            layer.register_parameter(name, BasevLLMParameter(data=torch.zeros((0,), dtype=torch.int32, device=device),
                                                             weight_loader=_make_loader(name)))
        layer.register_parameter("weight", BasevLLMParameter(data=torch.empty((1,), dtype=torch.uint8, device=device),
                                                             weight_loader=_discard_loader))
        for name in ("weight_scale_inv", "weight_scale"):
            layer.register_parameter(name, BasevLLMParameter(
                data=torch.empty((1,), dtype=torch.float16, device=device), weight_loader=_discard_loader))
        layer.register_buffer("huff_max_len", torch.tensor(int(self.params.max_len), dtype=torch.int32, device=device),
                              persistent=False)
        layer.register_buffer("huff_in_features_i32", torch.tensor(int(input_size), dtype=torch.int32, device=device),
                              persistent=False)
        layer.register_buffer("huff_out_features_i32",
                              torch.tensor(int(output_size), dtype=torch.int32, device=device), persistent=False)

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        for name in [n for n, _ in HUFF_PARAMS] + list(_PACK_PARAMS):
            p = getattr(layer, name)
            if not isinstance(p, torch.nn.Parameter):
                setattr(layer, name, torch.nn.Parameter(p, requires_grad=False))
        prefix = getattr(layer, "prefix", None)
        if isinstance(prefix, str) and prefix:
            _PREFIX_TO_LAYER[prefix] = layer
        layer._fp8_huff_state = {}

    # ------------------------------------------------------------------ decode
    @staticmethod
    def _shards(layer: torch.nn.Module) -> List[Dict[str, torch.Tensor]]:
        """The layer's sidecars in row order: [{param name: tensor}] (one entry unless merged)."""
        per = getattr(layer, "_huff_fp8_u8_shards", None)
        if isinstance(per, dict) and per:
            order = sorted(per.keys())
            out = [{name: getattr(layer, f"_{name}_shards")[i] for name, _ in HUFF_PARAMS} for i in order]
            if any(int(s["huff_fp8_u8"].numel()) == 0 for s in out):
                # the reference falls back to the largest shard when one is empty (:495-524)
                best = max(out, key=lambda s: int(s["huff_fp8_u8"].numel()))
                if int(best["huff_fp8_u8"].numel()) <= 0:
                    raise RuntimeError("fp8_huffman: all shard sidecars are empty")
                return [best]
            return out
        return [{name: getattr(layer, name) for name, _ in HUFF_PARAMS}]

    @staticmethod
    def _fp8_2d(t: torch.Tensor, m_in: int) -> torch.Tensor:
        if t.numel() == 0:
            raise RuntimeError(f"fp8_huffman: encountered empty fp8_u8 tensor (shape={tuple(t.shape)}). "
                               "This usually indicates missing/incorrect shard_id remapping during weight loading.")
        if t.dim() == 2:
            return t
        if t.dim() == 1:
            if m_in <= 0 or t.numel() % m_in != 0:
                raise ValueError(f"fp8_huffman: invalid fp8_u8 flat shape={tuple(t.shape)} for m_in={m_in}")
            return t.view(-1, m_in)
        raise ValueError(f"fp8_huffman: invalid fp8_u8 dim={t.dim()} shape={tuple(t.shape)}")

    def _plan(self, layer: torch.nn.Module, m_in: int, slot: int):
        """(DecodePlan, BF16 [N, K] weight view) decoding every shard into its row slice."""
        from .decode import DecodePlan

        state = layer.__dict__.setdefault("_fp8_huff_state", {})
        cached = state.get(("plan", slot))
        if cached is not None:
            return cached
        shards = self._shards(layer)
        fp8s = [self._fp8_2d(s["huff_fp8_u8"], m_in) for s in shards]
        k = int(fp8s[0].shape[1])
        if any(int(f.shape[1]) != k for f in fp8s):
            raise ValueError("fp8_huffman: shards of one layer must share the input dimension")
        n_total = sum(int(f.shape[0]) for f in fp8s)
        device = fp8s[0].device
        if os.environ.get("MPSERVE_FP8_HUFFMAN_CACHE", "0") == "1":
            flat = torch.empty(n_total * k, dtype=torch.bfloat16, device=device)
        else:
            flat = SCRATCH.get(device, n_total * k, slot)
        items = []
        row = 0
        for f, s in zip(fp8s, shards):
            n = int(f.shape[0])
            items.append((f.contiguous(), s, flat[row * k:(row + n) * k]))
            row += n
        plan = DecodePlan(items)
        weight = flat.view(n_total, k)
        state[("plan", slot)] = (plan, weight)
        return plan, weight

    def decoded_weight(self, layer: torch.nn.Module, m_in: int, slot: int = 0,
                       stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """Enqueue the layer's decode on ``stream`` (default: current) and return the BF16 [N, K] weight."""
        plan, weight = self._plan(layer, m_in, slot)
        state = layer.__dict__.setdefault("_fp8_huff_state", {})
        if os.environ.get("MPSERVE_FP8_HUFFMAN_CACHE", "0") == "1" and state.get("decoded"):
            return weight
        plan.decode(stream)
        state["decoded"] = True
        return weight

    def prefetch(self, layer: torch.nn.Module, m_in: int, stream: torch.cuda.Stream, slot: int = 1) -> None:
        """Decode ``layer`` on ``stream`` into scratch ``slot``; its next ``apply()`` waits for it.

        The caller keeps ``slot`` apart from the scratch a running GEMM reads (alternate
        slots between consecutive layers of one size).
        """
        weight = self.decoded_weight(layer, m_in, slot=slot, stream=stream)
        ev = torch.cuda.Event()
        ev.record(stream)
        layer.__dict__.setdefault("_fp8_huff_state", {})["pending"] = (ev, weight)

    # ------------------------------------------------------------------ apply
    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        if not x.is_cuda:
            raise ValueError("fp8_huffman requires CUDA tensors")
        if x.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("fp8_huffman expects activations in bf16 or fp16")
        if x.numel() == 0:
            out_features = 0
            if hasattr(layer, "huff_out_features_i32"):
                out_features = int(getattr(layer, "huff_out_features_i32").item())
            if out_features <= 0 and hasattr(layer, "output_size"):
                out_features = int(getattr(layer, "output_size"))
            if out_features <= 0:
                raise RuntimeError("fp8_huffman: cannot infer out_features for empty-token run "
                                   f"(prefix={getattr(layer, 'prefix', None)!r}, "
                                   f"layer_type={type(layer).__name__})")
            out = torch.empty(x.shape[:-1] + (out_features,), dtype=x.dtype, device=x.device)
            if bias is not None and out.numel() > 0:
                out.add_(bias)
            return out

        x2d = x.reshape(-1, x.shape[-1])
        m_in = int(x2d.shape[1])
        w = self._packed_weight(layer, m_in)
        if w is None:
            state = layer.__dict__.setdefault("_fp8_huff_state", {})
            pending = state.pop("pending", None)
            if pending is not None:
                ev, w = pending
                torch.cuda.current_stream(x.device).wait_event(ev)
            else:
                w = self.decoded_weight(layer, m_in, slot=0)
        if x.dtype == torch.float16 and w.dtype != torch.float16:
            w = w.to(torch.float16)
        out = torch.matmul(x2d, w.t())
        if bias is not None:
            out.add_(bias)
        return out.reshape(x.shape[:-1] + (out.shape[-1],))

    # The layer-pack path (reference :559-655): a layer whose huff_attn_block_*
    # metadata is non-empty is a row slice of its layer's leader (o_proj).
    @staticmethod
    def _pack_meta(layer: torch.nn.Module) -> Optional[Tuple[int, int]]:
        d_rs = getattr(layer, "_huff_attn_block_row_start_i32_shards", None)
        d_rl = getattr(layer, "_huff_attn_block_row_len_i32_shards", None)
        if isinstance(d_rs, dict) and isinstance(d_rl, dict) and d_rs:
            spans = []
            for si, rs in d_rs.items():
                rl = d_rl.get(si)
                if isinstance(rs, torch.Tensor) and isinstance(rl, torch.Tensor) and rs.numel() and rl.numel():
                    s, ln = int(rs.reshape(-1)[0].item()), int(rl.reshape(-1)[0].item())
                    if ln > 0:
                        spans.append((s, s + ln))
            if spans:
                lo, hi = min(a for a, _ in spans), max(b for _, b in spans)
                return (lo, hi - lo) if hi > lo else None
        rs = getattr(layer, "huff_attn_block_row_start_i32", None)
        rl = getattr(layer, "huff_attn_block_row_len_i32", None)
        if isinstance(rs, torch.Tensor) and isinstance(rl, torch.Tensor) and rs.numel() and rl.numel():
            s, ln = int(rs.reshape(-1)[0].item()), int(rl.reshape(-1)[0].item())
            if ln > 0:
                return s, ln
        return None

    def _packed_weight(self, layer: torch.nn.Module, m_in: int) -> Optional[torch.Tensor]:
        meta = self._pack_meta(layer)
        if meta is None:
            return None
        prefix = getattr(layer, "prefix", None)
        if not isinstance(prefix, str) or not prefix:
            return None
        if ".self_attn." in prefix:
            leader_prefix = prefix.split(".self_attn.", 1)[0] + ".self_attn.o_proj"
        elif ".mlp." in prefix:
            leader_prefix = prefix.split(".mlp.", 1)[0] + ".self_attn.o_proj"
        else:
            return None
        leader = _PREFIX_TO_LAYER.get(leader_prefix, None)
        if leader is None:
            raise RuntimeError(f"fp8_huffman: cannot find layer-pack leader {leader_prefix!r} for {prefix!r}")
        method = getattr(leader, "quant_method", None)
        method = method if isinstance(method, FP8HuffmanLinearMethod) else self
        w_full = method.decoded_weight(leader, m_in, slot=0)
        row_start, row_len = meta
        return w_full[row_start:row_start + row_len]
