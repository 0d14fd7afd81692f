"""vLLM quantization method ``fp8_huffman`` on ROCm / MI355X.

The surface vLLM sees is the reference plugin's
(scripts/mpserve_vllm_fp8_huffman.py): the registration name
``"fp8_huffman"`` (:95), ``FP8HuffmanConfig`` with its ``max_len`` /
``include_regex`` / ``ignore_regex`` keys and the
``MPSERVE_ENABLE_FP8_HUFFMAN=1`` gate (:98-148), and
``FP8HuffmanLinearMethod`` with the same thirteen ``huff_*`` parameters, the
discarded ``weight`` / ``weight_scale_inv`` / ``weight_scale`` parameters, the
three buffers and the shard map of merged layers (:155-360). ``apply()``
returns what the reference's does (:389-665): ``x @ W.T`` (+ bias) for the BF16
weight W rebuilt bit-exact from FP8 bytes + sidecar.

How it gets there is this build's own:

* Loading keeps each shard's sidecar tensors per shard index; at
  ``process_weights_after_loading`` every layer gets a ``_LayerDecode``: the
  sidecars in row order, their layer-pack rows (if any), and one
  ``DecodePlan`` that decodes every shard straight into its row slice of one
  BF16 weight buffer (one launch; the reference decodes shard by shard into
  fresh tensors and concatenates them, :526-543). Plan creation happens there,
  after loading: it synchronises the current stream once and allocates; a
  forward pass then only launches.
* The weight buffer is a scratch slot shared by every layer of the same size
  (``ScratchPool``); plans are relocatable, so slot 1 serves ``prefetch()``,
  which decodes the next layer on a side stream while the current GEMM runs.
  ``MPSERVE_FP8_HUFFMAN_CACHE=1`` instead gives each layer its own buffer,
  decoded once at load time (the memory of a BF16 model, no decode per step).
* A layer of a packed attention/MLP block (non-empty
  ``huff_attn_block_row_*``) multiplies by its row slice of its leader's
  (the block's ``o_proj``) decoded weight, as the reference does (:559-655);
  the leader itself, when it carries pack rows, multiplies by its own slice.
  The leader's weight is decoded at most once per forward pass for the whole
  block: the scratch pool records which layer's weight each buffer holds (and
  in which graph capture and vLLM forward context it was written), and the
  block's later layers reuse it (the reference caches it per forward context,
  :559-577).

Importing this module requires vLLM (as the reference's does); it registers
the method as a side effect.
"""
from __future__ import annotations

import ctypes
import os
import re
import weakref
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

from vllm.model_executor.layers.linear import LinearBase, LinearMethodBase  # noqa: E402
from vllm.model_executor.layers.linear import UnquantizedLinearMethod  # noqa: E402
from vllm.model_executor.layers.quantization import register_quantization_config  # noqa: E402
from vllm.model_executor.layers.quantization.base_config import (  # noqa: E402
    QuantizationConfig,
    QuantizeMethodBase,
)
from vllm.model_executor.parameter import BasevLLMParameter  # noqa: E402

ENV_ENABLE = "MPSERVE_ENABLE_FP8_HUFFMAN"
ENV_CACHE = "MPSERVE_FP8_HUFFMAN_CACHE"

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
PACK_PARAMS = ("huff_attn_block_row_start_i32", "huff_attn_block_row_len_i32")
# shard id -> row-block index of a merged layer (reference :176-184)
SHARD_INDEX: Dict[object, int] = {0: 0, 1: 1, "q": 0, "k": 1, "v": 2, "gate": 0, "up": 1}
# the reference's default ignore list (:105)
DEFAULT_IGNORE = r"(^lm_head$|^model\.visual\.|.*\.mlp\.gate$|.*\.mlp\.shared_expert_gate$)"

# prefix -> layer, so that a packed layer finds its block's leader
_LAYERS_BY_PREFIX: "weakref.WeakValueDictionary[str, torch.nn.Module]" = weakref.WeakValueDictionary()


@dataclass(frozen=True)
class FP8HuffmanParams:
    max_len: int = 7


class _PrefixFilter:
    """Which linear layers the method takes: none on the ignore list; of the
    rest, all when there is no include pattern, else those it matches."""

    def __init__(self, include: Optional[str], ignore: Optional[str]):
        self._include = re.compile(include) if include else None
        self._ignore = re.compile(ignore) if ignore else None

    def accepts(self, prefix: str) -> bool:
        if self._ignore is not None and self._ignore.search(prefix):
            return False
        return self._include is None or self._include.search(prefix) is not None


@register_quantization_config("fp8_huffman")
class FP8HuffmanConfig(QuantizationConfig):
    """Config of the ``fp8_huffman`` method (reference :95-148)."""

    # config.json keys and their defaults (from_config)
    _KEYS = (("max_len", 7), ("include_regex", None), ("ignore_regex", None))

    def __init__(self, *, max_len: int = 7, include_regex: str | None = None,
                 ignore_regex: str | None = DEFAULT_IGNORE) -> None:
        super().__init__()
        if int(max_len) != 7:
            raise ValueError("fp8_huffman currently requires max_len=7")
        self.params = FP8HuffmanParams(max_len=int(max_len))
        self.include_regex = include_regex
        self.ignore_regex = ignore_regex
        self._filter = _PrefixFilter(include_regex, ignore_regex)
        self._enabled = os.environ.get(ENV_ENABLE, "0") == "1"

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
        kw = {k: config.get(k, d) for k, d in cls._KEYS}
        kw["max_len"] = int(kw["max_len"])
        return cls(**kw)

    def get_quant_method(self, layer: torch.nn.Module, prefix: str) -> Optional[QuantizeMethodBase]:
        # gate off: every layer stays unquantized (the reference returns that for any layer)
        if not self._enabled:
            return UnquantizedLinearMethod()
        if not isinstance(layer, LinearBase):
            return None
        if self._filter.accepts(prefix):
            return FP8HuffmanLinearMethod(self.params)
        return UnquantizedLinearMethod()


class ScratchPool:
    """BF16 weight buffers keyed by (device, elements, slot), shared by every
    layer of that size: slot 0 is the weight apply() multiplies by, slot 1 the
    one prefetch() fills for the next layer.

    It also records, per buffer, the token of the last decode enqueued into it
    (the layer's state, the capture id of the stream, the vLLM forward
    context), so that a packed block's layers can reuse their leader's decoded
    weight while nothing else has been decoded into that buffer since."""

    def __init__(self) -> None:
        self._bufs: Dict[Tuple[int, int, int], torch.Tensor] = {}
        self._owner: Dict[int, tuple] = {}

    @staticmethod
    def _key(device: torch.device, numel: int, slot: int) -> Tuple[int, int, int]:
        return (device.index if device.index is not None else torch.cuda.current_device(), int(numel), int(slot))

    def get(self, device: torch.device, numel: int, slot: int) -> torch.Tensor:
        key = self._key(device, numel, slot)
        buf = self._bufs.get(key)
        if buf is None:
            buf = self._bufs[key] = torch.empty(int(numel), dtype=torch.bfloat16, device=device)
        return buf

    def existing(self, device: torch.device, numel: int, slot: int) -> Optional[torch.Tensor]:
        return self._bufs.get(self._key(device, numel, slot))

    def mark(self, buf: torch.Tensor, token: tuple) -> None:
        """A decode with ``token`` was just enqueued into ``buf``."""
        self._owner[buf.data_ptr()] = token

    def holds(self, buf: torch.Tensor, token: tuple) -> bool:
        """Whether the last decode enqueued into ``buf`` carried ``token`` (objects
        compared by identity, integers by value)."""
        t = self._owner.get(buf.data_ptr())
        return t is not None and len(t) == len(token) and all(
            a is b or (type(a) is int and type(b) is int and a == b) for a, b in zip(t, token))

    def clear(self) -> None:
        self._bufs.clear()
        self._owner.clear()


SCRATCH = ScratchPool()


class _HuffParamLoader:
    """weight_loader of one ``huff_*`` parameter.

    A lazily loaded tensor (one that materialises on ``[:]``) is read and moved
    to the parameter's device. Without a shard id (or for an unmerged layer) it
    replaces the parameter's data, unless it is smaller than the placeholder.
    With one, it is kept as that shard's array in the layer's
    ``_fp8_huff_shards[row block][name]``; the reference keeps the same arrays
    per parameter name (:200-229).
    """

    def __init__(self, layer: torch.nn.Module, name: str, merged: bool):
        self.layer_ref = weakref.ref(layer)
        self.name = name
        self.merged = merged

    def __call__(self, param: torch.Tensor, loaded_weight, shard_id: object | None = None, *args, **kwargs) -> None:
        src = loaded_weight if isinstance(loaded_weight, torch.Tensor) else loaded_weight[:]
        t = src.to(device=param.device).contiguous()
        if not self.merged or shard_id is None:
            if t.numel() >= param.data.numel():
                param.data = t
            return
        if shard_id not in SHARD_INDEX:
            raise ValueError(f"Unknown shard_id for fp8_huffman: {shard_id!r}")
        layer = self.layer_ref()
        layer.__dict__.setdefault("_fp8_huff_shards", {}).setdefault(SHARD_INDEX[shard_id], {})[self.name] = t


def _discard(param: torch.Tensor, loaded_weight, *args, **kwargs) -> None:
    """weight_loader of the checkpoint's FP8 weight and scales: the sidecar carries them."""


@dataclass(eq=False)
class _LayerDecode:
    """What a layer needs at apply(): set up once, by process_weights_after_loading."""
    out_features: int
    in_features: int
    pack: Optional[Tuple[int, int]] = None           # (first row, rows) in the block leader's weight
    leader: Optional[str] = None                     # the block leader's prefix, when packed
    plan: Optional[object] = None                    # DecodePlan into `weight`'s buffer
    weight: Optional[torch.Tensor] = None            # BF16 [N, K] the plan decodes into
    cached: bool = False                             # weight decoded once, kept
    pending: Optional[Tuple[torch.cuda.Event, torch.Tensor]] = None  # a prefetch's (event, weight)
    extra: Dict[str, object] = field(default_factory=dict)


def _as_2d(fp8: torch.Tensor, k: int) -> torch.Tensor:
    """A shard's FP8 bytes as [rows, k]: stored 2-D, or flat with a multiple of k bytes."""
    if fp8.numel() == 0:
        raise RuntimeError(f"fp8_huffman: a shard's huff_fp8_u8 is empty (shape {tuple(fp8.shape)}): "
                           "its sidecar was not loaded (is the shard id mapped?)")
    if fp8.dim() == 2:
        return fp8
    if fp8.dim() == 1 and k > 0 and fp8.numel() % k == 0:
        return fp8.view(-1, k)
    raise ValueError(f"fp8_huffman: huff_fp8_u8 of shape {tuple(fp8.shape)} does not hold rows of {k} bytes")


def _capture_id(device: torch.device) -> int:
    """Id of the graph capture the current stream is in (0: not capturing)."""
    if not torch.cuda.is_current_stream_capturing():
        return 0
    from . import _native

    v = ctypes.c_uint64(0)
    h = torch.cuda.current_stream(device).cuda_stream
    _native.check(_native.lib().mps_stream_capture_id(ctypes.c_void_p(h), ctypes.byref(v)))
    return int(v.value)


def _forward_context() -> object:
    """vLLM's current forward context object, or None outside one (or without
    vllm.forward_context): a new object per forward pass."""
    try:
        from vllm.forward_context import get_forward_context, is_forward_context_available
    except Exception:
        return None
    try:
        return get_forward_context() if is_forward_context_available() else None
    except Exception:
        return None


def _leader_prefix(prefix: object) -> Optional[str]:
    """The block leader of a layer: ``<block>.self_attn.o_proj`` for a layer of
    an attention or MLP block, else None (reference :579-587)."""
    if not isinstance(prefix, str) or not prefix:
        return None
    for part in (".self_attn.", ".mlp."):
        if part in prefix:
            return prefix.split(part, 1)[0] + ".self_attn.o_proj"
    return None


def _first_int(t: Optional[torch.Tensor]) -> Optional[int]:
    if isinstance(t, torch.Tensor) and t.numel() > 0:
        return int(t.reshape(-1)[0].item())
    return None


class FP8HuffmanLinearMethod(LinearMethodBase):
    """Linear method that rebuilds BF16 weights from FP8 + Huffman sidecar (reference :151-665)."""

    def __init__(self, params: FP8HuffmanParams):
        self.params = params

    # ------------------------------------------------------------------ weights
    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: List[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs) -> None:
        if int(getattr(layer, "tp_rank", 0)) != 0 or int(getattr(layer, "tp_size", 1)) != 1:
            raise NotImplementedError("fp8_huffman MVP only supports tp_size=1")
        device = torch.device("cuda" if torch.cuda.is_available() else "cpu")
        merged = len(output_partition_sizes) > 1

        def param(data: torch.Tensor, loader) -> BasevLLMParameter:
            return BasevLLMParameter(data=data, weight_loader=loader)

        for name, dtype in HUFF_PARAMS:
            layer.register_parameter(name, param(torch.empty((1,), dtype=dtype, device=device),
                                                 _HuffParamLoader(layer, name, merged)))
        for name in PACK_PARAMS:
            layer.register_parameter(name, param(torch.zeros((0,), dtype=torch.int32, device=device),
                                                 _HuffParamLoader(layer, name, merged)))
        layer.register_parameter("weight", param(torch.empty((1,), dtype=torch.uint8, device=device), _discard))
        for name in ("weight_scale_inv", "weight_scale"):
            layer.register_parameter(name, param(torch.empty((1,), dtype=torch.float16, device=device), _discard))
        for name, value in (("huff_max_len", self.params.max_len), ("huff_in_features_i32", input_size),
                            ("huff_out_features_i32", output_size)):
            layer.register_buffer(name, torch.tensor(int(value), dtype=torch.int32, device=device), persistent=False)
        layer._fp8_huff_sizes = (int(output_size), int(input_size))

    # ------------------------------------------------------------------ after loading
    @staticmethod
    def _sidecars(layer: torch.nn.Module) -> List[Dict[str, torch.Tensor]]:
        """The layer's sidecars in row order (one unless merged). When a shard's
        FP8 bytes are empty the reference decodes only the largest shard
        (:495-524); so does this."""
        per = layer.__dict__.get("_fp8_huff_shards")
        if not per:
            return [{name: getattr(layer, name).data for name, _ in HUFF_PARAMS}]
        shards = [per[i] for i in sorted(per)]
        sizes = [int(s["huff_fp8_u8"].numel()) if "huff_fp8_u8" in s else 0 for s in shards]
        if min(sizes) > 0:
            return shards
        if max(sizes) <= 0:
            raise RuntimeError("fp8_huffman: all shard sidecars are empty")
        return [shards[sizes.index(max(sizes))]]

    @staticmethod
    def _pack_rows(layer: torch.nn.Module) -> Optional[Tuple[int, int]]:
        """The layer's rows (first, count) in its block leader's weight, when it is
        part of a packed block: the span of its shards' row ranges, or its own."""
        spans = []
        for shard in (layer.__dict__.get("_fp8_huff_shards") or {}).values():
            start = _first_int(shard.get(PACK_PARAMS[0]))
            rows = _first_int(shard.get(PACK_PARAMS[1]))
            if start is not None and rows is not None and rows > 0:
                spans.append((start, start + rows))
        if not spans:
            start = _first_int(getattr(layer, PACK_PARAMS[0], None))
            rows = _first_int(getattr(layer, PACK_PARAMS[1], None))
            if start is not None and rows is not None and rows > 0:
                spans.append((start, start + rows))
        if not spans:
            return None
        lo, hi = min(a for a, _ in spans), max(b for _, b in spans)
        return (lo, hi - lo) if hi > lo else None

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        from .decode import DecodePlan

        for name in [n for n, _ in HUFF_PARAMS] + list(PACK_PARAMS):
            p = getattr(layer, name)
            if not isinstance(p, torch.nn.Parameter):
                setattr(layer, name, torch.nn.Parameter(p, requires_grad=False))
        prefix = getattr(layer, "prefix", None)
        if isinstance(prefix, str) and prefix:
            _LAYERS_BY_PREFIX[prefix] = layer
        out_features, in_features = getattr(layer, "_fp8_huff_sizes", (0, 0))
        pack = self._pack_rows(layer)
        # Pack rows count only inside an attention or MLP block, whose leader is
        # its o_proj; elsewhere the reference decodes the layer's own sidecar (:609-629).
        leader = _leader_prefix(prefix) if pack is not None else None
        st = _LayerDecode(out_features=out_features, in_features=in_features,
                          pack=pack if leader is not None else None, leader=leader)
        layer._fp8_huff = st
        if leader is not None and leader != prefix:
            return  # a member of a packed block: decoded through its leader
        sidecars = self._sidecars(layer)
        fp8s = [_as_2d(s["huff_fp8_u8"], in_features) for s in sidecars]
        if not fp8s[0].is_cuda:
            return  # no GPU: the layer loads, and apply() (CUDA only) reports it
        k = int(fp8s[0].shape[1])
        if any(int(f.shape[1]) != k for f in fp8s):
            raise ValueError("fp8_huffman: the shards of one layer must share the input dimension")
        rows = sum(int(f.shape[0]) for f in fp8s)
        device = fp8s[0].device
        st.cached = os.environ.get(ENV_CACHE, "0") == "1"
        flat = (torch.empty(rows * k, dtype=torch.bfloat16, device=device) if st.cached
                else SCRATCH.get(device, rows * k, 0))
        items, row = [], 0
        for f, s in zip(fp8s, sidecars):
            n = int(f.shape[0])
            items.append((f.contiguous(), s, flat[row * k:(row + n) * k]))
            row += n
        st.plan = DecodePlan(items)  # synchronises the current stream once; allocates the plan
        st.weight = flat.view(rows, k)
        if st.cached:
            st.plan.decode()

    # ------------------------------------------------------------------ decode
    @staticmethod
    def _state(layer: torch.nn.Module) -> _LayerDecode:
        st = layer.__dict__.get("_fp8_huff")
        if st is None:
            raise RuntimeError(f"fp8_huffman: process_weights_after_loading has not run for "
                               f"{getattr(layer, 'prefix', type(layer).__name__)!r}")
        return st

    def _token(self, st: _LayerDecode) -> tuple:
        return (st, _capture_id(st.weight.device), _forward_context())

    def decoded_weight(self, layer: torch.nn.Module, m_in: Optional[int] = None, slot: int = 0,
                       stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """The layer's BF16 [N, K] weight (for a packed block's leader, the whole
        block's), its decode enqueued on ``stream`` (default: current) into
        scratch ``slot`` (or the layer's own buffer in cache mode, decoded once).

        Launches of a layer's plan on different streams may overlap: the plan
        gives each stream its own work queue, and a graph replays with the
        queue of the stream it was captured on. What they write is the caller's
        to order: two decodes into one slot on two streams, or a decode into the
        slot a GEMM on another stream still reads, race."""
        st = self._state(layer)
        if st.plan is None:
            if st.leader is not None and st.leader != getattr(layer, "prefix", None):
                raise RuntimeError("fp8_huffman: a packed layer's weight is its leader's (see apply)")
            raise RuntimeError("fp8_huffman: the layer's sidecar is not on a GPU")
        if st.cached:
            return st.weight
        s = stream if stream is not None else torch.cuda.current_stream(st.weight.device)
        if slot == 0:
            st.plan.decode(s)
            out = st.weight
        else:
            buf = SCRATCH.get(st.weight.device, st.weight.numel(), slot)
            st.plan.decode_into(buf, s)
            out = buf.view(st.weight.shape)
        SCRATCH.mark(out, self._token(st))
        return out

    def prefetch(self, layer: torch.nn.Module, m_in: Optional[int] = None, stream: Optional[torch.cuda.Stream] = None,
                 slot: int = 1) -> None:
        """Decode ``layer`` on ``stream`` into scratch ``slot``; its next ``apply()``
        waits for that decode instead of decoding. The caller keeps ``slot`` apart
        from the scratch a running GEMM reads (alternate slots between consecutive
        layers of one size). The first prefetch into a slot of a new size
        allocates that slot."""
        st = self._state(layer)
        w = self.decoded_weight(layer, slot=slot, stream=stream)
        ev = torch.cuda.Event()
        ev.record(stream if stream is not None else torch.cuda.current_stream(w.device))
        st.pending = (ev, w)

    def _take_pending(self, st: _LayerDecode) -> Optional[torch.Tensor]:
        """A prefetched weight, once the current stream waits for its decode."""
        if st.pending is None:
            return None
        ev, w = st.pending
        st.pending = None
        torch.cuda.current_stream(w.device).wait_event(ev)
        return w

    def _block_weight(self, leader: torch.nn.Module) -> torch.Tensor:
        """A packed block's decoded weight: its leader's, decoded at most once per
        forward pass (the reference's forward-context cache, :559-577). It is
        reused while the scratch buffer that holds it has had nothing else
        decoded into it, in the same graph capture (or none) and the same vLLM
        forward context."""
        st = self._state(leader)
        if st.plan is None:
            raise RuntimeError(f"fp8_huffman: the layer-pack leader {getattr(leader, 'prefix', None)!r} "
                               "has no decoded weight (its sidecar is not on a GPU)")
        if st.cached:
            return st.weight
        w = self._take_pending(st)
        if w is not None:
            return w
        token = self._token(st)
        for slot in (0, 1):
            buf = st.weight if slot == 0 else SCRATCH.existing(st.weight.device, st.weight.numel(), slot)
            if buf is not None and SCRATCH.holds(buf, token):
                return buf.view(st.weight.shape)
        return self.decoded_weight(leader)

    def _leader_weight(self, layer: torch.nn.Module, st: _LayerDecode) -> torch.Tensor:
        """A packed layer's rows of its block leader's (``<block>.self_attn.o_proj``)
        weight; the leader's own rows when the layer is the leader."""
        prefix = getattr(layer, "prefix", "") or ""
        if st.leader == prefix:
            leader, method = layer, self
        else:
            leader = _LAYERS_BY_PREFIX.get(st.leader)
            if leader is None:
                raise RuntimeError(f"fp8_huffman: cannot find layer-pack leader {st.leader!r} for {prefix!r}")
            method = getattr(leader, "quant_method", None)
            method = method if isinstance(method, FP8HuffmanLinearMethod) else self
        w_full = method._block_weight(leader)
        start, rows = st.pack
        return w_full[start:start + rows]

    def _weight_for_apply(self, layer: torch.nn.Module) -> torch.Tensor:
        st = self._state(layer)
        if st.pack is not None:
            return self._leader_weight(layer, st)
        w = self._take_pending(st)
        return w if w is not None else self.decoded_weight(layer)

    # ------------------------------------------------------------------ apply
    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        if not x.is_cuda:
            raise ValueError("fp8_huffman requires CUDA tensors")
        if x.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("fp8_huffman expects activations in bf16 or fp16")
        st = self._state(layer)
        if x.numel() == 0:
            n_out = st.out_features or int(getattr(layer, "output_size", 0) or 0)
            if n_out <= 0:
                raise RuntimeError(f"fp8_huffman: no output size known for {getattr(layer, 'prefix', None)!r}")
            y = torch.empty(x.shape[:-1] + (n_out,), dtype=x.dtype, device=x.device)
            return y.add_(bias) if bias is not None and y.numel() > 0 else y
        w = self._weight_for_apply(layer)
        if x.dtype == torch.float16:
            w = w.to(torch.float16)
        y = torch.matmul(x.reshape(-1, x.shape[-1]), w.t())
        if bias is not None:
            y.add_(bias)
        return y.reshape(x.shape[:-1] + (y.shape[-1],))
