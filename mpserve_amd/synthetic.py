"""Seeded synthetic FP8 checkpoints of the benchmark configurations.

A weight is ``w = (randn * sigma).to(bf16)``; its per-output-channel FP32 scale
is ``absmax_row(w) / 448``; the FP8 e4m3 bytes are
``clamp(w / s, -448, 448).to(float8_e4m3fn)``; the scale key the sidecar
builder groups rows by is the FP16 bit pattern of ``s``, as the reference's
compress script derives it (scripts/compress_llm_fp8_huffman.py:96-104).
Optional outliers (config 3) replace a Bernoulli(p) subset with exactly
+-k*sigma before the BF16 cast.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import torch

FP8_MAX = 448.0

LLAMA3_8B_LAYER: List[Tuple[str, int, int]] = [
    ("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("v_proj", 1024, 4096), ("o_proj", 4096, 4096),
    ("gate_proj", 14336, 4096), ("up_proj", 14336, 4096), ("down_proj", 4096, 14336),
]
LLAMA3_70B_LAYER: List[Tuple[str, int, int]] = [
    ("q_proj", 8192, 8192), ("k_proj", 1024, 8192), ("v_proj", 1024, 8192), ("o_proj", 8192, 8192),
    ("gate_proj", 28672, 8192), ("up_proj", 28672, 8192), ("down_proj", 8192, 28672),
]
LLAMA3_8B_LM_HEAD = ("lm_head", 128256, 4096)


def config_weights(workload: str) -> List[Tuple[str, int, int, int, float, float]]:
    """(name, n, m, seed, sigma, outlier_p) of every weight of a benchmark configuration.

    ``layer8b`` (config 2): one Llama-3-8B layer; ``layer70b`` (config 3): one
    Llama-3-70B layer, sigma 0.015 with 0.1% outliers at +-8 sigma;
    ``model8b`` (config 5): 32 Llama-3-8B layers plus lm_head. Seeds are fixed
    per (layer, projection), so every caller builds the same inputs.
    """
    if workload == "layer70b":
        return [(f"layers.0.{name}", n, m, 200 + j, 0.015, 1e-3) for j, (name, n, m) in enumerate(LLAMA3_70B_LAYER)]
    if workload not in ("layer8b", "model8b"):
        raise ValueError(f"unknown workload {workload!r}")
    layers = 32 if workload == "model8b" else 1
    out = [(f"layers.{layer}.{name}", n, m, 100 + 16 * layer + j, 0.02, 0.0)
           for layer in range(layers) for j, (name, n, m) in enumerate(LLAMA3_8B_LAYER)]
    if workload == "model8b":
        name, n, m = LLAMA3_8B_LM_HEAD
        out.append((name, n, m, 99, 0.02, 0.0))
    return out


@dataclass
class SyntheticWeight:
    bf16: torch.Tensor        # [n, m] bfloat16
    fp8_u8: torch.Tensor      # [n, m] uint8 (e4m3 bit patterns)
    scale_f32: torch.Tensor   # [n, 1] float32
    scale_u16: torch.Tensor   # [n] uint16: FP16 bits of the scale


def quantize_per_row(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(fp8 bytes, FP32 scale [n,1], u16 scale key [n]) of a BF16 [n, m] weight."""
    wf = w.float()
    s = wf.abs().amax(dim=1, keepdim=True) / FP8_MAX
    s = torch.where(s > 0, s, torch.ones_like(s))
    q = (wf / s).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn).view(torch.uint8)
    key = s.to(torch.float16).view(torch.uint16).reshape(-1)
    return q.contiguous(), s, key.contiguous()


def make_weight(n: int, m: int, sigma: float = 0.02, seed: int = 0, outlier_p: float = 0.0,
                outlier_k: float = 8.0, device: str | torch.device = "cpu") -> SyntheticWeight:
    """Seeded BF16 weight and its per-row FP8 quantization, generated on ``device``."""
    g = torch.Generator(device=device).manual_seed(int(seed))
    w = torch.randn((n, m), generator=g, device=device, dtype=torch.float32) * sigma
    if outlier_p > 0.0:
        mask = torch.rand((n, m), generator=g, device=device) < outlier_p
        sign = torch.where(torch.rand((n, m), generator=g, device=device) < 0.5, -1.0, 1.0)
        w = torch.where(mask, sign * (outlier_k * sigma), w)
    w = w.to(torch.bfloat16)
    q, s, key = quantize_per_row(w)
    return SyntheticWeight(w.contiguous(), q, s, key)


@dataclass
class SyntheticAwqWeight:
    bf16: torch.Tensor       # [n, m] bfloat16
    int4_u8: torch.Tensor    # [n, m] uint8, int4 values 0..15
    scale_u16: torch.Tensor  # [n, m // group] (or [n] when group is None) uint16: BF16 bits of the scale


def make_awq_weight(n: int, m: int, group: int | None = 128, sigma: float = 0.02, seed: int = 0,
                    device: str | torch.device = "cpu") -> SyntheticAwqWeight:
    """Seeded BF16 weight and an AWQ-style int4 quantisation of it.

    The scale of each group of ``group`` columns of a row (of a whole row when
    ``group`` is None) is ``absmax / 7`` rounded to BF16, and the int4 value is
    ``clamp(round(w / s) + 8, 0, 15)`` (zero point 8). The sidecar the AWQ
    builders write depends only on these three tensors, not on how the int4
    values were chosen.
    """
    g = torch.Generator(device=device).manual_seed(int(seed))
    w = (torch.randn((n, m), generator=g, device=device, dtype=torch.float32) * sigma).to(torch.bfloat16)
    wf = w.float()
    gs = m if group is None else int(group)
    if gs <= 0 or m % gs != 0:
        raise ValueError(f"group ({gs}) must divide the column count ({m})")
    amax = wf.reshape(n, m // gs, gs).abs().amax(dim=2)
    s = (amax / 7.0).to(torch.bfloat16)
    s = torch.where(s.float() > 0, s, torch.ones_like(s))
    sf = s.float().repeat_interleave(gs, dim=1)
    q = (torch.round(wf / sf) + 8).clamp(0, 15).to(torch.uint8)
    key = s.view(torch.uint16)
    if group is None:
        key = key.reshape(n)
    return SyntheticAwqWeight(w.contiguous(), q.contiguous(), key.contiguous())
