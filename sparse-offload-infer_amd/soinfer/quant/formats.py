"""Symmetric integer weight quantization (no zero-point).

W ~= scale * q with q in [-qmax, qmax], qmax = 2^(bits-1) - 1; the most
negative code is never produced. Quantization runs along the last dimension
K of a [..., N, K] tensor. Same formats, configuration object and rounding
rules as the reference's python/soinfer/quant/formats.py (:24-123):

  per_tensor   one scale, [1, 1]
  per_channel  one scale per row, [..., N, 1]
  group        one scale per (row, group of group_size along K), K zero-padded
               up to a multiple of group_size, scale [..., N, ceil(K/gs)]
  block32      group with group_size 32
  mx_e8m0      block32 with each scale rounded to the nearest power of two

q = clamp(round_half_even(w / scale), -qmax, qmax); the division is an IEEE
binary32 division on any device.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional

import torch

from . import calibrate

GRANULARITIES = ("per_tensor", "per_channel", "group", "block32", "mx_e8m0")
BLOCK32 = 32


def qmax_for_bits(bits: int) -> int:
    return (1 << (bits - 1)) - 1


@dataclass
class QuantConfig:
    bits: int
    granularity: str
    group_size: Optional[int] = None

    def __post_init__(self) -> None:
        if self.granularity not in GRANULARITIES:
            raise ValueError(f"unknown granularity {self.granularity!r}; expected one of {GRANULARITIES}")
        if self.granularity in ("block32", "mx_e8m0"):
            self.group_size = BLOCK32
        elif self.granularity == "group" and not self.group_size:
            raise ValueError("granularity 'group' needs a group_size")


@dataclass
class QuantTensor:
    qweight: torch.Tensor  # int8 [..., N, K or padded K]
    scale: torch.Tensor  # float32 [..., N, num_groups] ([1, 1] for per_tensor)
    config: QuantConfig
    orig_k: int


def _divide(w: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return w / scale.expand_as(w)


def _to_codes(values: torch.Tensor, scale: torch.Tensor, qmax: int) -> torch.Tensor:
    return torch.clamp(torch.round(_divide(values, scale)), -qmax, qmax).to(torch.int8)


def round_to_pow2(scale: torch.Tensor) -> torch.Tensor:
    """Nearest power of two of a non-negative scale (E8M0 style); 0 stays 0."""
    positive = scale > 0
    safe = torch.where(positive, scale, torch.ones_like(scale))
    return torch.where(positive, torch.exp2(torch.round(torch.log2(safe))), torch.zeros_like(scale))


def quantize(w: torch.Tensor, config: QuantConfig, scale_fn: Optional[Callable] = None) -> QuantTensor:
    w = w.float()
    qmax = qmax_for_bits(config.bits)
    fn = scale_fn or calibrate.min_max
    K = w.shape[-1]

    if config.granularity == "per_tensor":
        flat = w.reshape(-1)
        scale = fn(flat, flat.abs().max(), qmax).reshape(1, 1).float()
        return QuantTensor(_to_codes(w, scale, qmax), scale, config, K)

    if config.granularity == "per_channel":
        scale = fn(w, w.abs().amax(dim=-1), qmax).unsqueeze(-1).float()
        return QuantTensor(_to_codes(w, scale, qmax), scale, config, K)

    gs = int(config.group_size)
    G = -(-K // gs)
    if G * gs != K:
        w = torch.nn.functional.pad(w, (0, G * gs - K))
    grouped = w.reshape(*w.shape[:-1], G, gs)
    scale = fn(grouped, grouped.abs().amax(dim=-1), qmax)
    if config.granularity == "mx_e8m0":
        scale = round_to_pow2(scale)
    scale = scale.float()
    q = _to_codes(grouped, scale.unsqueeze(-1), qmax).reshape(*w.shape[:-1], G * gs)
    return QuantTensor(q, scale, config, K)


def dequantize(qt: QuantTensor) -> torch.Tensor:
    q = qt.qweight.float()
    if qt.config.granularity in ("per_tensor", "per_channel"):
        return q * qt.scale
    gs = int(qt.config.group_size)
    G = q.shape[-1] // gs
    w = (q.reshape(*q.shape[:-1], G, gs) * qt.scale.unsqueeze(-1)).reshape(q.shape)
    return w[..., : qt.orig_k]


def fraction_exact_zero(qt: QuantTensor) -> float:
    """Fraction of real (unpadded) codes that quantized to exactly 0."""
    return (qt.qweight[..., : qt.orig_k] == 0).float().mean().item()
