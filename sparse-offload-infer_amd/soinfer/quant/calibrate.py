"""Scale selection for the quantizer.

A scale function maps (grouped values [..., g], amax [...], qmax) to a scale
[...]. min_max is the one the decode path uses: scale = amax / qmax floored
at the smallest normal float32, as in the reference's calibrate.min_max
(python/soinfer/quant/calibrate.py:19,22-27). The division is done
tensor-by-tensor so it is an IEEE division on every device (a division by a
Python scalar may be lowered to a reciprocal multiply on the GPU).
"""
from __future__ import annotations

import torch

TINY = torch.finfo(torch.float32).tiny


def min_max(grouped: torch.Tensor, amax: torch.Tensor, qmax: int) -> torch.Tensor:
    denom = torch.full_like(amax, float(qmax))
    return torch.clamp(amax / denom, min=TINY)


def percentile(grouped: torch.Tensor, amax: torch.Tensor, qmax: int, pct: float = 99.9) -> torch.Tensor:
    """Clip amax to the pct-th percentile of |values| (never above amax) before scaling."""
    clipped = torch.quantile(grouped.abs().float(), pct / 100.0, dim=-1)
    clipped = torch.minimum(clipped, amax)
    return torch.clamp(clipped / torch.full_like(clipped, float(qmax)), min=TINY)
