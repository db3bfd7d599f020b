"""The reference's own CPU path for a quantized GEMV, restated in torch (CPU tensors).

TEST AND BENCH INFRASTRUCTURE ONLY. bench.py's cpu_baseline leg times it as
the CPU baseline, and tests/ check it. The product never imports it.

The reference checks its GEMV kernels against dequantize-then-matmul on the
host side: W_dequant = formats.dequantize(qt) (python/soinfer/quant/
formats.py:113-123: fp32 codes times the fp32 group scale, padded K cut back
to the true K), then expected = torch.mv(W_dequant.float(), x[:K].float())
.half() (tests/test_m4_kernels.py:157-165). The same two steps are what a CPU
user of the reference runs for a GEMV. This module states them as functions
of the unpacked int8 codes and fp32 scales, the inputs formats.quantize
produces.

Pinned by tests/test_oracle_cpu.py: dequantize_group equals the C oracle's
soi_ref_dequant_int4 bit for bit (the same binary32 product fl(q*s) per
element); gemv_dequant_mv is within binary16 rounding of the binary64 oracle
GEMV and returns the binary16 rounding of a column for a basis vector x.
"""
from __future__ import annotations

import torch


def dequantize_group(q: torch.Tensor, scale: torch.Tensor, orig_k: int, group_size: int) -> torch.Tensor:
    """fp32 [N, orig_k] weights from int8 codes q [N, G*group_size] and fp32 scales [N, G] (formats.py:113-123):
    each code times its group's scale in binary32, then the zero padding past orig_k dropped."""
    N, Kp = q.shape
    G = Kp // group_size
    w = q.float().reshape(N, G, group_size) * scale.float().reshape(N, G, 1)
    return w.reshape(N, Kp)[:, :orig_k]


def gemv_dequant_mv(q: torch.Tensor, scale: torch.Tensor, x: torch.Tensor, orig_k: int,
                    group_size: int) -> torch.Tensor:
    """fp16 [N] = torch.mv(dequantize(q, scale), x[:orig_k] as fp32), rounded to fp16 (test_m4_kernels.py:157-165)."""
    return torch.mv(dequantize_group(q, scale, orig_k, group_size), x[:orig_k].float()).half()


def gemv_mv_predequantized(W: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """The matmul half alone, on an fp32 W [N, K] dequantized beforehand."""
    return torch.mv(W, x[: W.shape[1]].float()).half()
