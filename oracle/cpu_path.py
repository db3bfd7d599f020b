"""The reference's own CPU paths for the hot-path operators, restated in torch (CPU tensors).

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

The other operators' CPU oracles in the reference's tests are restated the
same way: top-k as torch.topk (tests/test_m7_kernels.py:19-20), gathers as
index_select (tests/test_gather_rows.py:41), the sparse accumulate as
(h.float() @ W_dequant.float()).half() (tests/test_m7_sparse_gemv.py:63-71)
and attention as decode_attention_ref (tests/test_m5_kernels.py:157-170).

Pinned by tests/test_oracle_cpu.py: dequantize_group equals the C oracle's
soi_ref_dequant_int4 bit for bit (the same binary32 product fl(q*s) per
element); gemv_dequant_mv is within binary16 rounding of the binary64 oracle
GEMV and returns the binary16 rounding of a column for a basis vector x;
topk_indices gives the rule-A set on distinct values, gather_rows equals
numpy indexing, sparse_accumulate_ref is within binary16 rounding of the
binary64 sparse accumulate, decode_attention_ref within the attention
tolerance of the binary64 attention.
"""
from __future__ import annotations

import math

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


def topk_indices(abs_g: torch.Tensor, k: int) -> torch.Tensor:
    """The reference test's top-k: torch.topk over fp32 |gate| (tests/test_m7_kernels.py:19-20), indices only."""
    return torch.topk(abs_g, k).indices


def gather_rows(matrix: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """matrix.index_select(0, indices) (tests/test_gather_rows.py:41): the rows' bytes."""
    return matrix.index_select(0, indices)


def sparse_accumulate_ref(h_sel: torch.Tensor, W_dequant_sel: torch.Tensor) -> torch.Tensor:
    """fp16 [H] = (h.float() @ W_dequant.float()).half() over the selected rows of down^T
    (tests/test_m7_sparse_gemv.py:63-71)."""
    return (h_sel.float() @ W_dequant_sel.float()).half()


def decode_attention_ref(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, cur_len: int) -> torch.Tensor:
    """Per query head: softmax(K q / sqrt(hd)) V over the first cur_len timesteps of its KV head, in fp32, fp16
    out (tests/test_m5_kernels.py:157-170)."""
    nq, hd = q.shape
    rep = nq // k_cache.shape[0]
    scale = 1.0 / math.sqrt(hd)
    out = torch.empty_like(q)
    for h in range(nq):
        kv = h // rep
        scores = torch.mv(k_cache[kv, :cur_len].float(), q[h].float()) * scale
        out[h] = torch.mv(v_cache[kv, :cur_len].float().t(), torch.softmax(scores, dim=0)).half()
    return out
