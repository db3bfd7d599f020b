"""Dynamic Input Pruning (DIP) SwiGLU MLP for one decoder layer at batch 1.

Operation sequence of the reference's run_decoder_layer_dip /
run_decoder_layer_cached_dip MLP half (python/soinfer/runtime/generate.py:
276-310 and 367-404):

    gate  = INT4 GEMV(W_gate, x)                       dense, [I]
    idx   = topk_threshold_select(|gate| as fp32, k)   ascending indices
    u     = INT4 GEMV over rows idx of W_up            [k]
    h     = fp16(silu(fp32(gate[idx])) * fp32(u))      torch glue, as the reference
    y     = sum_j h_j * row idx_j of W_down^T          [H]

On MI355X all weights stay resident in HBM (288 GB), so the selected rows are
read in place through the index list (no host gather). dip_mlp_gathered runs
the reference's gather-then-GEMV shape on device buffers, and cached_dip_mlp
the hot-cache + staging shape; all three return bit-identical outputs for the
same inputs, because every path feeds the same kernel bodies the same
logical rows.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F

from .. import ops
from ..offload.hot_cache import HotCache


@dataclass
class DipMLPWeights:
    """INT4 g-group weights of one SwiGLU MLP. down is stored transposed ([I, H]) so that selecting
    intermediate channels is a row selection for both up and down (reference
    python/soinfer/offload/load_hf_checkpoint.py:90-111)."""

    gate_Wq: torch.Tensor  # [I, ceil(H/8)*4] uint8
    gate_scale: torch.Tensor  # [I, ceil(H/gs)] fp32
    up_Wq: torch.Tensor  # [I, ceil(H/8)*4]
    up_scale: torch.Tensor
    down_T_Wq: torch.Tensor  # [I, ceil(H/8)*4]
    down_T_scale: torch.Tensor  # [I, ceil(H/gs)]
    hidden_size: int
    group_size: int

    @property
    def intermediate_size(self) -> int:
        return int(self.gate_Wq.shape[0])


def select_channels(w: DipMLPWeights, x: torch.Tensor, dip_k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """gate = W_gate x (dense) and the DIP selection idx (int32 [dip_k], ascending)."""
    gate = ops.gemv_w4a16_group_lop3(w.gate_Wq, w.gate_scale, x, w.hidden_size, w.group_size)
    abs_g = gate.float().abs().contiguous()
    idx = ops.topk_threshold_select(abs_g, dip_k)
    return gate, idx


def silu_gate(gate: torch.Tensor, idx: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """h_j = fp16(silu(fp32(gate[idx_j])) * fp32(u_j)) (generate.py:304-305)."""
    g_sel = gate.index_select(0, idx.long())
    return (F.silu(g_sel.float()) * u.float()).half()


def dip_mlp(w: DipMLPWeights, x: torch.Tensor, dip_k: int, channel_counts: Optional[torch.Tensor] = None):
    """Resident-weight DIP MLP. Returns (y [H] fp16, idx [dip_k] int32)."""
    gate, idx = select_channels(w, x, dip_k)
    if channel_counts is not None:
        channel_counts.scatter_add_(0, idx.long(), torch.ones(idx.shape[0], dtype=channel_counts.dtype,
                                                              device=idx.device))
    u = ops.gemv_w4a16_indexed(w.up_Wq, w.up_scale, idx, x, w.hidden_size, w.group_size)
    h = silu_gate(gate, idx, u)
    y = ops.gemv_w4a16_indexed_accumulate(w.down_T_Wq, w.down_T_scale, idx, h, w.hidden_size, w.group_size)
    return y, idx


def dip_mlp_gathered(w: DipMLPWeights, x: torch.Tensor, dip_k: int):
    """Reference-shaped DIP MLP: gather the selected up / down^T rows into compact buffers first, then
    gemv_w4a16_group_lop3 and gemv_w4a16_sparse_accumulate. Returns (y, idx)."""
    gate, idx = select_channels(w, x, dip_k)
    k = idx.shape[0]
    idx_l = idx.long()
    up_sel = torch.empty(k, w.up_Wq.shape[1], dtype=torch.uint8, device=x.device)
    down_sel = torch.empty(k, w.down_T_Wq.shape[1], dtype=torch.uint8, device=x.device)
    ops.gather_rows_device(w.up_Wq, idx, up_sel)
    ops.gather_rows_device(w.down_T_Wq, idx, down_sel)
    u = ops.gemv_w4a16_group_lop3(up_sel, w.up_scale.index_select(0, idx_l), x, w.hidden_size, w.group_size)
    h = silu_gate(gate, idx, u)
    y = ops.gemv_w4a16_sparse_accumulate(down_sel, w.down_T_scale.index_select(0, idx_l), h, w.hidden_size,
                                         w.group_size)
    return y, idx


def cached_dip_mlp(w: DipMLPWeights, cache: HotCache, x: torch.Tensor, dip_k: int,
                   host_up: Optional[torch.Tensor] = None, host_down_T: Optional[torch.Tensor] = None,
                   staging: Optional[torch.Tensor] = None, miss_bytes: Optional[list] = None):
    """Cache-aware DIP MLP: selected channels resident in `cache` are read from it, the misses from a
    staging buffer; one fused kernel per direction. Misses are fetched from the device-resident weights
    (default) or, when host_up / host_down_T (pinned [I, row_nbytes]) are given, from pinned host memory
    through `staging` (pinned, >= dip_k * row_nbytes) with the staged H2D gather. Bit-identical to dip_mlp.
    Returns (y, idx, miss_count)."""
    gate, idx = select_channels(w, x, dip_k)
    desc, miss_channels, miss_count = ops.build_dip_descriptors(idx, cache.slot_of)
    mc = int(miss_count.item())
    miss = miss_channels[:mc]
    miss_l = miss.long()
    dev = x.device
    up_st = torch.empty(mc, w.up_Wq.shape[1], dtype=torch.uint8, device=dev)
    down_st = torch.empty(mc, w.down_T_Wq.shape[1], dtype=torch.uint8, device=dev)
    if mc:
        if host_up is not None and host_down_T is not None:
            miss_cpu = miss_l.cpu()
            ops.gather_rows_staged(host_up, miss_cpu, staging, up_st)
            torch.cuda.current_stream().synchronize()  # staging reused for the second gather
            ops.gather_rows_staged(host_down_T, miss_cpu, staging, down_st)
        else:
            ops.gather_rows_device(w.up_Wq, miss, up_st)
            ops.gather_rows_device(w.down_T_Wq, miss, down_st)
    if miss_bytes is not None:
        miss_bytes.append(mc * (w.up_Wq.shape[1] + w.down_T_Wq.shape[1]))
    up_st_scale = w.up_scale.index_select(0, miss_l)
    down_st_scale = w.down_T_scale.index_select(0, miss_l)
    u = ops.gemv_dip_fused_up(cache.up_Wq, cache.up_scale, up_st, up_st_scale, desc, x, w.hidden_size,
                              w.group_size)
    h = silu_gate(gate, idx, u)
    y = ops.gemv_dip_fused_down(cache.down_Wq, cache.down_scale, down_st, down_st_scale, desc, h,
                                w.hidden_size, w.group_size)
    return y, idx, mc


def cached_dip_mlp_direct(w: DipMLPWeights, cache: HotCache, x: torch.Tensor, dip_k: int,
                          full_up: Optional[torch.Tensor] = None, full_down_T: Optional[torch.Tensor] = None,
                          workspace: Optional[torch.Tensor] = None):
    """Cache-aware DIP MLP with the misses read in place: the up GEMV and the down accumulate resolve every
    selected channel through cache.slot_of themselves, reading hits from the cache and misses from full_up /
    full_down_T (pinned host memory read through its device mapping, or device tensors; default: the
    resident weights). No descriptors, no gather, no staging buffer and no host sync; the SiLU gating is the
    up GEMV's epilogue. Bit-identical to dip_mlp and cached_dip_mlp. Returns (y, idx)."""
    from .. import _C

    gate, idx = select_channels(w, x, dip_k)
    full_up = w.up_Wq if full_up is None else full_up
    full_down_T = w.down_T_Wq if full_down_T is None else full_down_T
    H, gs = w.hidden_size, w.group_size
    h = torch.empty(dip_k, dtype=torch.float16, device=x.device)
    _C.gemv_dip_cached_up_silu_into(cache.up_Wq, cache.up_scale, full_up, w.up_scale, cache.slot_of, idx, x, gate,
                                    h, H, gs)
    if workspace is None:
        workspace = torch.zeros(max(1, _C.sparse_accumulate_workspace_bytes(H, dip_k)), dtype=torch.uint8,
                                device=x.device)
    y = torch.empty(H, dtype=torch.float16, device=x.device)
    _C.gemv_dip_cached_down_into(cache.down_Wq, cache.down_scale, full_down_T, w.down_T_scale, cache.slot_of, idx,
                                 h, y, H, gs, workspace)
    return y, idx


def calibrate_channel_frequencies(w: DipMLPWeights, xs: torch.Tensor, dip_k: int) -> torch.Tensor:
    """counts[c] = number of calibration inputs whose DIP selection contains channel c
    (generate.py:579-609, one layer). xs: [n, H] fp16."""
    counts = torch.zeros(w.intermediate_size, dtype=torch.int64, device=xs.device)
    for i in range(xs.shape[0]):
        dip_mlp(w, xs[i].contiguous(), dip_k, channel_counts=counts)
    return counts
