"""Quantize a local safetensors checkpoint's decoder linears into a PinnedWeightStore, one tensor at a time.

Same arena format and entry points as the reference's loader
(python/soinfer/offload/load_hf_checkpoint.py:32-148):

  * every decoder layer's 7 linear weights (LINEAR_SUFFIXES order) are
    quantized to INT4 (symmetric, group_size along K, fp32 scales) and packed
    in AWQ nibble order, then registered in that order, layer by layer;
  * with include_down_proj_t, down_proj is also registered transposed
    ([intermediate, hidden]) right after it, under the synthetic name
    "model.layers.{i}.mlp.down_proj_T.weight", so that selecting
    intermediate channels is a row selection for both up and down;
  * the arena is sized exactly beforehand from the shards' headers
    (plan_arena_bytes), because a pinned arena is one fixed allocation;
  * scales stay on the GPU (LoadedMatrix.scale), packed rows in the arena.

Only a local directory with model.safetensors.index.json and its shards is
read (no download). Quantization runs on the CPU in IEEE binary32, as the
reference does, so the arena bytes are a pure function of the checkpoint.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass
from typing import Optional

import torch

from ..quant import formats, pack
from .weight_store import PinnedWeightStore, WeightHandle

LINEAR_SUFFIXES = (
    "self_attn.q_proj.weight",
    "self_attn.k_proj.weight",
    "self_attn.v_proj.weight",
    "self_attn.o_proj.weight",
    "mlp.gate_proj.weight",
    "mlp.up_proj.weight",
    "mlp.down_proj.weight",
)
DOWN_PROJ_SUFFIX = "mlp.down_proj.weight"
DOWN_PROJ_T_SUFFIX = "mlp.down_proj_T.weight"  # synthetic: down_proj transposed, registered by this loader only


@dataclass
class LoadedMatrix:
    handle: WeightHandle
    scale: torch.Tensor  # [N, num_groups] fp32 on the GPU
    packed_k: int  # K after zero-padding to a multiple of the group size (the GEMV's K)
    n: int
    k: int


def packed_int4_bytes(n: int, k: int) -> int:
    """Bytes of an [n, k] INT4 matrix: n rows of ceil(k/8) 32-bit words."""
    return n * ((k + 7) // 8) * 4


class _Shards:
    """Tensor name -> safetensors shard, with one open handle per shard."""

    def __init__(self, model_dir: str):
        from safetensors import safe_open

        self._open = safe_open
        self.dir = model_dir
        with open(os.path.join(model_dir, "model.safetensors.index.json")) as f:
            self.weight_map = json.load(f)["weight_map"]
        self._handles: dict[str, object] = {}

    def _shard(self, name: str):
        file = self.weight_map[name]
        if file not in self._handles:
            self._handles[file] = self._open(os.path.join(self.dir, file), framework="pt")
        return self._handles[file]

    def shape(self, name: str) -> tuple[int, int]:
        n, k = self._shard(name).get_slice(name).get_shape()  # header only
        return int(n), int(k)

    def tensor(self, name: str) -> torch.Tensor:
        return self._shard(name).get_tensor(name)


def plan_arena_bytes(model_dir: str, num_layers: int, suffixes: tuple = LINEAR_SUFFIXES,
                     transpose: bool = False, group_size: Optional[int] = None) -> int:
    """Exact arena bytes for the INT4-packed matrices of `suffixes` over num_layers layers, from the shard
    headers only; transpose=True plans them transposed (the down_proj_T registration). With group_size, K is
    first padded to a multiple of it, as the quantizer pads before packing (the reference plans the unpadded K,
    which is the same whenever group_size divides K)."""
    shards = _Shards(model_dir)
    total = 0
    for layer in range(num_layers):
        for suffix in suffixes:
            n, k = shards.shape(f"model.layers.{layer}.{suffix}")
            if transpose:
                n, k = k, n
            if group_size:
                k = -(-k // group_size) * group_size
            total += packed_int4_bytes(n, k)
    return total


def _quantize_int4(w: torch.Tensor, group_size: int):
    qt = formats.quantize(w.float(), formats.QuantConfig(bits=4, granularity="group", group_size=group_size))
    packed, packed_k = pack.pack_int4(qt.qweight)
    return packed.contiguous(), qt.scale.contiguous(), packed_k


def stream_load_layers(model_dir: str, num_layers: int, group_size: int = 128, log_every: int = 8,
                       include_down_proj_t: bool = False, device: Optional[str] = "cuda"):
    """Quantize and register every layer's linears (and down_proj_T when asked). Returns (store, matrices)
    with matrices["model.layers.{i}.{suffix}"] = LoadedMatrix. At most one source tensor is materialized at a
    time."""
    shards = _Shards(model_dir)
    total = plan_arena_bytes(model_dir, num_layers, group_size=group_size)
    if include_down_proj_t:
        total += plan_arena_bytes(model_dir, num_layers, suffixes=(DOWN_PROJ_SUFFIX,), transpose=True,
                                  group_size=group_size)
    store = PinnedWeightStore(total)
    matrices: dict[str, LoadedMatrix] = {}

    def put(name: str, w: torch.Tensor) -> None:
        n, k = w.shape
        packed, scale, packed_k = _quantize_int4(w, group_size)
        handle = store.register(name, packed)
        matrices[name] = LoadedMatrix(handle, scale.to(device) if device else scale, packed_k, int(n), int(k))

    for layer in range(num_layers):
        for suffix in LINEAR_SUFFIXES:
            name = f"model.layers.{layer}.{suffix}"
            w = shards.tensor(name)
            put(name, w)
            if include_down_proj_t and suffix == DOWN_PROJ_SUFFIX:
                put(f"model.layers.{layer}.{DOWN_PROJ_T_SUFFIX}", w.t().contiguous())
            del w
        if log_every and ((layer + 1) % log_every == 0 or layer == num_layers - 1):
            print(f"  loaded layer {layer + 1}/{num_layers} ({store.bytes_used / 1e9:.2f} GB in arena)")
    return store, matrices
