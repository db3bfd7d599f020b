"""Hot-channel cache for cache-aware Dynamic Input Pruning.

StaticFrequencyPolicy picks the cache_size most frequently selected
intermediate channels from calibration counts, ties broken by the lower
channel index (reference python/soinfer/offload/hot_cache.py:67-95).
LRUPolicy and LFUDecayPolicy are the online alternatives the reference
evaluates against it in trace-driven simulation (hot_cache.py:98-187), and
compare_policies runs all three over one trace (hot_cache.py:190-218). The
simulations are host bookkeeping only.

HotCache holds, for those channels in ascending order, their up_proj rows and
down_proj^T rows (packed INT4 + fp32 scales) in device memory, and slot_of
[I] int32 mapping a channel to its cache slot or -1 (reference
hot_cache.py:228-315). build_dip_descriptors reads slot_of directly.
On MI355X the full weights are resident in HBM, so the cache is filled with
a device-side row gather; from_host builds it from a pinned host arena with
the staged H2D gather instead (the reference's offload setting).
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass
from typing import Iterable, Optional, Sequence

import torch


def _sorted_ints(selected) -> list[int]:
    if isinstance(selected, torch.Tensor):
        selected = selected.tolist()
    return sorted(int(c) for c in selected)


@dataclass
class SimulationResult:
    policy: str
    cache_size: int
    hits: int
    total: int

    @property
    def hit_rate(self) -> float:
        return self.hits / self.total if self.total else 0.0


class StaticFrequencyPolicy:
    """Fixed hot set: the cache_size channels of highest frequency, lower index first on ties."""

    name = "static"

    def __init__(self, frequencies: torch.Tensor | Sequence[int], cache_size: int):
        freq = torch.as_tensor(frequencies).to(torch.int64).cpu()
        n = freq.numel()
        self.cache_size = min(int(cache_size), n)
        # stable sort by descending frequency keeps ascending index among equals
        order = torch.sort(-freq, stable=True).indices
        self.hot_indices = torch.sort(order[: self.cache_size]).values
        self.hot_set = frozenset(self.hot_indices.tolist())

    def simulate(self, trace: Iterable) -> SimulationResult:
        hits = total = 0
        for selected in trace:
            for c in _sorted_ints(selected):
                total += 1
                hits += c in self.hot_set
        return SimulationResult(self.name, self.cache_size, hits, total)


class LRUPolicy:
    """Least-recently-selected eviction, no calibration (hot_cache.py:98-141).

    A token's selected channels are all looked up against the cache as it stood at the end of the previous
    token (hits become most recent); only then are the token's misses inserted, in ascending channel order,
    each evicting the least recently used entry when the cache is full. This is how the device cache behaves
    per token (descriptors for the whole selection, then one update), and it keeps cross-token reuse visible
    when one token selects more channels than the cache holds."""

    name = "lru"

    def __init__(self, cache_size: int):
        self.cache_size = int(cache_size)

    def simulate(self, trace: Iterable) -> SimulationResult:
        cache: "OrderedDict[int, None]" = OrderedDict()  # first = least recently used
        hits = total = 0
        for selected in trace:
            chans = _sorted_ints(selected)
            total += len(chans)
            missed = []
            for c in chans:
                if c in cache:
                    cache.move_to_end(c)
                    hits += 1
                else:
                    missed.append(c)
            if self.cache_size <= 0:
                continue
            for c in missed:
                if len(cache) >= self.cache_size:
                    cache.popitem(last=False)
                cache[c] = None
        return SimulationResult(self.name, self.cache_size, hits, total)


class LFUDecayPolicy:
    """Lowest-frequency eviction with periodic decay (hot_cache.py:144-187).

    Every selection adds 1 to its channel's frequency (before the lookup); a miss into a full cache evicts
    the cached channel of lowest frequency, the higher index on ties (the lower index stays, as in
    StaticFrequencyPolicy). After every decay_every tokens all tracked frequencies are multiplied by
    decay in (0, 1], so stale popularity fades."""

    name = "lfu_decay"

    def __init__(self, cache_size: int, decay: float = 0.98, decay_every: int = 50):
        if not (0.0 < decay <= 1.0):
            raise ValueError("decay must be in (0, 1]")
        self.cache_size = int(cache_size)
        self.decay = float(decay)
        self.decay_every = int(decay_every)

    def simulate(self, trace: Iterable) -> SimulationResult:
        freq: dict = {}
        cache: set = set()
        hits = total = 0
        for step, selected in enumerate(trace):
            for c in _sorted_ints(selected):
                total += 1
                freq[c] = freq.get(c, 0.0) + 1.0
                if c in cache:
                    hits += 1
                    continue
                if self.cache_size <= 0:
                    continue
                if len(cache) >= self.cache_size:
                    # lowest frequency first; among equal frequencies the highest index goes
                    cache.remove(min(cache, key=lambda x: (freq[x], -x)))
                cache.add(c)
            if self.decay_every > 0 and (step + 1) % self.decay_every == 0:
                for ch in freq:
                    freq[ch] *= self.decay
        return SimulationResult(self.name, self.cache_size, hits, total)


def compare_policies(trace: Sequence, cache_sizes: Sequence[int], frequencies: Optional[Sequence[int]] = None,
                     **lfu_kwargs) -> list:
    """Static, LRU and LFU-with-decay over the same trace at each cache size (hot_cache.py:190-218).

    frequencies (for the static policy) default to the trace's own per-channel selection counts, i.e. the
    static policy's best case; pass calibration counts to evaluate it on held-out traffic instead."""
    trace = list(trace)
    if frequencies is None:
        counts: dict = {}
        for selected in trace:
            for c in _sorted_ints(selected):
                counts[c] = counts.get(c, 0) + 1
        n = max(counts) + 1 if counts else 0
        frequencies = [counts.get(c, 0) for c in range(n)]
    out = []
    for size in cache_sizes:
        out.append(StaticFrequencyPolicy(frequencies, size).simulate(trace))
        out.append(LRUPolicy(size).simulate(trace))
        out.append(LFUDecayPolicy(size, **lfu_kwargs).simulate(trace))
    return out


@dataclass
class HotCache:
    slot_of: torch.Tensor  # [I] int32 device, -1 if not cached
    hot_indices: torch.Tensor  # [C] int64 device, ascending
    up_Wq: torch.Tensor  # [C, up_row_nbytes] uint8 device
    up_scale: torch.Tensor  # [C, up_groups] fp32 device
    down_Wq: torch.Tensor  # [C, down_row_nbytes] uint8 device
    down_scale: torch.Tensor  # [C, down_groups] fp32 device

    @property
    def cache_size(self) -> int:
        return int(self.hot_indices.shape[0])

    @staticmethod
    def _slots(I: int, hot: torch.Tensor, device) -> torch.Tensor:
        slot_of = torch.full((I,), -1, dtype=torch.int32, device=device)
        if hot.numel():
            slot_of[hot.to(device)] = torch.arange(hot.numel(), dtype=torch.int32, device=device)
        return slot_of

    @staticmethod
    def build(up_Wq: torch.Tensor, up_scale: torch.Tensor, down_T_Wq: torch.Tensor, down_T_scale: torch.Tensor,
              hot_indices) -> "HotCache":
        """Cache built from device-resident weights with the device row gather."""
        from .. import ops

        device = up_Wq.device
        hot = torch.as_tensor(_sorted_ints(hot_indices), dtype=torch.int64)
        C = hot.numel()
        hot_d = hot.to(device)
        idx32 = hot_d.to(torch.int32)
        up_c = torch.empty(C, up_Wq.shape[1], dtype=torch.uint8, device=device)
        down_c = torch.empty(C, down_T_Wq.shape[1], dtype=torch.uint8, device=device)
        if C:
            ops.gather_rows_device(up_Wq, idx32, up_c)
            ops.gather_rows_device(down_T_Wq, idx32, down_c)
        return HotCache(
            slot_of=HotCache._slots(up_Wq.shape[0], hot, device),
            hot_indices=hot_d,
            up_Wq=up_c,
            up_scale=up_scale.index_select(0, hot_d).contiguous(),
            down_Wq=down_c,
            down_scale=down_T_scale.index_select(0, hot_d).contiguous(),
        )

    @staticmethod
    def from_host(up_host: torch.Tensor, up_scale: torch.Tensor, down_T_host: torch.Tensor,
                  down_T_scale: torch.Tensor, hot_indices, device="cuda") -> "HotCache":
        """Cache built from pinned host rows with the staged H2D gather (scales already on the device)."""
        from .. import ops

        hot = torch.as_tensor(_sorted_ints(hot_indices), dtype=torch.int64)
        C = hot.numel()
        up_c = torch.empty(C, up_host.shape[1], dtype=torch.uint8, device=device)
        down_c = torch.empty(C, down_T_host.shape[1], dtype=torch.uint8, device=device)
        if C:
            st = torch.empty(C, max(up_host.shape[1], down_T_host.shape[1]), dtype=torch.uint8, pin_memory=True)
            ops.gather_rows_staged(up_host, hot, st, up_c)
            torch.cuda.current_stream().synchronize()  # staging is reused for the second gather
            ops.gather_rows_staged(down_T_host, hot, st, down_c)
            torch.cuda.current_stream().synchronize()
        hot_d = hot.to(device)
        return HotCache(
            slot_of=HotCache._slots(up_host.shape[0], hot, device),
            hot_indices=hot_d,
            up_Wq=up_c,
            up_scale=up_scale.index_select(0, hot_d).contiguous(),
            down_Wq=down_c,
            down_scale=down_T_scale.index_select(0, hot_d).contiguous(),
        )
