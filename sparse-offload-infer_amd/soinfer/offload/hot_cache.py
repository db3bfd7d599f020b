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

import heapq
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


class _TraceSimulator:
    """Replays a selection trace token by token and counts cache hits. A token is the set of channels one
    decode step selects (sorted ascending here, whatever order the trace gives); a subclass's _step(t, chans)
    returns how many of them hit and updates its cache. cache_size <= 0 means no cache (every lookup misses)."""

    name = ""

    def __init__(self, cache_size: int):
        self.cache_size = int(cache_size)

    def _begin(self) -> None:
        """Forget the state of a previous replay."""

    def _step(self, t: int, chans: list) -> int:
        raise NotImplementedError

    def simulate(self, trace: Iterable) -> SimulationResult:
        self._begin()
        hits = total = 0
        for t, selected in enumerate(trace):
            chans = _sorted_ints(selected)
            total += len(chans)
            hits += self._step(t, chans)
        return SimulationResult(self.name, self.cache_size, hits, total)


class StaticFrequencyPolicy(_TraceSimulator):
    """Fixed hot set: the cache_size channels of highest frequency, lower index first on ties
    (hot_cache.py:67-95 of the reference)."""

    name = "static"

    def __init__(self, frequencies: torch.Tensor | Sequence[int], cache_size: int):
        freq = torch.as_tensor(frequencies).to(torch.int64).cpu()
        super().__init__(min(int(cache_size), freq.numel()))
        # a stable sort on -frequency leaves equal frequencies in ascending channel order
        ranked = torch.sort(-freq, stable=True).indices
        self.hot_indices = torch.sort(ranked[: self.cache_size]).values
        self.hot_set = frozenset(self.hot_indices.tolist())

    def _step(self, t: int, chans: list) -> int:
        return sum(1 for c in chans if c in self.hot_set)


class LRUPolicy(_TraceSimulator):
    """Online cache that evicts the channel selected longest ago; needs no calibration (reference
    hot_cache.py:98-141).

    Per token, as the device cache works (every selected channel resolved against the cache, then one update):
    first every channel of the token is looked up in the cache as the previous token left it, each hit
    refreshing its recency (ascending channel order); then the token's misses go in, ascending, each evicting
    the least recently used channel while the cache is full. Looking up and inserting channel by channel
    instead would let a token that selects more channels than the cache holds evict everything the previous
    token left before it is looked up. Recency is a tick per touch; the eviction order is a heap of (tick,
    channel) entries, where entries whose channel was touched again since are skipped when they surface."""

    name = "lru"

    def _begin(self) -> None:
        self._tick = 0
        self._last = {}  # cached channel -> tick of its latest touch
        self._heap = []  # (tick, channel); stale entries skipped on pop

    def _touch(self, c: int) -> None:
        self._tick += 1
        self._last[c] = self._tick
        heapq.heappush(self._heap, (self._tick, c))

    def _step(self, t: int, chans: list) -> int:
        hit = [c for c in chans if c in self._last]
        for c in hit:
            self._touch(c)
        if self.cache_size <= 0:
            return len(hit)
        for c in chans:
            if c in self._last:
                continue
            while len(self._last) >= self.cache_size:
                tick, old = heapq.heappop(self._heap)
                if self._last.get(old) == tick:  # the entry is current: old is the least recently used
                    del self._last[old]
            self._touch(c)
        return len(hit)


class LFUDecayPolicy(_TraceSimulator):
    """Online cache that evicts the channel of lowest decayed frequency (reference hot_cache.py:144-187).

    Each selection first adds 1 to its channel's frequency, then looks the channel up; a miss into a full
    cache replaces the cached channel of lowest frequency (of two equal, the higher index leaves, as the
    static policy keeps the lower one). Every decay_every tokens every frequency seen so far is multiplied by
    decay (0 < decay <= 1), so a channel popular long ago loses its claim."""

    name = "lfu_decay"

    def __init__(self, cache_size: int, decay: float = 0.98, decay_every: int = 50):
        if not 0.0 < decay <= 1.0:
            raise ValueError(f"LFUDecayPolicy: decay must satisfy 0 < decay <= 1, got {decay}")
        super().__init__(cache_size)
        self.decay = float(decay)
        self.decay_every = int(decay_every)

    def _begin(self) -> None:
        self._freq = {}  # channel -> decayed selection count
        self._cached = set()

    def _step(self, t: int, chans: list) -> int:
        f, cached = self._freq, self._cached
        n_hit = 0
        for c in chans:
            f[c] = f.get(c, 0.0) + 1.0
            if c in cached:
                n_hit += 1
            elif self.cache_size > 0:
                if len(cached) >= self.cache_size:
                    cached.remove(min(cached, key=lambda x: (f[x], -x)))
                cached.add(c)
        if self.decay_every > 0 and (t + 1) % self.decay_every == 0:
            for c in f:
                f[c] *= self.decay
        return n_hit


def compare_policies(trace: Sequence, cache_sizes: Sequence[int], frequencies: Optional[Sequence[int]] = None,
                     **lfu_kwargs) -> list:
    """For each cache size, the static, LRU and LFU-with-decay results over one trace, in that order
    (reference hot_cache.py:190-218).

    Without frequencies the static policy ranks channels by their counts in the trace itself (its best case);
    calibration counts from other tokens evaluate it on held-out traffic instead."""
    tokens = [_sorted_ints(sel) for sel in trace]
    if frequencies is None:
        n = 1 + max((c for tok in tokens for c in tok), default=-1)
        frequencies = [0] * n
        for tok in tokens:
            for c in tok:
                frequencies[c] += 1
    results = []
    for size in cache_sizes:
        for sim in (StaticFrequencyPolicy(frequencies, size), LRUPolicy(size), LFUDecayPolicy(size, **lfu_kwargs)):
            results.append(sim.simulate(tokens))
    return results


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
