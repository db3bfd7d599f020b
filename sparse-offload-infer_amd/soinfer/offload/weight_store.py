"""One pinned host arena holding quantized weight matrices, rows as the addressable unit.

Same interface and semantics as the reference's PinnedWeightStore
(python/soinfer/offload/weight_store.py:26-117): a single pinned allocation
sized up front, matrices registered once in order at fixed byte offsets, each
row one contiguous span, so any subset of a matrix's rows can be fetched
without touching the rest.

On MI355X the arena is also read in place by the GPU: pinned host memory is
mapped into the device address space, and device_address() gives the address
kernels use (the hot-cache GEMVs and the device row gather read miss rows
straight from it over PCIe, with no staging copy).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable

import torch


@dataclass(frozen=True)
class WeightHandle:
    """One matrix's rows inside a PinnedWeightStore arena (offset is the store's business)."""

    name: str
    offset: int  # byte offset into the arena
    num_rows: int
    row_nbytes: int

    @property
    def nbytes(self) -> int:
        return self.num_rows * self.row_nbytes


def plan_bytes(shapes: Iterable[tuple[int, int]]) -> int:
    """Arena size for matrices of the given [num_rows, row_nbytes] shapes, registered back to back."""
    total = 0
    for rows, row_nbytes in shapes:
        if rows < 0 or row_nbytes < 0:
            raise ValueError("negative matrix shape")
        total += rows * row_nbytes
    return total


class PinnedWeightStore:
    """A single pinned host allocation holding quantized matrices row-major. total_bytes is fixed at
    construction: pinned memory is page-locked, so the whole model gets one allocation instead of many small
    ones."""

    def __init__(self, total_bytes: int):
        if total_bytes <= 0:
            raise ValueError("total_bytes must be positive")
        self.arena = torch.empty(total_bytes, dtype=torch.uint8, pin_memory=True)
        self._write_offset = 0
        self._handles: dict[str, WeightHandle] = {}
        self._device_base = None

    def register(self, name: str, data: torch.Tensor) -> WeightHandle:
        """Copy data ([num_rows, row_nbytes] uint8, any device) into the next free span; returns its handle.
        Registration order fixes the layout."""
        if name in self._handles:
            raise ValueError(f"weight {name!r} already registered")
        if data.dtype != torch.uint8 or data.dim() != 2:
            raise ValueError(f"register({name!r}): data must be 2D uint8 [num_rows, row_nbytes], got "
                             f"{tuple(data.shape)} {data.dtype}")
        num_rows, row_nbytes = data.shape
        nbytes = num_rows * row_nbytes
        end = self._write_offset + nbytes
        if end > self.arena.numel():
            raise ValueError(f"register({name!r}): arena overflow -- {nbytes} bytes requested, "
                             f"{self.arena.numel() - self._write_offset} remain")
        self.arena[self._write_offset:end].view(num_rows, row_nbytes).copy_(data)
        handle = WeightHandle(name, self._write_offset, num_rows, row_nbytes)
        self._handles[name] = handle
        self._write_offset = end
        return handle

    def handle(self, name: str) -> WeightHandle:
        return self._handles[name]

    def matrix_view(self, handle: WeightHandle) -> torch.Tensor:
        """[num_rows, row_nbytes] uint8 view of the pinned arena (no copy)."""
        return self.arena[handle.offset:handle.offset + handle.nbytes].view(handle.num_rows, handle.row_nbytes)

    def row_view(self, handle: WeightHandle, row: int) -> torch.Tensor:
        """One row, [row_nbytes] uint8 view (no copy)."""
        if not 0 <= row < handle.num_rows:
            raise IndexError(f"row {row} out of range for {handle.name!r} (num_rows={handle.num_rows})")
        start = handle.offset + row * handle.row_nbytes
        return self.arena[start:start + handle.row_nbytes]

    def rows_view(self, handle: WeightHandle, rows: torch.Tensor) -> torch.Tensor:
        """The selected rows (1D int64 indices) gathered into a new contiguous tensor (a copy)."""
        return self.matrix_view(handle).index_select(0, rows).contiguous()

    def device_address(self, handle: WeightHandle) -> int:
        """Device-visible address of the matrix's first byte (the arena's device mapping + offset), for kernels
        that read rows in place."""
        if self._device_base is None:
            from .. import _C

            self._device_base = _C.host_device_pointer(self.arena)
        return self._device_base + handle.offset

    @property
    def bytes_used(self) -> int:
        return self._write_offset

    @property
    def bytes_total(self) -> int:
        return self.arena.numel()
