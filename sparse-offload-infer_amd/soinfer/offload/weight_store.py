"""Pinned host arena for packed weight matrices, addressable row by row.

Public surface of the reference's PinnedWeightStore / WeightHandle
(python/soinfer/offload/weight_store.py:26-117, used by load_hf_checkpoint.py
:95-146, generate.py:114,287,294 and hot_cache.py:300-304): one page-locked
allocation sized up front, matrices appended in registration order with no
padding between them, each row one contiguous byte span, so any subset of a
matrix's rows can be copied or read without touching the rest.

Design here: the arena is a ledger of spans. Each registered matrix is a
WeightHandle (name, byte offset, rows, row width) appended to an ordered list;
the next free byte is the end of the last span, so the ledger is the only
state. The arena is also a GPU-visible buffer: pinned host memory is mapped
into the device address space, and device_address() returns where a kernel
finds a matrix through that mapping (the hot-cache GEMVs and the device row
gather read miss rows in place over PCIe, with no staging copy).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable, Iterator

import torch


@dataclass(frozen=True)
class WeightHandle:
    """Where one matrix lives in a PinnedWeightStore: rows [offset, offset + nbytes) of the arena, each
    row_nbytes wide."""

    name: str
    offset: int
    num_rows: int
    row_nbytes: int

    @property
    def nbytes(self) -> int:
        return self.num_rows * self.row_nbytes

    @property
    def end(self) -> int:
        return self.offset + self.nbytes

    def row_span(self, row: int) -> tuple[int, int]:
        """[start, stop) arena byte range of one row."""
        start = self.offset + row * self.row_nbytes
        return start, start + self.row_nbytes


def plan_bytes(shapes: Iterable[tuple[int, int]]) -> int:
    """Arena bytes for matrices of the given (num_rows, row_nbytes) shapes appended back to back."""
    need = 0
    for shape in shapes:
        rows, width = (int(v) for v in shape)
        if min(rows, width) < 0:
            raise ValueError(f"plan_bytes: a matrix shape cannot be negative, got {tuple(shape)}")
        need += rows * width
    return need


class PinnedWeightStore:
    """One pinned uint8 arena of total_bytes holding row-major packed matrices. The size is fixed: the whole
    model is page-locked in a single allocation rather than many small ones."""

    def __init__(self, total_bytes: int):
        total_bytes = int(total_bytes)
        if total_bytes < 1:
            raise ValueError(f"PinnedWeightStore needs a positive size, got {total_bytes} bytes")
        self.arena = torch.empty(total_bytes, dtype=torch.uint8, pin_memory=True)
        self._ledger: list[WeightHandle] = []
        self._index: dict[str, int] = {}
        self._mapped_base: int | None = None

    # ---- layout ----
    @property
    def bytes_used(self) -> int:
        return self._ledger[-1].end if self._ledger else 0

    @property
    def bytes_total(self) -> int:
        return self.arena.numel()

    def __len__(self) -> int:
        return len(self._ledger)

    def __contains__(self, name: str) -> bool:
        return name in self._index

    def __iter__(self) -> Iterator[WeightHandle]:
        return iter(self._ledger)

    def register(self, name: str, data: torch.Tensor) -> WeightHandle:
        """Append data ([num_rows, row_nbytes] uint8 on any device) right after the previous matrix and return
        its handle. The registration order is the arena layout."""
        if name in self._index:
            raise ValueError(f"PinnedWeightStore.register: the name {name!r} is taken")
        if not (isinstance(data, torch.Tensor) and data.dtype == torch.uint8 and data.dim() == 2):
            got = (tuple(data.shape), data.dtype) if isinstance(data, torch.Tensor) else type(data).__name__
            raise ValueError(f"PinnedWeightStore.register({name!r}): expected a 2-D uint8 matrix, got {got}")
        h = WeightHandle(name, self.bytes_used, int(data.shape[0]), int(data.shape[1]))
        if h.end > self.bytes_total:
            raise ValueError(f"PinnedWeightStore.register({name!r}): {h.nbytes} bytes do not fit, only "
                             f"{self.bytes_total - h.offset} of the {self.bytes_total}-byte arena are free")
        self.matrix_view(h).copy_(data)
        self._index[name] = len(self._ledger)
        self._ledger.append(h)
        return h

    def handle(self, name: str) -> WeightHandle:
        return self._ledger[self._index[name]]

    # ---- views (no copies) and gathers ----
    def matrix_view(self, handle: WeightHandle) -> torch.Tensor:
        """The matrix as a [num_rows, row_nbytes] view of the arena."""
        return self.arena.narrow(0, handle.offset, handle.nbytes).view(handle.num_rows, handle.row_nbytes)

    def row_view(self, handle: WeightHandle, row: int) -> torch.Tensor:
        """Row `row` of the matrix as a [row_nbytes] view of the arena."""
        if row < 0 or row >= handle.num_rows:
            raise IndexError(f"{handle.name!r} has rows 0..{handle.num_rows - 1}; row {row} does not exist")
        start, _ = handle.row_span(row)
        return self.arena.narrow(0, start, handle.row_nbytes)

    def rows_view(self, handle: WeightHandle, rows: torch.Tensor) -> torch.Tensor:
        """A new contiguous [len(rows), row_nbytes] tensor holding the listed rows (int64 indices, any order)."""
        return torch.index_select(self.matrix_view(handle), 0, rows)

    # ---- device mapping ----
    def device_address(self, handle: WeightHandle) -> int:
        """Address of the matrix's first byte in the GPU's mapping of the arena, for kernels that read its rows
        in place."""
        if self._mapped_base is None:
            from .. import _C

            self._mapped_base = int(_C.host_device_pointer(self.arena))
        return self._mapped_base + handle.offset
