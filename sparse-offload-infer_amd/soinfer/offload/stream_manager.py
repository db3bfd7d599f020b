"""Copy streams for double / triple buffered weight prefetch, with write-after-read protection.

Public surface of the reference's StreamManager
(python/soinfer/offload/stream_manager.py:10-86, driven by WeightPipeline in
generate.py:85-138): prefetch(i, dst, src) starts an asynchronous copy of
pinned host bytes into device buffer i, wait(i) orders the current stream
after it, mark_read_done(i) records where the kernels reading buffer i were
issued, and the next prefetch into buffer i starts only after that point, so
a transfer never overwrites data a kernel launched earlier is still reading.
synchronize(i) blocks the host until buffer i's copy has landed.

Design here: each buffer is a CopySlot that owns its copy stream and two
events, `landed` (its latest copy is complete) and `released` (its latest
readers were issued before this point), plus a flag telling whether
`released` has ever been recorded: the first transfer into a buffer has no
reader to wait for. All streams keep the default priority; the copies are
hipMemcpyAsync from pinned memory, run by the SDMA engines.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class CopySlot:
    """One prefetch buffer's stream and its two fences."""

    stream: torch.cuda.Stream
    landed: torch.cuda.Event = field(default_factory=torch.cuda.Event)
    released: torch.cuda.Event = field(default_factory=torch.cuda.Event)
    has_reader: bool = False

    def start_copy(self, dst: torch.Tensor, src: torch.Tensor) -> None:
        if self.has_reader:
            self.stream.wait_event(self.released)
        with torch.cuda.stream(self.stream):
            dst.copy_(src, non_blocking=True)
            self.landed.record()

    def release(self, on: torch.cuda.Stream) -> None:
        self.released.record(on)
        self.has_reader = True


class StreamManager:
    """num_buffers copy slots (2 for double buffering, 3 for triple). shared_stream=True gives every slot the same
    copy stream (an addition to the reference's interface): the copies then run one after another in the order
    they were queued instead of splitting the host link between concurrent transfers."""

    def __init__(self, num_buffers: int = 2, shared_stream: bool = False):
        if int(num_buffers) < 1:
            raise ValueError(f"StreamManager needs at least one buffer, got {num_buffers}")
        self.num_buffers = int(num_buffers)
        if shared_stream:
            one = torch.cuda.Stream()
            self.slots = [CopySlot(one) for _ in range(self.num_buffers)]
        else:
            self.slots = [CopySlot(torch.cuda.Stream()) for _ in range(self.num_buffers)]

    def _slot(self, buf_idx: int) -> CopySlot:
        if not 0 <= buf_idx < self.num_buffers:
            raise IndexError(f"buffer {buf_idx} does not exist (this manager has {self.num_buffers})")
        return self.slots[buf_idx]

    def prefetch(self, buf_idx: int, gpu_buffer: torch.Tensor, host_data: torch.Tensor) -> None:
        """Queue host_data (pinned) -> gpu_buffer on buffer buf_idx's copy stream, behind the buffer's previous
        readers. Returns at once."""
        slot = self._slot(buf_idx)
        if not host_data.is_pinned():
            raise ValueError("StreamManager.prefetch: an asynchronous host->device copy needs pinned host_data "
                             "(e.g. a PinnedWeightStore view)")
        if tuple(gpu_buffer.shape) != tuple(host_data.shape):
            raise ValueError(f"StreamManager.prefetch: destination {tuple(gpu_buffer.shape)} and source "
                             f"{tuple(host_data.shape)} differ in shape")
        slot.start_copy(gpu_buffer, host_data)

    def wait(self, buf_idx: int) -> None:
        """Make the current stream wait (on the device) for buffer buf_idx's latest copy."""
        torch.cuda.current_stream().wait_event(self._slot(buf_idx).landed)

    def mark_read_done(self, buf_idx: int) -> None:
        """Declare that every kernel reading buffer buf_idx has been issued on the current stream; the next
        prefetch into the buffer waits for them to finish."""
        self._slot(buf_idx).release(torch.cuda.current_stream())

    def synchronize(self, buf_idx: int) -> None:
        """Block the host until buffer buf_idx's latest copy has landed."""
        self._slot(buf_idx).landed.synchronize()
