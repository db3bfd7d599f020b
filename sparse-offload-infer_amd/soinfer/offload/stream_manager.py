"""Copy streams with transfer-done and read-done events for double / triple buffered weight prefetch.

Same interface and semantics as the reference's StreamManager
(python/soinfer/offload/stream_manager.py:10-86): buffer i has its own copy
stream, an event marking "transfer into buffer i done" and an event marking
"the last reader of buffer i done". prefetch(i) first makes the copy stream
wait for buffer i's read-done event, so a new transfer never overwrites data a
kernel launched earlier is still reading (the write-after-read hazard the
reference hit once kernels got fast); wait(i) orders the current stream after
the transfer; mark_read_done(i) records the reader's completion point.

All streams use the default priority. On MI355X the copies are
hipMemcpyAsync from pinned host memory, executed by the SDMA engines.
"""
from __future__ import annotations

import torch


class StreamManager:
    def __init__(self, num_buffers: int = 2):
        if num_buffers < 1:
            raise ValueError("num_buffers must be >= 1")
        self.num_buffers = num_buffers
        self.streams = [torch.cuda.Stream() for _ in range(num_buffers)]
        self.events = [torch.cuda.Event() for _ in range(num_buffers)]
        # never recorded until the first mark_read_done: waiting on an unrecorded event is a no-op, which is
        # right for a buffer's first transfer
        self.read_done_events = [torch.cuda.Event() for _ in range(num_buffers)]

    def prefetch(self, buf_idx: int, gpu_buffer: torch.Tensor, host_data: torch.Tensor) -> None:
        """Asynchronous copy host_data (pinned) -> gpu_buffer on buffer buf_idx's stream, after that buffer's
        last reader; records the transfer-done event. Returns immediately."""
        if not host_data.is_pinned():
            raise ValueError("prefetch: host_data must be pinned (PinnedWeightStore) for an asynchronous copy")
        if gpu_buffer.shape != host_data.shape:
            raise ValueError(f"prefetch: gpu_buffer shape {tuple(gpu_buffer.shape)} != host_data shape "
                             f"{tuple(host_data.shape)}")
        stream = self.streams[buf_idx]
        stream.wait_event(self.read_done_events[buf_idx])
        with torch.cuda.stream(stream):
            gpu_buffer.copy_(host_data, non_blocking=True)
        self.events[buf_idx].record(stream)

    def wait(self, buf_idx: int) -> None:
        """Order the current stream after buffer buf_idx's transfer (a device-side wait, not a host sync)."""
        torch.cuda.current_stream().wait_event(self.events[buf_idx])

    def mark_read_done(self, buf_idx: int) -> None:
        """Record, on the current stream, that the kernels reading buffer buf_idx have been issued; the next
        prefetch into buf_idx waits for them."""
        self.read_done_events[buf_idx].record(torch.cuda.current_stream())

    def synchronize(self, buf_idx: int) -> None:
        """Host-side wait for buffer buf_idx's transfer (tests and timing)."""
        self.events[buf_idx].synchronize()
