"""What stands in for a checkpointed layer's input between its forward and
its backward (the role of grinnder/autograd/checkpoint.py:31-83).

The trainer runs each partition's layer under
``torch.utils.checkpoint.checkpoint(..., use_reentrant=True)``, which saves
only the layer's gathered input rows.  These saved-tensor hooks replace that
tensor by a small handle with one method, ``restore()``, called when the
backward recomputes the layer:

- ``ScatteredCheckpoint`` (GriNNder mode) keeps nothing.  Its handle names
  the partition's block in a DeviceBuffer; before the backward the trainer
  gathers the partition's rows into that buffer again, and ``restore`` waits
  for that gather's stream and hands out the block.
- ``HongtuCheckpoint`` (the HongTu baseline) snapshots the rows to pinned
  host memory on the current stream, and ``restore`` copies them back into a
  fresh block of the buffer, ordered after the snapshot by an event.

The block handed out by ``restore`` is a new tensor, so it is given the
``requires_grad`` flag the saved input had: the recompute must see the
input as differentiable for GradOffload's backward (the halo-gradient
scatter) to run.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor
from torch.autograd.graph import saved_tensors_hooks

from grinnder_amd.buffer.device import DeviceBuffer


@dataclass(frozen=True)
class RegatherHandle:
    """The saved input is re-gathered into `buffer` on `stream` by the trainer."""

    buffer: DeviceBuffer
    pid: int
    stream: torch.cuda.Stream
    requires_grad: bool

    def restore(self) -> Tensor:
        self.buffer.h2d_synchronize(self.stream)
        torch.cuda.current_stream().wait_stream(self.stream)
        return self.buffer[self.pid].requires_grad_(self.requires_grad)


@dataclass(frozen=True)
class HostSnapshot:
    """The saved input's rows, held in host memory until the backward."""

    buffer: DeviceBuffer
    pid: int
    rows: Tensor
    copied: torch.cuda.Event
    requires_grad: bool

    @staticmethod
    def take(buffer: DeviceBuffer, pid: int, t: Tensor) -> "HostSnapshot":
        rows = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        rows.copy_(t.detach(), non_blocking=True)
        copied = torch.cuda.Event()
        copied.record()
        return HostSnapshot(buffer, pid, rows, copied, t.requires_grad)

    def restore(self) -> Tensor:
        block = self.buffer.allocate(self.pid)
        torch.cuda.current_stream().wait_event(self.copied)
        block.copy_(self.rows, non_blocking=True)
        return block.requires_grad_(self.requires_grad)


def _restore(handle) -> Tensor:
    return handle.restore()


class ScatteredCheckpoint(saved_tensors_hooks):
    def __init__(self, pid: int, device_buffer: DeviceBuffer, h2d_stream: torch.cuda.Stream):
        def pack(t: Tensor) -> RegatherHandle:
            if not (device_buffer.is_allocated(pid) and t is device_buffer[pid]):
                raise RuntimeError(
                    f"ScatteredCheckpoint: the saved tensor is not partition {pid}'s block of "
                    "the device buffer, so it could not be gathered again")
            return RegatherHandle(device_buffer, pid, h2d_stream, t.requires_grad)

        super().__init__(pack, _restore)


class HongtuCheckpoint(saved_tensors_hooks):
    def __init__(self, pid: int, device_buffer: DeviceBuffer):
        def pack(t: Tensor) -> HostSnapshot:
            return HostSnapshot.take(device_buffer, pid, t)

        super().__init__(pack, _restore)
