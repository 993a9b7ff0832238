"""HBM blocks of one layer's per-partition rows (the role of grinnder/buffer/device.py).

A partition's block exists only while the partition is in flight.
``allocate`` creates it from torch's caching allocator, on the current
stream like any tensor; ``release`` drops it and returns its storage at
once, even if a stale Python reference to the tensor is still around.  A
double-buffered epoch therefore holds at most a few partitions of a layer
in HBM.  Blocks are fp32 [rows, dim], rows = the partition's size in this
buffer (expanded sizes for gathered inputs, partition sizes for gradients).
"""

from __future__ import annotations

from typing import Dict, List, Optional

import torch
from torch import Tensor

from grinnder_amd import _C
from grinnder_amd.buffer.host import HostBuffer


class DeviceBuffer:
    def __init__(self, num_parts: int, part_sizes: List[int], embedding_dim: int,
                 device: str = "cuda:0"):
        if len(part_sizes) != num_parts:
            raise ValueError(f"{len(part_sizes)} partition sizes for {num_parts} partitions")
        self.num_parts = num_parts
        self.part_sizes = [int(s) for s in part_sizes]
        self.embedding_dim = int(embedding_dim)
        self.device = torch.device(device)
        self._blocks: Dict[int, Tensor] = {}

    def __len__(self) -> int:
        return self.num_parts

    def __getitem__(self, pid: int) -> Tensor:
        """The partition's block; without one, a shape-only (meta) tensor of
        the partition's logical shape, which holds no memory."""
        block = self._blocks.get(pid)
        if block is not None:
            return block
        if not 0 <= pid < self.num_parts:
            raise IndexError(f"partition {pid} outside [0, {self.num_parts})")
        return torch.empty((self.part_sizes[pid], self.embedding_dim), dtype=torch.float32,
                           device="meta")

    def allocate(self, pid: int) -> Tensor:
        """The partition's block, created on first use."""
        block = self._blocks.get(pid)
        if block is None:
            if not 0 <= pid < self.num_parts:
                raise IndexError(f"partition {pid} outside [0, {self.num_parts})")
            block = torch.empty((self.part_sizes[pid], self.embedding_dim),
                                dtype=torch.float32, device=self.device)
            self._blocks[pid] = block
        return block

    def release(self, pid: int) -> None:
        block = self._blocks.pop(pid, None)
        if block is not None:
            block.grad = None
            block.untyped_storage().resize_(0)

    def is_allocated(self, pid: int) -> bool:
        return pid in self._blocks

    def allocated_pids(self) -> List[int]:
        return sorted(self._blocks)

    @property
    def resident_bytes(self) -> int:
        return sum(b.untyped_storage().nbytes() for b in self._blocks.values())

    def async_gather(self, pid: int, host_buffer: HostBuffer,
                     boundaries: List[Optional[Tensor]], stream: torch.cuda.Stream) -> None:
        """Queues the partition's [intra | halo] rows from the host buffers
        into its block on `stream` (see HostBuffer.async_gather)."""
        host_buffer.async_gather(pid, self.allocate(pid), boundaries, stream)

    def h2d_synchronize(self, stream: torch.cuda.Stream) -> None:
        """Waits for the oldest queued upload (errors are raised, not
        swallowed) and for `stream`."""
        _C.h2d_synchronize()
        stream.synchronize()

    def reset(self) -> None:
        for pid in list(self._blocks):
            self.release(pid)
