"""DeviceBuffer: per-partition GPU tensors with lazy allocation (grinnder/buffer/device.py).

Tensor objects keep their logical shape; storage is resized to zero on
release so only the partitions in flight (double buffering) occupy HBM.
"""

from __future__ import annotations

from typing import List, Optional

import torch
from torch import Tensor

from grinnder_amd import _C
from grinnder_amd.buffer.host import HostBuffer


class DeviceBuffer:
    def __init__(self, num_parts: int, part_sizes: List[int], embedding_dim: int,
                 device: str = "cuda:0"):
        self.num_parts = num_parts
        self.part_sizes = list(part_sizes)
        self.embedding_dim = embedding_dim
        self.device = device
        self._tensors: List[Tensor] = []
        for i in range(num_parts):
            t = torch.empty(part_sizes[i], embedding_dim, dtype=torch.float32, device=device)
            t.untyped_storage().resize_(0)
            self._tensors.append(t)

    def __getitem__(self, pid: int) -> Tensor:
        return self._tensors[pid]

    def __len__(self) -> int:
        return self.num_parts

    def allocate(self, pid: int) -> Tensor:
        t = self._tensors[pid]
        nbytes = t.numel() * t.element_size()
        if t.untyped_storage().size() < nbytes:
            t.untyped_storage().resize_(nbytes)
        return t

    def release(self, pid: int) -> None:
        t = self._tensors[pid]
        t.untyped_storage().resize_(0)
        t.grad = None

    def is_allocated(self, pid: int) -> bool:
        return self._tensors[pid].untyped_storage().size() > 0

    def allocated_pids(self) -> List[int]:
        return [p for p in range(self.num_parts) if self.is_allocated(p)]

    @property
    def resident_bytes(self) -> int:
        return sum(t.untyped_storage().size() for t in self._tensors)

    def async_gather(self, pid: int, host_buffer: HostBuffer,
                     boundaries: List[Optional[Tensor]], stream: torch.cuda.Stream) -> None:
        self.allocate(pid)
        host_buffer.async_gather(pid, self._tensors[pid], boundaries, stream)

    def h2d_synchronize(self, stream: torch.cuda.Stream) -> None:
        _C.h2d_synchronize()
        stream.synchronize()

    def reset(self) -> None:
        for i in range(self.num_parts):
            self.release(i)
