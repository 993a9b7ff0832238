"""Activation checkpointing hooks (grinnder/autograd/checkpoint.py:31-83).

Used around ``torch.utils.checkpoint.checkpoint(fn, ..., x, use_reentrant=True)``
so that only the gathered input x is saved:

HongtuCheckpoint: pack copies x to host memory; unpack copies it back into
    the partition's device buffer (a snapshot per partition and layer).
ScatteredCheckpoint: pack keeps a reference to the device buffer only;
    unpack waits for the trainer's re-gather of x from the host buffers (no
    snapshot) and returns the buffer.
"""

from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd.graph import saved_tensors_hooks

from grinnder_amd.buffer.device import DeviceBuffer


class HongtuCheckpoint(saved_tensors_hooks):
    def __init__(self, pid: int, device_buffer: DeviceBuffer):
        def pack(tensor: Tensor):
            return (tensor.device, tensor.cpu(), device_buffer)

        def unpack(packed):
            _, cpu_tensor, dbuf = packed
            dbuf.allocate(pid)
            dbuf[pid].copy_(cpu_tensor)
            return dbuf[pid]

        super().__init__(pack, unpack)


class ScatteredCheckpoint(saved_tensors_hooks):
    def __init__(self, pid: int, device_buffer: DeviceBuffer, h2d_stream: torch.cuda.Stream):
        def pack(tensor: Tensor):
            assert tensor is device_buffer[pid], (
                "ScatteredCheckpoint: saved tensor is not device_buffer[pid]")
            return (tensor.device, device_buffer, h2d_stream)

        def unpack(packed):
            _, dbuf, stream = packed
            dbuf.h2d_synchronize(stream)
            torch.cuda.current_stream().wait_stream(stream)
            return dbuf[pid]

        super().__init__(pack, unpack)
