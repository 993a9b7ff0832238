"""Storage backend: tensors in files on local storage (the role of
grinnder/storage/backend.py:21-163).

Every file is `{storage_dir}/{file_id}.pt` and holds the tensor's raw
row-major bytes, nothing else: the reference's format, so files written by
either side can be read by the other.

- Host side: IoUringEngine (grinnder_amd._C; a pread/pwrite thread pool),
  asynchronous, with integer handles for wait().
- Device side: the reference uses kvikio (GPUDirect Storage), which is not
  available here.  gpu_write / gpu_read stage the rows through a pinned host
  buffer: a D2H on the given stream, then a file write (and the reverse).
  Both return when the data is in place, as kvikio's calls do.
"""

from __future__ import annotations

import os
import shutil
from typing import Optional

import torch
from torch import Tensor

from grinnder_amd.utils import ensure_dir


class StorageBackend:
    def __init__(self, storage_dir: str, queue_depth: int = 64):
        from grinnder_amd._C import IoUringEngine

        self._storage_dir = ensure_dir(storage_dir)
        self._io_engine = IoUringEngine(queue_depth)

    @property
    def storage_dir(self) -> str:
        return self._storage_dir

    def _path(self, file_id: str) -> str:
        return os.path.join(self._storage_dir, f"{file_id}.pt")

    # ------------------------------------------------------------ device side

    @staticmethod
    def _stream(tensor: Tensor, stream: Optional[torch.cuda.Stream]) -> torch.cuda.Stream:
        s = stream if stream is not None else torch.cuda.current_stream(tensor.device)
        s.wait_stream(torch.cuda.current_stream(tensor.device))
        return s

    def gpu_write(self, tensor: Tensor, file_id: str,
                  stream: Optional[torch.cuda.Stream] = None) -> None:
        """Writes a device tensor's rows to the file (data only: no autograd)."""
        if not tensor.is_cuda:
            raise RuntimeError("gpu_write requires a GPU tensor")
        src = tensor.detach()
        staging = torch.empty(src.shape, dtype=src.dtype, pin_memory=True)
        s = self._stream(src, stream)
        with torch.cuda.stream(s):
            staging.copy_(src, non_blocking=True)
        s.synchronize()
        self.wait(self.host_write(staging, file_id))

    def gpu_read(self, file_id: str, tensor: Tensor,
                 stream: Optional[torch.cuda.Stream] = None) -> None:
        """Reads the file into a contiguous device tensor."""
        if not tensor.is_cuda or not tensor.is_contiguous():
            raise RuntimeError("gpu_read requires a contiguous GPU tensor")
        staging = torch.empty(tensor.shape, dtype=tensor.dtype, pin_memory=True)
        self.wait(self.host_read(file_id, staging))
        s = self._stream(tensor, stream)
        with torch.cuda.stream(s):
            tensor.copy_(staging, non_blocking=True)
        s.synchronize()

    # -------------------------------------------------------------- host side

    def host_write(self, tensor: Tensor, file_id: str, async_: bool = True) -> int:
        """Queues a write of a contiguous CPU tensor; returns its handle."""
        if tensor.is_cuda or not tensor.is_contiguous():
            raise RuntimeError("host_write requires a contiguous CPU tensor")
        h = self._io_engine.submit_write(self._path(file_id), tensor, 0,
                                         tensor.numel() * tensor.element_size())
        if not async_:
            self.wait(h)
        return h

    def host_read(self, file_id: str, tensor: Tensor, async_: bool = True) -> int:
        """Queues a read of the file into a contiguous CPU tensor; returns its handle."""
        if tensor.is_cuda or not tensor.is_contiguous():
            raise RuntimeError("host_read requires a contiguous CPU tensor")
        h = self._io_engine.submit_read(self._path(file_id), tensor, 0,
                                        tensor.numel() * tensor.element_size())
        if not async_:
            self.wait(h)
        return h

    def wait(self, handle: int) -> None:
        self._io_engine.wait(handle)

    def wait_all(self) -> None:
        self._io_engine.wait_all()

    # ------------------------------------------------------- file management

    def exists(self, file_id: str) -> bool:
        return os.path.exists(self._path(file_id))

    def remove(self, file_id: str) -> None:
        try:
            os.remove(self._path(file_id))
        except FileNotFoundError:
            pass

    def cleanup(self) -> None:
        """Removes every file under the storage directory."""
        self.wait_all()
        if os.path.exists(self._storage_dir):
            shutil.rmtree(self._storage_dir)
        ensure_dir(self._storage_dir)

    def file_size(self, file_id: str) -> int:
        path = self._path(file_id)
        return os.path.getsize(path) if os.path.exists(path) else 0
