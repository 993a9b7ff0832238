"""StorageTensor: one tensor that lives either in host memory or in a storage
file (the role of grinnder/storage/tensor.py:13-182).

State machine: 'host' (the rows are in a CPU tensor) and 'storage' (only the
file has them; no host memory is held).  Moves are asynchronous: to_storage /
to_host queue the I/O and the finish_* call (or synchronize) completes it;
with async_=False they complete at once.  Device copies are always transient
(to_gpu, fill_from_gpu).  Host memory is pageable unless pinned=True.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
from torch import Tensor


class StorageTensor:
    def __init__(self, shape: tuple, dtype: torch.dtype, backend, file_id: str,
                 pinned: bool = False):
        self._shape = tuple(shape)
        self._dtype = dtype
        self._backend = backend
        self._file_id = file_id
        self._pinned = bool(pinned) and torch.cuda.is_available()
        self._numel = math.prod(self._shape)
        self._element_size = torch.empty((), dtype=dtype).element_size()
        self._nbytes = self._numel * self._element_size
        self._host_tensor: Optional[Tensor] = self._new_host()
        self._location = "host"
        self._io_handle = -1

    # ------------------------------------------------------------------ state

    @property
    def shape(self) -> tuple:
        return self._shape

    @property
    def dtype(self) -> torch.dtype:
        return self._dtype

    @property
    def location(self) -> str:
        return self._location

    @property
    def file_id(self) -> str:
        return self._file_id

    @property
    def host_data(self) -> Tensor:
        if self._location != "host" or self._host_tensor is None:
            raise RuntimeError(f"{self._file_id}: the data is in storage; call to_host() first")
        return self._host_tensor

    def synchronize(self) -> None:
        """Completes the queued I/O, if any."""
        if self._io_handle >= 0:
            handle, self._io_handle = self._io_handle, -1
            self._backend.wait(handle)

    # ------------------------------------------------------------------ moves

    def to_storage(self, async_: bool = True) -> None:
        """Writes the host rows to the file; the host memory is dropped when
        the write completes (finish_to_storage)."""
        if self._location == "storage":
            return
        self.synchronize()
        self._io_handle = self._backend.host_write(self._host_tensor, self._file_id)
        if not async_:
            self.finish_to_storage()

    def finish_to_storage(self) -> None:
        self.synchronize()
        self._host_tensor = None
        self._location = "storage"

    def to_host(self, async_: bool = True) -> None:
        """Reads the file back into (new) host memory."""
        if self._location == "host":
            return
        self.synchronize()
        if self._host_tensor is None:
            self._host_tensor = self._new_host()
        self._io_handle = self._backend.host_read(self._file_id, self._host_tensor)
        if not async_:
            self.finish_to_host()

    def finish_to_host(self) -> None:
        self.synchronize()
        self._location = "host"

    # ----------------------------------------------------------- device side

    def to_gpu(self, target: Tensor, stream: Optional[torch.cuda.Stream] = None) -> None:
        """Copies the host rows into a device tensor (non-blocking on `stream`)."""
        src = self.host_data
        if stream is None:
            target.copy_(src)
            return
        with torch.cuda.stream(stream):
            target.copy_(src, non_blocking=True)

    def fill_from_gpu(self, source: Tensor, stream: Optional[torch.cuda.Stream] = None) -> None:
        """Copies a device tensor into the host rows (D2H)."""
        dst = self.host_data
        if stream is None:
            dst.copy_(source)
            return
        with torch.cuda.stream(stream):
            dst.copy_(source, non_blocking=True)

    def bypass_from_gpu(self, source: Tensor,
                        stream: Optional[torch.cuda.Stream] = None) -> None:
        """Writes a device tensor straight to the file; no host copy is kept."""
        self.synchronize()
        self._backend.gpu_write(source, self._file_id, stream)
        self._host_tensor = None
        self._location = "storage"

    def reset(self) -> None:
        """Back to host, zeroed."""
        if self._host_tensor is None:
            self._host_tensor = self._new_host()
        self._host_tensor.zero_()
        self._location = "host"
        self._io_handle = -1

    def _new_host(self) -> Tensor:
        return torch.empty(self._shape, dtype=self._dtype, pin_memory=self._pinned)

    def __repr__(self) -> str:
        return (f"StorageTensor(shape={self._shape}, dtype={self._dtype}, "
                f"location={self._location}, file_id={self._file_id})")
