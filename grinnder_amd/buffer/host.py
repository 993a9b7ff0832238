"""HostBuffer: one layer of per-partition host tensors (grinnder/buffer/host.py:55-478).

Transfers go through the native op table (grinnder_amd._C).  With
``pin_memory=True`` (what the Trainer uses) partitions live in pinned host
memory, so the halo gather and the gradient scatter-add run as device kernels
reading / updating the host rows in place over PCIe.  Synchronisation waits
on the transfer stream only, never on the whole device.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional

import torch
from torch import Tensor

from grinnder_amd import _C, _lib


PINNED_STATS = {"bytes": 0, "blocks": 0, "fallbacks": 0, "fallback_bytes": 0}


class _PinnedBlock:
    """Owns one exact-size pinned host allocation (gr_host_alloc).

    Ownership runs one way, tensor -> ctypes array -> block, so the
    allocation is released as soon as the last tensor over it dies, not at
    some later cyclic garbage collection (a dropped Trainer would otherwise
    keep tens of GB pinned)."""

    def __init__(self, nbytes: int):
        ptr = ctypes.c_void_p()
        _lib.call("gr_host_alloc", nbytes, ctypes.byref(ptr))
        self.ptr = ptr.value
        PINNED_STATS["bytes"] += nbytes
        PINNED_STATS["blocks"] += 1
        self.nbytes = nbytes

    def array(self) -> ctypes.Array:
        """A ctypes view of the block that keeps the block alive."""
        arr = (ctypes.c_char * self.nbytes).from_address(self.ptr)
        arr._owner = self
        return arr

    def __del__(self):
        ptr = getattr(self, "ptr", None)
        if ptr:
            self.ptr = None
            try:
                PINNED_STATS["bytes"] -= self.nbytes
                PINNED_STATS["blocks"] -= 1
                _lib.load().gr_host_free(ptr)
            except Exception:  # interpreter shutdown: the process frees it anyway
                pass


def pinned_empty(rows: int, cols: int) -> Tensor:
    """Exact-size pinned fp32 host tensor; pageable if pinning is refused
    (the reference's HostBuffer also falls back, grinnder/buffer/host.py:36-45)."""
    nbytes = rows * cols * 4
    if nbytes == 0:
        return torch.empty((rows, cols), dtype=torch.float32)
    try:
        block = _PinnedBlock(nbytes)
    except _lib.GrError:
        PINNED_STATS["fallbacks"] += 1
        PINNED_STATS["fallback_bytes"] += nbytes
        return torch.empty((rows, cols), dtype=torch.float32)
    return torch.frombuffer(block.array(), dtype=torch.float32).view(rows, cols)


def _empty_host_tensor(rows: int, cols: int, *, pin_memory: bool, allocate: bool) -> Tensor:
    if not allocate:
        return torch.empty((0, cols), dtype=torch.float32)
    if pin_memory:
        return pinned_empty(rows, cols)
    return torch.empty((rows, cols), dtype=torch.float32)


def _none_to_empty(pid: int, boundaries: List[Optional[Tensor]], num_parts: int) -> List[Tensor]:
    out = []
    for i in range(num_parts):
        b = boundaries[i] if i < len(boundaries) else None
        out.append(torch.empty(0, dtype=torch.long) if (i == pid or b is None) else b)
    return out


class HostBuffer:
    """Partition-wise fp32 tensors on the host.

    Gather layout on the device: [intra(pid) | boundary_from_p0 | ... ]; the
    scatter uses the same layout and accumulates (+=) into host partitions.
    Storage is allocated lazily per partition and can be released.
    """

    def __init__(self, num_parts: int, part_sizes: List[int], embedding_dim: int,
                 backend=None, file_prefix: str = "host", lazy: bool = True,
                 pin_memory: bool = False):
        self._backend = backend
        self.num_parts = num_parts
        self.part_sizes = list(part_sizes)
        self.embedding_dim = embedding_dim
        self._file_prefix = file_prefix
        self._element_size = 4
        self._lazy = lazy
        self._pin_memory = pin_memory
        self._zero_initialized = [False] * num_parts
        # Partitions whose host rows may differ from their storage copy (the
        # copy is rewritten before such a partition is evicted).
        self._dirty = [False] * num_parts
        self._tensors: List[Tensor] = []
        # D2H entries (fills, scatters) this buffer queued and nobody waited
        # for yet; the library's D2H completion queue is FIFO.
        self.d2h_queued = 0
        for i in range(num_parts):
            t = _empty_host_tensor(part_sizes[i], embedding_dim, pin_memory=pin_memory,
                                   allocate=not lazy)
            if not lazy:
                t.zero_()
                self._zero_initialized[i] = True
            self._tensors.append(t)

    def __getitem__(self, pid: int) -> Tensor:
        self.allocate(pid)
        self._dirty[pid] = True  # the caller may write through the tensor
        return self._tensors[pid]

    def __len__(self) -> int:
        return self.num_parts

    def partition_nbytes(self, pid: int) -> int:
        return self.part_sizes[pid] * self.embedding_dim * self._element_size

    @property
    def total_nbytes(self) -> int:
        return sum(self.partition_nbytes(p) for p in range(self.num_parts))

    def allocate(self, pid: int) -> Tensor:
        t = self._tensors[pid]
        expected = self.partition_nbytes(pid)
        if t.untyped_storage().size() < expected:
            if self._pin_memory:
                t = pinned_empty(self.part_sizes[pid], self.embedding_dim)
                self._tensors[pid] = t
            else:
                t.untyped_storage().resize_(expected)
        shape = (self.part_sizes[pid], self.embedding_dim)
        if tuple(t.shape) != shape:
            t.set_(t.untyped_storage(), 0, shape, (self.embedding_dim, 1))
        return t

    def release(self, pid: int) -> None:
        self._tensors[pid] = _empty_host_tensor(self.part_sizes[pid], self.embedding_dim,
                                                pin_memory=self._pin_memory, allocate=False)
        self._zero_initialized[pid] = False
        self._dirty[pid] = False

    def release_all(self) -> None:
        for pid in range(self.num_parts):
            self.release(pid)

    def is_allocated(self, pid: int) -> bool:
        return self._tensors[pid].untyped_storage().size() >= self.partition_nbytes(pid)

    def allocated_pids(self) -> List[int]:
        return [p for p in range(self.num_parts) if self.is_allocated(p)]

    def zero_partition(self, pid: int) -> None:
        self.allocate(pid).zero_()
        self._zero_initialized[pid] = True
        self._dirty[pid] = True

    @property
    def resident_bytes(self) -> int:
        return sum(self.partition_nbytes(p) for p in range(self.num_parts)
                   if self.is_allocated(p))

    # ---------------------------------------------------------- GPU -> host

    def async_fill(self, pid: int, gpu_data: Tensor, stream: torch.cuda.Stream) -> None:
        """D2H copy of a partition's [B, D] device tensor into host partition pid."""
        assert gpu_data.is_cuda
        self.allocate(pid)
        stream.wait_stream(torch.cuda.current_stream(gpu_data.device))
        with torch.cuda.stream(stream):
            _C.d2h_copy_async(gpu_data.contiguous(), self._tensors[pid])
        self.d2h_queued += 1
        self._zero_initialized[pid] = True
        self._dirty[pid] = True

    def d2h_synchronize(self, stream: torch.cuda.Stream) -> None:
        """Waits for the oldest queued D2H entry, then for `stream` itself."""
        self.d2h_wait_oldest()
        stream.synchronize()

    def d2h_wait_oldest(self) -> None:
        """Waits for the oldest queued D2H entry only (no stream synchronize)."""
        _C.d2h_synchronize()
        self.d2h_queued = max(0, self.d2h_queued - 1)

    # ---------------------------------------------------------- host -> GPU

    def async_upload(self, pid: int, gpu_target: Tensor, stream: torch.cuda.Stream) -> None:
        assert gpu_target.is_cuda
        if not self.is_allocated(pid):
            raise RuntimeError(f"HostBuffer partition {pid} is not resident for upload")
        stream.wait_stream(torch.cuda.current_stream(gpu_target.device))
        with torch.cuda.stream(stream):
            _C.h2d_copy_async(self._tensors[pid], gpu_target)

    def h2d_synchronize(self, stream: torch.cuda.Stream) -> None:
        _C.h2d_synchronize()
        stream.synchronize()

    # ---------------------------------------------------------------- gather

    def async_gather(self, pid: int, gpu_target: Tensor, boundaries: List[Optional[Tensor]],
                     stream: torch.cuda.Stream) -> None:
        """gpu_target = [self[pid] | self[p][boundaries[p]] for p ascending]."""
        assert gpu_target.is_cuda
        required = {pid}
        for p, b in enumerate(boundaries):
            if p != pid and b is not None and b.numel() > 0:
                required.add(p)
        missing = [p for p in sorted(required) if not self.is_allocated(p)]
        if missing:
            raise RuntimeError(f"HostBuffer partitions {missing} are not resident for gather")
        bnd = _none_to_empty(pid, boundaries, self.num_parts)
        stream.wait_stream(torch.cuda.current_stream(gpu_target.device))
        with torch.cuda.stream(stream):
            _C.gather_partitions(pid, self._tensors, gpu_target, bnd)

    # --------------------------------------------------------------- scatter

    def async_scatter(self, pid: int, gpu_source: Tensor, boundaries: List[Optional[Tensor]],
                      stream: torch.cuda.Stream) -> None:
        """Accumulates gpu_source (gather layout) into the host partitions."""
        assert gpu_source.is_cuda
        for p, b in enumerate(boundaries):
            if p == pid or (b is not None and b.numel() > 0):
                self.allocate(p)
                if not self._zero_initialized[p]:
                    self._tensors[p].zero_()
                    self._zero_initialized[p] = True
                self._dirty[p] = True
        bnd = _none_to_empty(pid, boundaries, self.num_parts)
        with torch.cuda.stream(stream):
            _C.scatter_partitions(pid, gpu_source, self._tensors, bnd)
        self.d2h_queued += 1

    # ------------------------------------------------------------- utilities

    def initialize_zeros(self, lazy: bool = False) -> None:
        """Every partition becomes zero: now, or (lazy) when first touched;
        storage copies of the old values are dropped."""
        if lazy:
            self.release_all()
            if self._backend is not None:
                for pid in range(self.num_parts):
                    self._backend.remove(self._file_id(pid))
            return
        for pid in range(self.num_parts):
            self.allocate(pid).zero_()
            self._zero_initialized[pid] = True
            self._dirty[pid] = True

    def reset(self) -> None:
        self.initialize_zeros()

    # ------------------------------------------------- host <-> storage files

    def attach_backend(self, backend) -> None:
        """Gives the buffer a storage backend after construction (the
        trainer sets up the storage tier only when host memory is short)."""
        self._backend = backend

    def _file_id(self, pid: int) -> str:
        return f"{self._file_prefix}_p{pid}"

    def _require_backend(self, what: str):
        if self._backend is None:
            raise RuntimeError(f"HostBuffer.{what}: no storage backend")
        return self._backend

    def storage_exists(self, pid: int) -> bool:
        """Whether partition pid has a copy in storage."""
        return self._backend is not None and self._backend.exists(self._file_id(pid))

    def ensure_storage_copy(self, pid: int) -> None:
        """Writes a resident partition to storage unless an up-to-date copy
        exists there (the reference skips the write whenever any copy exists,
        which would drop rows that changed since it was written)."""
        if self._backend is None:
            return
        if self.storage_exists(pid) and not (self.is_allocated(pid) and self._dirty[pid]):
            return
        if not self.is_allocated(pid):
            raise RuntimeError(f"HostBuffer partition {pid} is neither resident nor in storage")
        self.cpu_to_storage(pid)

    def _pids(self, pid: Optional[int]) -> List[int]:
        return list(range(self.num_parts)) if pid is None else [pid]

    def storage_to_cpu(self, pid: Optional[int] = None) -> None:
        """Loads partition pid (all partitions with a storage copy, when pid is
        None) from storage into host memory, allocating it again if it was
        released.  The reads run in parallel; returns when they are done."""
        backend = self._require_backend("storage_to_cpu")
        pids = self._pids(pid)
        if pid is None:
            pids = [p for p in pids if self.storage_exists(p)]
        handles = [backend.host_read(self._file_id(p), self.allocate(p)) for p in pids]
        for h in handles:
            backend.wait(h)
        for p in pids:
            self._zero_initialized[p] = True
            self._dirty[p] = False

    def cpu_to_storage(self, pid: Optional[int] = None) -> None:
        """Writes partition pid (every partition, when pid is None) to storage;
        returns when the writes are done.  Host memory is kept."""
        backend = self._require_backend("cpu_to_storage")
        pids = self._pids(pid)
        handles = [backend.host_write(self.allocate(p), self._file_id(p)) for p in pids]
        for h in handles:
            backend.wait(h)
        for p in pids:
            self._dirty[p] = False

    def async_bypass_to_storage(self, pid: int, gpu_data: Tensor,
                                stream: torch.cuda.Stream) -> None:
        """Writes a partition's device rows straight to storage, without a
        resident host copy (the reference's GPUDirect bypass,
        grinnder/buffer/host.py:392-405): ordered after the current stream's
        work, on `stream`, complete on return."""
        backend = self._require_backend("async_bypass_to_storage")
        stream.wait_stream(torch.cuda.current_stream(gpu_data.device))
        backend.gpu_write(gpu_data, self._file_id(pid), stream)
