"""The reference's native op table (grinnder._C, csrc/grinnder_ops.cpp:7-34) on the C ABI.

Same names, argument meaning and preconditions as the pybind module, so the
buffer and autograd layers call them unchanged:

  h2d_copy_async(src_cpu, dst_gpu)           csrc/cuda/async_transfer.cu:40-58
  d2h_copy_async(src_gpu, dst_cpu)           :20-38
  h2d_synchronize() / d2h_synchronize()      :17-18 (oldest queued entry)
  gather_partitions(pid, srcs, dst, bnds)    :60-120
  scatter_partitions(pid, src, dsts, bnds)   :122-186
  build_subgraph(rowptr, col, value, idx, bipartite)   csrc/cpu/subgraph.cpp

Differences by design: work is enqueued on the current stream from the
calling thread (no worker thread is needed for pinned buffers), errors are
raised immediately or by the next *_synchronize (never swallowed), and
pinned host partitions are moved by device kernels over PCIe.

  IoUringEngine(queue_depth)                 csrc/cpu/io_uring_engine.cpp:15-245
      submit_read / submit_write(path, tensor, offset, nbytes) -> handle,
      wait(handle), wait_all(), poll(handle), pending(), has_io_uring()
      The storage tier's host <-> file engine.  liburing is absent, so
      requests run on a pread/pwrite thread pool (gr_io_*); has_io_uring()
      is therefore False.  Failed or short transfers raise at wait().
"""

from __future__ import annotations

from typing import List, Optional

import torch
from torch import Tensor

from grinnder_amd import _lib
from grinnder_amd.aggregation import KernelTimer
from grinnder_amd.data.partition import build_subgraph  # noqa: F401  (re-export)

__all__ = [
    "h2d_copy_async", "d2h_copy_async", "h2d_synchronize", "d2h_synchronize",
    "gather_partitions", "scatter_partitions", "build_subgraph", "IoUringEngine",
]


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _nondefault_stream(device: torch.device, what: str) -> torch.cuda.Stream:
    stream = torch.cuda.current_stream(device)
    _require(stream != torch.cuda.default_stream(device),
             f"Async {what} requires a non-default CUDA stream")
    return stream


def _check_same_dtype(a: Tensor, b: Tensor) -> None:
    _require(a.dtype == b.dtype, f"dtype mismatch: {a.dtype} vs {b.dtype}")


def d2h_copy_async(src: Tensor, dst: Tensor) -> None:
    _require(src.is_cuda, "Source must be a CUDA tensor")
    _require(not dst.is_cuda, "Destination must be a CPU tensor")
    _require(src.is_contiguous(), "Source must be contiguous")
    _require(dst.is_contiguous(), "Destination must be contiguous")
    _check_same_dtype(src, dst)
    _require(src.numel() == dst.numel(), "d2h_copy_async: size mismatch")
    stream = _nondefault_stream(src.device, "D2H")
    _lib.call("gr_d2h_copy_async", src.data_ptr(), dst.data_ptr(),
              src.numel() * src.element_size(), stream.cuda_stream)


def h2d_copy_async(src: Tensor, dst: Tensor) -> None:
    _require(not src.is_cuda, "Source must be a CPU tensor")
    _require(dst.is_cuda, "Destination must be a CUDA tensor")
    _require(src.is_contiguous(), "Source must be contiguous")
    _require(dst.is_contiguous(), "Destination must be contiguous")
    _check_same_dtype(src, dst)
    _require(src.numel() == dst.numel(), "h2d_copy_async: size mismatch")
    stream = _nondefault_stream(dst.device, "H2D")
    _lib.call("gr_h2d_copy_async", src.data_ptr(), dst.data_ptr(),
              src.numel() * src.element_size(), stream.cuda_stream)


def h2d_synchronize() -> None:
    _lib.call("gr_h2d_synchronize")


def d2h_synchronize() -> None:
    _lib.call("gr_d2h_synchronize")


def _boundary_arrays(pid: int, boundaries: List[Optional[Tensor]], num_parts: int):
    _require(len(boundaries) == num_parts, "boundaries must have one entry per partition")
    keep = []
    ptrs, lens = [], []
    for p, b in enumerate(boundaries):
        if p == pid or b is None or b.numel() == 0:
            ptrs.append(None)
            lens.append(0)
            continue
        _require(not b.is_cuda, "boundaries must be CPU tensors")
        b = b.to(torch.int64).contiguous()
        keep.append(b)
        ptrs.append(b.data_ptr())
        lens.append(b.numel())
    return keep, _lib.ptr_array(ptrs), _lib.i64_array(lens)


def gather_partitions(pid: int, srcs: List[Tensor], dst: Tensor,
                      boundaries: List[Optional[Tensor]]) -> None:
    """dst = [srcs[pid] | srcs[p][boundaries[p]] for p ascending, p != pid]."""
    _require(dst.is_cuda, "Destination must be a CUDA tensor")
    _require(dst.is_contiguous(), "Destination must be contiguous")
    for s in srcs:
        _require(not s.is_cuda, "Sources must be CPU tensors")
        _require(s.is_contiguous(), "Sources must be contiguous")
        _check_same_dtype(s, dst)
    stream = _nondefault_stream(dst.device, "gather")
    P = len(srcs)
    row_bytes = (dst.numel() // max(dst.size(0), 1)) * dst.element_size() if dst.dim() else 0
    for s in srcs:
        if s.numel():
            _require(s.numel() // s.size(0) * s.element_size() == row_bytes,
                     "Gather: source row width differs from destination")
    keep, bptr, blen = _boundary_arrays(pid, boundaries, P)
    src_ptrs = _lib.ptr_array([s.data_ptr() if s.numel() else None for s in srcs])
    src_rows = _lib.i64_array([s.size(0) if s.dim() else 0 for s in srcs])
    with KernelTimer.region("halo_gather", dst.size(0) * row_bytes, 0, row_bytes // 4):
        _lib.call("gr_gather_partitions", pid, P, src_ptrs, src_rows, dst.data_ptr(),
                  dst.size(0), max(row_bytes, 1), bptr, blen, stream.cuda_stream)
    del keep


def scatter_partitions(pid: int, src: Tensor, dsts: List[Tensor],
                       boundaries: List[Optional[Tensor]]) -> None:
    """fp32 accumulate: dsts[pid] += src[:B]; dsts[p][boundaries[p]] += next rows."""
    _require(src.is_cuda, "Source must be a CUDA tensor")
    _require(src.is_contiguous(), "Source must be contiguous")
    _require(src.dtype == torch.float32, "scatter_partitions supports float32")
    for d in dsts:
        _require(not d.is_cuda, "Destinations must be CPU tensors")
        _require(d.is_contiguous(), "Destinations must be contiguous")
        _check_same_dtype(d, src)
    stream = _nondefault_stream(src.device, "scatter")
    P = len(dsts)
    dim = src.numel() // max(src.size(0), 1)
    keep, bptr, blen = _boundary_arrays(pid, boundaries, P)
    dst_ptrs = _lib.ptr_array([d.data_ptr() if d.numel() else None for d in dsts])
    dst_rows = _lib.i64_array([d.size(0) for d in dsts])
    with KernelTimer.region("halo_scatter", src.numel() * 4, 0, dim):
        _lib.call("gr_scatter_partitions", pid, P, src.data_ptr(), src.size(0), max(dim, 1),
                  dst_ptrs, dst_rows, bptr, blen, stream.cuda_stream)
    del keep


class IoUringEngine:
    """Asynchronous host <-> file I/O (the reference's IoUringEngine API).

    `queue_depth` bounds the worker threads (at most 16): each request is
    split into 8 MiB chunks that the workers read or write in parallel.
    A submitted tensor must stay alive, and unchanged for a write, until
    the request is waited for; the engine keeps a reference to it until then.
    """

    def __init__(self, queue_depth: int = 64):
        import ctypes

        if queue_depth < 1:
            raise ValueError("queue_depth must be >= 1")
        handle = ctypes.c_void_p()
        _lib.call("gr_io_create", max(1, min(16, int(queue_depth))), ctypes.byref(handle))
        self._engine = handle.value
        self._inflight = {}

    def has_io_uring(self) -> bool:
        return False

    def _submit(self, write: bool, path: str, tensor: Tensor, offset: int, nbytes: int) -> int:
        import ctypes

        what = "submit_write" if write else "submit_read"
        _require(not tensor.is_cuda, f"{what}: tensor must be on CPU")
        _require(tensor.is_contiguous(), f"{what}: tensor must be contiguous")
        _require(0 <= nbytes <= tensor.numel() * tensor.element_size(),
                 f"{what}: {nbytes} bytes do not fit the tensor")
        h = ctypes.c_int64()
        _lib.call("gr_io_submit", self._engine, int(write), str(path).encode(),
                  tensor.data_ptr() if nbytes else None, int(offset), int(nbytes),
                  ctypes.byref(h))
        self._inflight[h.value] = tensor
        return h.value

    def submit_read(self, path: str, tensor: Tensor, offset: int, nbytes: int) -> int:
        return self._submit(False, path, tensor, offset, nbytes)

    def submit_write(self, path: str, tensor: Tensor, offset: int, nbytes: int) -> int:
        return self._submit(True, path, tensor, offset, nbytes)

    def wait(self, handle: int) -> None:
        try:
            _lib.call("gr_io_wait", self._engine, int(handle))
        finally:
            self._inflight.pop(handle, None)

    def wait_all(self) -> None:
        try:
            _lib.call("gr_io_wait_all", self._engine)
        finally:
            self._inflight.clear()

    def poll(self, handle: int) -> bool:
        import ctypes

        done = ctypes.c_int32()
        _lib.call("gr_io_poll", self._engine, int(handle), ctypes.byref(done))
        return bool(done.value)

    def pending(self) -> int:
        import ctypes

        n = ctypes.c_int64()
        _lib.call("gr_io_pending", self._engine, ctypes.byref(n))
        return int(n.value)

    def __del__(self):
        engine = getattr(self, "_engine", None)
        if engine:
            self._engine = None
            try:
                _lib.load().gr_io_destroy(engine)
            except Exception:  # interpreter shutdown
                pass
