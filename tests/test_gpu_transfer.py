"""GPU: the grinnder._C transfer ops (h2d/d2h, halo gather, gradient scatter-add)
against the reference's fixtures and the oracle, for pinned and pageable
host partitions.  Gather/scatter are integer/byte work: bit-exact."""

import numpy as np
import pytest
import torch

import oracle
from grinnder_amd import _C
from grinnder_amd._lib import GrError
from grinnder_amd.buffer.host import HostBuffer

pytestmark = pytest.mark.gpu


def _on_side_stream(fn):
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        fn()
    s.synchronize()


def test_h2d_d2h_copy(gpu):
    """tests/test_cpp_extensions.py:117-142."""
    for pinned in (True, False):
        src = torch.randn(10, 4, pin_memory=pinned)
        dst = torch.empty(10, 4, device=gpu)
        _on_side_stream(lambda: _C.h2d_copy_async(src, dst))
        _C.h2d_synchronize()
        assert torch.equal(dst.cpu(), src)
        back = torch.empty(10, 4, pin_memory=pinned)
        _on_side_stream(lambda: _C.d2h_copy_async(dst, back))
        _C.d2h_synchronize()
        assert torch.equal(back, src)


def test_default_stream_rejected(gpu):
    """The reference asserts a non-default current stream (async_transfer.cu:27,47)."""
    with pytest.raises(RuntimeError):
        _C.h2d_copy_async(torch.zeros(2), torch.zeros(2, device=gpu))


@pytest.mark.parametrize("pinned", [True, False])
def test_gather_reference_fixture(gpu, pinned):
    """tests/test_cpp_extensions.py:144-171 (arange partitions, pid 0)."""
    p0 = torch.arange(8, dtype=torch.float).reshape(4, 2)
    p1 = torch.arange(8, 14, dtype=torch.float).reshape(3, 2)
    p2 = torch.arange(14, 24, dtype=torch.float).reshape(5, 2)
    srcs = [t.pin_memory() if pinned else t for t in (p0, p1, p2)]
    bnd = [torch.empty(0, dtype=torch.long), torch.tensor([0, 2]), torch.tensor([3])]
    dst = torch.empty(7, 2, device=gpu)
    _on_side_stream(lambda: _C.gather_partitions(0, srcs, dst, bnd))
    _C.h2d_synchronize()
    assert dst.cpu().tolist() == [[0, 1], [2, 3], [4, 5], [6, 7], [8, 9], [12, 13], [20, 21]]


@pytest.mark.parametrize("pinned", [True, False])
def test_scatter_reference_fixture(gpu, pinned):
    """tests/test_cpp_extensions.py:173-202 and tests/test_host_buffer_ops.py:40-60."""
    dsts = [torch.zeros(4, 2), torch.zeros(3, 2), torch.zeros(5, 2)]
    if pinned:
        dsts = [d.pin_memory() for d in dsts]
    bnd = [torch.empty(0, dtype=torch.long), torch.tensor([0, 2]), torch.tensor([3])]
    src = torch.ones(7, 2, device=gpu)
    _on_side_stream(lambda: _C.scatter_partitions(0, src, dsts, bnd))
    _C.d2h_synchronize()
    assert torch.equal(dsts[0], torch.ones(4, 2))
    assert dsts[1].tolist() == [[1, 1], [0, 0], [1, 1]]
    assert dsts[2][3].tolist() == [1, 1] and float(dsts[2].sum()) == 2.0
    dsts[0].fill_(1.0)
    src2 = torch.full((7, 2), 2.0, device=gpu)
    _on_side_stream(lambda: _C.scatter_partitions(0, src2, dsts, bnd))
    _C.d2h_synchronize()
    assert torch.equal(dsts[0], torch.full((4, 2), 3.0))


def _random_layout(seed, P=5, dim=37):
    g = torch.Generator().manual_seed(seed)
    sizes = [int(x) for x in torch.randint(50, 400, (P,), generator=g)]
    srcs = [torch.randn(n, dim, generator=g) for n in sizes]
    pid = seed % P
    bnd = []
    for p in range(P):
        if p == pid or (p + seed) % 4 == 0:
            bnd.append(None)
        else:
            k = int(torch.randint(1, sizes[p], (1,), generator=g))
            bnd.append(torch.randperm(sizes[p], generator=g)[:k])
    return pid, srcs, bnd


@pytest.mark.parametrize("seed,pinned,dim", [(0, True, 37), (1, False, 37), (2, True, 100),
                                             (3, True, 256), (4, False, 64)])
def test_gather_scatter_match_oracle(gpu, seed, pinned, dim):
    pid, srcs, bnd = _random_layout(seed, dim=dim)
    if pinned:
        srcs = [s.pin_memory() for s in srcs]
    ref = oracle.gather_partitions(pid, srcs, bnd)
    dst = torch.empty(ref.shape, device=gpu)
    b64 = [torch.empty(0, dtype=torch.long) if b is None else b for b in bnd]
    _on_side_stream(lambda: _C.gather_partitions(pid, srcs, dst, b64))
    _C.h2d_synchronize()
    assert np.array_equal(dst.cpu().numpy(), ref)

    grad = torch.randn(ref.shape, generator=torch.Generator().manual_seed(seed + 9))
    dsts = [torch.randn(s.shape, generator=torch.Generator().manual_seed(i)) for i, s in
            enumerate(srcs)]
    if pinned:
        dsts = [d.pin_memory() for d in dsts]
    expect = oracle.scatter_partitions(pid, grad, dsts, bnd)
    gd = grad.to(gpu)
    _on_side_stream(lambda: _C.scatter_partitions(pid, gd, dsts, b64))
    _C.d2h_synchronize()
    for d, e in zip(dsts, expect):
        assert np.array_equal(d.numpy(), e)


def test_scatter_repeated_indices_pinned_falls_back_ordered(gpu):
    dsts = [torch.zeros(2, 1).pin_memory(), torch.zeros(3, 1).pin_memory()]
    bnd = [torch.empty(0, dtype=torch.long), torch.tensor([1, 1, 2])]
    src = torch.tensor([[1.0], [2.0], [3.0], [4.0], [5.0]], device=gpu)
    _on_side_stream(lambda: _C.scatter_partitions(0, src, dsts, bnd))
    _C.d2h_synchronize()
    assert dsts[1].reshape(-1).tolist() == [0.0, 7.0, 5.0]


def test_size_mismatch_and_bad_index_raise(gpu):
    srcs = [torch.zeros(4, 2), torch.zeros(3, 2)]
    dst = torch.empty(6, 2, device=gpu)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with pytest.raises(GrError, match="size mismatch"):
            _C.gather_partitions(0, srcs, dst, [torch.empty(0, dtype=torch.long),
                                                torch.tensor([0])])
        with pytest.raises(GrError, match="out of range"):
            _C.gather_partitions(0, srcs, dst, [torch.empty(0, dtype=torch.long),
                                                torch.tensor([0, 5])])
        with pytest.raises(GrError, match="size mismatch"):
            _C.scatter_partitions(0, torch.zeros(9, 2, device=gpu), srcs,
                                  [torch.empty(0, dtype=torch.long), torch.tensor([0])])
    s.synchronize()


def test_host_buffer_fill_upload_gather_scatter(gpu):
    """tests/test_host_buffer_ops.py:14-60 and tests/test_buffers.py:49-76."""
    for pin in (False, True):
        buf = HostBuffer(num_parts=2, part_sizes=[5, 3], embedding_dim=4, pin_memory=pin)
        buf.initialize_zeros()
        data = torch.randn(5, 4, device=gpu)
        stream = torch.cuda.Stream()
        buf.async_fill(0, data, stream)
        buf.d2h_synchronize(stream)
        assert torch.equal(buf[0], data.cpu())
        tgt = torch.empty(5, 4, device=gpu)
        buf.async_upload(0, tgt, stream)
        buf.h2d_synchronize(stream)
        assert torch.equal(tgt, data)

        buf = HostBuffer(num_parts=3, part_sizes=[4, 3, 5], embedding_dim=2, pin_memory=pin)
        buf[0].copy_(torch.arange(8).reshape(4, 2).float())
        buf[1].copy_(torch.arange(8, 14).reshape(3, 2).float())
        buf[2].copy_(torch.arange(14, 24).reshape(5, 2).float())
        bnd = [None, torch.tensor([0, 2]), torch.tensor([3])]
        out = torch.empty(7, 2, device=gpu)
        buf.async_gather(0, out, bnd, stream)
        buf.h2d_synchronize(stream)
        assert out.cpu().tolist() == [[0, 1], [2, 3], [4, 5], [6, 7], [8, 9], [12, 13],
                                      [20, 21]]
        buf.initialize_zeros()
        buf[0].fill_(1.0)
        buf.async_scatter(0, torch.full((7, 2), 2.0, device=gpu), bnd, stream)
        buf.d2h_synchronize(stream)
        assert torch.equal(buf[0], torch.full((4, 2), 3.0))
        assert buf[1].tolist() == [[2, 2], [0, 0], [2, 2]]


def test_pageable_paths_span_several_staging_chunks(gpu):
    """Pageable gather / scatter larger than one 64 MiB staging chunk."""
    g = torch.Generator().manual_seed(0)
    dim = 64
    sizes = [150_000, 200_000, 180_000]
    srcs = [torch.randn(n, dim, generator=g) for n in sizes]
    bnd = [None, torch.randperm(sizes[1], generator=g)[:170_000],
           torch.randperm(sizes[2], generator=g)[:160_000]]
    ref = oracle.gather_partitions(0, srcs, bnd)
    dst = torch.empty(ref.shape, device=gpu)
    b64 = [torch.empty(0, dtype=torch.long) if b is None else b for b in bnd]
    _on_side_stream(lambda: _C.gather_partitions(0, srcs, dst, b64))
    _C.h2d_synchronize()
    assert np.array_equal(dst.cpu().numpy(), ref)
    grad = torch.randn(ref.shape, generator=g)
    dsts = [torch.randn(n, dim, generator=g) for n in sizes]
    expect = oracle.scatter_partitions(0, grad, dsts, bnd)
    gd = grad.to(gpu)
    _on_side_stream(lambda: _C.scatter_partitions(0, gd, dsts, b64))
    _C.d2h_synchronize()
    for d, e in zip(dsts, expect):
        assert np.array_equal(d.numpy(), e)
