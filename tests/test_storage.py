"""CPU tests of the storage tier: the I/O engine (IoUringEngine on gr_io_*),
StorageBackend, StorageTensor, HostBuffer's storage operations and the
PartitionCache policies (reference tests test_storage.py, test_cache.py)."""

import os

import numpy as np
import pytest
import torch

from grinnder_amd import _lib
from grinnder_amd._C import IoUringEngine
from grinnder_amd.buffer.host import HostBuffer
from grinnder_amd.cache import PartitionCache
from grinnder_amd.storage import StorageBackend, StorageTensor


@pytest.fixture
def backend(tmp_path):
    return StorageBackend(str(tmp_path / "store"))


# ------------------------------------------------------------- the engine --

def test_engine_round_trip_in_parallel_chunks(tmp_path):
    """A 20 MB tensor (3 chunks of 8 MiB), written and read back; the file
    holds the raw row-major bytes and nothing else."""
    e = IoUringEngine(8)
    assert not e.has_io_uring()
    t = torch.randn(5_000_001)
    path = str(tmp_path / "a.pt")
    h = e.submit_write(path, t, 0, t.numel() * 4)
    e.wait(h)
    assert os.path.getsize(path) == t.numel() * 4
    assert np.array_equal(np.fromfile(path, dtype=np.float32), t.numpy())
    u = torch.empty_like(t)
    h = e.submit_read(path, u, 0, u.numel() * 4)
    e.wait(h)
    assert torch.equal(u, t)
    # an offset read of the tail
    v = torch.empty(10)
    e.wait(e.submit_read(path, v, (t.numel() - 10) * 4, 40))
    assert torch.equal(v, t[-10:])


def test_engine_poll_pending_wait_all(tmp_path):
    e = IoUringEngine(4)
    t = torch.arange(1000, dtype=torch.float32)
    hs = [e.submit_write(str(tmp_path / f"f{i}.pt"), t, 0, 4000) for i in range(16)]
    assert e.pending() <= 16
    e.wait_all()
    assert e.pending() == 0
    h = e.submit_read(str(tmp_path / "f3.pt"), torch.empty(1000), 0, 4000)
    while not e.poll(h):
        pass
    e.wait(h)
    with pytest.raises(_lib.GrError, match="unknown or already waited"):
        e.wait(hs[0])


def test_engine_reports_errors(tmp_path):
    e = IoUringEngine(2)
    with pytest.raises(_lib.GrError, match="cannot open"):
        e.submit_read(str(tmp_path / "missing.pt"), torch.empty(4), 0, 16)
    path = str(tmp_path / "short.pt")
    e.wait(e.submit_write(path, torch.ones(4), 0, 16))
    h = e.submit_read(path, torch.empty(8), 0, 32)
    with pytest.raises(_lib.GrError, match="shorter"):
        e.wait(h)
    with pytest.raises(RuntimeError, match="contiguous"):
        e.submit_write(path, torch.ones(4, 4).t(), 0, 64)
    with pytest.raises(RuntimeError, match="do not fit"):
        e.submit_write(path, torch.ones(4), 0, 17)


def test_engine_failed_chunk_fails_the_request(tmp_path):
    """A read of 5 chunks from a file truncated inside the fourth: the other
    chunks succeed, and wait() must still report the failure (the request
    completes only once every chunk has published its result).  Repeated
    with many workers so that the failing chunk is not reliably the last."""
    chunk = 8 << 20
    path = str(tmp_path / "trunc.pt")
    full = torch.arange(5 * chunk // 4, dtype=torch.int32).view(torch.float32)
    e = IoUringEngine(8)
    e.wait(e.submit_write(path, full, 0, full.numel() * 4))
    os.truncate(path, 3 * chunk + 1234)
    for _ in range(20):
        u = torch.zeros_like(full)
        h = e.submit_read(path, u, 0, u.numel() * 4)
        with pytest.raises(_lib.GrError, match="shorter"):
            e.wait(h)
        # the chunks before the cut still arrived
        assert torch.equal(u[:3 * chunk // 4].view(torch.int32),
                           full[:3 * chunk // 4].view(torch.int32))
    assert e.pending() == 0


# ------------------------------------------------------------- the backend --

def test_backend_host_write_read_and_files(backend):
    """tests/test_storage.py:31-62 of the reference."""
    t = torch.randn(10, 5)
    backend.wait(backend.host_write(t, "test1"))
    assert backend.exists("test1") and backend.file_size("test1") == 200
    assert os.path.exists(os.path.join(backend.storage_dir, "test1.pt"))
    out = torch.empty_like(t)
    backend.wait(backend.host_read("test1", out))
    assert torch.equal(t, out)
    backend.remove("test1")
    assert not backend.exists("test1")
    backend.host_write(torch.randn(5), "a", async_=False)
    backend.host_write(torch.randn(5), "b", async_=False)
    backend.cleanup()
    assert not backend.exists("a") and not backend.exists("b")


def test_storage_tensor_lifecycle(backend):
    """tests/test_storage.py:65-107 of the reference."""
    st = StorageTensor((10, 5), torch.float32, backend, "st_test")
    assert st.location == "host" and not st.host_data.is_pinned()
    st.host_data.fill_(3.14)
    st.to_storage(async_=False)
    assert st.location == "storage"
    with pytest.raises(RuntimeError):
        st.host_data
    st.to_host()
    st.finish_to_host()
    assert st.location == "host" and torch.equal(st.host_data, torch.full((10, 5), 3.14))
    st.reset()
    assert bool((st.host_data == 0).all())


def test_host_buffer_storage_round_trip(backend):
    hb = HostBuffer(3, [10, 15, 12], 8, backend=backend, file_prefix="feat_l1")
    for p in range(3):
        hb[p].copy_(torch.randn(hb.part_sizes[p], 8))
    before = [hb[p].clone() for p in range(3)]
    hb.cpu_to_storage()
    assert all(backend.exists(f"feat_l1_p{p}") for p in range(3))
    hb.release_all()
    assert hb.allocated_pids() == []
    hb.storage_to_cpu(1)
    assert hb.allocated_pids() == [1] and torch.equal(hb[1], before[1])
    hb.storage_to_cpu()
    assert all(torch.equal(hb[p], before[p]) for p in range(3))


def test_eviction_rewrites_changed_rows(backend):
    """A partition changed since its storage copy was written is written
    again before it is released, so the stale copy is never read back."""
    hb = HostBuffer(1, [4], 2, backend=backend, file_prefix="x")
    hb[0].fill_(1.0)
    hb.ensure_storage_copy(0)
    hb.storage_to_cpu(0)            # clean: loaded from its copy
    hb.ensure_storage_copy(0)       # nothing to write
    hb[0].fill_(2.0)                # changed
    hb.ensure_storage_copy(0)
    hb.release(0)
    hb.storage_to_cpu(0)
    assert bool((hb[0] == 2.0).all())


# ------------------------------------------------------------- the cache --

class FakeBackend:
    """In-memory stand-in with the backend's host API (reference test_cache.py:18-33)."""

    def __init__(self):
        self.store = {}

    def host_write(self, tensor, file_id, async_=True):
        self.store[file_id] = tensor.detach().clone()
        return file_id

    def host_read(self, file_id, tensor, async_=True):
        tensor.copy_(self.store[file_id])
        return file_id

    def wait(self, handle):
        return None

    def exists(self, file_id):
        return file_id in self.store


def _gb(nbytes):
    return nbytes / float(1 << 30)


def _make_cache(num_parts, num_layers, dim, num_nodes, backend, mode, budget_gb=100,
                fixed=0, margin=0, deps=None, part_sizes=None):
    dims = [dim] * (num_layers + 1)
    sizes = part_sizes or [num_nodes // num_parts] * num_parts
    hbs = [HostBuffer(num_parts, sizes, dim, backend=backend, file_prefix=f"feat_l{l}")
           for l in range(num_layers + 1)]
    gbs = [None] + [HostBuffer(num_parts, sizes, dim, backend=backend, file_prefix=f"grad_l{l}")
                    for l in range(1, num_layers)]
    cache = PartitionCache(num_parts, num_layers, dims, num_nodes, hbs, gbs, backend, mode=mode,
                           host_memory_budget_gb=budget_gb, fixed_resident_bytes=fixed,
                           safety_margin_bytes=margin, dependency_sets=deps)
    return cache, hbs, gbs


@pytest.mark.parametrize("use_files", [False, True])
def test_cache_auto_detect_and_accounting(backend, use_files):
    """tests/test_cache.py:91-172 of the reference."""
    be = backend if use_files else FakeBackend()
    cache, _, _ = _make_cache(4, 3, 4, 100, be, mode="auto", budget_gb=100)
    assert cache.mode == "lru_layer"
    layer = 100 * 4 * 4
    cache, _, _ = _make_cache(4, 3, 4, 100, be, mode="auto", budget_gb=_gb(2 * layer - 1))
    assert cache.mode == "partition_lru"
    plan = cache.memory_plan
    assert plan.layer_working_set_bytes == 2 * layer
    assert plan.all_layer_residency_bytes == 6 * layer
    assert cache.activation_cache_budget_bytes == cache.remaining_cache_bytes
    # room = budget - fixed - margin; lru_layer keeps a gradient layer free
    cache, _, _ = _make_cache(4, 3, 4, 100, be, mode="auto", budget_gb=_gb(4 * layer),
                              fixed=layer // 2, margin=layer // 2)
    assert cache.mode == "lru_layer" and cache.remaining_cache_bytes == 3 * layer
    assert cache.activation_cache_budget_bytes == 2 * layer
    cache, _, _ = _make_cache(4, 3, 4, 100, be, mode="auto", budget_gb=_gb(4 * layer - 1),
                              fixed=layer // 2, margin=layer // 2)
    assert cache.mode == "partition_lru"
    with pytest.raises(ValueError, match="Unsupported cache mode"):
        _make_cache(4, 3, 4, 100, be, mode="full_layer")


def test_cache_lru_layer_hits_and_eviction_order(backend):
    """tests/test_cache.py:175-249: a miss loads from storage, a second
    access hits; a produced layer stays resident and the oldest is evicted
    (written back first)."""
    layer_bytes = 2 * 10 * 1 * 4
    cache, bufs, _ = _make_cache(2, 2, 1, 20, backend, mode="lru_layer",
                                 budget_gb=_gb(layer_bytes * 2), part_sizes=[10, 10])
    for pid in range(2):
        bufs[0][pid].fill_(1.0)
        bufs[0].cpu_to_storage(pid)
        bufs[0].release(pid)
    cache.ensure_in_host(0)
    assert cache._misses == 1 and all(bufs[0].is_allocated(p) for p in range(2))
    cache.ensure_in_host(0)
    assert cache._hits == 1
    for pid in range(2):
        bufs[1][pid].fill_(2.0)
    cache.on_layer_complete(0)
    for pid in range(2):
        bufs[2][pid].fill_(3.0)
    cache.on_layer_complete(1)
    assert all(backend.exists(f"feat_l1_p{pid}") for pid in range(2))
    assert not any(bufs[1].is_allocated(p) for p in range(2))
    assert all(bufs[2].is_allocated(p) for p in range(2))
    assert list(cache._cached_layers) == [2]
    cache.ensure_in_host(1)  # evicts layer 2, reloads layer 1 with its values
    assert bool((bufs[1][0] == 2.0).all()) and list(cache._cached_layers) == [1]
    assert 0 < cache.hit_rate < 1


def test_cache_partition_lru_dependency_sets(backend):
    """tests/test_cache.py:252-296: pairs outside the target's dependency set
    are evicted in least-recently-used order; shared ones stay."""
    cache, bufs, _ = _make_cache(3, 1, 1, 30, backend, mode="partition_lru",
                                 budget_gb=_gb(80), part_sizes=[10, 10, 10])
    for pid in range(3):
        bufs[0][pid].fill_(float(pid))
        bufs[0].cpu_to_storage(pid)
    bufs[0].release_all()
    cache.ensure_dependencies_in_host(0, 0, dependencies={0, 2})
    assert [bufs[0].is_allocated(p) for p in range(3)] == [True, False, True]
    cache.ensure_dependencies_in_host(0, 1, dependencies={1, 2})
    assert [bufs[0].is_allocated(p) for p in range(3)] == [False, True, True]
    assert set(cache._cached_partitions) == {(0, 1), (0, 2)}
    assert cache._hits == 1 and cache._misses == 3
    assert float(bufs[0][2][0, 0]) == 2.0
    with pytest.raises(MemoryError):
        cache.ensure_dependencies_in_host(0, 0, dependencies={0, 1, 2})
    bnd = [None, torch.tensor([1, 2]), torch.empty(0, dtype=torch.long)]
    cache.ensure_dependencies_in_host(0, 0, boundaries=bnd)  # depends on {0, 1}
    assert set(cache._cached_partitions) == {(0, 0), (0, 1)}


def test_cache_gradient_flush_and_reset(backend):
    """tests/test_cache.py:299-355."""
    cache, bufs, grads = _make_cache(4, 3, 8, 100, backend, mode="lru_layer")
    grads[1][0].fill_(3.14)
    cache.on_backward_layer_complete(1)
    assert backend.exists("grad_l1_p0")
    cache, _, grads = _make_cache(4, 3, 8, 100, backend, mode="partition_lru")
    grads[1].initialize_zeros(lazy=True)
    grads[1][2].fill_(2.0)
    backend.remove("grad_l1_p0")
    cache.on_backward_layer_complete(1)
    assert backend.exists("grad_l1_p2") and not backend.exists("grad_l1_p0")
    assert not any(grads[1].is_allocated(p) for p in range(4))
    cache, bufs, _ = _make_cache(4, 3, 4, 100, backend, mode="lru_layer")
    for pid in range(4):
        bufs[0][pid].fill_(1.0)
        bufs[0].cpu_to_storage(pid)
        bufs[0].release(pid)
    cache.ensure_in_host(0)
    cache.ensure_in_host(0)
    cache.reset()
    assert cache._hits == 0 and cache._misses == 0 and cache.hit_rate == 0.0
    assert not any(bufs[0].is_allocated(p) for p in range(4))


def test_partitioned_graph_stores_adjacency(backend):
    """build_partitioned_graph(backend=...) also writes each partition's CSR
    (grinnder/data/partition.py:373-379)."""
    from grinnder_amd.config import GriNNderConfig
    from grinnder_amd.data import synthetic
    from grinnder_amd.data.partition import build_partitioned_graph

    ei = synthetic.banded_graph(40, 3)
    m = torch.ones(40, dtype=torch.bool)
    g = build_partitioned_graph(ei, torch.randn(40, 4), torch.zeros(40, dtype=torch.long), m, m,
                                m, GriNNderConfig(num_parts=3), backend=backend)
    for pid, (rp, c, v) in enumerate(g.adj_csr):
        got = torch.empty_like(c)
        backend.wait(backend.host_read(f"adj_col_p{pid}", got))
        assert torch.equal(got, c) and backend.file_size(f"adj_val_p{pid}") == 4 * v.numel()
