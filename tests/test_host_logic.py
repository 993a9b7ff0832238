"""CPU tests of the boundary and host logic: the C ABI loads and exports every
declared symbol, the native bookkeeping is bit-exact with the oracle (and the
compiled reference), plans/transposes are consistent, and the host-side
mirrors of the reference API behave like the reference (no GPU needed)."""

import ctypes

import numpy as np
import re
from pathlib import Path

import pytest
import torch

import oracle
from grinnder_amd import _lib
from grinnder_amd.buffer.host import HostBuffer
from grinnder_amd.config import GriNNderConfig
from grinnder_amd.data import synthetic
from grinnder_amd.data.adjacency import build_plan
from grinnder_amd.data.graph import PartitionedGraph
from grinnder_amd.data.partition import (_build_partition_subgraph, build_partitioned_graph,
                                         build_subgraph)

ROOT = Path(__file__).resolve().parent.parent


# ------------------------------------------------------------- the C ABI --

def test_library_exports_every_declared_symbol():
    header = (ROOT / "include" / "grinnder_amd.h").read_text()
    declared = set(re.findall(r"^\s*(?:int|const char\*)\s+(gr_\w+)\(", header, re.M))
    assert len(declared) >= 19
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(_lib.EXPORTED)
    assert _lib.load().gr_abi_version() == 100


def test_loader_refuses_a_stale_library(monkeypatch):
    """The library carries the hash of the sources it was built from; the
    loader refuses it when the sources beside it hash differently."""
    lib = _lib.load()
    assert lib.gr_source_hash().decode() == _lib.source_hash()
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "source_hash", lambda: "0" * 64)
    with pytest.raises(ImportError, match="other sources"):
        _lib.load()
    monkeypatch.undo()
    assert _lib.load() is lib


def test_errors_are_reported_not_swallowed():
    with pytest.raises(_lib.GrError, match="spmm_plan"):
        _lib.call("gr_spmm_plan", None, 5, 16, None, None, None, None, None)
    bad = torch.tensor([0, 2, 1])  # non-monotone rowptr
    n = torch.zeros(3, dtype=torch.int64)
    with pytest.raises(_lib.GrError, match="monotone"):
        _lib.call("gr_spmm_plan", bad.data_ptr(), 2, 16, None, n.data_ptr(), None,
                  n[1:].data_ptr(), n[2:].data_ptr())


def test_aggregation_refuses_fewer_slots_than_the_plan_has():
    """A plan with n_fix split rows has at least 2 * n_fix split units, each
    writing a slot of its own: a smaller n_slots would put their partial
    sums past the workspace (or the no-alloc scratch).  Both entry points
    refuse it before anything is launched, so no GPU is needed here."""
    rowptr = torch.tensor([0, 700, 705, 1400])  # rows 0 and 2 split at seg_len 256
    units_n = torch.zeros(3, dtype=torch.int64)
    _lib.call("gr_spmm_plan", rowptr.data_ptr(), 3, 256, None, units_n.data_ptr(), None,
              units_n[1:].data_ptr(), units_n[2:].data_ptr())
    n_units, n_fix, n_slots = units_n.tolist()
    assert (n_fix, n_slots) == (2, 6)
    units = torch.zeros(n_units * 4, dtype=torch.int32)
    fixups = torch.zeros(n_fix * 3, dtype=torch.int32)
    _lib.call("gr_spmm_plan", rowptr.data_ptr(), 3, 256, units.data_ptr(),
              units_n.data_ptr(), fixups.data_ptr(), units_n[1:].data_ptr(),
              units_n[2:].data_ptr())
    fake = 1 << 20  # never dereferenced: the call is refused first
    common = (units.data_ptr(), n_units, fixups.data_ptr(), n_fix, fake, fake, fake, 8,
              fake, 8, None, 3, 8)
    for short in (0, 3):
        with pytest.raises(_lib.GrError, match="below the 2 \\* n_fix"):
            _lib.call("gr_gcn_aggregate", *common, fake, short, None)
        with pytest.raises(_lib.GrError, match="below the 2 \\* n_fix"):
            _lib.call("gr_gcn_aggregate_noalloc", *common, short, None)


def test_single_hip_runtime_loaded():
    _lib.load()
    maps = Path("/proc/self/maps").read_text().splitlines()
    runtimes = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(runtimes) == 1, runtimes


# ------------------------------------------------------- build_subgraph --

def test_build_subgraph_known_answers():
    """tests/test_cpp_extensions.py:64-106."""
    rowptr = torch.tensor([0, 2, 3, 4, 4])
    col = torch.tensor([1, 2, 2, 3])
    r, c, v, n_id = build_subgraph(rowptr, col, None, torch.tensor([0, 1]), True)
    assert r.tolist() == [0, 2, 3] and c.tolist() == [1, 2, 2] and n_id.tolist() == [0, 1, 2]
    assert v is None
    value = torch.tensor([0.5, 0.3, 0.7, 0.1])
    r, c, v, n_id = build_subgraph(rowptr, col, value, torch.tensor([0]), True)
    assert v.shape[0] == c.shape[0] and v.tolist() == pytest.approx([0.5, 0.3])
    r, c, v, n_id = build_subgraph(torch.tensor([0, 2, 3, 3]), torch.tensor([1, 2, 2]), None,
                                   torch.tensor([0]), False)
    assert r.shape[0] == n_id.shape[0] + 1


@pytest.mark.parametrize("seed", range(4))
def test_build_subgraph_bit_exact(seed):
    g = torch.Generator().manual_seed(seed)
    n = 300
    ei = torch.randint(0, n, (2, 2500), generator=g)
    rowptr, col, _ = oracle.edge_index_to_csr(ei, n)
    val = torch.rand(col.numel(), generator=g)
    idx = torch.randperm(n, generator=g)[:90]
    idx[5] = idx[3]  # repeated seed: last assignment wins, as in the reference
    ref = oracle.ref_build_subgraph()
    for bip in (True, False):
        got = build_subgraph(rowptr, col, val, idx, bip)
        exp = oracle.build_subgraph(rowptr, col, val, idx, bip)
        for a, b in zip(got, exp):
            assert torch.equal(a, b)
        if ref is not None:
            for a, b in zip(got, ref(rowptr, col, val, idx, bip)):
                assert torch.equal(a, b)


def test_partition_subgraph_and_pipeline_bit_exact():
    for n, reach, parts in [(20, 3, 4), (57, 4, 5), (200, 6, 3)]:
        ei = synthetic.banded_graph(n, reach)
        x = torch.randn(n, 4)
        y = torch.zeros(n, dtype=torch.long)
        m = torch.ones(n, dtype=torch.bool)
        g = build_partitioned_graph(ei, x, y, m, m, m, GriNNderConfig(num_parts=parts))
        ref = oracle.partition_pipeline(ei, n, g.perm, g.ptr)
        for pid in range(parts):
            _, adj, bnd, expanded, batch = ref[pid]
            for a, b in zip(g.adj_csr[pid], adj):
                assert torch.equal(a, b)
            for a, b in zip(g.boundaries[pid], bnd):
                assert (a is None and b is None) or torch.equal(a, b)
            assert g.expanded_sizes[pid] == expanded and g.partition_sizes[pid] == batch
    # uniform random graph (C1 shape, reduced)
    ei = synthetic.uniform_graph(3000, 12000, seed=1)
    nd = synthetic.node_data(3000, 8, 5)
    g = build_partitioned_graph(ei, nd.x, nd.y, nd.train_mask, nd.val_mask, nd.test_mask,
                                GriNNderConfig(num_parts=3))
    ref = oracle.partition_pipeline(ei, 3000, g.perm, g.ptr)
    for pid in range(3):
        for a, b in zip(g.adj_csr[pid], ref[pid][1]):
            assert torch.equal(a, b)


def _assert_same_partitions(g, ref):
    for pid in range(g.num_parts):
        _, adj, bnd, expanded, batch = ref[pid]
        for a, b in zip(g.adj_csr[pid], adj):
            assert torch.equal(a, b), pid
        for a, b in zip(g.boundaries[pid], bnd):
            assert (a is None and b is None) or torch.equal(a, b), pid
        assert (g.expanded_sizes[pid], g.partition_sizes[pid]) == (expanded, batch), pid


@pytest.mark.parametrize("parts", [4, 16])
def test_directed_rmat_pipeline_bit_exact(parts):
    """A directed R-MAT graph (power-law, 50k nodes), where CSR orientation
    and the degree's side are observable: the whole preprocessing pipeline
    is bit-exact with the oracle's, whose orientation the known answer and
    the brute-force check in tests/test_oracle.py pin."""
    n = 50_000
    ei = synthetic.rmat_graph(n, 400_000, scale=16, seed=5, undirected=False)
    assert not torch.equal(torch.sort(ei[0] * n + ei[1]).values,
                           torch.sort(ei[1] * n + ei[0]).values)  # really directed
    nd = synthetic.node_data(n, 4, 5)
    g = build_partitioned_graph(ei, nd.x, nd.y, nd.train_mask, nd.val_mask, nd.test_mask,
                                GriNNderConfig(num_parts=parts))
    _assert_same_partitions(g, oracle.partition_pipeline(ei, n, g.perm, g.ptr))


def test_native_directed_pipeline_known_answer_and_brute_force():
    """The product's pipeline (partition_adjacency, the steps after the
    partitioner) against the hand-derived directed answer and the brute-force
    orientation check, serial and on worker threads."""
    from grinnder_amd.data.partition import partition_adjacency
    from tests.test_oracle import check_directed_brute_force, check_directed_known_answer

    for workers in (1, 3):
        fn = lambda ei, n, perm, ptr: partition_adjacency(ei, n, perm, ptr, workers=workers)
        check_directed_known_answer(fn)
        for seed in range(3):
            check_directed_brute_force(fn, seed)


def test_native_partition_subgraph_halo_order_known_answer():
    """The hand-derived halo layout of grinnder/data/partition.py:195-225."""
    from tests.test_oracle import check_halo_known_answer

    check_halo_known_answer(_build_partition_subgraph)


@pytest.mark.parametrize("seed", range(3))
def test_native_partition_subgraph_halo_layout_property(seed):
    from tests.test_oracle import check_halo_layout_property

    check_halo_layout_property(_build_partition_subgraph, seed)


def test_partition_cache_round_trip(tmp_path):
    """tests/test_partition.py:165-205 (cache written then reloaded identically)."""
    ei = synthetic.banded_graph(20, 3)
    x = torch.randn(20, 8)
    y = torch.randint(0, 3, (20,))
    m = torch.ones(20, dtype=torch.bool)
    cfg = GriNNderConfig(num_parts=4)
    path = tmp_path / "cache.pt"
    g1 = build_partitioned_graph(ei, x, y, m, m, m, cfg, cache_path=path)
    assert path.exists()
    g2 = build_partitioned_graph(ei, x, y, m, m, m, cfg, cache_path=path)
    assert g1.partition_sizes == g2.partition_sizes and g1.expanded_sizes == g2.expanded_sizes
    for a, b in zip(g1.adj_csr, g2.adj_csr):
        for s, t in zip(a, b):
            assert torch.equal(s, t)


# -------------------------------------------------- transpose and plans --

def test_csr_transpose_is_stable_and_complete():
    g = torch.Generator().manual_seed(3)
    rows, cols = 70, 90
    ei = torch.stack([torch.randint(0, rows, (900,), generator=g),
                      torch.randint(0, cols, (900,), generator=g)])
    rowptr, col, _ = oracle.edge_index_to_csr(ei, rows)
    val = torch.rand(col.numel(), generator=g)
    colptr = torch.empty(cols + 1, dtype=torch.int64)
    ri = torch.empty(col.numel(), dtype=torch.int32)
    vt = torch.empty(col.numel())
    pm = torch.empty(col.numel(), dtype=torch.int32)
    _lib.call("gr_csr_transpose", rowptr.data_ptr(), col.data_ptr(), val.data_ptr(), rows, cols,
              colptr.data_ptr(), ri.data_ptr(), vt.data_ptr(), pm.data_ptr())
    assert torch.equal(colptr[1:] - colptr[:-1], torch.bincount(col, minlength=cols))
    assert torch.equal(torch.sort(pm.long()).values, torch.arange(col.numel()))
    row_of_edge = torch.repeat_interleave(torch.arange(rows), rowptr[1:] - rowptr[:-1])
    assert torch.equal(ri.long(), row_of_edge[pm.long()])
    assert torch.equal(vt, val[pm.long()])
    for c in range(cols):
        seg = pm[colptr[c]:colptr[c + 1]].long()
        assert torch.equal(col[seg], torch.full_like(seg, c))
        assert torch.equal(seg, torch.sort(seg).values)  # stable: CSR order kept


def test_spmm_plan_covers_every_edge_once():
    deg = torch.tensor([0, 3, 1000, 17, 0, 2049, 5, 4096, 1])
    rowptr = torch.zeros(deg.numel() + 1, dtype=torch.int64)
    rowptr[1:] = deg.cumsum(0)
    p = build_plan(rowptr, deg.numel(), 512, "cpu")
    u = p.units.long()
    covered = torch.zeros(int(rowptr[-1]), dtype=torch.int64)
    for row, b, e, slot in u.tolist():
        assert rowptr[row] <= b <= e <= rowptr[row + 1] and e - b <= 512
        covered[b:e] += 1
    assert torch.equal(covered, torch.ones_like(covered))
    assert p.n_units == (deg.numel() - 3) + 2 + 5 + 8  # 6 whole rows + split rows 2049, 4096, 1000
    split = {r: (f, n) for r, f, n in p.fixups.tolist()}
    assert set(split) == {2, 5, 7}
    slots = sorted(s for *_, s in u.tolist() if s >= 0)
    assert slots == list(range(p.n_slots))
    for row, (first, n) in split.items():
        units = [x for x in u.tolist() if x[0] == row]
        assert [x[3] for x in units] == list(range(first, first + n))
    assert all(x[3] >= 0 for x in u.tolist()[:15]) and all(x[3] < 0 for x in u.tolist()[15:])


def test_spmm_plan_blocked_orders_whole_rows_by_block():
    """gr_spmm_plan_blocked: the same split units, fixups and slots as
    gr_spmm_plan, and the same whole-row units, reordered so that each
    block's rows come together (length classes longest first within a
    block, row order within a class)."""
    g = torch.Generator().manual_seed(4)
    deg = torch.randint(0, 40, (300,), generator=g)
    deg[[7, 150, 299]] = torch.tensor([1300, 600, 2049])
    rowptr = torch.zeros(deg.numel() + 1, dtype=torch.int64)
    rowptr[1:] = deg.cumsum(0)
    blocks = torch.tensor([0, 100, 100, 220, 300])
    a = build_plan(rowptr, deg.numel(), 512, "cpu")
    b = build_plan(rowptr, deg.numel(), 512, "cpu", blocks)
    assert (a.n_units, a.n_fix, a.n_slots) == (b.n_units, b.n_fix, b.n_slots)
    assert torch.equal(a.fixups, b.fixups)
    ua, ub = a.units.tolist(), b.units.tolist()
    nsplit = sum(1 for x in ua if x[3] >= 0)
    assert ua[:nsplit] == ub[:nsplit]
    assert sorted(ua[nsplit:]) == sorted(ub[nsplit:])
    whole = ub[nsplit:]

    def key(x):
        r, lo, hi, _ = x
        blk = int(torch.searchsorted(blocks, torch.tensor(r), right=True)) - 1
        return (blk, -(hi - lo).bit_length(), r)
    assert whole == sorted(whole, key=key)
    with pytest.raises(_lib.GrError, match="blocks"):
        build_plan(rowptr, deg.numel(), 512, "cpu", torch.tensor([0, 100, 299]))


def test_whole_adjacency_is_the_full_graph_in_partition_order():
    """PartitionedGraph.whole_adjacency (the adjacency merged layers run on):
    the per-partition CSRs stacked with every column mapped to its global row
    equal, row by row and edge by edge, the full graph's CSR built directly
    from the relabelled edge list (self-loops and GCN weights as the
    partition pipeline adds them); its forward plan runs block by block
    over the partitions (row_blocks = ptr)."""
    from grinnder_amd.data.datasets import append_self_loops, compute_gcn_norm
    from grinnder_amd.data.partition import _edge_index_to_csr

    n = 3000
    gen = torch.Generator().manual_seed(1)
    ei = torch.randint(0, n, (2, 15000), generator=gen)  # directed: one orientation fits
    ei = ei[:, ei[0] != ei[1]]
    nd = synthetic.node_data(n, 8, 5)
    g = build_partitioned_graph(ei, nd.x, nd.y, nd.train_mask, nd.val_mask, nd.test_mask,
                                GriNNderConfig(num_parts=4))
    w = g.whole_adjacency()
    assert w.sparse_sizes() == (n, n) and torch.equal(w.row_blocks, g.ptr.to(torch.int64))
    inv = torch.empty_like(g.perm)
    inv[g.perm] = torch.arange(n)
    e = inv[ei]
    val = compute_gcn_norm(e, n, add_self_loops=True)
    e = append_self_loops(e, n)
    # The reference's orientation: rows are edge_index[0]
    # (grinnder/data/partition.py:79-87).  The graph is directed, so the
    # transposed CSR differs and would fail here.
    rowptr, col, perm = _edge_index_to_csr(e, n)
    v = val[perm]
    rt, _, _ = _edge_index_to_csr(e.flip(0), n)
    assert not torch.equal(rt, rowptr)
    assert torch.equal(rowptr, w.rowptr)
    for r in range(n):
        a, b = int(rowptr[r]), int(rowptr[r + 1])
        ka = sorted(zip(w.col[a:b].tolist(), w.value[a:b].tolist()))
        kb = sorted(zip(col[a:b].tolist(), v[a:b].tolist()))
        assert ka == kb, r
    assert g.whole_adjacency() is w


def test_rmat_stream_independent_of_threads():
    a = synthetic.rmat_sample(7, 20, 1000, 200000, nthreads=1)
    b = synthetic.rmat_sample(7, 20, 1000, 200000, nthreads=8)
    c = synthetic.rmat_sample(7, 20, 101000, 100000, nthreads=3)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert torch.equal(a[0][100000:], c[0]) and torch.equal(a[1][100000:], c[1])
    # quadrant frequencies at the first level follow (a, b, c, d)
    s, d = a
    top_s, top_d = s >> 19, d >> 19
    q = torch.bincount(top_s * 2 + top_d, minlength=4).double() / s.numel()
    assert torch.allclose(q, torch.tensor([0.57, 0.19, 0.19, 0.05], dtype=torch.float64),
                          atol=0.01)


def test_rmat_graph_exact_edge_count_and_symmetry():
    ei = synthetic.rmat_graph(5000, 30000, seed=3, batch=1 << 15)
    assert ei.size(1) == 60000
    assert (ei[0] != ei[1]).all() and int(ei.max()) < 5000
    key = ei[0] * 5000 + ei[1]
    assert torch.unique(key).numel() == 60000
    rev = ei[1] * 5000 + ei[0]
    assert torch.equal(torch.sort(key).values, torch.sort(rev).values)


# ------------------------------------------------------- host mirrors --

def test_host_buffer_lazy_allocation():
    """tests/test_buffers.py:10-47."""
    buf = HostBuffer(num_parts=3, part_sizes=[10, 15, 12], embedding_dim=8)
    assert len(buf) == 3 and buf[0].shape == (10, 8) and not buf[0].is_pinned()
    buf = HostBuffer(num_parts=2, part_sizes=[5, 7], embedding_dim=4)
    assert not buf.is_allocated(0) and buf.resident_bytes == 0
    assert tuple(buf._tensors[0].shape) == (0, 4)
    t = buf[0]
    assert t.shape == (5, 4) and buf.resident_bytes == buf.partition_nbytes(0)
    buf.release(0)
    assert not buf.is_allocated(0) and buf.resident_bytes == 0
    buf = HostBuffer(num_parts=2, part_sizes=[5, 5], embedding_dim=4)
    buf[0].fill_(1.0)
    buf.initialize_zeros()
    assert (buf[0] == 0).all() and (buf[1] == 0).all()
    buf[0].fill_(1.0)
    buf.initialize_zeros(lazy=True)
    assert not buf.is_allocated(0) and not buf.is_allocated(1)


def test_config_defaults_and_env(monkeypatch):
    """tests/test_config.py."""
    c = GriNNderConfig()
    assert c.mode == "grinnder" and c.num_parts == 8 and c.pool_size == 2
    assert c.cache_mode == "auto" and c.device == "cuda:0" and c.num_gpus == 1
    monkeypatch.setenv("GRINNDER_PARTITION_THREADS", "3")
    assert GriNNderConfig().preprocess_workers == 3
    assert GriNNderConfig().partitioner_kwargs["num_threads"] == 3


def test_partitioned_graph_accessors():
    """tests/test_data.py:60-90."""
    g = PartitionedGraph(num_nodes=10, num_edges=20, num_parts=2, partition_sizes=[6, 4],
                         adj_csr=[], boundaries=[], expanded_sizes=[8, 6],
                         features=torch.randn(10, 3), labels=torch.tensor([0, 1] * 5),
                         train_mask=torch.ones(10, dtype=torch.bool),
                         val_mask=torch.zeros(10, dtype=torch.bool),
                         test_mask=torch.zeros(10, dtype=torch.bool), perm=torch.arange(10),
                         ptr=torch.tensor([0, 6, 10]))
    assert g.feat_dim == 3 and g.num_classes == 2
    assert g.partition_features(1).shape == (4, 3) and g.partition_train_mask(0).sum() == 6


def test_product_path_has_no_cpu_fallback():
    """The aggregation entry points refuse CPU tensors instead of computing."""
    from grinnder_amd.aggregation import gat_attention, gcn_aggregate
    from grinnder_amd.data.adjacency import Adjacency

    adj = Adjacency(torch.tensor([0, 1]), torch.tensor([0]), None, (1, 1))
    with pytest.raises(RuntimeError, match="GPU"):
        gcn_aggregate(torch.randn(1, 4), adj)
    with pytest.raises(RuntimeError, match="GPU"):
        gat_attention(torch.randn(1, 4), adj, torch.randn(1, 1, 4), torch.randn(1, 1, 4), None,
                      1, 4)


# ------------------------------------------------------------ partitioner --

@pytest.mark.parametrize("order", ["bfs", "natural"])
def test_partitioner_is_a_balanced_permutation(order):
    from grinnder_amd.data.partition import partition_nodes

    ei = synthetic.rmat_graph(3000, 20000, seed=5, batch=1 << 15)
    for P in (1, 3, 8):
        perm, ptr = partition_nodes(ei, 3000, P, capacity=1.1, order=order)
        assert torch.equal(torch.sort(perm).values, torch.arange(3000))
        assert int(ptr[0]) == 0 and int(ptr[-1]) == 3000
        sizes = (ptr[1:] - ptr[:-1]).tolist()
        assert max(sizes) <= int(np.ceil(1.1 * 3000 / P))
        again = partition_nodes(ei, 3000, P, capacity=1.1, order=order)
        assert torch.equal(perm, again[0]) and torch.equal(ptr, again[1])


def test_partitioner_keeps_banded_graph_local():
    from grinnder_amd.data.partition import partition_nodes

    ei = synthetic.banded_graph(400, 3)
    perm, ptr = partition_nodes(ei, 400, 4, capacity=1.1)
    g = build_partitioned_graph(ei, torch.randn(400, 2), torch.zeros(400, dtype=torch.long),
                                *(torch.ones(400, dtype=torch.bool),) * 3,
                                GriNNderConfig(num_parts=4))
    assert g.halo_amplification() < 1.2  # a random cut would be ~ 2.7


def test_gemm_tn_split_heuristic_and_argument_checks():
    """Host-side planning of the split-K weight-gradient GEMM; the argument
    checks reject a short workspace before anything reaches the device."""
    from grinnder_amd.dense import gemm_tn_splits

    for m, n, k in [(256, 256, 2_449_029), (47, 256, 10), (1, 1, 0), (256, 100, 100_000)]:
        s, ws = gemm_tn_splits(m, n, k)
        assert 1 <= s <= 4096 and ws == s * m * n
    s, _ = gemm_tn_splits(256, 256, 2_449_029)
    assert s % 8 == 0 and s * 4 >= 1024
    fake = 256  # non-NULL pointers: the call must fail before any device access
    with pytest.raises(_lib.GrError, match="workspace"):
        _lib.call("gr_gemm_tn", fake, 8, fake, 8, 8, 8, 100, 0.0, fake, fake, 128, 7, None)
    with pytest.raises(_lib.GrError, match="leading dimension"):
        _lib.call("gr_gemm_tn", fake, 4, fake, 8, 8, 8, 100, 0.0, fake, fake, 10**6, 1, None)
    with pytest.raises(_lib.GrError, match="in-place"):
        _lib.call("gr_bias_ln_act", fake, 12, None, fake, fake, 1e-5, 0, 4, 8, fake, fake, fake,
                  fake, None)
    with pytest.raises(_lib.GrError, match="activation"):
        _lib.call("gr_bias_ln_act", fake, 8, None, fake, fake, 1e-5, 7, 4, 8, fake, fake, fake,
                  fake, None)


def test_loss_mask_codes_and_argument_checks():
    from grinnder_amd.loss import mask_codes

    b = lambda v: torch.tensor(v, dtype=torch.bool)  # noqa: E731
    codes = mask_codes(b([1, 0, 1, 0]), b([0, 1, 1, 0]), b([0, 0, 1, 1]))
    assert codes.dtype == torch.uint8 and codes.tolist() == [1, 2, 7, 4]
    fake = 256  # rejected before any device access
    with pytest.raises(_lib.GrError, match="ldg"):
        _lib.call("gr_xent_forward", fake, 10, 5, 10, fake, fake, 0, None, fake, 4, fake, fake,
                  fake, 7168, None)
    with pytest.raises(_lib.GrError, match="workspace"):
        _lib.call("gr_xent_forward", fake, 10, 5, 10, fake, fake, 0, None, None, 0, fake, fake,
                  fake, 3, None)
