"""Pins the CPU oracle against the reference's known answers, the compiled
reference code (oracle/_ref) and independent closed forms (CPU only)."""

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle
from tests.graphs import random_bipartite


# ---------------------------------------------------------------- gcn norm --

def test_gcn_norm_triangle_known_answer():
    """tests/test_data.py:11-20 of the reference (weights in (0, 1]): on the
    triangle + self-loops every degree is 3, so every weight is the fp32
    square of fp32(3^-1/2), within one ulp of 1/3."""
    ei = torch.tensor([[0, 1, 1, 2, 0, 2], [1, 0, 2, 1, 2, 0]])
    w = oracle.compute_gcn_norm(ei, 3, True)
    assert w.shape == (9,)
    assert (w > 0).all() and (w <= 1).all()
    r = np.float32(1.0) / np.sqrt(np.float32(3.0))
    assert torch.equal(w, torch.full((9,), float(np.float32(r * r))))
    assert abs(float(w[0]) - 1.0 / 3.0) <= float(np.spacing(np.float32(1.0 / 3.0)))


def test_gcn_norm_matches_brute_force_degrees():
    g = torch.Generator().manual_seed(0)
    n = 40
    ei = torch.randint(0, n, (2, 300), generator=g)
    ei[:, :5] = torch.tensor([[3] * 5, [7] * 5])  # repeated edges are kept
    w = oracle.compute_gcn_norm(ei, n, True)
    full = torch.cat([ei, torch.arange(n).repeat(2, 1)], dim=1)
    deg = [0] * n
    for c in full[1].tolist():
        deg[c] += 1
    for e, (r, c) in enumerate(full.t().tolist()):
        expect = np.float32(1.0 / np.sqrt(np.float32(deg[r]))) * np.float32(1.0 / np.sqrt(np.float32(deg[c])))
        assert w[e].item() == pytest.approx(float(expect), rel=2e-7)


def test_pow_minus_half_is_reciprocal_sqrt():
    """deg.pow(-0.5) on integer degrees equals the correctly rounded
    1/sqrt (so a C restatement 1.0f/sqrtf(d) is bit-exact)."""
    d = torch.arange(1, 200001, dtype=torch.float32)
    a = d.pow(-0.5)
    b = torch.from_numpy((np.float32(1.0) / np.sqrt(d.numpy())).astype(np.float32))
    assert torch.equal(a, b)


def test_gcn_norm_isolated_node_weight_zero_not_inf():
    ei = torch.tensor([[0], [1]])
    w = oracle.compute_gcn_norm(ei, 3, add_loops=False)
    assert torch.isfinite(w).all()


# --------------------------------------------------------------------- CSR --

def test_csr_rows_and_permutation():
    g = torch.Generator().manual_seed(1)
    n = 50
    ei = torch.randint(0, n, (2, 700), generator=g)
    rowptr, col, perm = oracle.edge_index_to_csr(ei, n)
    counts = torch.bincount(ei[0], minlength=n)
    assert torch.equal(rowptr[1:] - rowptr[:-1], counts)
    assert torch.equal(col, ei[1][perm])
    for r in range(n):
        got = sorted(col[rowptr[r]:rowptr[r + 1]].tolist())
        expect = sorted(ei[1][ei[0] == r].tolist())
        assert got == expect


# --------------------------------------------------------- build_subgraph --

def test_build_subgraph_reference_known_answer():
    """tests/test_cpp_extensions.py:64-84."""
    rowptr = torch.tensor([0, 2, 3, 4, 4])
    col = torch.tensor([1, 2, 2, 3])
    r, c, v, n_id = oracle.build_subgraph(rowptr, col, None, torch.tensor([0, 1]), True)
    assert r.tolist() == [0, 2, 3]
    assert c.tolist() == [1, 2, 2]
    assert n_id.tolist() == [0, 1, 2]
    assert v is None


def test_build_subgraph_values_and_non_bipartite():
    """tests/test_cpp_extensions.py:86-106."""
    rowptr = torch.tensor([0, 2, 3, 4, 4])
    col = torch.tensor([1, 2, 2, 3])
    value = torch.tensor([0.5, 0.3, 0.7, 0.1])
    r, c, v, n_id = oracle.build_subgraph(rowptr, col, value, torch.tensor([0]), True)
    assert v.tolist() == pytest.approx([0.5, 0.3])
    assert c.tolist() == [1, 2] and n_id.tolist() == [0, 1, 2]
    rowptr = torch.tensor([0, 2, 3, 3])
    col = torch.tensor([1, 2, 2])
    r, c, v, n_id = oracle.build_subgraph(rowptr, col, None, torch.tensor([0]), False)
    assert r.numel() == n_id.numel() + 1
    assert r.tolist() == [0, 2, 2, 2]


def _random_csr(n, m, seed):
    g = torch.Generator().manual_seed(seed)
    ei = torch.randint(0, n, (2, m), generator=g)
    rowptr, col, _ = oracle.edge_index_to_csr(ei, n)
    val = torch.rand(col.numel(), generator=g)
    return rowptr, col, val


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_build_subgraph_matches_compiled_reference(seed):
    ref = oracle.ref_build_subgraph()
    if ref is None:
        pytest.skip("reference build (oracle/_ref) not present")
    rowptr, col, val = _random_csr(120, 900, seed)
    g = torch.Generator().manual_seed(seed + 10)
    idx = torch.randperm(120, generator=g)[:37]
    for bip in (True, False):
        a = oracle.build_subgraph(rowptr, col, val, idx, bip)
        b = ref(rowptr, col, val, idx, bip)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
        assert torch.equal(a[2], b[2]) and torch.equal(a[3], b[3])


def test_build_subgraph_brute_force_relabel():
    """Every output edge maps back to an input edge of the same seed row."""
    rowptr, col, val = _random_csr(60, 400, 5)
    idx = torch.tensor([5, 17, 3, 44])
    r, c, v, n_id = oracle.build_subgraph(rowptr, col, val, idx, True)
    for i, s in enumerate(idx.tolist()):
        got = [(int(n_id[x]), float(y)) for x, y in zip(c[r[i]:r[i + 1]], v[r[i]:r[i + 1]])]
        exp = [(int(x), float(y)) for x, y in zip(col[rowptr[s]:rowptr[s + 1]],
                                                   val[rowptr[s]:rowptr[s + 1]])]
        assert got == exp
    assert len(set(n_id.tolist())) == n_id.numel()


# ---------------------------------------------- partition subgraph / pipeline --

def _banded(n, reach):
    edges = set()
    for i in range(n):
        for j in range(max(0, i - reach), min(n, i + reach + 1)):
            if i != j:
                edges.add((i, j))
    return torch.tensor([[e[0] for e in edges], [e[1] for e in edges]], dtype=torch.long)


def test_partition_subgraph_serial_equals_parallel():
    """tests/test_partition.py:207-249: banded 20-node graph, ptr [0,5,10,15,20]."""
    ei = _banded(20, 3)
    w = oracle.compute_gcn_norm(ei, 20, True)
    ei = oracle.add_self_loops(ei, 20)
    rowptr, col, sp = oracle.edge_index_to_csr(ei, 20)
    w = w[sp]
    ptr = torch.tensor([0, 5, 10, 15, 20])
    serial = [oracle.build_partition_subgraph(p, ptr, rowptr, col, w, 4) for p in range(4)]
    with ThreadPoolExecutor(4) as ex:
        par = list(ex.map(lambda p: oracle.build_partition_subgraph(p, ptr, rowptr, col, w, 4),
                          range(4)))
    for s, q in zip(serial, par):
        assert s[0] == q[0] and s[3:] == q[3:]
        for a, b in zip(s[1], q[1]):
            assert torch.equal(a, b)
        for a, b in zip(s[2], q[2]):
            assert (a is None and b is None) or torch.equal(a, b)
    for pid, (rp, c, v), bnd, expanded, batch in serial:
        assert rp.numel() == batch + 1
        assert bnd[pid] is None
        assert int(c.max()) < expanded


def test_partition_subgraph_gather_invariant():
    """Gathering rows in the [intra | halo by owner] layout and aggregating with
    the remapped columns equals aggregating the global rows directly."""
    ei = _banded(30, 4)
    n = 30
    w = oracle.compute_gcn_norm(ei, n, True)
    ei = oracle.add_self_loops(ei, n)
    rowptr, col, sp = oracle.edge_index_to_csr(ei, n)
    w = w[sp]
    ptr = torch.tensor([0, 8, 17, 30])
    x = torch.randn(n, 5, generator=torch.Generator().manual_seed(3))
    full = oracle.spmm(rowptr, col, w, x)
    for pid in range(3):
        _, (rp, c, v), bnd, expanded, batch = oracle.build_partition_subgraph(
            pid, ptr, rowptr, col, w, 3)
        srcs = [x[ptr[p]:ptr[p + 1]] for p in range(3)]
        gathered = torch.from_numpy(oracle.gather_partitions(pid, srcs, bnd))
        assert gathered.shape[0] == expanded
        part = oracle.spmm(rp, c, v, gathered)
        assert np.allclose(part, full[int(ptr[pid]):int(ptr[pid + 1])], rtol=0, atol=1e-12)


# Hand-derived known answer for the halo layout of
# grinnder/data/partition.py:195-225 (derivation written out below).
# 8 nodes, 3 partitions ptr=[0,3,5,8]: p0={0,1,2}, p1={3,4}, p2={5,6,7}.
# Neighbour lists are chosen so that discovery order within an owner is
# NOT ascending (a sorted-within-owner restatement gives different lists).
HALO_ROWS = [[7, 3, 5], [4, 6, 0], [5, 3, 7, 1], [6, 1, 3, 0], [2, 7, 5, 1], [5, 4, 0], [],
             [2, 7, 3, 0, 4]]
HALO_PTR = [0, 3, 5, 8]
# pid 0: first-seen halo ids 7,3,5,4,6 -> owner p1: 3,4 ; owner p2: 7,5,6
#   layout [0,1,2 | 3,4 | 7,5,6]; row 0 (7,3,5) -> (5,3,6) ...
# pid 1: first-seen 6,1,0,2,7,5 -> p0: 1,0,2 ; p2: 6,7,5
#   layout [3,4 | 1,0,2 | 6,7,5]
# pid 2: first-seen 4,0,2,3 -> p0: 0,2 ; p1: 4,3
#   layout [5,6,7 | 0,2 | 4,3]
HALO_EXPECTED = {
    0: dict(rowptr=[0, 3, 6, 10], col=[5, 3, 6, 4, 7, 0, 6, 3, 5, 1],
            boundaries=[None, [0, 1], [2, 0, 1]], expanded=8, batch=3),
    1: dict(rowptr=[0, 4, 8], col=[5, 2, 0, 3, 4, 6, 7, 2],
            boundaries=[[1, 0, 2], None, [1, 2, 0]], expanded=8, batch=2),
    2: dict(rowptr=[0, 3, 3, 8], col=[0, 5, 3, 4, 2, 6, 3, 5],
            boundaries=[[0, 2], [1, 0], None], expanded=7, batch=3),
}


def _halo_csr():
    rowptr = torch.tensor([0] + np.cumsum([len(r) for r in HALO_ROWS]).tolist())
    col = torch.tensor([c for r in HALO_ROWS for c in r])
    val = torch.arange(col.numel(), dtype=torch.float32) + 0.5
    return rowptr, col, val


def check_halo_known_answer(fn):
    """Checks fn(pid, ptr, rowptr, col, w, P) against HALO_EXPECTED."""
    rowptr, col, val = _halo_csr()
    ptr = torch.tensor(HALO_PTR)
    for pid, exp in HALO_EXPECTED.items():
        got_pid, (rp, c, v), bnd, expanded, batch = fn(pid, ptr, rowptr, col, val, 3)
        assert got_pid == pid
        assert rp.tolist() == exp["rowptr"], pid
        assert c.tolist() == exp["col"], pid
        seeds = range(HALO_PTR[pid], HALO_PTR[pid + 1])
        assert v.tolist() == [float(val[j]) for s in seeds
                              for j in range(int(rowptr[s]), int(rowptr[s + 1]))]
        assert [None if b is None else b.tolist() for b in bnd] == exp["boundaries"], pid
        assert (expanded, batch) == (exp["expanded"], exp["batch"])


def check_halo_layout_property(fn, seed):
    """Independent restatement of the layout: the concatenated global ids of
    the boundaries are n_id[B:] stably sorted by owning partition, and each
    remapped column addresses the same global node as before the remap."""
    g = torch.Generator().manual_seed(seed)
    n, parts = 120, 5
    ei = torch.randint(0, n, (2, 900), generator=g)
    rowptr, col, _ = oracle.edge_index_to_csr(ei, n)
    val = torch.rand(col.numel(), generator=g)
    cuts = torch.sort(torch.randperm(n - 1, generator=g)[:parts - 1] + 1).values
    ptr = torch.cat([torch.tensor([0]), cuts, torch.tensor([n])])
    for pid in range(parts):
        lo, hi = int(ptr[pid]), int(ptr[pid + 1])
        _, _, _, n_id = oracle.build_subgraph(rowptr, col, val, torch.arange(lo, hi), True)
        halo = n_id[hi - lo:]
        owner = torch.searchsorted(ptr, halo, right=True) - 1
        order = torch.sort(owner, stable=True).indices
        _, (rp, c, v), bnd, expanded, batch = fn(pid, ptr, rowptr, col, val, parts)
        got = [b + ptr[p] for p, b in enumerate(bnd) if b is not None]
        got = torch.cat(got) if got else torch.zeros(0, dtype=torch.long)
        assert torch.equal(got, halo[order])
        layout = torch.cat([torch.arange(lo, hi), got])
        assert expanded == layout.numel() and batch == hi - lo
        assert torch.equal(layout[c], col[int(rowptr[lo]):int(rowptr[hi])])
        for p, b in enumerate(bnd):
            assert (b is None) == (p == pid or not bool((owner == p).any()))


def _sorted_within_owner(pid, ptr, rowptr, col, w, parts):
    """A plausible slip: the oracle with halo ids sorted within each owner."""
    out = oracle.build_partition_subgraph(pid, ptr, rowptr, col, w, parts)
    _, (rp, c, v), bnd, expanded, batch = out
    layout_old = torch.cat([torch.arange(int(ptr[pid]), int(ptr[pid + 1]))]
                           + [b + ptr[p] for p, b in enumerate(bnd) if b is not None])
    bnd = [None if b is None else torch.sort(b).values for b in bnd]
    layout = torch.cat([torch.arange(int(ptr[pid]), int(ptr[pid + 1]))]
                       + [b + ptr[p] for p, b in enumerate(bnd) if b is not None])
    pos = {int(g): i for i, g in enumerate(layout.tolist())}
    c = torch.tensor([pos[int(layout_old[k])] for k in c.tolist()], dtype=torch.long)
    return pid, (rp, c, v), bnd, expanded, batch


def test_partition_subgraph_halo_order_known_answer():
    check_halo_known_answer(oracle.build_partition_subgraph)


@pytest.mark.parametrize("seed", range(3))
def test_partition_subgraph_halo_layout_property(seed):
    check_halo_layout_property(oracle.build_partition_subgraph, seed)


def test_halo_checks_reject_sorted_within_owner():
    """The two checks above fail for an oracle that sorts halo ids within an
    owner (the mistake is planted in a copy of the oracle, on the CPU)."""
    with pytest.raises(AssertionError):
        check_halo_known_answer(_sorted_within_owner)
    with pytest.raises(AssertionError):
        check_halo_layout_property(_sorted_within_owner, 0)


# ------------------------------------------- orientation on directed graphs --
# The reference takes CSR rows from edge_index[0] (grinnder/data/partition.py:
# 79-87) but counts degrees on edge_index[1] (grinnder/data/datasets.py:356-
# 360).  On a symmetric graph neither choice is observable; these checks use
# directed graphs.  `fn(edge_index, n, perm, ptr)` returns the per-partition
# list [(pid, (rowptr, col, value), boundaries, expanded, batch)].

# 0->1, 0->3, 1->2, 3->0, 4->0, 4->2, 2->4 (edge_index[0] -> edge_index[1])
DIRECTED_EI = [[0, 0, 1, 3, 4, 4, 2], [1, 3, 2, 0, 0, 2, 4]]


def check_directed_known_answer(fn):
    """Hand-derived on DIRECTED_EI with identity perm and ptr [0, 3, 5].
    Degrees on edge_index[1] plus the self-loop: [3, 2, 3, 2, 2].  Rows are
    edge_index[0] (out-neighbours plus self).  Partition 0 (rows 0-2) finds
    halo 3 in row 0, then 4 in row 2; partition 1 (rows 3-4) finds 0 in row
    3, then 2 in row 4.  Within-row order is argsort's, so rows compare as
    multisets of (local column, weight)."""
    r2, r3 = np.float32(1) / np.sqrt(np.float32(2)), np.float32(1) / np.sqrt(np.float32(3))
    w = {(a, b): float(a * b) for a in (r2, r3) for b in (r2, r3)}
    d = [r3, r2, r3, r2, r2]
    expect = {
        0: dict(rows=[{(1, w[d[0], d[1]]), (3, w[d[0], d[3]]), (0, w[d[0], d[0]])},
                      {(2, w[d[1], d[2]]), (1, w[d[1], d[1]])},
                      {(4, w[d[2], d[4]]), (2, w[d[2], d[2]])}],
                boundaries=[None, [0, 1]], expanded=5, batch=3),
        1: dict(rows=[{(2, w[d[3], d[0]]), (0, w[d[3], d[3]])},
                      {(2, w[d[4], d[0]]), (3, w[d[4], d[2]]), (1, w[d[4], d[4]])}],
                boundaries=[[0, 2], None], expanded=4, batch=2),
    }
    out = fn(torch.tensor(DIRECTED_EI), 5, torch.arange(5), torch.tensor([0, 3, 5]))
    for pid, (got_pid, (rp, c, v), bnd, expanded, batch) in enumerate(out):
        exp = expect[pid]
        assert got_pid == pid
        rows = [set(zip(c[int(rp[r]):int(rp[r + 1])].tolist(),
                        v[int(rp[r]):int(rp[r + 1])].tolist())) for r in range(batch)]
        assert rows == exp["rows"], pid
        assert [None if b is None else b.tolist() for b in bnd] == exp["boundaries"], pid
        assert (expanded, batch) == (exp["expanded"], exp["batch"]), pid


def check_directed_brute_force(fn, seed, n=300, m=2500, parts=4):
    """A random directed multigraph under a random perm and random cuts: every
    partition row r (new id) holds exactly the out-edges r -> j of the
    relabelled edge list plus its self-loop, each weighted fp32(deg[r]^-1/2)
    * fp32(deg[j]^-1/2) with deg[j] counted by brute force over the edges'
    targets (plus 1); columns resolve to global ids through the layout
    [own rows | boundaries by owner]."""
    g = torch.Generator().manual_seed(seed)
    ei = torch.randint(0, n, (2, m), generator=g)
    ei = ei[:, ei[0] != ei[1]]
    perm = torch.randperm(n, generator=g)
    cuts = torch.sort(torch.randperm(n - 1, generator=g)[:parts - 1] + 1).values
    ptr = torch.cat([torch.tensor([0]), cuts, torch.tensor([n])])
    inv = [0] * n
    for new, old in enumerate(perm.tolist()):
        inv[old] = new
    src = [inv[s] for s in ei[0].tolist()]
    dst = [inv[t] for t in ei[1].tolist()]
    deg = [1] * n
    for t in dst:
        deg[t] += 1
    rs = [np.float32(1) / np.sqrt(np.float32(k)) for k in deg]
    out_edges = [[] for _ in range(n)]
    for s, t in zip(src + list(range(n)), dst + list(range(n))):
        out_edges[s].append((t, float(rs[s] * rs[t])))
    for pid, (_, (rp, c, v), bnd, expanded, batch) in enumerate(fn(ei, n, perm, ptr)):
        lo = int(ptr[pid])
        layout = [lo + k for k in range(batch)]
        for p, b in enumerate(bnd):
            if b is not None:
                layout += [int(ptr[p]) + k for k in b.tolist()]
        assert len(layout) == expanded
        for r in range(batch):
            a, e = int(rp[r]), int(rp[r + 1])
            got = sorted(zip((layout[k] for k in c[a:e].tolist()), v[a:e].tolist()))
            assert got == sorted(out_edges[lo + r]), (pid, r)


def _swapped_pipeline(ei, n, perm, ptr):
    """A plausible slip: the pipeline with edge_index[0] and [1] swapped
    (rows from the targets, degrees on the sources)."""
    return oracle.partition_pipeline(ei.flip(0), n, perm, ptr)


def _row_degree_pipeline(ei, n, perm, ptr):
    """A plausible slip: degrees counted on edge_index[0] instead of [1].
    The oracle's structure is kept and every weight recomputed from the
    out-degrees (plus the self-loop)."""
    out = oracle.partition_pipeline(ei, n, perm, ptr)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(n)
    e = inv[ei]
    deg = torch.bincount(e[0], minlength=n).to(torch.float32) + 1
    rs = deg.pow(-0.5)
    fixed = []
    for pid, (rp, c, v), bnd, expanded, batch in out:
        lo = int(ptr[pid])
        layout = torch.tensor([lo + k for k in range(batch)]
                              + [int(ptr[p]) + k for p, b in enumerate(bnd) if b is not None
                                 for k in b.tolist()], dtype=torch.long)
        rows = torch.repeat_interleave(torch.arange(batch), rp[1:] - rp[:-1]) + lo
        fixed.append((pid, (rp, c, rs[rows] * rs[layout[c]]), bnd, expanded, batch))
    return fixed


def test_directed_pipeline_known_answer():
    check_directed_known_answer(oracle.partition_pipeline)


@pytest.mark.parametrize("seed", range(3))
def test_directed_pipeline_brute_force(seed):
    check_directed_brute_force(oracle.partition_pipeline, seed)


def test_directed_checks_reject_swapped_orientation_and_row_degrees():
    """Both checks fail for a pipeline that swaps edge_index[0] and [1], and
    for one that counts degrees on edge_index[0] (the mistakes are planted
    in copies of the oracle, on the CPU)."""
    for slip in (_swapped_pipeline, _row_degree_pipeline):
        with pytest.raises(AssertionError):
            check_directed_known_answer(slip)
        with pytest.raises(AssertionError):
            check_directed_brute_force(slip, 0)


# ----------------------------------------------------------- arithmetic --

def _dense(rowptr, col, val, rows, cols):
    a = torch.zeros(rows, cols, dtype=torch.float64)
    for i in range(rows):
        for e in range(int(rowptr[i]), int(rowptr[i + 1])):
            a[i, col[e]] += float(val[e])
    return a


def test_spmm_matches_dense_brute_force():
    rowptr, col, val = random_bipartite(40, 55, 6, seed=2, long_rows=1, long_len=90)
    x = torch.randn(55, 9, dtype=torch.float32, generator=torch.Generator().manual_seed(0))
    b = torch.randn(9)
    a = _dense(rowptr, col, val, 40, 55)
    ref = a @ x.double() + b.double()
    got = oracle.spmm(rowptr, col, val, x, b)
    assert np.allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)
    g = torch.randn(40, 9)
    got_t = oracle.spmm_t(rowptr, col, val, g, 55)
    assert np.allclose(got_t, (a.t() @ g.double()).numpy(), rtol=1e-12, atol=1e-12)


def test_spmm_rows_matches_dense_brute_force():
    """The row-subset driver (used at full size on sampled rows): repeated and
    unordered row ids, empty rows, a bias, and any thread count."""
    rowptr, col, val = random_bipartite(60, 70, 7, seed=12, long_rows=2, long_len=150)
    x = torch.randn(70, 6, generator=torch.Generator().manual_seed(1))
    b = torch.randn(6)
    ref = (_dense(rowptr, col, val, 60, 70) @ x.double() + b.double()).numpy()
    rows = torch.tensor([59, 3, 3, 0, 17, 42, 8, 8, 31])
    for threads in (1, 4, 16):
        got = oracle.spmm_rows(rowptr, col, val, x, rows, b, threads=threads)
        assert np.allclose(got, ref[rows.numpy()], rtol=0, atol=1e-12)
    with pytest.raises(IndexError):
        oracle.spmm_rows(rowptr, col, val, x, torch.tensor([60]))


def test_spmm_special_cases():
    # identity adjacency (self-loops only): Y = X + b
    n = 7
    rowptr = torch.arange(n + 1)
    col = torch.arange(n)
    val = torch.ones(n)
    x = torch.randn(n, 4)
    assert np.array_equal(oracle.spmm(rowptr, col, val, x), x.double().numpy())
    # all-ones features: each output row equals its row's weight sum
    rowptr, col, val = random_bipartite(20, 30, 5, seed=9)
    ones = torch.ones(30, 3)
    rs = torch.zeros(20, dtype=torch.float64)
    for i in range(20):
        rs[i] = val[rowptr[i]:rowptr[i + 1]].double().sum()
    got = oracle.spmm(rowptr, col, val, ones)
    assert np.allclose(got, rs[:, None].expand(20, 3).numpy(), atol=1e-12)


def _dense_gat(a_mask, hs, att_src, att_dst, bias, H, C, concat):
    """Dense float64 GAT: masked logits, softmax with max subtraction and +1e-16."""
    B = a_mask.shape[0]
    h3 = hs.view(-1, H, C)
    s = (h3 * att_src.view(1, H, C)).sum(-1)  # [E,H]
    d = (h3[:B] * att_dst.view(1, H, C)).sum(-1)  # [B,H]
    t = s.t().unsqueeze(1) + d.t().unsqueeze(2)  # [H,B,E]
    v = torch.nn.functional.leaky_relu(t, 0.2)
    cnt = a_mask.unsqueeze(0).to(torch.float64)  # multiplicity of each (i, j)
    neg = torch.finfo(torch.float64).min
    m = torch.where(cnt > 0, v, torch.full_like(v, neg)).amax(-1, keepdim=True).detach()
    m = torch.where(m == neg, torch.zeros_like(m), m)  # rows without edges
    p = torch.exp(torch.where(cnt > 0, v - m, torch.zeros_like(v))) * cnt
    den = p.sum(-1, keepdim=True) + 1e-16
    alpha = p / den  # [H,B,E] (summed over duplicate edges)
    o = torch.einsum("hbe,ehc->bhc", alpha, h3)
    out = o.reshape(B, H * C) if concat else o.mean(1)
    return out + bias


@pytest.mark.parametrize("H,C,concat", [(1, 5, True), (3, 4, True), (2, 3, False)])
def test_gat_oracle_matches_dense_autograd(H, C, concat):
    B, E = 9, 13
    rowptr, col, _ = random_bipartite(B, E, 3, seed=H + C, empty_frac=0.1)
    # dense multiplicity matrix (duplicates allowed)
    mask = torch.zeros(B, E)
    for i in range(B):
        for e in range(int(rowptr[i]), int(rowptr[i + 1])):
            mask[i, col[e]] += 1
    g = torch.Generator().manual_seed(4)
    hs = torch.randn(E, H * C, generator=g)
    a_s = torch.randn(1, H, C, generator=g)
    a_d = torch.randn(1, H, C, generator=g)
    out_w = H * C if concat else C
    b = torch.randn(out_w, generator=g)
    gy = torch.randn(B, out_w, generator=g)

    ref_out, alpha, tpre = oracle.gat_forward(rowptr, col, hs, H, C, a_s, a_d, b, concat)
    dhs, das, dad, db = oracle.gat_backward(rowptr, col, hs, H, C, a_s, a_d, concat, alpha,
                                            tpre, gy)

    hs64 = hs.double().requires_grad_(True)
    as64 = a_s.double().requires_grad_(True)
    ad64 = a_d.double().requires_grad_(True)
    b64 = b.double().requires_grad_(True)
    out = _dense_gat(mask, hs64, as64, ad64, b64, H, C, concat)
    out.backward(gy.double())
    assert np.allclose(ref_out, out.detach().numpy(), rtol=1e-10, atol=1e-10)
    assert np.allclose(dhs, hs64.grad.numpy(), rtol=1e-9, atol=1e-10)
    assert np.allclose(das, as64.grad.reshape(-1).numpy(), rtol=1e-9, atol=1e-10)
    assert np.allclose(dad, ad64.grad.reshape(-1).numpy(), rtol=1e-9, atol=1e-10)
    assert np.allclose(db, b64.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_dense_gat_gradcheck():
    """The dense restatement itself is differentiated correctly (finite differences)."""
    B, E, H, C = 4, 6, 2, 3
    rowptr, col, _ = random_bipartite(B, E, 2, seed=1, empty_frac=0.0)
    mask = torch.zeros(B, E)
    for i in range(B):
        for e in range(int(rowptr[i]), int(rowptr[i + 1])):
            mask[i, col[e]] += 1
    g = torch.Generator().manual_seed(0)
    hs = torch.randn(E, H * C, generator=g, dtype=torch.float64, requires_grad=True)
    a_s = torch.randn(1, H, C, generator=g, dtype=torch.float64, requires_grad=True)
    a_d = torch.randn(1, H, C, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(H * C, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(
        lambda h, s, d, bb: _dense_gat(mask, h, s, d, bb, H, C, True), (hs, a_s, a_d, b))


# ------------------------------------------------------- gather / scatter --

def _arange_fixture():
    """tests/test_cpp_extensions.py:144-171 / tests/test_buffers.py:49-76."""
    p0 = torch.arange(8, dtype=torch.float).reshape(4, 2)
    p1 = torch.arange(8, 14, dtype=torch.float).reshape(3, 2)
    p2 = torch.arange(14, 24, dtype=torch.float).reshape(5, 2)
    return [p0, p1, p2], [None, torch.tensor([0, 2]), torch.tensor([3])]


def test_gather_reference_fixture():
    srcs, bnd = _arange_fixture()
    out = oracle.gather_partitions(0, srcs, bnd)
    assert out.shape == (7, 2)
    assert np.array_equal(out[:4], srcs[0].numpy())
    assert np.array_equal(out[4:6], srcs[1][[0, 2]].numpy())
    assert np.array_equal(out[6:7], srcs[2][[3]].numpy())
    assert out.tolist() == [[0, 1], [2, 3], [4, 5], [6, 7], [8, 9], [12, 13], [20, 21]]


def test_scatter_reference_fixtures():
    # tests/test_cpp_extensions.py:173-202: ones into zeros
    dsts = [torch.zeros(4, 2), torch.zeros(3, 2), torch.zeros(5, 2)]
    bnd = [None, torch.tensor([0, 2]), torch.tensor([3])]
    out = oracle.scatter_partitions(0, torch.ones(7, 2), dsts, bnd)
    assert np.array_equal(out[0], np.ones((4, 2), np.float32))
    assert out[1].tolist() == [[1, 1], [0, 0], [1, 1]]
    assert out[2][3].tolist() == [1, 1] and out[2].sum() == 2
    # tests/test_host_buffer_ops.py:40-60: 1.0 + 2.0 = 3.0 on the self block
    dsts = [torch.ones(4, 2), torch.zeros(3, 2), torch.zeros(5, 2)]
    out = oracle.scatter_partitions(0, torch.full((7, 2), 2.0), dsts, bnd)
    assert np.array_equal(out[0], np.full((4, 2), 3.0, np.float32))


def test_scatter_repeated_indices_accumulate_in_order():
    """index_put_(accumulate=True) semantics: repeated indices all add."""
    dsts = [torch.zeros(2, 1), torch.zeros(3, 1)]
    bnd = [None, torch.tensor([1, 1, 2])]
    src = torch.tensor([[1.0], [2.0], [3.0], [4.0], [5.0]])
    out = oracle.scatter_partitions(0, src, dsts, bnd)
    assert out[1].reshape(-1).tolist() == [0.0, 7.0, 5.0]


# ------------------------------------- the GPU epoch tests' torch restatements --

def test_gat_restatement_matches_oracle():
    """tests/restate.py's one-head GAT attention (the float64 model checker of
    the epoch-level GPU tests) equals the oracle's GATConv forward and
    backward on a small square graph, rows from the CSR."""
    from tests.restate import gat_attention_full

    n, c = 150, 12
    rowptr, col, _ = random_bipartite(n, n, 6, seed=3, long_rows=2, long_len=40)
    g = torch.Generator().manual_seed(4)
    hs = torch.randn(n, c, generator=g, dtype=torch.float64)
    a_s = torch.randn(1, 1, c, generator=g, dtype=torch.float64)
    a_d = torch.randn(1, 1, c, generator=g, dtype=torch.float64)
    b = torch.randn(c, generator=g, dtype=torch.float64)
    gy = torch.randn(n, c, generator=g, dtype=torch.float64)
    dst = torch.repeat_interleave(torch.arange(n), rowptr[1:] - rowptr[:-1])
    leaves = [t.clone().requires_grad_(True) for t in (hs, a_s, a_d, b)]
    out = gat_attention_full(*leaves, dst, col, n)
    out.backward(gy)
    ref_o, alpha, tpre = oracle.gat_forward(rowptr, col, hs.float(), 1, c, a_s.float(),
                                            a_d.float(), b.float(), True)
    refs = oracle.gat_backward(rowptr, col, hs.float(), 1, c, a_s.float(), a_d.float(), True,
                               alpha, tpre, gy.float())
    # The oracle takes fp32 inputs (accumulating in float64): compare at fp32 input rounding.
    assert torch.allclose(out.detach(), torch.from_numpy(ref_o), rtol=1e-5, atol=1e-5)
    for got, ref in zip(leaves, refs):
        ref = torch.as_tensor(ref).reshape(got.shape)
        assert torch.allclose(got.grad, ref, rtol=1e-4, atol=1e-4), (got.grad - ref).abs().max()


def test_gcn_restatement_matches_dense():
    """tests/restate.py's GCN layers equal a dense float64 restatement."""
    from grinnder_amd.nn import GCN
    from tests.restate import gcn_layers

    n = 120
    rowptr, col, val = random_bipartite(n, n, 5, seed=8)
    a = torch.sparse_csr_tensor(rowptr, col, val.double(), (n, n))
    dense = a.to_dense()
    torch.manual_seed(1)
    model = GCN(16, 24, 5, num_layers=3, dropout=0.0, norm=True).double()
    x = torch.randn(n, 16, dtype=torch.float64)
    got = gcn_layers(model, a, x)
    h = x
    for i, conv in enumerate(model.convs):
        h = dense @ (h @ conv.lin.weight.t()) + conv.bias
        if i < 2:
            h = torch.relu(model.norms[i](h))
    assert torch.allclose(got, h, rtol=1e-12, atol=1e-12)
