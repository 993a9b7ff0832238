"""Seeded synthetic graphs and node data for the benchmark configurations.

The reference trains on downloaded OGB / IGB datasets; with no network, the
benchmark configurations are defined on seeded synthetic graphs of the same
shape: a uniform random graph (plumbing case) and R-MAT graphs
(a, b, c, d) = (.57, .19, .19, .05) with a seeded vertex permutation.

R-MAT samples come from gr_rmat_sample (counter-based, so the stream does not
depend on thread count); deduplication keeps the first K distinct valid pairs
in stream order, computed with torch ops on whichever device is given.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch
from torch import Tensor

from grinnder_amd import _lib


@dataclass
class NodeData:
    x: Tensor
    y: Tensor
    train_mask: Tensor
    val_mask: Tensor
    test_mask: Tensor


def uniform_graph(num_nodes: int, num_pairs: int, seed: int = 42) -> Tensor:
    """Undirected uniform random graph: `num_pairs` sampled pairs u != v,
    deduplicated and symmetrised (no self-loops).  Returns int64 [2, M]."""
    g = torch.Generator().manual_seed(seed)
    u = torch.randint(0, num_nodes, (num_pairs,), generator=g)
    v = torch.randint(0, num_nodes, (num_pairs,), generator=g)
    keep = u != v
    u, v = u[keep], v[keep]
    lo, hi = torch.minimum(u, v), torch.maximum(u, v)
    key = torch.unique(lo * num_nodes + hi)
    a, b = key // num_nodes, key % num_nodes
    return torch.stack([torch.cat([a, b]), torch.cat([b, a])])


def banded_graph(num_nodes: int, reach: int) -> Tensor:
    """Symmetric band graph |i - j| <= reach, i != j, in (i, j) lexicographic
    order (the construction of the reference's small test graphs)."""
    rows, cols = [], []
    for i in range(num_nodes):
        for j in range(max(0, i - reach), min(num_nodes, i + reach + 1)):
            if i != j:
                rows.append(i)
                cols.append(j)
    return torch.tensor([rows, cols], dtype=torch.long)


def rmat_sample(seed: int, scale: int, first: int, n: int, a: float = 0.57, b: float = 0.19,
                c: float = 0.19, nthreads: int = 0) -> Tuple[Tensor, Tensor]:
    """Samples [first, first+n) of the seeded R-MAT stream (CPU int64)."""
    src = torch.empty(max(n, 1), dtype=torch.int64)
    dst = torch.empty(max(n, 1), dtype=torch.int64)
    _lib.call("gr_rmat_sample", seed, scale, a, b, c, first, n, src.data_ptr(), dst.data_ptr(),
              nthreads)
    return src[:n], dst[:n]


def rmat_graph(num_nodes: int, num_edges: int, scale: Optional[int] = None, seed: int = 42,
               undirected: bool = True, device: str = "cpu", batch: int = 1 << 25,
               a: float = 0.57, b: float = 0.19, c: float = 0.19) -> Tensor:
    """R-MAT graph on `num_nodes` nodes with exactly `num_edges` distinct pairs.

    Vertex ids of the 2^scale R-MAT grid are shuffled by a seeded permutation,
    samples with an endpoint >= num_nodes or u == v are rejected, and the
    first `num_edges` distinct pairs (unordered if `undirected`) in stream
    order are kept.  Undirected graphs are returned symmetrised:
    [2, 2 * num_edges] as [(u, v) all, then (v, u) all].
    """
    if scale is None:
        scale = max(1, (num_nodes - 1).bit_length())
    if num_nodes > (1 << scale):
        raise ValueError("num_nodes exceeds 2^scale")
    g = torch.Generator().manual_seed(seed)
    relabel = torch.randperm(1 << scale, generator=g).to(device)
    keys = []
    n_valid = 0
    first = 0
    uniq_count = 0
    while True:
        s, d = rmat_sample(seed, scale, first, batch, a, b, c)
        first += batch
        s = relabel[s.to(device)]
        d = relabel[d.to(device)]
        ok = (s < num_nodes) & (d < num_nodes) & (s != d)
        s, d = s[ok], d[ok]
        if undirected:
            s, d = torch.minimum(s, d), torch.maximum(s, d)
        keys.append(s * num_nodes + d)
        n_valid += s.numel()
        if n_valid >= num_edges:
            allk = torch.cat(keys)
            keys = [allk]
            uniq_count = int(torch.unique(allk).numel())
            if uniq_count >= num_edges:
                break
    allk = keys[0]
    uniq, inv = torch.unique(allk, return_inverse=True)
    first_pos = torch.full((uniq.numel(),), allk.numel(), dtype=torch.int64, device=allk.device)
    first_pos.scatter_reduce_(0, inv, torch.arange(allk.numel(), device=allk.device), "amin")
    order = first_pos.argsort()[:num_edges]
    sel = uniq[order]
    u, v = sel // num_nodes, sel % num_nodes
    if undirected:
        ei = torch.stack([torch.cat([u, v]), torch.cat([v, u])])
    else:
        ei = torch.stack([u, v])
    return ei.cpu()


def node_data(num_nodes: int, feat_dim: int, num_classes: int, seed: int = 42,
              split=(0.6, 0.2), device: str = "cpu") -> NodeData:
    """x ~ N(0,1) fp32, uniform labels, random 60/20/20 train/val/test masks."""
    g = torch.Generator(device=device).manual_seed(seed + 1)
    x = torch.randn((num_nodes, feat_dim), generator=g, dtype=torch.float32, device=device)
    gc = torch.Generator().manual_seed(seed + 2)
    y = torch.randint(0, num_classes, (num_nodes,), generator=gc)
    order = torch.randperm(num_nodes, generator=gc)
    n_tr = int(split[0] * num_nodes)
    n_va = int(split[1] * num_nodes)
    train = torch.zeros(num_nodes, dtype=torch.bool)
    val = torch.zeros(num_nodes, dtype=torch.bool)
    test = torch.zeros(num_nodes, dtype=torch.bool)
    train[order[:n_tr]] = True
    val[order[n_tr:n_tr + n_va]] = True
    test[order[n_tr + n_va:]] = True
    return NodeData(x, y, train, val, test)


class SyntheticFeatures:
    """A [num_nodes, dim] N(0,1) fp32 feature matrix that is never materialised.

    Row v is generated from (seed, v) by gr_gaussian_rows, so partitions are
    produced on demand (the role of the reference's memory-mapped
    NumpyFeatureStore, grinnder/data/datasets.py:59-100): ``partition(start,
    end)`` returns the rows at new positions [start, end) after
    ``with_permutation(perm)``.
    """

    def __init__(self, num_nodes: int, dim: int, seed: int = 42,
                 perm: Optional[Tensor] = None):
        self.num_nodes = num_nodes
        self.dim = dim
        self.seed = seed
        self.perm = perm

    @property
    def shape(self):
        return (self.num_nodes, self.dim)

    def size(self, i: Optional[int] = None):
        return self.shape if i is None else self.shape[i]

    def with_permutation(self, perm: Tensor) -> "SyntheticFeatures":
        base = perm if self.perm is None else self.perm[perm]
        return SyntheticFeatures(self.num_nodes, self.dim, self.seed, base)

    def rows(self, ids: Tensor, out: Optional[Tensor] = None) -> Tensor:
        ids = ids.to(torch.int64).contiguous()
        if out is None:
            out = torch.empty((ids.numel(), self.dim), dtype=torch.float32)
        _lib.call("gr_gaussian_rows", self.seed, ids.data_ptr(), ids.numel(), self.dim,
                  out.data_ptr(), 0)
        return out

    def partition(self, start: int, end: int) -> Tensor:
        ids = torch.arange(start, end) if self.perm is None else self.perm[start:end]
        return self.rows(ids)

    def __getitem__(self, idx):
        if isinstance(idx, slice):
            start, stop, step = idx.indices(self.num_nodes)
            if step == 1:
                return self.partition(start, stop)
        ids = torch.arange(self.num_nodes)[idx]
        if self.perm is not None:
            ids = self.perm[ids]
        return self.rows(ids.reshape(-1))
