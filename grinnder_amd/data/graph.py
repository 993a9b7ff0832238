"""PartitionedGraph (grinnder/data/graph.py:12-84), plus cached adjacencies."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Tuple

import torch
from torch import Tensor

from grinnder_amd.data.adjacency import Adjacency


@dataclass
class PartitionedGraph:
    """A graph partitioned into contiguous node ranges ``ptr[p]:ptr[p+1]``.

    adj_csr[p] = (rowptr [B_p+1], col [nnz_p] in [0, E_p), value [nnz_p]) is the
    bipartite adjacency of partition p: rows are its B_p nodes, columns its
    E_p = B_p + halo gathered rows laid out [intra | halo from p'=0..P-1].
    boundaries[p][p'] = local row indices (int64) in partition p' of the halo
    rows p needs from p' (None for p' == p or when empty).
    """

    num_nodes: int
    num_edges: int
    num_parts: int
    partition_sizes: List[int]
    adj_csr: List[Tuple[Tensor, Tensor, Optional[Tensor]]]
    boundaries: List[List[Optional[Tensor]]]
    expanded_sizes: List[int]
    features: Any
    labels: Tensor
    train_mask: Tensor
    val_mask: Tensor
    test_mask: Tensor
    perm: Tensor
    ptr: Tensor
    _adjs: Dict[int, Adjacency] = field(default_factory=dict, repr=False, compare=False)
    _whole: Optional[Adjacency] = field(default=None, repr=False, compare=False)

    @property
    def feat_dim(self) -> int:
        return self.features.shape[1]

    @property
    def num_classes(self) -> int:
        return int(self.labels.max().item()) + 1

    def _range(self, pid: int) -> Tuple[int, int]:
        return int(self.ptr[pid].item()), int(self.ptr[pid + 1].item())

    def partition_features(self, pid: int) -> Tensor:
        start, end = self._range(pid)
        if hasattr(self.features, "partition"):
            return self.features.partition(start, end)
        return self.features[start:end]

    def partition_labels(self, pid: int) -> Tensor:
        start, end = self._range(pid)
        return self.labels[start:end]

    def partition_train_mask(self, pid: int) -> Tensor:
        start, end = self._range(pid)
        return self.train_mask[start:end]

    def partition_val_mask(self, pid: int) -> Tensor:
        start, end = self._range(pid)
        return self.val_mask[start:end]

    def partition_test_mask(self, pid: int) -> Tensor:
        start, end = self._range(pid)
        return self.test_mask[start:end]

    def adjacency(self, pid: int) -> Adjacency:
        """The partition's adjacency object (device plans are built on first use)."""
        adj = self._adjs.get(pid)
        if adj is None:
            rowptr, col, value = self.adj_csr[pid]
            adj = Adjacency(rowptr, col, value,
                            (self.partition_sizes[pid], self.expanded_sizes[pid]))
            self._adjs[pid] = adj
        return adj

    def gathered_rows(self, pid: int) -> Tensor:
        """Global ids (int64, host) of partition pid's E_p gathered rows, in
        the column order of adj_csr[pid]: its own rows, then the halo rows
        from p' = 0..P-1."""
        lo, hi = self._range(pid)
        parts = [torch.arange(lo, hi, dtype=torch.int64)]
        for q, b in enumerate(self.boundaries[pid]):
            if q != pid and b is not None and b.numel() > 0:
                parts.append(b.to(torch.int64) + int(self.ptr[q]))
        rows = torch.cat(parts)
        if rows.numel() != self.expanded_sizes[pid]:
            raise RuntimeError(f"partition {pid}: {rows.numel()} gathered rows, "
                               f"expected {self.expanded_sizes[pid]}")
        return rows

    def whole_adjacency(self) -> Adjacency:
        """Every partition's adjacency as one [N, N] adjacency over global
        row ids (built on first use, cached): row r of partition p is global
        row ptr[p] + r with the same edges in the same order, each column
        mapped through gathered_rows(p).  Its forward plan runs the
        partitions' rows partition by partition (row_blocks = ptr)."""
        if self._whole is None:
            n = int(self.ptr[-1])
            rowptr = torch.empty(n + 1, dtype=torch.int64)
            cols, vals = [], []
            off = 0
            for pid in range(self.num_parts):
                rp, col, val = self.adj_csr[pid]
                lo, hi = self._range(pid)
                rowptr[lo:hi] = rp[:-1].to(torch.int64) + off
                off += int(rp[-1])
                cols.append(self.gathered_rows(pid)[col.to(torch.int64)])
                vals.append(val.to(torch.float32) if val is not None
                            else torch.ones(col.numel(), dtype=torch.float32))
            rowptr[n] = off
            self._whole = Adjacency(rowptr, torch.cat(cols), torch.cat(vals), (n, n),
                                    row_blocks=self.ptr.to(torch.int64).clone())
        return self._whole

    def halo_amplification(self) -> float:
        """sum_p E_p / N: gathered rows per node per layer."""
        return sum(self.expanded_sizes) / max(1, self.num_nodes)
