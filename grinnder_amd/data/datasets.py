"""GCN normalisation on the full graph (grinnder/data/datasets.py:334-362).

The reference computes it with PyG's ``add_self_loops`` (append (i, i) for
every node, no deduplication) and ``degree`` (scatter-add of fp32 ones over
``edge_index[1]``), then ``deg.pow(-0.5)`` with inf -> 0.  The same torch CPU
ops are used here so the weights are bit-identical.
"""

from __future__ import annotations

import torch
from torch import Tensor


def append_self_loops(edge_index: Tensor, num_nodes: int) -> Tensor:
    """Appends the N self-loops (i, i) after the existing edges (PyG add_self_loops)."""
    loops = torch.arange(num_nodes, dtype=edge_index.dtype, device=edge_index.device)
    return torch.cat([edge_index, torch.stack([loops, loops])], dim=1)


def degree(index: Tensor, num_nodes: int, dtype=torch.float32) -> Tensor:
    """Number of occurrences of each node id in `index` (as `dtype`)."""
    out = torch.zeros(num_nodes, dtype=dtype, device=index.device)
    return out.scatter_add_(0, index, torch.ones(index.numel(), dtype=dtype,
                                                 device=index.device))


def compute_gcn_norm(edge_index: Tensor, num_nodes: int, add_self_loops: bool = True) -> Tensor:
    """w_e = deg^-1/2[row_e] * deg^-1/2[col_e], deg counted over edge_index[1].

    Returns one weight per edge of ``edge_index`` followed (when
    ``add_self_loops``) by one per appended self-loop.
    """
    if add_self_loops:
        edge_index = append_self_loops(edge_index, num_nodes)
    row, col = edge_index[0], edge_index[1]
    deg = degree(col, num_nodes, dtype=torch.float32)
    deg_inv_sqrt = deg.pow(-0.5)
    deg_inv_sqrt[deg_inv_sqrt == float("inf")] = 0
    return deg_inv_sqrt[row] * deg_inv_sqrt[col]
