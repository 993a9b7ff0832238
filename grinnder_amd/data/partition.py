"""Graph partitioning and per-partition subgraph construction.

Follows build_partitioned_graph (grinnder/data/partition.py:231-416):
  1. partition -> (perm, ptr) with contiguous node ranges per partition,
  2. reorder features / labels / masks and relabel edges by inv_perm,
  3. GCN normalisation on the full reordered graph (before splitting),
  4. append self-loops, CSR by ``row.argsort()``,
  5. per partition: 1-hop bipartite subgraph (build_subgraph), boundaries
     by owning partition ascending and column remap to that order.
Steps 2-4 use the reference's torch CPU ops (bit-identical outputs); step 5
runs in the native library (gr_build_subgraph, gr_partition_boundaries), which
replaces the reference's unordered_map extraction and its per-element Python
remap loop (partition.py:217-219).

The reference delegates step 1 to grdpart, which is not available; the
partitioner here is this package's own (see ``partition_nodes``).
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from pathlib import Path
from typing import Any, Dict, List, Optional, Tuple, Union

import torch
from torch import Tensor

from grinnder_amd import _lib
from grinnder_amd.config import GriNNderConfig
from grinnder_amd.data.datasets import append_self_loops, compute_gcn_norm
from grinnder_amd.data.graph import PartitionedGraph

PARTITION_CACHE_VERSION = 1


def _edge_index_to_csr(edge_index: Tensor, num_nodes: int) -> Tuple[Tensor, Tensor, Tensor]:
    """COO -> CSR ordered by ``row.argsort()`` (same torch call as the reference)."""
    row, col = edge_index[0], edge_index[1]
    perm = row.argsort()
    row = row[perm]
    col = col[perm]
    rowptr = torch.zeros(num_nodes + 1, dtype=torch.long)
    rowptr.scatter_add_(0, row + 1, torch.ones_like(row))
    rowptr = rowptr.cumsum(0)
    return rowptr, col, perm


def build_subgraph(rowptr: Tensor, col: Tensor, value: Optional[Tensor], idx: Tensor,
                   bipartite: bool):
    """1-hop subgraph with contiguous relabelling (native; csrc/cpu/subgraph.cpp:8-114).

    Seeds get ids [0, len(idx)); unseen neighbours get the next ids in
    first-seen order.  Returns (rowptr, col, value or None, n_id).
    """
    for name, t in (("rowptr", rowptr), ("col", col), ("idx", idx)):
        if t.is_cuda:
            raise RuntimeError(f"{name} must be a CPU tensor")
        if t.dtype != torch.int64:
            raise RuntimeError(f"{name} must be int64")
    rowptr = rowptr.contiguous()
    col = col.contiguous()
    idx = idx.contiguous()
    if value is not None:
        if value.is_cuda:
            raise RuntimeError("value must be a CPU tensor")
        if value.dim() != 1:
            raise RuntimeError("value must be 1D")
        value = value.contiguous()
    num_rows = rowptr.numel() - 1
    nnz = torch.zeros(1, dtype=torch.int64)
    nn = torch.zeros(1, dtype=torch.int64)
    vptr = value.data_ptr() if value is not None else None
    vsz = value.element_size() if value is not None else 0
    _lib.call("gr_build_subgraph", rowptr.data_ptr(), col.data_ptr(), vptr, vsz, num_rows,
              idx.data_ptr(), idx.numel(), int(bipartite), None, None, None, None,
              nnz.data_ptr(), nn.data_ptr())
    n_edges, n_nodes = int(nnz), int(nn)
    out_rowptr = torch.empty((idx.numel() if bipartite else n_nodes) + 1, dtype=torch.int64)
    out_col = torch.empty(max(n_edges, 1), dtype=torch.int64)
    out_val = torch.empty(max(n_edges, 1), dtype=value.dtype) if value is not None else None
    n_id = torch.empty(max(n_nodes, 1), dtype=torch.int64)
    _lib.call("gr_build_subgraph", rowptr.data_ptr(), col.data_ptr(), vptr, vsz, num_rows,
              idx.data_ptr(), idx.numel(), int(bipartite), out_rowptr.data_ptr(),
              out_col.data_ptr(), _lib.ptr(out_val), n_id.data_ptr(), nnz.data_ptr(),
              nn.data_ptr())
    return (out_rowptr, out_col[:n_edges], out_val[:n_edges] if out_val is not None else None,
            n_id[:n_nodes])


def _build_partition_subgraph(pid: int, ptr: Tensor, rowptr: Tensor, col: Tensor,
                              edge_weight: Tensor, num_parts: int, build_subgraph_fn=None):
    """One partition's bipartite adjacency and boundaries (partition.py:178-228).

    Returns (pid, (rowptr, col, value), boundaries, expanded_size, batch_size).
    """
    fn = build_subgraph_fn or build_subgraph
    start, end = int(ptr[pid]), int(ptr[pid + 1])
    batch_size = end - start
    seeds = torch.arange(start, end, dtype=torch.long)
    sub_rowptr, sub_col, sub_value, n_id = fn(rowptr, col, edge_weight, seeds, True)
    halo = n_id[batch_size:].contiguous()
    n_halo = halo.numel()
    ptr64 = ptr.to(torch.int64).contiguous()
    sub_col = sub_col.contiguous()
    flat = torch.empty(max(n_halo, 1), dtype=torch.int64)
    lens = torch.zeros(num_parts, dtype=torch.int64)
    _lib.call("gr_partition_boundaries", pid, num_parts, ptr64.data_ptr(), batch_size,
              halo.data_ptr() if n_halo else None, n_halo, sub_col.data_ptr(), sub_col.numel(),
              flat.data_ptr(), lens.data_ptr())
    boundaries: List[Optional[Tensor]] = [None] * num_parts
    off = 0
    for p, n in enumerate(lens.tolist()):
        if p != pid and n > 0:
            boundaries[p] = flat[off:off + n].clone()
        off += n if p != pid else 0
    return pid, (sub_rowptr, sub_col, sub_value), boundaries, batch_size + n_halo, batch_size


def partition_nodes(edge_index: Tensor, num_nodes: int, num_parts: int,
                    partitioner: str = "grinnder", capacity: float = 1.1,
                    order: str = "bfs", **_unused) -> Tuple[Tensor, Tensor]:
    """Returns (perm, ptr): new position -> old node id, and partition pointers.

    grdpart is not available, so both partitioner names map to this package's
    deterministic partitioner (gr_partition_graph): breadth-first visit order
    (``order="bfs"``; ``"natural"`` keeps id order) and linear deterministic
    greedy assignment under ``capacity`` (the reference's partitioner_kwargs
    key).  Partition quality changes only halo sizes, never results: training
    is partition-invariant.
    """
    if partitioner not in ("grinnder", "spinner"):
        raise ValueError(
            f"Unsupported partitioner {partitioner!r}. "
            "Supported partitioners are 'grinnder' and 'spinner'."
        )
    if num_parts < 1 or num_parts > max(1, num_nodes):
        raise ValueError(f"num_parts={num_parts} invalid for {num_nodes} nodes")
    if order not in ("bfs", "natural"):
        raise ValueError(f"unknown visit order {order!r}")
    ei = edge_index.to(torch.int64)
    src = ei[0].contiguous()
    dst = ei[1].contiguous()
    perm = torch.empty(num_nodes, dtype=torch.int64)
    ptr = torch.empty(num_parts + 1, dtype=torch.int64)
    _lib.call("gr_partition_graph", src.data_ptr(), dst.data_ptr(), src.numel(), num_nodes,
              num_parts, float(capacity), int(order == "bfs"), perm.data_ptr(), ptr.data_ptr())
    return perm, ptr


def partition_adjacency(edge_index: Tensor, num_nodes: int, perm: Tensor, ptr: Tensor,
                        workers: int = 1):
    """Steps 2-6 of build_partitioned_graph (grinnder/data/partition.py:302-363)
    for a given partition (perm, ptr): relabel the edges by inv_perm, weight
    them on the full graph (degree counted on edge_index[1] after the
    self-loops), append the self-loops, build the CSR with edge_index[0] as
    the row, then every partition's adjacency and boundaries.  Returns
    [(pid, (rowptr, col, value), boundaries, expanded_size, batch_size)] in
    partition order."""
    inv_perm = torch.empty_like(perm)
    inv_perm[perm] = torch.arange(num_nodes, dtype=torch.long)
    if not torch.equal(perm, torch.arange(num_nodes)):
        edge_index = inv_perm[edge_index]
    edge_weight = compute_gcn_norm(edge_index, num_nodes, add_self_loops=True)
    edge_index = append_self_loops(edge_index, num_nodes)
    rowptr, col, sort_perm = _edge_index_to_csr(edge_index, num_nodes)
    edge_weight = edge_weight[sort_perm]
    del sort_perm, edge_index
    P = int(ptr.numel()) - 1
    args = (ptr, rowptr, col, edge_weight, P)
    workers = max(1, min(int(workers), P))
    if workers == 1:
        return [_build_partition_subgraph(pid, *args) for pid in range(P)]
    with ThreadPoolExecutor(max_workers=workers) as ex:
        return list(ex.map(lambda pid: _build_partition_subgraph(pid, *args), range(P)))


def _reorder_graph_payload(x: Any, y: Tensor, train_mask: Tensor, val_mask: Tensor,
                           test_mask: Tensor, perm: Tensor):
    if hasattr(x, "with_permutation"):
        x = x.with_permutation(perm)
    else:
        x = x[perm]
    return x, y[perm], train_mask[perm], val_mask[perm], test_mask[perm]


def _store_adjacency(backend, adj_csr) -> None:
    """With a storage backend, each partition's CSR is also written to
    storage as adj_rowptr_p{pid}, adj_col_p{pid}, adj_val_p{pid} (raw int64 /
    fp32; grinnder/data/partition.py:373-379); the graph keeps them in RAM."""
    if backend is None:
        return
    for pid, (rp, c, v) in enumerate(adj_csr):
        backend.host_write(rp.contiguous(), f"adj_rowptr_p{pid}", async_=False)
        backend.host_write(c.contiguous(), f"adj_col_p{pid}", async_=False)
        if v is not None:
            backend.host_write(v.contiguous(), f"adj_val_p{pid}", async_=False)


def _cache_matches(cache: Dict[str, Any], *, num_nodes: int, num_edges: int, num_parts: int,
                   partitioner: str) -> bool:
    return (cache.get("version") == PARTITION_CACHE_VERSION
            and cache.get("num_nodes") == num_nodes
            and cache.get("input_num_edges") == num_edges
            and cache.get("num_parts") == num_parts
            and cache.get("partitioner") == partitioner)


def build_partitioned_graph(edge_index: Tensor, x: Any, y: Tensor, train_mask: Tensor,
                            val_mask: Tensor, test_mask: Tensor, config: GriNNderConfig,
                            backend=None, cache_path: Optional[Union[str, Path]] = None,
                            save_cache: bool = True) -> PartitionedGraph:
    """Partitions a graph and builds every partition's adjacency and boundaries."""
    num_nodes = int(x.size(0))
    input_num_edges = int(edge_index.size(1))

    if cache_path is not None and Path(cache_path).is_file():
        cache = torch.load(cache_path, map_location="cpu", weights_only=True)
        if _cache_matches(cache, num_nodes=num_nodes, num_edges=input_num_edges,
                          num_parts=config.num_parts, partitioner=config.partitioner):
            perm = cache["perm"]
            x, y, train_mask, val_mask, test_mask = _reorder_graph_payload(
                x, y, train_mask, val_mask, test_mask, perm)
            _store_adjacency(backend, cache["adj_csr"])
            return PartitionedGraph(
                num_nodes=cache["num_nodes"], num_edges=cache["num_edges"],
                num_parts=cache["num_parts"], partition_sizes=cache["partition_sizes"],
                adj_csr=cache["adj_csr"], boundaries=cache["boundaries"],
                expanded_sizes=cache["expanded_sizes"], features=x, labels=y,
                train_mask=train_mask, val_mask=val_mask, test_mask=test_mask, perm=perm,
                ptr=cache["ptr"])

    perm, ptr = partition_nodes(edge_index, num_nodes, config.num_parts, config.partitioner,
                                **config.partitioner_kwargs)
    x, y, train_mask, val_mask, test_mask = _reorder_graph_payload(
        x, y, train_mask, val_mask, test_mask, perm)
    P = config.num_parts
    results = partition_adjacency(edge_index, num_nodes, perm, ptr,
                                  workers=int(config.preprocess_workers))
    graph_num_edges = int(edge_index.size(1)) + num_nodes  # with the appended self-loops

    adj_csr: List[Tuple[Tensor, Tensor, Optional[Tensor]]] = []
    boundaries: List[List[Optional[Tensor]]] = []
    expanded_sizes: List[int] = []
    partition_sizes: List[int] = []
    for _, adj, bnd, expanded, batch in results:
        adj_csr.append(adj)
        boundaries.append(bnd)
        expanded_sizes.append(expanded)
        partition_sizes.append(batch)

    _store_adjacency(backend, adj_csr)
    if cache_path is not None and save_cache:
        path = Path(cache_path)
        path.parent.mkdir(parents=True, exist_ok=True)
        tmp = path.with_suffix(path.suffix + ".tmp")
        torch.save({
            "version": PARTITION_CACHE_VERSION, "num_nodes": num_nodes,
            "input_num_edges": input_num_edges, "num_edges": graph_num_edges,
            "num_parts": P, "partitioner": config.partitioner,
            "partition_sizes": partition_sizes, "adj_csr": adj_csr, "boundaries": boundaries,
            "expanded_sizes": expanded_sizes, "perm": perm, "ptr": ptr,
        }, tmp)
        tmp.replace(path)

    return PartitionedGraph(
        num_nodes=num_nodes, num_edges=graph_num_edges, num_parts=P,
        partition_sizes=partition_sizes, adj_csr=adj_csr, boundaries=boundaries,
        expanded_sizes=expanded_sizes, features=x, labels=y, train_mask=train_mask,
        val_mask=val_mask, test_mask=test_mask, perm=perm, ptr=ptr)
