"""CPU oracle for the partitioned GNN layer hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package, as the checker (or the timed CPU baseline); the
product package ``grinnder_amd`` never imports it.

Contents, each a restatement of the reference's algorithm:

* ``compute_gcn_norm`` / ``add_self_loops`` — grinnder/data/datasets.py:334-362
  with PyG's ``add_self_loops`` (append, no dedup) and ``degree``
  (scatter_add of fp32 ones) — same torch CPU ops, hence bit-exact.
* ``edge_index_to_csr`` — grinnder/data/partition.py:75-88 (same unstable
  ``argsort`` call as the reference).
* ``build_subgraph`` — csrc/cpu/subgraph.cpp:8-114 and its Python fallback
  grinnder/data/partition.py:29-72 (pure-Python dict loops, small inputs).
* ``build_partition_subgraph`` — grinnder/data/partition.py:178-228.
* ``partition_pipeline`` — grinnder/data/partition.py:302-363 given (perm, ptr).
* GCN / GAT layer arithmetic and the halo gather / scatter-add — C functions
  in ``oracle.c`` (double accumulation), loaded through ctypes.

How each part is pinned (the checks live in tests/test_oracle.py):
  gcn_norm: the reference's triangle known answer (all weights 1/3),
      brute-force degree counts, pow(-0.5) == 1/sqrt for integer degrees.
  CSR: brute-force per-row multisets, rowptr == cumulative counts, and
      col == col_in[perm].
  build_subgraph: reference known answers (tests/test_cpp_extensions.py:
      64-106), bit-exact against the reference's own subgraph.cpp compiled
      into oracle/_ref (when the reference tree is present), brute force.
  build_partition_subgraph: serial == parallel on the reference's banded
      20-node graph with ptr [0,5,10,15,20] (tests/test_partition.py:207-249),
      plus the invariant gathered-x[col'] == x[n_id-order col].
  GCN/GAT arithmetic: dense float64 torch restatements (different code path)
      and torch.autograd.gradcheck.
  gather/scatter: the reference's arange / ones / 1+2=3 fixtures
      (tests/test_cpp_extensions.py:144-202, tests/test_buffers.py:49-76,
      tests/test_host_buffer_ops.py:40-60).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch
from torch import Tensor

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"
REF_DIR = ORACLE_DIR / "_ref"

_lib = None


def build() -> None:
    """Builds liboracle.so (and oracle/_ref when the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        i32 = ctypes.c_int32
        L.orc_spmm_csr.argtypes = [i64, P, P, P, P, i64, i64, P, P]
        L.orc_spmm_csr_t.argtypes = [i64, i64, P, P, P, P, i64, P]
        L.orc_spmm_rows.argtypes = [i64, P, P, P, P, P, i64, i64, P, P]
        L.orc_gat_forward.argtypes = [i64, i64, P, P, P, i64, i64, P, P, P, i32, P, P, P]
        L.orc_gat_backward.argtypes = [i64, i64, P, P, P, i64, i64, P, P, i32, P, P, P, P, P,
                                       P, P]
        L.orc_gather_partitions.argtypes = [i32, i32, P, P, i64, P, P, P]
        L.orc_gather_partitions.restype = i64
        L.orc_scatter_partitions.argtypes = [i32, i32, P, i64, P, P, P, P]
        L.orc_scatter_partitions.restype = i64
        _lib = L
    return _lib


def _np(t: Tensor, dtype) -> np.ndarray:
    return np.ascontiguousarray(t.detach().cpu().numpy().astype(dtype, copy=False))


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


# ----------------------------------------------------------- bookkeeping --

def add_self_loops(edge_index: Tensor, num_nodes: int) -> Tensor:
    """PyG add_self_loops without attributes: append (i, i) for every node."""
    loop = torch.arange(num_nodes, dtype=edge_index.dtype).unsqueeze(0).repeat(2, 1)
    return torch.cat([edge_index, loop], dim=1)


def compute_gcn_norm(edge_index: Tensor, num_nodes: int, add_loops: bool = True) -> Tensor:
    """grinnder/data/datasets.py:334-362 (degree over edge_index[1])."""
    if add_loops:
        edge_index = add_self_loops(edge_index, num_nodes)
    row, col = edge_index[0], edge_index[1]
    deg = torch.zeros(num_nodes, dtype=torch.float32).scatter_add_(
        0, col, torch.ones(col.size(0), dtype=torch.float32))
    dinv = deg.pow(-0.5)
    dinv[dinv == float("inf")] = 0
    return dinv[row] * dinv[col]


def edge_index_to_csr(edge_index: Tensor, num_nodes: int) -> Tuple[Tensor, Tensor, Tensor]:
    """grinnder/data/partition.py:75-88."""
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
    """csrc/cpu/subgraph.cpp:8-114 in pure Python (small inputs only)."""
    rp = rowptr.tolist()
    cl = col.tolist()
    seeds = idx.tolist()
    vals = value.tolist() if value is not None else None
    node_map: Dict[int, int] = {}
    boundary: List[int] = []
    for i, v in enumerate(seeds):
        node_map[v] = i
    out_rowptr = [0]
    out_col: List[int] = []
    out_val: List[float] = []
    for v in seeds:
        for j in range(rp[v], rp[v + 1]):
            w = cl[j]
            if w not in node_map:
                node_map[w] = len(seeds) + len(boundary)
                boundary.append(w)
            out_col.append(node_map[w])
            if vals is not None:
                out_val.append(vals[j])
        out_rowptr.append(len(out_col))
    if not bipartite:
        out_rowptr.extend([len(out_col)] * len(boundary))
    out_v = torch.tensor(out_val, dtype=value.dtype) if value is not None else None
    n_id = torch.tensor(seeds + boundary, dtype=torch.long)
    return (torch.tensor(out_rowptr, dtype=torch.long), torch.tensor(out_col, dtype=torch.long),
            out_v, n_id)


def build_partition_subgraph(pid: int, ptr: Tensor, rowptr: Tensor, col: Tensor,
                             edge_weight: Tensor, num_parts: int):
    """grinnder/data/partition.py:178-228 (boundaries by owner ascending, discovery
    order within an owner; halo columns remapped to that order)."""
    start, end = int(ptr[pid]), int(ptr[pid + 1])
    batch = end - start
    seeds = torch.arange(start, end, dtype=torch.long)
    sub_rowptr, sub_col, sub_val, n_id = build_subgraph(rowptr, col, edge_weight, seeds, True)
    halo = n_id[batch:].tolist()
    boundaries: List[Optional[Tensor]] = [None] * num_parts
    order: List[int] = []
    for p in range(num_parts):
        if p == pid:
            continue
        lo, hi = int(ptr[p]), int(ptr[p + 1])
        pos = [k for k, g in enumerate(halo) if lo <= g < hi]
        if pos:
            order.extend(pos)
            boundaries[p] = torch.tensor([halo[k] - lo for k in pos], dtype=torch.long)
    if halo and order:
        inv = {old: new for new, old in enumerate(order)}
        sub_col = torch.tensor([c if c < batch else batch + inv[c - batch]
                                for c in sub_col.tolist()], dtype=torch.long)
    return pid, (sub_rowptr, sub_col, sub_val), boundaries, batch + len(halo), batch


def partition_pipeline(edge_index: Tensor, num_nodes: int, perm: Tensor, ptr: Tensor):
    """Steps 2-6 of build_partitioned_graph (grinnder/data/partition.py:302-363)
    for a given partition (perm, ptr).  Returns per-partition results."""
    inv_perm = torch.empty_like(perm)
    inv_perm[perm] = torch.arange(num_nodes, dtype=torch.long)
    ei = inv_perm[edge_index]
    w = compute_gcn_norm(ei, num_nodes, True)
    ei = add_self_loops(ei, num_nodes)
    rowptr, col, sort_perm = edge_index_to_csr(ei, num_nodes)
    w = w[sort_perm]
    P = ptr.numel() - 1
    return [build_partition_subgraph(p, ptr, rowptr, col, w, P) for p in range(P)]


# ------------------------------------------------------------ arithmetic --

def spmm(rowptr: Tensor, col: Tensor, val: Optional[Tensor], x: Tensor,
         bias: Optional[Tensor] = None) -> np.ndarray:
    """Y = A X (+ bias) in float64 accumulation (oracle.c orc_spmm_csr)."""
    rows = rowptr.numel() - 1
    rp, cl = _np(rowptr, np.int64), _np(col, np.int64)
    v = None if val is None else _np(val, np.float32)
    xx = _np(x, np.float32)
    b = None if bias is None else _np(bias, np.float32)
    out = np.zeros((rows, xx.shape[1]), dtype=np.float64)
    lib().orc_spmm_csr(rows, _p(rp), _p(cl), _p(v), _p(xx), xx.shape[1], xx.shape[1], _p(b),
                       _p(out))
    return out


def spmm_rows(rowptr: Tensor, col: Tensor, val: Optional[Tensor], x: Tensor, rows: Tensor,
              bias: Optional[Tensor] = None, threads: int = 16) -> np.ndarray:
    """Rows `rows` of A X (+ bias), float64 accumulation (oracle.c
    orc_spmm_rows), split over `threads` host threads (ctypes releases the
    GIL).  The inputs are converted once, so X may be a full-size matrix."""
    from concurrent.futures import ThreadPoolExecutor

    rp, cl = _np(rowptr, np.int64), _np(col, np.int64)
    v = None if val is None else _np(val, np.float32)
    xx = _np(x, np.float32)
    b = None if bias is None else _np(bias, np.float32)
    sel = _np(rows, np.int64)
    dim = xx.shape[1]
    out = np.zeros((sel.size, dim), dtype=np.float64)
    if sel.size and (sel.min() < 0 or sel.max() >= rp.size - 1):
        raise IndexError("spmm_rows: row id out of range")
    if cl.size and (cl.min() < 0 or cl.max() >= xx.shape[0]):
        raise IndexError("spmm_rows: column id out of range")
    chunks = np.array_split(np.arange(sel.size), max(1, min(threads, sel.size)))

    def run(idx):
        if idx.size == 0:
            return
        k0 = int(idx[0])
        lib().orc_spmm_rows(idx.size, sel.ctypes.data + 8 * k0, _p(rp), _p(cl), _p(v), _p(xx),
                            dim, dim, _p(b), out.ctypes.data + 8 * dim * k0)

    with ThreadPoolExecutor(len(chunks)) as ex:
        list(ex.map(run, chunks))
    return out


def spmm_t(rowptr: Tensor, col: Tensor, val: Optional[Tensor], g: Tensor,
           num_cols: int) -> np.ndarray:
    """dZ = A^T G in float64 accumulation (scatter form, no transpose built)."""
    rows = rowptr.numel() - 1
    rp, cl = _np(rowptr, np.int64), _np(col, np.int64)
    v = None if val is None else _np(val, np.float32)
    gg = _np(g, np.float32)
    out = np.zeros((num_cols, gg.shape[1]), dtype=np.float64)
    lib().orc_spmm_csr_t(rows, num_cols, _p(rp), _p(cl), _p(v), _p(gg), gg.shape[1], _p(out))
    return out


def gat_forward(rowptr, col, hs, heads, channels, att_src, att_dst, bias, concat):
    """PyG GATConv attention forward (oracle.c orc_gat_forward).
    Returns (out float64, alpha [nnz,H], t [nnz,H])."""
    B = rowptr.numel() - 1
    E = hs.size(0)
    rp, cl = _np(rowptr, np.int64), _np(col, np.int64)
    h = _np(hs, np.float32)
    a_s, a_d = _np(att_src.reshape(-1), np.float32), _np(att_dst.reshape(-1), np.float32)
    b = None if bias is None else _np(bias, np.float32)
    nnz = cl.size
    out_w = heads * channels if concat else channels
    out = np.zeros((B, out_w), dtype=np.float64)
    alpha = np.zeros((max(nnz, 1), heads), dtype=np.float64)
    tpre = np.zeros((max(nnz, 1), heads), dtype=np.float64)
    lib().orc_gat_forward(B, E, _p(rp), _p(cl), _p(h), heads, channels, _p(a_s), _p(a_d), _p(b),
                          int(concat), _p(out), _p(alpha), _p(tpre))
    return out, alpha[:nnz], tpre[:nnz]


def gat_backward(rowptr, col, hs, heads, channels, att_src, att_dst, concat, alpha, tpre, gy):
    """Gradient of gat_forward (oracle.c orc_gat_backward).
    Returns (dhs, datt_src [H*C], datt_dst [H*C], dbias) as float64."""
    B = rowptr.numel() - 1
    E = hs.size(0)
    rp, cl = _np(rowptr, np.int64), _np(col, np.int64)
    h = _np(hs, np.float32)
    a_s, a_d = _np(att_src.reshape(-1), np.float32), _np(att_dst.reshape(-1), np.float32)
    g = _np(gy, np.float32)
    HC = heads * channels
    out_w = HC if concat else channels
    al = np.ascontiguousarray(alpha if alpha.size else np.zeros((1, heads)))
    tp = np.ascontiguousarray(tpre if tpre.size else np.zeros((1, heads)))
    dhs = np.zeros((E, HC))
    das = np.zeros(HC)
    dad = np.zeros(HC)
    db = np.zeros(out_w)
    lib().orc_gat_backward(B, E, _p(rp), _p(cl), _p(h), heads, channels, _p(a_s), _p(a_d),
                           int(concat), _p(al), _p(tp), _p(g), _p(dhs), _p(das), _p(dad), _p(db))
    return dhs, das, dad, db


# ------------------------------------------------------- gather / scatter --

def gather_partitions(pid: int, srcs: List[Tensor], boundaries: List[Optional[Tensor]]
                      ) -> np.ndarray:
    """[srcs[pid] | srcs[p][boundaries[p]] for p ascending, p != pid] (oracle.c)."""
    P = len(srcs)
    dim = srcs[0].size(1)
    arrs = [_np(s, np.float32) for s in srcs]
    bnd = [np.zeros(0, np.int64) if (p == pid or b is None) else _np(b, np.int64)
           for p, b in enumerate(boundaries)]
    total = arrs[pid].shape[0] + sum(b.size for p, b in enumerate(bnd) if p != pid)
    out = np.zeros((total, dim), dtype=np.float32)
    src_p = (ctypes.c_void_p * P)(*[a.ctypes.data for a in arrs])
    rows = (ctypes.c_int64 * P)(*[a.shape[0] for a in arrs])
    b_p = (ctypes.c_void_p * P)(*[b.ctypes.data if b.size else None for b in bnd])
    lens = (ctypes.c_int64 * P)(*[b.size if p != pid else 0 for p, b in enumerate(bnd)])
    n = lib().orc_gather_partitions(pid, P, src_p, rows, dim, b_p, lens, out.ctypes.data)
    assert n == total
    return out


def scatter_partitions(pid: int, src: Tensor, dsts: List[Tensor],
                       boundaries: List[Optional[Tensor]]) -> List[np.ndarray]:
    """fp32 accumulate of src into copies of dsts (oracle.c); returns the new dsts."""
    P = len(dsts)
    g = _np(src, np.float32)
    dim = g.shape[1]
    outs = [np.array(_np(d, np.float32), copy=True) for d in dsts]
    bnd = [np.zeros(0, np.int64) if (p == pid or b is None) else _np(b, np.int64)
           for p, b in enumerate(boundaries)]
    d_p = (ctypes.c_void_p * P)(*[o.ctypes.data for o in outs])
    rows = (ctypes.c_int64 * P)(*[o.shape[0] for o in outs])
    b_p = (ctypes.c_void_p * P)(*[b.ctypes.data if b.size else None for b in bnd])
    lens = (ctypes.c_int64 * P)(*[b.size if p != pid else 0 for p, b in enumerate(bnd)])
    n = lib().orc_scatter_partitions(pid, P, g.ctypes.data, dim, d_p, rows, b_p, lens)
    assert n == g.shape[0]
    return outs


def ref_build_subgraph():
    """The reference's compiled build_subgraph (oracle/_ref), or None if not built."""
    import importlib.util
    for so in REF_DIR.glob("ref_subgraph*.so"):
        spec = importlib.util.spec_from_file_location("ref_subgraph", so)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        return mod.build_subgraph
    return None
