"""Per-partition bipartite adjacency and its device-resident aggregation plans.

``Adjacency`` takes the role the reference gives torch_sparse.SparseTensor in
``Trainer._get_adj`` (grinnder/engine/trainer.py:288-302): rows are the B
destination nodes of a partition, columns the E = B + halo gathered source
rows, values the full-graph GCN normalisation.  Unlike the reference, which
re-uploads the int64 CSR and rebuilds the CSC on every call, the device form
(int32 indices, CSR and CSC work plans) is built once and cached per device.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch
from torch import Tensor

from grinnder_amd import _lib

# Rows longer than this many edges are split into several work units whose
# partial sums are combined by an ordered fixup pass.
DEFAULT_SEG_LEN = 512

# Whole rows longer than this run one per wavefront in the narrow attention
# kernels (gat_narrow.hip's kRowsMax); shorter ones eight to a wavefront.
LONG_ROW = 32


@dataclass
class Plan:
    """Work plan of one sparse pass (see gr_spmm_plan)."""

    rows: int
    units: Tensor  # int32 [n_units, 4] on device
    fixups: Tensor  # int32 [n_fix, 3] on device
    n_units: int
    n_fix: int
    n_slots: int
    # int32 [n_long] on device: the units that are split or longer than
    # LONG_ROW edges, in plan order (the one-per-wavefront kernels' work).
    long_units: Optional[Tensor] = None
    n_long: int = 0


@dataclass
class DevicePlan:
    """Device-resident CSR (forward) and CSC (backward) forms of an adjacency."""

    num_dst: int
    num_src: int
    nnz: int
    idx: Tensor  # int32 [nnz]  CSR column (source row) per edge
    val: Tensor  # fp32 [nnz]
    fwd: Plan
    row_idx: Tensor  # int32 [nnz]  CSC: destination row per entry
    val_t: Tensor  # fp32 [nnz]
    perm: Tensor  # int32 [nnz]  CSC entry -> CSR position
    bwd: Plan


def build_plan(rowptr: Tensor, rows: int, seg_len: int, device,
               blocks: Optional[Tensor] = None) -> Plan:
    """Builds the unit/fixup plan of a CSR row pointer (int64, CPU) on `device`;
    with `blocks` (int64 row boundaries [0, ..., rows]) the whole rows run
    block by block (gr_spmm_plan_blocked)."""
    rowptr = rowptr.to(torch.int64).contiguous()
    n_units = torch.zeros(1, dtype=torch.int64)
    n_fix = torch.zeros(1, dtype=torch.int64)
    n_slots = torch.zeros(1, dtype=torch.int64)
    if blocks is None:
        def plan(units, fixups):
            _lib.call("gr_spmm_plan", rowptr.data_ptr(), rows, seg_len, units,
                      n_units.data_ptr(), fixups, n_fix.data_ptr(), n_slots.data_ptr())
    else:
        blocks = blocks.to(torch.int64).contiguous()

        def plan(units, fixups):
            _lib.call("gr_spmm_plan_blocked", rowptr.data_ptr(), rows, seg_len,
                      blocks.data_ptr(), blocks.numel() - 1, units, n_units.data_ptr(),
                      fixups, n_fix.data_ptr(), n_slots.data_ptr())
    plan(None, None)
    nu, nf, ns = int(n_units), int(n_fix), int(n_slots)
    units = torch.empty((max(nu, 1), 4), dtype=torch.int32)
    fixups = torch.empty((max(nf, 1), 3), dtype=torch.int32)
    plan(units.data_ptr(), fixups.data_ptr())
    u = units[:nu]
    long_units = torch.nonzero((u[:, 3] >= 0) | (u[:, 2] - u[:, 1] > LONG_ROW)).flatten()
    return Plan(rows=rows, units=u.to(device), fixups=fixups[:nf].to(device),
                n_units=nu, n_fix=nf, n_slots=ns,
                long_units=long_units.to(torch.int32).to(device), n_long=long_units.numel())


def build_device_plan(rowptr: Tensor, col: Tensor, value: Optional[Tensor],
                      sizes: Tuple[int, int], device, seg_len: int = DEFAULT_SEG_LEN,
                      row_blocks: Optional[Tensor] = None) -> DevicePlan:
    """Uploads a host CSR (int64 rowptr/col, fp32 value) with its transpose and
    plans; `row_blocks`: row boundaries the forward plan runs block by block."""
    rows, cols = int(sizes[0]), int(sizes[1])
    rowptr = rowptr.to(torch.int64).contiguous()
    col = col.to(torch.int64).contiguous()
    nnz = int(rowptr[-1]) if rowptr.numel() else 0
    if rowptr.numel() != rows + 1:
        raise ValueError(f"rowptr has {rowptr.numel()} entries, expected {rows + 1}")
    if col.numel() != nnz:
        raise ValueError(f"col has {col.numel()} entries, expected {nnz}")
    if value is None:
        value = torch.ones(nnz, dtype=torch.float32)
    value = value.to(torch.float32).contiguous()
    if nnz > 0:
        cmin, cmax = int(col.min()), int(col.max())
        if cmin < 0 or cmax >= cols:
            raise ValueError(f"column index out of range [0, {cols}): [{cmin}, {cmax}]")

    colptr = torch.empty(cols + 1, dtype=torch.int64)
    row_idx = torch.empty(max(nnz, 1), dtype=torch.int32)
    val_t = torch.empty(max(nnz, 1), dtype=torch.float32)
    perm = torch.empty(max(nnz, 1), dtype=torch.int32)
    _lib.call("gr_csr_transpose", rowptr.data_ptr(), col.data_ptr(), value.data_ptr(), rows,
              cols, colptr.data_ptr(), row_idx.data_ptr(), val_t.data_ptr(), perm.data_ptr())
    fwd = build_plan(rowptr, rows, seg_len, device, row_blocks)
    bwd = build_plan(colptr, cols, seg_len, device)
    return DevicePlan(
        num_dst=rows,
        num_src=cols,
        nnz=nnz,
        idx=col.to(torch.int32).to(device),
        val=value.to(device),
        fwd=fwd,
        row_idx=row_idx[:nnz].to(device),
        val_t=val_t[:nnz].to(device),
        perm=perm[:nnz].to(device),
        bwd=bwd,
    )


class Adjacency:
    """Bipartite CSR adjacency of one partition: [num_dst, num_src], fp32 values.

    Provides ``sparse_sizes()`` as the reference's models expect
    (grinnder/nn/gat.py:72) and a cached device plan for the HIP kernels.
    """

    def __init__(self, rowptr: Tensor, col: Tensor, value: Optional[Tensor],
                 sparse_sizes: Tuple[int, int], seg_len: int = DEFAULT_SEG_LEN,
                 row_blocks: Optional[Tensor] = None):
        self.rowptr = rowptr
        self.col = col
        self.value = value
        self._sizes = (int(sparse_sizes[0]), int(sparse_sizes[1]))
        self.seg_len = seg_len
        # Row boundaries the forward plan runs block by block (the partitions
        # of a stacked adjacency), or None.
        self.row_blocks = row_blocks
        self._plans: Dict[str, DevicePlan] = {}

    def sparse_sizes(self) -> Tuple[int, int]:
        return self._sizes

    def nnz(self) -> int:
        return int(self.col.numel())

    def device_plan(self, device) -> DevicePlan:
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError(
                "grinnder_amd aggregation runs only on the GPU (HIP); got device "
                f"{dev}. There is no CPU implementation."
            )
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        key = str(dev)
        plan = self._plans.get(key)
        if plan is None:
            plan = build_device_plan(self.rowptr, self.col, self.value, self._sizes, dev,
                                     self.seg_len, self.row_blocks)
            self._plans[key] = plan
        return plan

    def has_device_plan(self, device) -> bool:
        """Whether the device plan for `device` is built already."""
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        return str(dev) in self._plans

    def release_device(self) -> None:
        """Drops cached device plans (device memory returns to torch's allocator)."""
        self._plans.clear()
