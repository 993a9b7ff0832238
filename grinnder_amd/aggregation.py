"""Autograd wrappers of the HIP aggregation kernels (GCN SpMM, GAT attention).

These replace the third-party calls the reference reaches through PyG:
torch_sparse ``spmm_sum`` and its ``csr2csc`` backward for GCNConv
(grinnder/nn/gcn.py:53-56,65), and GATConv's logits / segment softmax /
message aggregation (grinnder/nn/gat.py:54-61,73).
"""

from __future__ import annotations

import contextlib
import ctypes
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch
from torch import Tensor

from grinnder_amd import _lib
from grinnder_amd.data.adjacency import Adjacency, DevicePlan
from grinnder_amd.dense import OutputRows, output_block


@dataclass
class KernelRecord:
    """One timed aggregation pass: algorithmic bytes and edges, HIP events."""

    name: str
    nbytes: int
    edges: int
    dim: int
    start: "torch.cuda.Event"
    end: "torch.cuda.Event"
    flops: int = 0

    def ms(self) -> float:
        return self.start.elapsed_time(self.end)


class KernelTimer:
    """Records HIP events around every aggregation pass (and, as "dense_*"
    regions with their flop counts, every dense product) while active.

    Events are recorded on the stream the kernels are launched on (the
    current stream), so elapsed times are the passes' device durations.
    Algorithmic bytes per pass (fp32 features, int32 index + fp32 value
    per edge):
      GCN pass over R rows of width D: nnz*(4D + 8) + R*(4D + 4)
      GAT forward:  nnz*(4HC + 8H + 4) + B*(4HC + 4H + 4)
      GAT backward: nnz*(8HC + 16H + 8) + E*(4HC + 4H) + B*(4HC + 4H)
    """

    active: Optional["KernelTimer"] = None

    def __init__(self, capacity: int = 0):
        """capacity: events to create (and record once) up front, so that
        regions timed later take ready events instead of creating them; a
        timed epoch of many short kernels otherwise pays for event creation
        on the host between its launches."""
        self.records: List[KernelRecord] = []
        self._pool: List["torch.cuda.Event"] = []
        for _ in range(capacity):
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self._pool.append(ev)
        if capacity:
            torch.cuda.synchronize()

    def __enter__(self):
        KernelTimer.active = self
        return self

    def __exit__(self, *exc):
        KernelTimer.active = None
        return False

    def _event(self) -> "torch.cuda.Event":
        return self._pool.pop() if self._pool else torch.cuda.Event(enable_timing=True)

    @staticmethod
    @contextlib.contextmanager
    def region(name: str, nbytes: int, edges: int, dim: int, flops: int = 0):
        timer = KernelTimer.active
        if timer is None:
            yield
            return
        start = timer._event()
        end = timer._event()
        start.record()
        yield
        end.record()
        timer.records.append(KernelRecord(name, nbytes, edges, dim, start, end, flops))


def dense_region(name: str, rows: int, k: int, n: int):
    """Timer region of a dense product of 2 * rows * k * n flops."""
    return KernelTimer.region("dense_" + name, 0, 0, n, 2 * rows * k * n)


def _check_device_tensor(name: str, t: Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (HIP); got {t.device}")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32; got {t.dtype}")


def column_sum(g: Tensor, weights: Optional[Tensor] = None, group: int = 1,
               rows_of: Optional[Tensor] = None) -> Tensor:
    """Sum over the rows of a [rows, D] fp32 device matrix (deterministic HIP
    kernel); with `weights` [rows, ceil(D / group)], row i of column f is
    scaled by weights[i, f // group] first.  With `rows_of` (int32, [n]) the
    rows summed are g[rows_of[i]], i < n, read in place."""
    if g.stride(-1) != 1:
        g = g.contiguous()
    rows, dim = g.shape
    if rows_of is not None:
        if rows_of.dtype != torch.int32 or rows_of.dim() != 1:
            raise ValueError("column_sum: rows_of must be a 1-D int32 tensor")
        rows = rows_of.numel()
    out = torch.empty(dim, dtype=torch.float32, device=g.device)
    nblk = max(1, min(4096, (rows + 255) // 256))
    ws = torch.empty(nblk * dim, dtype=torch.float32, device=g.device)
    w = None
    if weights is not None:
        w = weights.contiguous()
        if w.dim() != 2 or w.size(0) != rows or w.size(1) * group < dim:
            raise ValueError("column_sum: weights must be [rows, ceil(D / group)]")
    _lib.call("gr_column_sum", g.data_ptr(), rows, dim, max(g.stride(0), dim),
              _lib.ptr(rows_of), _lib.ptr(w),
              w.size(1) if w is not None else 0, group, out.data_ptr(), ws.data_ptr(),
              ws.numel(), _lib.stream_handle())
    return out


def gather_rows(x: Tensor, rows: Tensor) -> Tensor:
    """x[rows] for fp32 [*, D] device rows x and int64 device row ids (HIP
    kernel, flat over elements, so narrow rows run near copy speed too);
    the same values as x.index_select(0, rows)."""
    if x.dim() != 2 or rows.dim() != 1:
        raise ValueError("gather_rows: x [*, D], rows [n]")
    if x.dtype != torch.float32 or rows.dtype != torch.int64:
        raise ValueError("gather_rows: fp32 x, int64 rows")
    if x.stride(-1) != 1 or (x.size(0) > 1 and x.stride(0) < x.size(1)):
        # Rows that overlap (a broadcast or expanded view) are made dense:
        # the kernel reads row r at r * stride(0).
        x = x.contiguous()
    rows = rows.contiguous()
    n, dim = rows.numel(), x.size(1)
    y = torch.empty(n, dim, dtype=torch.float32, device=x.device)
    _lib.call("gr_gather_rows", x.data_ptr(), x.size(0), max(x.stride(0), dim),
              rows.data_ptr(), n, dim, y.data_ptr(), dim, _lib.stream_handle())
    return y


def scatter_add_rows(x: Tensor, rows: Tensor, y: Tensor) -> None:
    """y[rows[r]] += x[r] in place on the current stream (HIP kernel, no
    atomics): fp32 [n, D] rows into fp32 [*, D] y, rows int64 on the device
    and distinct, which is what makes the result deterministic.  The same
    values as y.index_add_(0, rows, x) for distinct rows."""
    if x.dim() != 2 or y.dim() != 2 or x.size(1) != y.size(1) or rows.numel() != x.size(0):
        raise ValueError("scatter_add_rows: x [n, D], rows [n], y [*, D]")
    if x.dtype != torch.float32 or y.dtype != torch.float32 or rows.dtype != torch.int64:
        raise ValueError("scatter_add_rows: fp32 x and y, int64 rows")
    if x.stride(-1) != 1 or (x.size(0) > 1 and x.stride(0) < x.size(1)):
        x = x.contiguous()
    if y.stride(-1) != 1 or (y.size(0) > 1 and y.stride(0) < y.size(1)):
        raise ValueError("scatter_add_rows: y must hold distinct, contiguous rows")
    rows = rows.contiguous()
    n, dim = x.shape
    _lib.call("gr_scatter_add_rows", x.data_ptr(), n, dim, max(x.stride(0), dim),
              rows.data_ptr(), y.data_ptr(), y.size(0), max(y.stride(0), dim),
              _lib.stream_handle())


def _workspace(n_slots: int, width: int, device) -> Optional[Tensor]:
    if n_slots == 0:
        return None
    return torch.empty(n_slots * width, dtype=torch.float32, device=device)


def spmm(plan, idx: Tensor, val: Tensor, x: Tensor, rows: int,
         bias: Optional[Tensor] = None, out: Optional[Tensor] = None,
         name: str = "gcn_spmm") -> Tensor:
    """out[r] = sum_e val[e] * x[idx[e]] (+ bias) for the rows of `plan`."""
    dim = x.size(1)
    if out is None:
        out = torch.empty((rows, dim), dtype=torch.float32, device=x.device)
    ws = _workspace(plan.n_slots, dim, x.device)
    nnz = idx.numel()
    with KernelTimer.region(name, nnz * (4 * dim + 8) + rows * (4 * dim + 4), nnz, dim):
        _lib.call("gr_gcn_aggregate", plan.units.data_ptr(), plan.n_units,
                  plan.fixups.data_ptr() if plan.n_fix else None, plan.n_fix,
                  idx.data_ptr(), val.data_ptr(), x.data_ptr(), x.stride(0), out.data_ptr(),
                  out.stride(0), _lib.ptr(bias), rows, dim, _lib.ptr(ws), plan.n_slots,
                  _lib.stream_handle())
    return out


@dataclass
class ProjectedSink:
    """Where a partition's source rows live when they are read in place: the
    aggregation reads the whole matrix of all partitions' rows ([N, d])
    through `gidx`, the global row of each CSR edge's source, instead of a
    gathered copy.  With `dz`, the backward adds Aᵀ G into dz ([N, d]) at
    `rows`, the global row of each of the partition's E source rows
    (distinct), instead of returning a gradient for the matrix; `token` is
    then a zero-element tensor that requires grad, so that autograd records
    the aggregation although the matrix does not.  Without dz the source
    gets no gradient (a layer's input features)."""

    dz: Optional[Tensor]
    gidx: Tensor
    rows: Optional[Tensor] = None
    token: Optional[Tensor] = None
    # First global row of the partition's destination rows (its own rows,
    # the first num_dst of `rows`); read by the attention backward.
    lo: int = 0
    # `rows` are every row of dz once, in order (a merged layer's whole-graph
    # pass), and nothing else writes dz: the GCN backward then writes Aᵀ G
    # into dz (which needs no zeroing) instead of adding it.
    overwrite: bool = False


def spmm_into(plan, idx: Tensor, val: Tensor, x: Tensor, sink: ProjectedSink,
              name: str = "gcn_bwd") -> None:
    """sink.dz[sink.rows[r]] += sum_e val[e] * x[idx[e]] for the rows of `plan`."""
    dim = x.size(1)
    dz = sink.dz
    if dz.size(1) != dim or not dz.is_contiguous():
        raise ValueError("spmm_into: dz must be contiguous with the width of x")
    rows = plan.rows
    if sink.rows.numel() != rows:
        raise ValueError(f"spmm_into: {sink.rows.numel()} row ids for {rows} rows")
    if sink.overwrite:
        if dz.size(0) != rows:
            raise ValueError(f"spmm_into: overwrite needs dz's {dz.size(0)} rows to be the "
                             f"plan's {rows}")
        spmm(plan, idx, val, x, rows, out=dz, name=name)
        return
    ws = _workspace(plan.n_slots, dim, x.device)
    nnz = idx.numel()
    with KernelTimer.region(name, nnz * (4 * dim + 8) + rows * (8 * dim + 4), nnz, dim):
        _lib.call("gr_gcn_aggregate_into", plan.units.data_ptr(), plan.n_units,
                  plan.fixups.data_ptr() if plan.n_fix else None, plan.n_fix,
                  idx.data_ptr(), val.data_ptr(), x.data_ptr(), x.stride(0),
                  sink.rows.data_ptr(), dz.data_ptr(), dz.stride(0), rows, dim, _lib.ptr(ws),
                  plan.n_slots, _lib.stream_handle())


class _GCNAggregate(torch.autograd.Function):
    """Y = A Z + b forward; dZ = A^T G (CSC plan) and db = sum G backward."""

    @staticmethod
    def forward(ctx, z: Tensor, bias: Optional[Tensor], plan: DevicePlan,
                sink: Optional[ProjectedSink] = None, token: Optional[Tensor] = None) -> Tensor:
        z = z.contiguous()
        y = spmm(plan.fwd, plan.idx if sink is None else sink.gidx, plan.val, z, plan.num_dst,
                 bias.contiguous() if bias is not None else None, name="gcn_fwd")
        ctx.plan = plan
        ctx.sink = sink
        ctx.has_bias = bias is not None
        return y

    @staticmethod
    def backward(ctx, gy: Tensor):
        plan: DevicePlan = ctx.plan
        gy = gy.contiguous()
        dz = None
        if ctx.sink is not None:
            if ctx.sink.dz is not None:
                spmm_into(plan.bwd, plan.row_idx, plan.val_t, gy, ctx.sink)
        elif ctx.needs_input_grad[0]:
            dz = spmm(plan.bwd, plan.row_idx, plan.val_t, gy, plan.num_src, name="gcn_bwd")
        db = column_sum(gy) if (ctx.has_bias and ctx.needs_input_grad[1]) else None
        return dz, db, None, None, None


def _check_source(z: Tensor, plan: DevicePlan, sink: Optional[ProjectedSink]) -> None:
    if sink is None:
        if z.size(0) != plan.num_src:
            raise ValueError(f"z has {z.size(0)} rows, adjacency has {plan.num_src} columns")
        return
    if sink.gidx.numel() != plan.nnz:
        raise ValueError("sink: gidx does not match the adjacency")
    if sink.dz is None:
        return
    if sink.rows is None or sink.rows.numel() != plan.num_src or sink.token is None:
        raise ValueError("sink: a sink with dz needs rows for every source and a token")
    if sink.dz.shape != z.shape:
        raise ValueError(f"sink: dz {tuple(sink.dz.shape)} vs Z {tuple(z.shape)}")


def gcn_aggregate(z: Tensor, adj: Adjacency, bias: Optional[Tensor] = None,
                  sink: Optional[ProjectedSink] = None) -> Tensor:
    """GCN neighbour aggregation A·Z (+ bias) of one partition, on the GPU.
    With a sink, z is the layer's whole Z read through sink.gidx, and the
    backward adds into sink.dz."""
    _check_device_tensor("z", z)
    plan = adj.device_plan(z.device)
    _check_source(z, plan, sink)
    if sink is None or sink.dz is None:
        return _GCNAggregate.apply(z, bias, plan, sink)
    return _GCNAggregate.apply(z, bias, plan, sink, sink.token)


class _GCNLinearAggregatePadded(torch.autograd.Function):
    """Y = A (X Wᵀ) + b for an output width D that is not a multiple of 4.

    The product is formed with W padded by zero rows to Dp = round_up(D, 4)
    columns, so both aggregation passes move 16-byte row vectors instead of
    scalars; the pad columns stay exactly zero and are sliced off.  Backward:
    dZ = Aᵀ [gY | 0], dW = dZᵀ X (first D rows), dX = dZ Wp, db = sum gY.
    """

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, bias: Optional[Tensor],
                plan: DevicePlan) -> Tensor:
        from torch.nn.functional import pad

        from grinnder_amd.dense import gemm_nt
        d = weight.size(0)
        dp = (d + 3) // 4 * 4
        x = x.contiguous()
        wp = pad(weight, (0, 0, 0, dp - d))
        with dense_region("fwd", x.size(0), x.size(1), dp):
            z = gemm_nt(x, wp)
        bp = pad(bias, (0, dp - d)).contiguous() if bias is not None else None
        y = spmm(plan.fwd, plan.idx, plan.val, z, plan.num_dst, bp, name="gcn_fwd")
        ctx.save_for_backward(x, wp)
        ctx.plan = plan
        ctx.d = d
        ctx.has_bias = bias is not None
        ctx.ln_sink = LNProductSink.accepts(x, wp)
        ctx.x_shape = x.shape
        return y[:, :d]

    @staticmethod
    def backward(ctx, gy: Tensor):
        from torch.nn.functional import pad

        from grinnder_amd.dense import gemm_nt, gemm_tn
        x, wp = ctx.saved_tensors
        plan: DevicePlan = ctx.plan
        d, dp = ctx.d, wp.size(0)
        gyp = pad(gy, (0, dp - d)).contiguous()
        dz = spmm(plan.bwd, plan.row_idx, plan.val_t, gyp, plan.num_src, name="gcn_bwd")
        dx = dw = None
        if ctx.needs_input_grad[0] and ctx.ln_sink is not None:
            # dX = dZ Wp is formed inside the LayerNorm backward that consumes it.
            dx = ctx.ln_sink.hand_over(dz, wp, ctx.x_shape)
        elif ctx.needs_input_grad[0]:
            with dense_region("dx", dz.size(0), dp, wp.size(1)):
                dx = gemm_nt(dz, wp.t().contiguous())
        if ctx.needs_input_grad[1]:
            with dense_region("dw", dz.size(0), dp, x.size(1)):
                dw = gemm_tn(dz, x)[:d]
        db = column_sum(gyp)[:d] if (ctx.has_bias and ctx.needs_input_grad[2]) else None
        return dx, dw, db, None


def gcn_linear_aggregate(x: Tensor, weight: Tensor, adj: Adjacency,
                         bias: Optional[Tensor] = None) -> Tensor:
    """A·(x Wᵀ) + bias of one partition (GPU), for any output width."""
    _check_device_tensor("x", x)
    plan = adj.device_plan(x.device)
    if x.size(0) != plan.num_src:
        raise ValueError(f"x has {x.size(0)} rows, adjacency has {plan.num_src} columns")
    if weight.size(0) % 4 == 0:
        from grinnder_amd.dense import linear
        return _GCNAggregate.apply(linear(x, weight), bias, plan)
    return _GCNLinearAggregatePadded.apply(x, weight, bias, plan)


class RowDotSink:
    """Carries c_i = <dL/dO_i, O_i> of a GAT attention output O from the
    backward of the LayerNorm that consumes O + b (formed there while
    dL/dO is in registers) to the attention's own backward, which uses it
    only when the gradient it receives is that LayerNorm's output itself."""

    __slots__ = ("cdot", "grad_ptr")

    def __init__(self):
        self.cdot: Optional[Tensor] = None
        self.grad_ptr = 0


def ln_act_backward(gout: Tensor, h: Tensor, mean: Tensor, rstd: Tensor, gamma: Tensor,
                    beta: Tensor, with_bias: bool = False, act: str = "relu",
                    shift: Optional[Tensor] = None, rowdot: Optional[Tensor] = None):
    """(dL/dh, dgamma, dbeta, dbias or None) of out = act(LayerNorm(h)) given
    dL/dout (GPU); dbias = the column sums of dL/dh, formed in the same pass.
    With `rowdot` (a [rows] tensor) the pass also writes rowdot[r] =
    <dL/dh_r, h_r - shift> (shift None: 0)."""
    gout = gout.contiguous()
    B, D = h.shape
    dev = h.device
    gh = torch.empty_like(h)
    dgamma = torch.empty(D, dtype=torch.float32, device=dev)
    dbeta = torch.empty(D, dtype=torch.float32, device=dev)
    dbias = torch.empty(D, dtype=torch.float32, device=dev) if with_bias else None
    nwaves = min(8192, max(4, (B + 15) // 16))
    nwaves = (nwaves + 3) // 4 * 4
    ws = torch.empty(((3 if with_bias else 2) * nwaves + 1) * D, dtype=torch.float32,
                     device=dev)
    _lib.call("gr_ln_act_backward", gout.data_ptr(), h.data_ptr(), mean.data_ptr(),
              rstd.data_ptr(), gamma.data_ptr(), beta.data_ptr(), _lib.ACTIVATIONS[act], B, D,
              gh.data_ptr(), dgamma.data_ptr(), dbeta.data_ptr(), _lib.ptr(dbias),
              _lib.ptr(shift.contiguous() if shift is not None else None), _lib.ptr(rowdot),
              ws.data_ptr(), ws.numel(), _lib.stream_handle())
    return gh, dgamma, dbeta, dbias


class LNProductSink:
    """Hands a fused LayerNorm/activation backward its incoming gradient as a
    product.  The node that consumes the LayerNorm's output x (alone) and
    forms x Wᵀ with W of at most 64 rows leaves dZ (its gradient of x Wᵀ) and
    W here and returns `token`, a zero tensor of x's shape with zero strides,
    as x's gradient.  The LayerNorm's backward, receiving exactly that token,
    forms dL/dx = dZ W inside its own pass (gr_ln_act_backward_product)
    instead of reading a [rows, D] gradient that a separate product wrote.
    A gradient that is not the token (x had other consumers, whose gradients
    autograd summed with the token's zeros) is completed with dZ W before the
    usual backward."""

    __slots__ = ("dz", "w", "token")

    def __init__(self):
        self.dz: Optional[Tensor] = None
        self.w: Optional[Tensor] = None
        self.token: Optional[Tensor] = None

    @staticmethod
    def accepts(x: Tensor, w: Tensor) -> Optional["LNProductSink"]:
        """The sink of x when x's gradient can be handed over as dZ W for this
        W ([K, D], K <= 64 and a multiple of 4, D = x's width), else None."""
        sink = getattr(x, "_grinnder_ln_sink", None)
        if sink is None or not isinstance(sink, LNProductSink):
            return None
        k, d = w.shape
        if k > 64 or k % 4 != 0 or d != x.size(-1) or d not in (64, 128, 192, 256):
            return None
        return sink

    def hand_over(self, dz: Tensor, w: Tensor, shape) -> Tensor:
        self.dz, self.w = dz, w
        self.token = torch.zeros((), dtype=dz.dtype, device=dz.device).expand(shape)
        return self.token

    def take(self, gout: Tensor):
        """(dz, w, exact) left for this gradient, or None; clears the sink."""
        if self.dz is None:
            return None
        tok = self.token
        exact = (gout.data_ptr() == tok.data_ptr() and gout.stride() == tok.stride()
                 and gout.shape == tok.shape)
        out = (self.dz, self.w, exact)
        self.dz = self.w = self.token = None
        return out


def ln_act_backward_product(dz: Tensor, w: Tensor, h: Tensor, mean: Tensor, rstd: Tensor,
                            gamma: Tensor, beta: Tensor, with_bias: bool = False,
                            act: str = "relu", shift: Optional[Tensor] = None,
                            rowdot: Optional[Tensor] = None):
    """ln_act_backward with dL/dout = dz W formed inside the pass (GPU):
    dz [rows, K] (K <= 64, a multiple of 4), w [K, D] with D in {64, 128, 192,
    256}.  Returns (dL/dh, dgamma, dbeta, dbias or None); `shift` / `rowdot`
    as in ln_act_backward."""
    B, D = h.shape
    dz = dz.contiguous()
    w = w.contiguous()
    dev = h.device
    gh = torch.empty_like(h)
    dgamma = torch.empty(D, dtype=torch.float32, device=dev)
    dbeta = torch.empty(D, dtype=torch.float32, device=dev)
    dbias = torch.empty(D, dtype=torch.float32, device=dev) if with_bias else None
    nwaves = min(8192, max(4, (B + 15) // 16))
    nwaves = (nwaves + 3) // 4 * 4
    ws = torch.empty(((3 if with_bias else 2) * nwaves + 1) * D, dtype=torch.float32,
                     device=dev)
    _lib.call("gr_ln_act_backward_product", dz.data_ptr(), dz.size(1), dz.size(1),
              w.data_ptr(), h.data_ptr(), mean.data_ptr(), rstd.data_ptr(),
              gamma.data_ptr(), beta.data_ptr(), _lib.ACTIVATIONS[act], B, D, gh.data_ptr(),
              dgamma.data_ptr(), dbeta.data_ptr(), _lib.ptr(dbias),
              _lib.ptr(shift.contiguous() if shift is not None else None), _lib.ptr(rowdot),
              ws.data_ptr(), ws.numel(), _lib.stream_handle())
    return gh, dgamma, dbeta, dbias


class _GCNAggregateLNReLU(torch.autograd.Function):
    """out = ReLU(LayerNorm(A Z + b)) with the LayerNorm/ReLU fused into the
    aggregation epilogue; backward: fused LN/ReLU gradient, then dZ = A^T gh."""

    @staticmethod
    def forward(ctx, z: Tensor, bias: Optional[Tensor], gamma: Tensor, beta: Tensor,
                plan: DevicePlan, eps: float, sink: Optional[ProjectedSink] = None,
                dest: Optional[OutputRows] = None, ln_sink: Optional[LNProductSink] = None,
                token: Optional[Tensor] = None) -> Tensor:
        z = z.contiguous()
        idx = plan.idx if sink is None else sink.gidx
        dev = z.device
        B, D = plan.num_dst, z.size(1)
        f = plan.fwd
        h = torch.empty((B, D), dtype=torch.float32, device=dev)
        out = output_block(dest, B, D, dev)
        mean = torch.empty(B, dtype=torch.float32, device=dev)
        rstd = torch.empty(B, dtype=torch.float32, device=dev)
        ws = _workspace(f.n_slots, D, dev)
        b = bias.contiguous() if bias is not None else None
        g, bt = gamma.contiguous(), beta.contiguous()
        nnz = plan.nnz
        with KernelTimer.region("gcn_fwd", nnz * (4 * D + 8) + B * (4 * D + 4), nnz, D):
            _lib.call("gr_gcn_aggregate_ln_relu", f.units.data_ptr(), f.n_units,
                      f.fixups.data_ptr() if f.n_fix else None, f.n_fix, idx.data_ptr(),
                      plan.val.data_ptr(), z.data_ptr(), z.stride(0), _lib.ptr(b), g.data_ptr(),
                      bt.data_ptr(), float(eps), B, D, h.data_ptr(), out.data_ptr(),
                      mean.data_ptr(), rstd.data_ptr(), _lib.ptr(ws), f.n_slots,
                      _lib.stream_handle())
        ctx.save_for_backward(h, mean, rstd, g, bt)
        ctx.plan = plan
        ctx.sink = sink
        ctx.ln_sink = ln_sink
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, gout: Tensor):
        h, mean, rstd, g, bt = ctx.saved_tensors
        plan: DevicePlan = ctx.plan
        prod = ctx.ln_sink.take(gout) if ctx.ln_sink is not None else None
        if prod is not None and prod[2]:
            gh, dgamma, dbeta, db = ln_act_backward_product(prod[0], prod[1], h, mean, rstd, g,
                                                            bt, ctx.has_bias)
        else:
            if prod is not None:
                from grinnder_amd.dense import gemm_nt
                gout = gout + gemm_nt(prod[0], prod[1].t().contiguous())
            gh, dgamma, dbeta, db = ln_act_backward(gout, h, mean, rstd, g, bt, ctx.has_bias)
        dz = None
        if ctx.sink is not None:
            if ctx.sink.dz is not None:
                spmm_into(plan.bwd, plan.row_idx, plan.val_t, gh, ctx.sink)
        elif ctx.needs_input_grad[0]:
            dz = spmm(plan.bwd, plan.row_idx, plan.val_t, gh, plan.num_src, name="gcn_bwd")
        return dz, db, dgamma, dbeta, None, None, None, None, None, None


def gcn_aggregate_ln_relu(z: Tensor, adj: Adjacency, bias: Optional[Tensor], gamma: Tensor,
                          beta: Tensor, eps: float = 1e-5,
                          sink: Optional[ProjectedSink] = None,
                          dest: Optional[OutputRows] = None) -> Tensor:
    """ReLU(LayerNorm(A·Z + bias)) of one partition in one fused pass (GPU);
    a sink as in gcn_aggregate; `dest`: the output is written into that block
    (dense.OutputRows) and returned as a view of it."""
    _check_device_tensor("z", z)
    plan = adj.device_plan(z.device)
    _check_source(z, plan, sink)
    ln_sink = LNProductSink()
    if sink is None or sink.dz is None:
        out = _GCNAggregateLNReLU.apply(z, bias, gamma, beta, plan, eps, sink, dest, ln_sink)
    else:
        out = _GCNAggregateLNReLU.apply(z, bias, gamma, beta, plan, eps, sink, dest, ln_sink,
                                        sink.token)
    # A product that consumes the output alone may hand its input gradient
    # back as dZ W (LNProductSink).
    out._grinnder_ln_sink = ln_sink
    return out


# Rows of per-wavefront partial sums the in-place GAT backward may use for the
# attention-vector gradient (at most what the GPU holds at once is used; an
# MI355X holds 256 CUs x 32 wavefronts): 8192 x C floats, 8 MB at C = 256.
_ATT_PARTIAL_ROWS = 8192


def _gat_narrow_ok(hs: Tensor, heads: int, channels: int) -> bool:
    """One head of at most 24 channels, a multiple of 4, on 16-byte rows: the
    packed-line kernels of gr_gat_narrow_forward / _backward."""
    return (heads == 1 and channels % 4 == 0 and 4 <= channels <= 24
            and hs.data_ptr() % 16 == 0 and hs.stride(0) % 4 == 0)


def _gat_records_ok(hs: Tensor, heads: int, channels: int) -> bool:
    """One head whose rows the record-based kernels take (gr_gat_backward_src_h1:
    at most 256 vectors, 16-byte vectors when aligned): the forward then
    stores no alpha and the backward recomputes it from the destination
    records."""
    if heads != 1:
        return False
    if channels % 4 == 0 and hs.data_ptr() % 16 == 0 and hs.stride(0) % 4 == 0:
        return channels <= 1024
    return channels <= 256


def _attention_backward(plan: DevicePlan, hs: Tensor, a_src: Tensor, a_dst: Tensor, s: Tensor,
                        d: Tensor, alpha_or_m: Tensor, den: Tensor, go: Tensor, cdot: Tensor,
                        H: int, C: int, records: bool, zsink: Optional[ProjectedSink]):
    """dHs (None with zsink: added into zsink.dz), datt_src and datt_dst of the
    attention given go = dL/dO [B, H*C] and cdot = <go_i, O_i> [B, H].
    records: one head, the forward stored no alpha (alpha_or_m holds m); the
    source pass reads the destination records (gr_gat_backward_src_h1)."""
    HC = H * C
    E, B = plan.num_src, plan.num_dst
    dev = hs.device
    stream = _lib.stream_handle()
    nnz = plan.nnz
    region = KernelTimer.region(
        "gat_bwd", nnz * (8 * HC + 16 * H + 8) + E * (4 * HC + 4 * H) + B * (4 * HC + 4 * H),
        nnz, HC)
    region.__enter__()
    ds = torch.empty((E, H), dtype=torch.float32, device=dev)
    gt = torch.empty((max(plan.nnz, 1), H), dtype=torch.float32, device=dev)
    bw = plan.bwd
    ws_stride = ((HC + 3) // 4) * 4 + ((H + 3) // 4) * 4
    ws = _workspace(bw.n_slots, ws_stride, dev)
    rec = None
    if records:
        if go.data_ptr() % 16:
            go = go.clone()  # 16-byte rows for the vector loads
        rec = torch.empty((B, 4), dtype=torch.float32, device=dev)
        _lib.call("gr_gat_dst_record", d.data_ptr(), alpha_or_m.data_ptr(), den.data_ptr(),
                  cdot.data_ptr(), B, rec.data_ptr(), stream)
    if zsink is None:
        dhs = torch.empty((E, HC), dtype=torch.float32, device=dev)
        if rec is not None:
            _lib.call("gr_gat_backward_src_h1", bw.units.data_ptr(), bw.n_units,
                      bw.fixups.data_ptr() if bw.n_fix else None, bw.n_fix,
                      plan.row_idx.data_ptr(), plan.perm.data_ptr(), hs.data_ptr(),
                      hs.stride(0), None, go.data_ptr(), s.data_ptr(), rec.data_ptr(),
                      a_src.data_ptr(), C, dhs.data_ptr(), ds.data_ptr(), gt.data_ptr(),
                      _lib.ptr(ws), bw.n_slots, None, 0, None, stream)
        else:
            _lib.call("gr_gat_backward_src", bw.units.data_ptr(), bw.n_units,
                      bw.fixups.data_ptr() if bw.n_fix else None, bw.n_fix,
                      plan.row_idx.data_ptr(), plan.perm.data_ptr(), hs.data_ptr(),
                      hs.stride(0), go.data_ptr(), s.data_ptr(), d.data_ptr(),
                      alpha_or_m.data_ptr(), cdot.data_ptr(), a_src.data_ptr(), H, C,
                      dhs.data_ptr(), ds.data_ptr(), gt.data_ptr(), _lib.ptr(ws),
                      bw.n_slots, stream)
        dst_rows = dhs
    else:
        # dHs straight into dZ at the partition's global rows; the
        # destination part below adds into its own rows dZ[lo:lo+B].
        # The same pass forms per-wavefront partial sums of
        # datt_src = sum_j ds_j Hs_j while Hs_j is in its registers.
        dhs = None
        att_rows = min(bw.n_units, _ATT_PARTIAL_ROWS)
        att_part = torch.empty((max(att_rows, 1), HC), dtype=torch.float32, device=dev)
        att_waves = ctypes.c_int64(0)
        if rec is not None:
            _lib.call("gr_gat_backward_src_h1", bw.units.data_ptr(), bw.n_units,
                      bw.fixups.data_ptr() if bw.n_fix else None, bw.n_fix,
                      plan.row_idx.data_ptr(), plan.perm.data_ptr(), hs.data_ptr(),
                      hs.stride(0), zsink.rows.data_ptr(), go.data_ptr(), s.data_ptr(),
                      rec.data_ptr(), a_src.data_ptr(), C, zsink.dz.data_ptr(),
                      ds.data_ptr(), gt.data_ptr(), _lib.ptr(ws), bw.n_slots,
                      att_part.data_ptr(), att_part.size(0), ctypes.addressof(att_waves),
                      stream)
        else:
            _lib.call("gr_gat_backward_src_into", bw.units.data_ptr(), bw.n_units,
                      bw.fixups.data_ptr() if bw.n_fix else None, bw.n_fix,
                      plan.row_idx.data_ptr(), plan.perm.data_ptr(), hs.data_ptr(),
                      hs.stride(0), zsink.rows.data_ptr(), go.data_ptr(), s.data_ptr(),
                      d.data_ptr(), alpha_or_m.data_ptr(), cdot.data_ptr(),
                      a_src.data_ptr(), H, C, zsink.dz.data_ptr(), ds.data_ptr(),
                      gt.data_ptr(), _lib.ptr(ws), bw.n_slots, att_part.data_ptr(),
                      att_part.size(0), ctypes.addressof(att_waves), stream)
        dst_rows = zsink.dz[zsink.lo:zsink.lo + B]
    dd = torch.empty((B, H), dtype=torch.float32, device=dev)
    f = plan.fwd
    ws = _workspace(f.n_slots, H, dev)
    _lib.call("gr_gat_backward_dst", f.units.data_ptr(), f.n_units,
              f.fixups.data_ptr() if f.n_fix else None, f.n_fix, gt.data_ptr(),
              a_dst.data_ptr(), cdot.data_ptr(), den.data_ptr(), H, C, dd.data_ptr(),
              dst_rows.data_ptr(), _lib.ptr(ws), f.n_slots, stream)
    region.__exit__(None, None, None)
    # Attention-vector gradients: per head, ds[:,h]^T Hs[:, h] and dd[:,h]^T Hs[:B, h].
    if zsink is None:
        datt_src = column_sum(hs, ds, C)
        datt_dst = column_sum(hs[:B], dd, C)
    else:
        if att_waves.value > 0:
            datt_src = column_sum(att_part[:att_waves.value])
        else:  # no units: nothing summed
            datt_src = torch.zeros(HC, dtype=torch.float32, device=dev)
        datt_dst = column_sum(hs[zsink.lo:zsink.lo + B], dd, C)
    return dhs, datt_src, datt_dst


class _GATAttention(torch.autograd.Function):
    """Attention logits + edge softmax + weighted aggregation of GATConv."""

    @staticmethod
    def forward(ctx, hs: Tensor, att_src: Tensor, att_dst: Tensor, bias: Optional[Tensor],
                plan: DevicePlan, heads: int, channels: int, concat: bool,
                s_pre: Optional[Tensor] = None, d_pre: Optional[Tensor] = None,
                sink: Optional[RowDotSink] = None, zsink: Optional[ProjectedSink] = None,
                token: Optional[Tensor] = None, zx_pre: Optional[Tensor] = None) -> Tensor:
        # zsink: hs is the matrix of all partitions' rows ([N, H*C], s_pre
        # [N, H] alike), read in place through zsink.gidx; the backward adds
        # dHs into zsink.dz at zsink.rows.  zx_pre: hs's packed lines
        # (gat_scores(packed=True) over these rows), read by the narrow path.
        hs = hs.contiguous()
        dev = hs.device
        H, C = heads, channels
        HC = H * C
        E, B = plan.num_src, plan.num_dst
        a_src = att_src.reshape(-1).contiguous()
        a_dst = att_dst.reshape(-1).contiguous()
        stream = _lib.stream_handle()
        nnz = plan.nnz
        region = KernelTimer.region(
            "gat_fwd", nnz * (4 * HC + 8 * H + 4) + B * (4 * HC + 4 * H + 4), nnz, HC)
        region.__enter__()
        if zsink is None and _gat_narrow_ok(hs, H, C):
            return _GATAttention._forward_narrow(ctx, hs, a_src, a_dst, bias, plan, C, s_pre,
                                                 d_pre, region, att_src.shape, zx_pre)
        if s_pre is not None:
            # Scores formed beforehand (once per layer for all rows of a
            # projected matrix, by the same kernel): s_pre [E, H], d_pre [B, H].
            s, d = s_pre.contiguous(), d_pre.contiguous()
        else:
            s = torch.empty((E, H), dtype=torch.float32, device=dev)
            d = torch.empty((B, H), dtype=torch.float32, device=dev)
            _lib.call("gr_gat_scores", hs.data_ptr(), hs.stride(0), E, B, H, C, a_src.data_ptr(),
                      a_dst.data_ptr(), s.data_ptr(), d.data_ptr(), stream)
        m = torch.empty((B, H), dtype=torch.float32, device=dev)
        den = torch.empty((B, H), dtype=torch.float32, device=dev)
        # One head: alpha is not stored; the backward recomputes it from the
        # destination records (gr_gat_backward_src_h1).
        records = _gat_records_ok(hs, H, C)
        alpha = None if records else torch.empty((max(nnz, 1), H), dtype=torch.float32,
                                                 device=dev)
        f = plan.fwd
        o = torch.empty((B, HC), dtype=torch.float32, device=dev)
        fused_bias = (concat or H == 1) and bias is not None
        y = torch.empty((B, HC), dtype=torch.float32, device=dev) if fused_bias else None
        b = bias.contiguous() if fused_bias else None
        ws_width = (HC + 3) // 4 * 4 + (2 * H + 3) // 4 * 4
        ws = _workspace(f.n_slots, ws_width, dev)
        idx = plan.idx if zsink is None else zsink.gidx
        _lib.call("gr_gat_forward", f.units.data_ptr(), f.n_units,
                  f.fixups.data_ptr() if f.n_fix else None, f.n_fix, idx.data_ptr(),
                  hs.data_ptr(), hs.stride(0), s.data_ptr(), d.data_ptr(), B, H, C, _lib.ptr(b),
                  m.data_ptr(), den.data_ptr(), _lib.ptr(alpha), o.data_ptr(), _lib.ptr(y), HC,
                  _lib.ptr(ws), 0 if ws is None else ws.numel(), f.n_slots, stream)
        region.__exit__(None, None, None)
        if concat or H == 1:
            if y is None:
                y = o  # no bias: the output is O itself, also saved for the backward
        else:
            y = o.view(B, H, C).mean(dim=1)
            if bias is not None:
                y = y + bias
        ctx.save_for_backward(hs, a_src, a_dst, s, d, m if records else alpha, den, o)
        ctx.records = records
        ctx.plan = plan
        ctx.shape = (H, C, concat)
        ctx.has_bias = bias is not None
        ctx.att_shape = att_src.shape
        ctx.sink = sink
        ctx.zsink = zsink
        return y

    @staticmethod
    def _forward_narrow(ctx, hs, a_src, a_dst, bias, plan, C, s_pre, d_pre, region,
                        att_shape, zx_pre=None):
        """One head of C <= 24 channels: every row packed into a 128-byte line
        with its logit, an online softmax, no alpha stored.  zx_pre: the
        lines packed beforehand (with s_pre, d_pre)."""
        dev = hs.device
        E, B = plan.num_src, plan.num_dst
        f = plan.fwd
        packed = zx_pre is not None and s_pre is not None
        zx = zx_pre if packed else torch.empty((E, 32), dtype=torch.float32, device=dev)
        fstate = torch.empty((B, C + 4), dtype=torch.float32, device=dev)
        # With a bias only Y = O + bias is written; the backward takes
        # O = Y - bias.
        out = torch.empty((B, C), dtype=torch.float32, device=dev)
        b = bias.contiguous() if bias is not None else None
        if s_pre is None:
            s = None
            dvec = torch.empty((B, 1), dtype=torch.float32, device=dev)
        else:
            s, dvec = s_pre.contiguous(), d_pre.contiguous()
        ws = _workspace(f.n_slots, 52, dev)
        _lib.call("gr_gat_narrow_forward", f.units.data_ptr(), f.n_units,
                  f.fixups.data_ptr() if f.n_fix else None, f.n_fix,
                  _lib.ptr(f.long_units), f.n_long, plan.idx.data_ptr(),
                  None if packed else hs.data_ptr(),
                  hs.stride(0), E, B, C, _lib.ptr(s), None if s is None else dvec.data_ptr(),
                  a_src.data_ptr(), a_dst.data_ptr(), _lib.ptr(b),
                  zx.data_ptr(), None if b is not None else out.data_ptr(),
                  out.data_ptr() if b is not None else None, C,
                  dvec.data_ptr() if s is None else None, fstate.data_ptr(),
                  _lib.ptr(ws), 0 if ws is None else ws.numel(), f.n_slots,
                  _lib.stream_handle())
        region.__exit__(None, None, None)
        ctx.save_for_backward(hs, a_src, a_dst, zx, fstate, out, dvec, b)
        ctx.narrow = True
        ctx.plan = plan
        ctx.shape = (1, C, True)
        ctx.has_bias = bias is not None
        ctx.att_shape = att_shape
        return out

    @staticmethod
    def _backward_narrow(ctx, gy: Tensor):
        hs, a_src, a_dst, zx, fstate, out, dvec, b = ctx.saved_tensors
        plan: DevicePlan = ctx.plan
        C = ctx.shape[1]
        E, B = plan.num_src, plan.num_dst
        dev = hs.device
        go = gy.contiguous()
        if go.data_ptr() % 16:
            go = go.clone()
        db = column_sum(go) if ctx.has_bias else None
        nnz = plan.nnz
        region = KernelTimer.region(
            "gat_bwd", nnz * (8 * C + 16 + 8) + E * (4 * C + 4) + B * (4 * C + 4), nnz, C)
        region.__enter__()
        bw = plan.bwd
        gx = torch.empty((B, 32), dtype=torch.float32, device=dev)
        dhs = torch.empty((E, C), dtype=torch.float32, device=dev)
        ds = torch.empty((E, 1), dtype=torch.float32, device=dev)
        dd = torch.empty((B, 1), dtype=torch.float32, device=dev)
        ws = _workspace(bw.n_slots, 28, dev)
        _lib.call("gr_gat_narrow_backward", bw.units.data_ptr(), bw.n_units,
                  bw.fixups.data_ptr() if bw.n_fix else None, bw.n_fix,
                  _lib.ptr(bw.long_units), bw.n_long, plan.row_idx.data_ptr(), zx.data_ptr(),
                  dvec.data_ptr(), E, B, C, go.data_ptr(), go.stride(0), out.data_ptr(),
                  out.stride(0), _lib.ptr(b), fstate.data_ptr(),
                  a_src.data_ptr(), a_dst.data_ptr(), gx.data_ptr(), dhs.data_ptr(),
                  ds.data_ptr(), dd.data_ptr(), _lib.ptr(ws), 0 if ws is None else ws.numel(),
                  bw.n_slots, _lib.stream_handle())
        region.__exit__(None, None, None)
        datt_src = column_sum(hs, ds, C)
        datt_dst = column_sum(hs[:B], dd, C)
        return (dhs, datt_src.view(ctx.att_shape), datt_dst.view(ctx.att_shape), db,
                None, None, None, None, None, None, None, None, None, None)

    @staticmethod
    def backward(ctx, gy: Tensor):
        if getattr(ctx, "narrow", False):
            return _GATAttention._backward_narrow(ctx, gy)
        hs, a_src, a_dst, s, d, alpha_or_m, den, o = ctx.saved_tensors
        plan: DevicePlan = ctx.plan
        H, C, concat = ctx.shape
        HC = H * C
        E, B = plan.num_src, plan.num_dst
        dev = hs.device
        gy = gy.contiguous()
        if concat or H == 1:
            go = gy
        else:
            go = (gy / H).unsqueeze(1).expand(B, H, C).reshape(B, HC).contiguous()
        db = column_sum(gy) if ctx.has_bias else None
        stream = _lib.stream_handle()
        sink = ctx.sink
        if (sink is not None and sink.cdot is not None and H == 1
                and go.data_ptr() == sink.grad_ptr and sink.cdot.numel() == B):
            # c_i came with this gradient from the LayerNorm that consumed O.
            cdot = sink.cdot.view(B, 1)
            sink.cdot = None
        else:
            cdot = torch.empty((B, H), dtype=torch.float32, device=dev)
            _lib.call("gr_gat_row_dot", go.data_ptr(), go.stride(0), o.data_ptr(), o.stride(0),
                      B, H, C, cdot.data_ptr(), stream)
        zsink = ctx.zsink
        dhs, datt_src, datt_dst = _attention_backward(plan, hs, a_src, a_dst, s, d, alpha_or_m,
                                                      den, go, cdot, H, C, ctx.records, zsink)
        return (dhs, datt_src.view(ctx.att_shape), datt_dst.view(ctx.att_shape), db,
                None, None, None, None, None, None, None, None, None, None)


def gat_scores(hs: Tensor, att_src: Tensor, att_dst: Tensor, heads: int, channels: int,
               num_dst: int, packed: bool = False) -> tuple:
    """The attention logits' two halves of GATConv (no autograd): s[r, h] =
    <hs[r, h], att_src[h]> for every row and d[r, h] = <hs[r, h], att_dst[h]>
    for the first num_dst rows, by the kernel gat_attention uses.
    packed: for a head the narrow kernels take, also the packed source lines
    of these rows, (s, d, zx) (gr_gat_narrow_pack, same s and d): the
    attention over exactly these rows then reads them instead of packing."""
    _check_device_tensor("hs", hs)
    hs = hs.contiguous()
    E, H = hs.size(0), heads
    if hs.size(1) != heads * channels or not 0 <= num_dst <= E:
        raise ValueError("gat_scores: bad shape")
    s = torch.empty((E, H), dtype=torch.float32, device=hs.device)
    d = torch.empty((num_dst, H), dtype=torch.float32, device=hs.device)
    a_src = att_src.detach().reshape(-1).contiguous()
    a_dst = att_dst.detach().reshape(-1).contiguous()
    if packed and _gat_narrow_ok(hs, H, channels):
        zx = torch.empty((E, 32), dtype=torch.float32, device=hs.device)
        _lib.call("gr_gat_narrow_pack", hs.data_ptr(), hs.stride(0), E, num_dst, channels,
                  a_src.data_ptr(), a_dst.data_ptr(), zx.data_ptr(), s.data_ptr(),
                  d.data_ptr(), _lib.stream_handle())
        return s, d, zx
    _lib.call("gr_gat_scores", hs.data_ptr(), hs.stride(0), E, num_dst, H, channels,
              a_src.data_ptr(), a_dst.data_ptr(), s.data_ptr(), d.data_ptr(),
              _lib.stream_handle())
    return s, d


def gat_attention(hs: Tensor, adj: Adjacency, att_src: Tensor, att_dst: Tensor,
                  bias: Optional[Tensor], heads: int, channels: int,
                  concat: bool = True,
                  scores: Optional[Tuple[Tensor, Tensor]] = None,
                  rowdot_sink: Optional[RowDotSink] = None,
                  sink: Optional[ProjectedSink] = None) -> Tensor:
    """GATConv attention over a bipartite partition adjacency, on the GPU.

    hs = lin(x) for all E source rows; destination features are hs[:B].
    Returns [B, H*C] (concat) or [B, C] (mean over heads), bias added.
    `scores`, when given, are the logit halves (s [E, H], d [B, H]) formed
    beforehand by gat_scores, so they are not formed again here.
    `rowdot_sink`: shared with the bias_ln_act that consumes this output, so
    that its backward hands over c_i (one head).
    `sink`: hs is the [N, H*C] matrix of all partitions' rows (one head of a
    multiple of 4 in 68..1024 channels), read in place through sink.gidx with
    `scores` = (s of all N rows, d of the partition's rows); the backward adds
    dHs into sink.dz at sink.rows and returns no gradient for hs.
    """
    _check_device_tensor("hs", hs)
    plan = adj.device_plan(hs.device)
    if hs.size(1) != heads * channels:
        raise ValueError(f"hs has {hs.size(1)} features, expected {heads * channels}")
    if sink is not None:
        if heads != 1 or channels % 4 != 0 or not 64 < channels <= 1024 or scores is None:
            raise ValueError("gat_attention: reading hs in place needs one head of 68..1024 "
                             "channels (a multiple of 4) and precomputed scores")
        s, d = scores
        if (sink.gidx.numel() != plan.nnz or sink.rows.numel() != plan.num_src
                or sink.dz is None or tuple(sink.dz.shape) != tuple(hs.shape)
                or not sink.dz.is_contiguous() or s.size(0) != hs.size(0)
                or tuple(d.shape) != (plan.num_dst, 1)
                or not 0 <= sink.lo <= hs.size(0) - plan.num_dst):
            raise ValueError("gat_attention: sink does not match the adjacency and hs")
        return _GATAttention.apply(hs, att_src, att_dst, bias, plan, heads, channels, concat,
                                   s, d, rowdot_sink, sink, sink.token)
    if hs.size(0) != plan.num_src:
        raise ValueError(f"hs has {hs.size(0)} rows, adjacency has {plan.num_src} columns")
    if scores is None:
        return _GATAttention.apply(hs, att_src, att_dst, bias, plan, heads, channels, concat,
                                   None, None, rowdot_sink)
    s, d = scores[0], scores[1]
    if tuple(s.shape) != (plan.num_src, heads) or tuple(d.shape) != (plan.num_dst, heads):
        raise ValueError("gat_attention: scores do not match the adjacency and heads")
    zx = scores[2] if len(scores) > 2 else None
    if zx is not None and tuple(zx.shape) != (plan.num_src, 32):
        raise ValueError("gat_attention: packed rows do not match the adjacency")
    return _GATAttention.apply(hs, att_src, att_dst, bias, plan, heads, channels, concat, s, d,
                               rowdot_sink, None, None, zx)


class _GATAttentionLN(torch.autograd.Function):
    """One head: attention + conv bias + LayerNorm + activation in one pass
    (gr_gat_forward_ln: the epilogue in the attention kernel's row store, so
    O never reaches HBM).  Backward: the LayerNorm/activation backward (or
    its form with the consumer's product, LNProductSink), which also forms
    c_i = <dL/dO_i, O_i>, then the attention backward with the destination
    records."""

    @staticmethod
    def forward(ctx, hs: Tensor, att_src: Tensor, att_dst: Tensor, bias: Optional[Tensor],
                gamma: Tensor, beta: Tensor, token: Optional[Tensor], plan: DevicePlan,
                eps: float, act: str, s_pre: Optional[Tensor], d_pre: Optional[Tensor],
                zsink: Optional[ProjectedSink], dest: Optional[OutputRows],
                ln_sink) -> Tensor:
        hs = hs.contiguous()
        dev = hs.device
        C = hs.size(1)
        E, B = plan.num_src, plan.num_dst
        a_src = att_src.reshape(-1).contiguous()
        a_dst = att_dst.reshape(-1).contiguous()
        stream = _lib.stream_handle()
        nnz = plan.nnz
        region = KernelTimer.region("gat_fwd", nnz * (4 * C + 12) + B * (4 * C + 8), nnz, C)
        region.__enter__()
        if s_pre is not None:
            s, d = s_pre.contiguous(), d_pre.contiguous()
        else:
            s = torch.empty((E, 1), dtype=torch.float32, device=dev)
            d = torch.empty((B, 1), dtype=torch.float32, device=dev)
            _lib.call("gr_gat_scores", hs.data_ptr(), hs.stride(0), E, B, 1, C, a_src.data_ptr(),
                      a_dst.data_ptr(), s.data_ptr(), d.data_ptr(), stream)
        m = torch.empty((B, 1), dtype=torch.float32, device=dev)
        den = torch.empty((B, 1), dtype=torch.float32, device=dev)
        h = torch.empty((B, C), dtype=torch.float32, device=dev)
        out = output_block(dest, B, C, dev)
        mean = torch.empty(B, dtype=torch.float32, device=dev)
        rstd = torch.empty(B, dtype=torch.float32, device=dev)
        f = plan.fwd
        ws = _workspace(f.n_slots, C + 4, dev)
        b = bias.contiguous() if bias is not None else None
        g, bt = gamma.contiguous(), beta.contiguous()
        idx = plan.idx if zsink is None else zsink.gidx
        _lib.call("gr_gat_forward_ln", f.units.data_ptr(), f.n_units,
                  f.fixups.data_ptr() if f.n_fix else None, f.n_fix, idx.data_ptr(),
                  hs.data_ptr(), hs.stride(0), s.data_ptr(), d.data_ptr(), B, C, _lib.ptr(b),
                  g.data_ptr(), bt.data_ptr(), float(eps), _lib.ACTIVATIONS[act],
                  m.data_ptr(), den.data_ptr(), h.data_ptr(), out.data_ptr(), C,
                  mean.data_ptr(), rstd.data_ptr(), _lib.ptr(ws),
                  0 if ws is None else ws.numel(), f.n_slots, stream)
        region.__exit__(None, None, None)
        ctx.save_for_backward(hs, a_src, a_dst, s, d, m, den, h, mean, rstd, g, bt)
        ctx.plan = plan
        ctx.zsink = zsink
        ctx.bias = b
        ctx.act = act
        ctx.ln_sink = ln_sink
        ctx.att_shape = att_src.shape
        return out

    @staticmethod
    def backward(ctx, gout: Tensor):
        hs, a_src, a_dst, s, d, m, den, h, mean, rstd, g, bt = ctx.saved_tensors
        plan: DevicePlan = ctx.plan
        B, C = h.shape
        has_bias = ctx.bias is not None
        rowdot = torch.empty(B, dtype=torch.float32, device=h.device)
        prod = ctx.ln_sink.take(gout) if ctx.ln_sink is not None else None
        if prod is not None and prod[2]:
            gh, dgamma, dbeta, db = ln_act_backward_product(
                prod[0], prod[1], h, mean, rstd, g, bt, has_bias, ctx.act, shift=ctx.bias,
                rowdot=rowdot)
        else:
            if prod is not None:
                from grinnder_amd.dense import gemm_nt
                gout = gout + gemm_nt(prod[0], prod[1].t().contiguous())
            gh, dgamma, dbeta, db = ln_act_backward(gout, h, mean, rstd, g, bt, has_bias,
                                                    ctx.act, shift=ctx.bias, rowdot=rowdot)
        dhs, datt_src, datt_dst = _attention_backward(plan, hs, a_src, a_dst, s, d, m, den, gh,
                                                      rowdot.view(B, 1), 1, C, True,
                                                      ctx.zsink)
        return (dhs, datt_src.view(ctx.att_shape), datt_dst.view(ctx.att_shape), db, dgamma,
                dbeta, None, None, None, None, None, None, None, None, None)


def gat_attention_ln_ok(hs: Tensor, heads: int, channels: int, gamma: Tensor) -> bool:
    """Whether gat_attention_ln runs its fused kernel: one head of 132..1024
    channels (a multiple of 4, rows held by a whole wavefront) on 16-byte
    rows, with an affine LayerNorm over the full width."""
    return (heads == 1 and channels % 4 == 0 and 128 < channels <= 1024
            and hs.data_ptr() % 16 == 0 and hs.stride(0) % 4 == 0
            and gamma is not None and tuple(gamma.shape) == (channels,))


def gat_attention_ln(hs: Tensor, adj: Adjacency, att_src: Tensor, att_dst: Tensor,
                     bias: Optional[Tensor], gamma: Tensor, beta: Tensor, eps: float,
                     act: str = "elu", scores: Optional[Tuple[Tensor, Tensor]] = None,
                     sink: Optional[ProjectedSink] = None,
                     dest: Optional[OutputRows] = None) -> Tensor:
    """act(LayerNorm(GATConv attention + bias)) of one head (GAT.forward_layer's
    conv -> LayerNorm -> ELU, grinnder/nn/gat.py:74-78) as one pass per row;
    hs, scores and sink as gat_attention, dest as dense.bias_ln_act.  The
    caller checks gat_attention_ln_ok."""
    _check_device_tensor("hs", hs)
    plan = adj.device_plan(hs.device)
    C = hs.size(1)
    if act not in _lib.ACTIVATIONS:
        raise ValueError(f"unknown activation {act!r}")
    if not gat_attention_ln_ok(hs, 1, C, gamma):
        raise ValueError("gat_attention_ln: one head of 132..1024 channels on 16-byte rows")
    s_pre = d_pre = None
    if scores is not None:
        s_pre, d_pre = scores
    token = None
    if sink is not None:
        if scores is None or sink.gidx.numel() != plan.nnz or sink.rows.numel() != plan.num_src \
                or sink.dz is None or tuple(sink.dz.shape) != tuple(hs.shape):
            raise ValueError("gat_attention_ln: sink does not match the adjacency and hs")
        token = sink.token
    elif hs.size(0) != plan.num_src:
        raise ValueError(f"hs has {hs.size(0)} rows, adjacency has {plan.num_src} columns")
    if s_pre is not None and (tuple(d_pre.shape) != (plan.num_dst, 1)
                              or s_pre.size(0) != hs.size(0)):
        raise ValueError("gat_attention_ln: scores do not match the adjacency")
    ln_sink = LNProductSink()
    out = _GATAttentionLN.apply(hs, att_src, att_dst, bias, gamma, beta, token, plan, eps, act,
                                s_pre, d_pre, sink, dest, ln_sink)
    out._grinnder_ln_sink = ln_sink
    return out
