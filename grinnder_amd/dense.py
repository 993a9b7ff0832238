"""Dense per-layer transform of the conv layers, on the HIP kernels.

PyG's GCNConv / GATConv (grinnder/nn/gcn.py:53-56, grinnder/nn/gat.py:54-61)
apply a bias-free ``Linear`` to the node features.  All three of its
products run on this library's fp32 MFMA kernels: the forward x Wᵀ (+ b) and
the input gradient dy W on ``gr_gemm_nt`` (row-block tiles, K-contiguous
operands), the weight gradient dW = dyᵀ x, which reduces over all K node rows
of the partition with M, N <= a few hundred, on ``gr_gemm_tn`` (split-K,
partials summed in a fixed order).

``bias_ln_act`` is the dense counterpart of the fused aggregation epilogue:
LayerNorm + ReLU after a GCN layer that aggregates first and multiplies
afterwards, and LayerNorm + ELU after a GAT layer.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch
from torch import Tensor

from grinnder_amd import _lib


def _check(name: str, t: Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (HIP); got {t.device}")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be float32; got {t.dtype}")


class OutputRows:
    """A caller's fp32 [rows, D] block of device memory (rows contiguous, no
    gradient) that a fused layer epilogue writes its result into, instead of
    a new tensor.  The epilogue returns a view of the block as the layer's
    autograd output, so a caller that wanted the output there (the next
    layer's HBM-resident input rows) needs no copy.  The block is passed
    inside this holder, not as a tensor argument, so that autograd does not
    take it for an input of the epilogue."""

    __slots__ = ("rows",)

    def __init__(self, rows: Tensor):
        self.rows = rows


def output_block(dest: Optional[OutputRows], rows: int, dim: int, device) -> Tensor:
    """The tensor a fused epilogue writes its [rows, dim] result into:
    dest's block when one is given (checked to be exactly that shape, fp32,
    on the device and row-contiguous), else a new tensor."""
    if dest is None:
        return torch.empty((rows, dim), dtype=torch.float32, device=device)
    t = dest.rows
    if (t.dtype != torch.float32 or t.device != torch.device(device) or tuple(t.shape) != (rows, dim)
            or (rows > 1 and t.stride(0) != dim) or (dim > 1 and t.stride(1) != 1)
            or t.requires_grad):
        raise ValueError(f"output block must be a contiguous fp32 [{rows}, {dim}] tensor on "
                         f"{device} without gradient; got {tuple(t.shape)}, {t.dtype}, "
                         f"strides {t.stride()}, on {t.device}")
    return t


def gemm_tn_splits(m: int, n: int, k: int) -> Tuple[int, int]:
    """Default K split count and workspace floats of ``gemm_tn`` for a shape."""
    splits = ctypes.c_int64(0)
    ws = ctypes.c_int64(0)
    _lib.call("gr_gemm_tn_workspace", m, n, k, ctypes.addressof(splits), ctypes.addressof(ws))
    return splits.value, ws.value


def gemm_tn(a: Tensor, b: Tensor, out: Optional[Tensor] = None, beta: float = 0.0,
            splits: Optional[int] = None) -> Tensor:
    """C = a^T b (+ beta * out) for a [K, M], b [K, N] row-major fp32 device matrices."""
    _check("a", a)
    _check("b", b)
    if a.dim() != 2 or b.dim() != 2 or a.size(0) != b.size(0):
        raise ValueError(f"gemm_tn: a {tuple(a.shape)} and b {tuple(b.shape)} need equal rows")
    if a.stride(1) != 1:
        a = a.contiguous()
    if b.stride(1) != 1:
        b = b.contiguous()
    k, m = a.shape
    n = b.size(1)
    if out is None:
        if beta != 0.0:
            raise ValueError("gemm_tn: beta != 0 needs `out`")
        out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    elif out.shape != (m, n) or not out.is_contiguous():
        raise ValueError(f"gemm_tn: out must be a contiguous [{m}, {n}] matrix")
    default_splits, _ = gemm_tn_splits(m, n, k)
    s = default_splits if splits is None else int(splits)
    ws = torch.empty(max(1, s * m * n), dtype=torch.float32, device=a.device)
    _lib.call("gr_gemm_tn", a.data_ptr(), max(a.stride(0), m), b.data_ptr(),
              max(b.stride(0), n), m, n, k, float(beta), out.data_ptr(), ws.data_ptr(),
              ws.numel(), s, _lib.stream_handle())
    return out


def gemm_nt(a: Tensor, b: Tensor, bias: Optional[Tensor] = None,
            out: Optional[Tensor] = None) -> Tensor:
    """C = a bᵀ (+ bias) for a [M, K] and b [N, K] fp32 device matrices with
    unit column stride (rows may be strided) on the matrix cores, or, for a
    short reduction (K <= 64, N >= 64), as a stream of C's rows on the vector
    units; `out` is a [M, N] matrix with unit column stride (for example a
    column slice of a wider buffer), written in place."""
    _check("a", a)
    _check("b", b)
    if a.dim() != 2 or b.dim() != 2 or a.size(1) != b.size(1):
        raise ValueError(f"gemm_nt: a {tuple(a.shape)} and b {tuple(b.shape)} need equal columns")
    if a.stride(1) != 1 or (a.size(0) > 1 and a.stride(0) < a.size(1)):
        a = a.contiguous()
    if b.stride(1) != 1 or (b.size(0) > 1 and b.stride(0) < b.size(1)):
        b = b.contiguous()
    m, k = a.shape
    n = b.size(0)
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    else:
        _check("out", out)
        if out.shape != (m, n) or out.stride(1) != 1 or (m > 1 and out.stride(0) < n):
            raise ValueError(f"gemm_nt: out must be a [{m}, {n}] matrix with unit column "
                             f"stride; got {tuple(out.shape)} strides {out.stride()}")
    if bias is not None:
        _check("bias", bias)
        bias = bias.contiguous()
        if bias.numel() != n:
            raise ValueError(f"gemm_nt: bias of {bias.numel()} elements, {n} expected")
    if m == 0 or n == 0:
        return out
    if k == 0:
        return out.copy_(bias.expand(m, n) if bias is not None else torch.zeros_like(out))
    _lib.call("gr_gemm_nt", a.data_ptr(), max(a.stride(0), k), b.data_ptr(),
              max(b.stride(0), k), m, n, k, _lib.ptr(bias), out.data_ptr(),
              max(out.stride(0), n), _lib.stream_handle())
    return out


class _Linear(torch.autograd.Function):
    """y = x W^T (+ b) and dx = dy W (gr_gemm_nt), dW = dy^T x (gr_gemm_tn),
    db = sum dy.
    `reuse` (a one-element list, or None) holds y as an earlier forward
    computed it from the same x, W and b: it is returned instead of being
    recomputed, and the backward is the same."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, bias: Optional[Tensor],
                reuse: Optional[list] = None) -> Tensor:
        from grinnder_amd.aggregation import dense_region
        x2 = x.reshape(-1, x.size(-1))
        if reuse is not None:
            y = reuse[0].detach()
            if y.shape != (x2.size(0), weight.size(0)):
                raise ValueError(f"linear: reused product has shape {tuple(y.shape)}, "
                                 f"expected {(x2.size(0), weight.size(0))}")
        else:
            with dense_region("fwd", x2.size(0), x2.size(1), weight.size(0)):
                y = gemm_nt(x2, weight, bias)
        ctx.save_for_backward(x2, weight)
        ctx.in_shape = x.shape
        ctx.has_bias = bias is not None
        return y.reshape(*x.shape[:-1], weight.size(0))

    @staticmethod
    def backward(ctx, gy: Tensor):
        from grinnder_amd.aggregation import dense_region
        x2, weight = ctx.saved_tensors
        gy2 = gy.reshape(-1, weight.size(0)).contiguous()
        dx = dw = db = None
        rows, dout, din = gy2.size(0), weight.size(0), weight.size(1)
        if ctx.needs_input_grad[0]:
            with dense_region("dx", rows, dout, din):
                dx = gemm_nt(gy2, weight.t().contiguous()).reshape(ctx.in_shape)
        if ctx.needs_input_grad[1]:
            with dense_region("dw", rows, dout, din):
                dw = gemm_tn(gy2, x2)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            from grinnder_amd.aggregation import column_sum
            db = column_sum(gy2)
        return dx, dw, db, None


def linear(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None,
           reuse: Optional[Tensor] = None) -> Tensor:
    """``F.linear`` on the library's MFMA kernels (GPU): forward and input
    gradient on gr_gemm_nt, weight gradient on the split-K gr_gemm_tn.
    `reuse`: this product as an earlier forward formed it from the same
    operands (rows [-1, out]); it is returned instead of recomputed, with the
    same backward."""
    if not x.is_cuda:
        raise RuntimeError(f"linear: x must be a GPU tensor (HIP); got {x.device}")
    return _Linear.apply(x, weight, bias, None if reuse is None else [reuse])


class _BiasLNAct(torch.autograd.Function):
    """out = act(LayerNorm(z + b)); backward with gr_ln_act_backward, or
    with gr_ln_act_backward_product when the consumer of out handed its
    gradient over as a product (aggregation.LNProductSink)."""

    @staticmethod
    def forward(ctx, z: Tensor, bias: Optional[Tensor], gamma: Tensor, beta: Tensor,
                eps: float, act: str, sink=None, dest: Optional[OutputRows] = None,
                ln_sink=None) -> Tensor:
        z = z.contiguous()
        rows, dim = z.shape
        dev = z.device
        h = torch.empty_like(z)
        out = output_block(dest, rows, dim, dev)
        mean = torch.empty(rows, dtype=torch.float32, device=dev)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        b = bias.contiguous() if bias is not None else None
        g, bt = gamma.contiguous(), beta.contiguous()
        _lib.call("gr_bias_ln_act", z.data_ptr(), z.stride(0), _lib.ptr(b), g.data_ptr(),
                  bt.data_ptr(), float(eps), _lib.ACTIVATIONS[act], rows, dim, h.data_ptr(),
                  out.data_ptr(), mean.data_ptr(), rstd.data_ptr(), _lib.stream_handle())
        ctx.save_for_backward(h, mean, rstd, g, bt)
        ctx.has_bias = bias is not None
        ctx.act = act
        ctx.sink = sink
        ctx.ln_sink = ln_sink
        ctx.bias = b
        return out

    @staticmethod
    def backward(ctx, gout: Tensor):
        from grinnder_amd.aggregation import ln_act_backward, ln_act_backward_product
        h, mean, rstd, g, bt = ctx.saved_tensors
        rowdot = None
        if ctx.sink is not None:
            # <dL/dz_r, z_r> with z = h - b, for the attention that produced z.
            rowdot = torch.empty(h.size(0), dtype=torch.float32, device=h.device)
        prod = ctx.ln_sink.take(gout) if ctx.ln_sink is not None else None
        if prod is not None and prod[2]:
            gh, dgamma, dbeta, db = ln_act_backward_product(
                prod[0], prod[1], h, mean, rstd, g, bt, ctx.has_bias, ctx.act,
                shift=ctx.bias, rowdot=rowdot)
        else:
            if prod is not None:
                gout = gout + gemm_nt(prod[0], prod[1].t().contiguous())
            gh, dgamma, dbeta, db = ln_act_backward(gout, h, mean, rstd, g, bt, ctx.has_bias,
                                                    ctx.act, shift=ctx.bias, rowdot=rowdot)
        if ctx.sink is not None:
            ctx.sink.cdot = rowdot
            ctx.sink.grad_ptr = gh.data_ptr()
        return gh, db, dgamma, dbeta, None, None, None, None, None


def bias_ln_act(z: Tensor, bias: Optional[Tensor], gamma: Tensor, beta: Tensor,
                eps: float = 1e-5, act: str = "relu", rowdot_sink=None,
                dest: Optional[OutputRows] = None) -> Tensor:
    """act(LayerNorm(z + bias)) over the rows of z (GPU, one pass); act is
    "relu" or "elu" (alpha = 1).  `rowdot_sink` (an aggregation.RowDotSink
    shared with the GAT attention that produced z): the backward also forms
    <dL/dz_r, z_r> and leaves it there.  `dest`: write the result into that
    block and return a view of it."""
    from grinnder_amd.aggregation import LNProductSink
    _check("z", z)
    if act not in _lib.ACTIVATIONS:
        raise ValueError(f"unknown activation {act!r}")
    ln_sink = LNProductSink()
    out = _BiasLNAct.apply(z, bias, gamma, beta, eps, act, rowdot_sink, dest, ln_sink)
    # A product that consumes the output alone may hand its input gradient
    # back as dZ W (LNProductSink).
    out._grinnder_ln_sink = ln_sink
    return out


def bias_ln_relu(z: Tensor, bias: Optional[Tensor], gamma: Tensor, beta: Tensor,
                 eps: float = 1e-5) -> Tensor:
    """ReLU(LayerNorm(z + bias)) over the rows of z (GPU, one pass)."""
    return bias_ln_act(z, bias, gamma, beta, eps, "relu")


class _LinearLNAct(torch.autograd.Function):
    """out = act(LayerNorm(x Wᵀ + b)) with the LayerNorm in the GEMM epilogue
    (gr_linear_ln_act); backward: gr_ln_act_backward, then dW = ghᵀ x on the
    split-K kernel and dx = gh W."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, bias: Optional[Tensor], gamma: Tensor,
                beta: Tensor, eps: float, act: str,
                dest: Optional[OutputRows] = None) -> Tensor:
        x = x.contiguous()
        rows, din = x.shape
        dout = weight.size(0)
        dev = x.device
        w = weight.contiguous()
        wt = w.t().contiguous()
        h = torch.empty((rows, dout), dtype=torch.float32, device=dev)
        out = output_block(dest, rows, dout, dev)
        mean = torch.empty(rows, dtype=torch.float32, device=dev)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        b = bias.contiguous() if bias is not None else None
        g, bt = gamma.contiguous(), beta.contiguous()
        from grinnder_amd.aggregation import dense_region
        with dense_region("fwd_ln", rows, din, dout):
            _lib.call("gr_linear_ln_act", x.data_ptr(), x.stride(0), rows, din, wt.data_ptr(),
                      dout, _lib.ptr(b), g.data_ptr(), bt.data_ptr(), float(eps),
                      _lib.ACTIVATIONS[act], h.data_ptr(), out.data_ptr(), mean.data_ptr(),
                      rstd.data_ptr(), _lib.stream_handle())
        ctx.save_for_backward(x, w, h, mean, rstd, g, bt)
        ctx.has_bias = bias is not None
        ctx.act = act
        return out

    @staticmethod
    def backward(ctx, gout: Tensor):
        from grinnder_amd.aggregation import dense_region, ln_act_backward
        x, w, h, mean, rstd, g, bt = ctx.saved_tensors
        gh, dgamma, dbeta, db = ln_act_backward(gout, h, mean, rstd, g, bt, ctx.has_bias,
                                                ctx.act)
        dx = dw = None
        rows, din, dout = x.size(0), x.size(1), w.size(0)
        if ctx.needs_input_grad[0]:
            with dense_region("dx", rows, dout, din):
                dx = gemm_nt(gh, w.t().contiguous())
        if ctx.needs_input_grad[1]:
            with dense_region("dw", rows, dout, din):
                dw = gemm_tn(gh, x)
        return dx, dw, db, dgamma, dbeta, None, None, None


def linear_ln_act(x: Tensor, weight: Tensor, bias: Optional[Tensor], gamma: Tensor,
                  beta: Tensor, eps: float = 1e-5, act: str = "relu",
                  dest: Optional[OutputRows] = None) -> Tensor:
    """act(LayerNorm(x Wᵀ + bias)) (GPU).  One fused MFMA pass when the output
    width is a multiple of 16 up to 256; otherwise the product and the
    epilogue run as two passes.  `dest` as in bias_ln_act."""
    _check("x", x)
    if act not in _lib.ACTIVATIONS:
        raise ValueError(f"unknown activation {act!r}")
    dout = weight.size(0)
    if dout % 16 == 0 and dout <= 256 and x.dim() == 2:
        return _LinearLNAct.apply(x, weight, bias, gamma, beta, eps, act, dest)
    return bias_ln_act(linear(x, weight), bias, gamma, beta, eps, act, dest=dest)
