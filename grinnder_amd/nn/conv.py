"""GCNConv / GATConv layers backed by the HIP aggregation kernels.

Parameter names and shapes follow PyG (the reference instantiates
``GCNConv(in, out, normalize=False)`` and ``GATConv(in, out, heads,
concat, add_self_loops=False)``, grinnder/nn/gcn.py:53-56 and
grinnder/nn/gat.py:54-61), so state_dicts are interchangeable:
``lin.weight``, ``bias``, ``att_src``, ``att_dst``.  PyG < 2.5 named the GAT
projection ``lin_src``/``lin_dst``; both spellings load.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple, Union

import torch
import torch.nn.functional as F
from torch import Tensor
from torch.nn import Linear, Module, Parameter

from grinnder_amd.aggregation import (RowDotSink, gat_attention, gat_attention_ln,
                                      gat_attention_ln_ok, gat_scores, gcn_aggregate,
                                      gcn_linear_aggregate)
from grinnder_amd.data.adjacency import Adjacency
from grinnder_amd.dense import bias_ln_act, linear


def glorot_(t: Tensor) -> Tensor:
    """PyG's glorot: U(-a, a), a = sqrt(6 / (size(-2) + size(-1)))."""
    a = math.sqrt(6.0 / (t.size(-2) + t.size(-1)))
    with torch.no_grad():
        return t.uniform_(-a, a)


class GCNConv(Module):
    """out = A · (x Wᵀ) + b with the adjacency's precomputed GCN weights.

    Only ``normalize=False`` is supported: the normalisation is computed once
    on the full graph and stored as adjacency values, as in the reference.

    PyG multiplies first and aggregates the out_channels-wide product.  When
    the layer widens (in_channels < out_channels) this layer aggregates first,
    (A x) Wᵀ + b: the same function with the fp32 sums reassociated, but the
    neighbour gather moves in_channels-wide rows, and when x needs no gradient
    the backward has no aggregation at all.
    """

    def __init__(self, in_channels: int, out_channels: int, normalize: bool = False,
                 bias: bool = True):
        super().__init__()
        if normalize:
            raise ValueError("GCNConv expects precomputed full-graph normalisation "
                             "(normalize=False)")
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.lin = Linear(in_channels, out_channels, bias=False)
        self.bias = Parameter(torch.empty(out_channels)) if bias else None
        self.reset_parameters()

    def reset_parameters(self) -> None:
        glorot_(self.lin.weight)
        if self.bias is not None:
            torch.nn.init.zeros_(self.bias)

    def aggregate_first(self) -> bool:
        return self.in_channels < self.out_channels

    def forward(self, x: Tensor, adj: Adjacency) -> Tensor:
        if self.aggregate_first():
            return linear(gcn_aggregate(x, adj), self.lin.weight, self.bias)
        return gcn_linear_aggregate(x, self.lin.weight, adj, self.bias)

    def __repr__(self) -> str:
        return f"{self.__class__.__name__}({self.in_channels}, {self.out_channels})"


class GATConv(Module):
    """Graph attention over a bipartite partition adjacency (PyG GATConv semantics).

    Called as ``conv((x, x[:B]), adj)``; the destination features must be the
    first B rows of the source features (one shared projection), which is how
    the reference's GAT.forward_layer calls it.
    """

    def __init__(self, in_channels: int, out_channels: int, heads: int = 1,
                 concat: bool = True, negative_slope: float = 0.2, dropout: float = 0.0,
                 add_self_loops: bool = True, bias: bool = True):
        super().__init__()
        if add_self_loops:
            raise ValueError("bipartite partition adjacencies already contain self-loops; "
                             "use add_self_loops=False")
        if negative_slope != 0.2:
            raise ValueError("the attention kernels implement negative_slope=0.2")
        if dropout != 0.0:
            raise ValueError("attention dropout is not supported (the reference uses 0)")
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.heads = heads
        self.concat = concat
        self.lin = Linear(in_channels, heads * out_channels, bias=False)
        self.att_src = Parameter(torch.empty(1, heads, out_channels))
        self.att_dst = Parameter(torch.empty(1, heads, out_channels))
        self.bias = Parameter(torch.empty(heads * out_channels if concat else out_channels)) \
            if bias else None
        self.reset_parameters()

    def reset_parameters(self) -> None:
        glorot_(self.lin.weight)
        glorot_(self.att_src)
        glorot_(self.att_dst)
        if self.bias is not None:
            torch.nn.init.zeros_(self.bias)

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        old = prefix + "lin_src.weight"
        if old in state_dict and prefix + "lin.weight" not in state_dict:
            state_dict[prefix + "lin.weight"] = state_dict.pop(old)
            state_dict.pop(prefix + "lin_dst.weight", None)
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)

    def forward(self, x: Union[Tensor, Tuple[Tensor, Tensor]], adj: Adjacency,
                add_bias: bool = True, reuse: Optional[Tensor] = None,
                keep: Optional[list] = None, rowdot_sink=None) -> Tensor:
        """add_bias=False leaves the bias out of the output, for a caller that
        adds it in a fused epilogue (the LayerNorm of GAT.forward_layer).
        keep: a list that receives this call's projection hs of the source
        rows (detached); reuse: such an hs from an earlier call on the same
        rows and weights, taken instead of the projection product (the
        backward is unchanged).  rowdot_sink: see attend."""
        bias = self.bias if add_bias else None
        num_dst = adj.sparse_sizes()[0]
        if isinstance(x, tuple):
            x_src, x_dst = x
            same = (x_dst.size(0) == num_dst and x_dst.data_ptr() == x_src.data_ptr()
                    and x_dst.stride() == x_src.stride())
            if not same:
                raise ValueError("GATConv expects (x, x[:num_dst]) with a shared projection")
        else:
            x_src = x
        if self.heads == 1 and self.out_channels % 4 != 0:
            # One head of C channels, C not a multiple of 4: run the attention
            # on C rounded up to 4 with zero-padded W, att_src, att_dst and
            # bias.  The pad channel is zero in Hs and in both attention
            # vectors, so the logits, alpha and the first C output channels
            # are unchanged; the kernels then move 16-byte row vectors.
            pad = (-self.out_channels) % 4
            w = F.pad(self.lin.weight, (0, 0, 0, pad))
            a_s = F.pad(self.att_src, (0, pad))
            a_d = F.pad(self.att_dst, (0, pad))
            b = F.pad(bias, (0, pad)) if bias is not None else None
            hs = linear(x_src, w, reuse=reuse)
            if keep is not None:
                keep.append(hs.detach())
            y = gat_attention(hs, adj, a_s, a_d, b, 1, self.out_channels + pad, self.concat)
            return y[:, :self.out_channels]
        hs = linear(x_src, self.lin.weight, reuse=reuse)
        if keep is not None:
            keep.append(hs.detach())
        return self.attend(hs, adj, add_bias, rowdot_sink=rowdot_sink)

    def _padded(self) -> int:
        """Zero columns added to one head of C channels, C not a multiple of 4."""
        return (-self.out_channels) % 4 if self.heads == 1 else 0

    def _pad_rows(self, hs: Tensor) -> Tensor:
        """hs with the padded head's zero columns: hs itself when it has them
        already (a projected matrix held at the padded width, whose pad
        columns the projection leaves zero)."""
        width = self.out_channels + self._padded()
        if hs.size(-1) == width:
            return hs
        if hs.size(-1) != self.out_channels:
            raise ValueError(f"GATConv: rows of {hs.size(-1)} channels for {self.out_channels}")
        return F.pad(hs, (0, width - self.out_channels))

    def attend(self, hs: Tensor, adj: Adjacency, add_bias: bool = True,
               scores: Optional[Tuple[Tensor, Tensor]] = None, rowdot_sink=None,
               sink=None) -> Tensor:
        """The layer after its projection: attention over hs = lin(x) for all
        source rows.  One head of C channels, C not a multiple of 4, runs on hs
        and the attention parameters zero-padded to a multiple of 4 (as in
        forward).  `scores`: the logit halves of these rows from scores().
        `rowdot_sink` (aggregation.RowDotSink): shared with the bias_ln_act
        that consumes this output, whose backward then hands the attention's
        backward c_i = <dL/dO_i, O_i> instead of it being formed again.
        `sink` (aggregation.ProjectedSink): hs is the matrix of all
        partitions' rows, read in place (gat_attention)."""
        bias = self.bias if add_bias else None
        pad = self._padded()
        if pad:
            if sink is not None:
                raise ValueError("GATConv.attend: a padded head reads gathered rows")
            b = F.pad(bias, (0, pad)) if bias is not None else None
            y = gat_attention(self._pad_rows(hs), adj, F.pad(self.att_src, (0, pad)),
                              F.pad(self.att_dst, (0, pad)), b, 1, self.out_channels + pad,
                              self.concat, scores)
            return y[:, :self.out_channels]
        return gat_attention(hs, adj, self.att_src, self.att_dst, bias, self.heads,
                             self.out_channels, self.concat, scores, rowdot_sink, sink)

    def attend_ln(self, hs: Tensor, adj: Adjacency, norm, act: str = "elu",
                  scores: Optional[Tuple[Tensor, Tensor]] = None, sink=None,
                  dest=None) -> Tensor:
        """act(norm(attend(hs) + bias)): the layer, its bias and the LayerNorm
        and activation that follow it in GAT.forward_layer
        (grinnder/nn/gat.py:74-78).  One head of 132..1024 channels runs it as
        one pass per row (gat_attention_ln: the epilogue in the attention
        kernel); otherwise the attention and then bias_ln_act, which hands
        the attention's backward c_i.  `dest`: as bias_ln_act."""
        if self._padded() == 0 and gat_attention_ln_ok(hs, self.heads, self.out_channels,
                                                        norm.weight):
            return gat_attention_ln(hs, adj, self.att_src, self.att_dst, self.bias,
                                    norm.weight, norm.bias, norm.eps, act, scores, sink, dest)
        dot = RowDotSink()
        x = self.attend(hs, adj, add_bias=False, scores=scores, rowdot_sink=dot, sink=sink)
        return bias_ln_act(x, self.bias, norm.weight, norm.bias, norm.eps, act, dot, dest=dest)

    def project(self, x_src: Tensor, reuse: Optional[Tensor] = None,
                keep: Optional[list] = None) -> Tensor:
        """hs = lin(x_src) for a head width that needs no padding, as forward
        forms it (with reuse / keep)."""
        hs = linear(x_src, self.lin.weight, reuse=reuse)
        if keep is not None:
            keep.append(hs.detach())
        return hs

    def scores(self, hs: Tensor, packed: bool = False) -> tuple:
        """The logit halves (s, d) of every row of hs, as attend forms them
        (padding included), for callers that hold hs for many partitions.
        packed: also the packed lines a narrow head's attention over exactly
        these rows reads, (s, d, zx), when the head takes them."""
        pad = self._padded()
        if pad:
            return gat_scores(self._pad_rows(hs), F.pad(self.att_src, (0, pad)),
                              F.pad(self.att_dst, (0, pad)), 1, self.out_channels + pad,
                              hs.size(0), packed)
        return gat_scores(hs, self.att_src, self.att_dst, self.heads, self.out_channels,
                          hs.size(0), packed)

    def __repr__(self) -> str:
        return (f"{self.__class__.__name__}({self.in_channels}, {self.out_channels}, "
                f"heads={self.heads})")
