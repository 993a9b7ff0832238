"""GAT model (grinnder/nn/gat.py:17-87) on the HIP GATConv."""

from __future__ import annotations

from typing import List

import torch
import torch.nn.functional as F
from torch import Tensor
from torch.nn import LayerNorm, ModuleList

from grinnder_amd.aggregation import RowDotSink
from grinnder_amd.dense import bias_ln_act
from grinnder_amd.nn.base import GriNNderModel
from grinnder_amd.nn.conv import GATConv


class GAT(GriNNderModel):
    """Graph Attention Network on bipartite partition inputs (x, x[:num_dst]).

    Layer l: dropout(x) -> GATConv -> (LayerNorm) -> ELU, except the last
    layer (one head, mean over heads, no activation).
    """

    def __init__(self, in_channels: int, hidden_channels: int, out_channels: int,
                 num_layers: int, heads: int = 8, dropout: float = 0.6, norm: bool = False):
        super().__init__(num_layers)
        self.dropout = dropout
        self.heads = heads
        self.convs = ModuleList()
        self.convs.append(GATConv(in_channels, hidden_channels, heads=heads,
                                  add_self_loops=False))
        for _ in range(num_layers - 2):
            self.convs.append(GATConv(hidden_channels * heads, hidden_channels, heads=heads,
                                      add_self_loops=False))
        self.convs.append(GATConv(hidden_channels * heads, out_channels, heads=1, concat=False,
                                  add_self_loops=False))
        self.norms = None
        if norm:
            self.norms = ModuleList(LayerNorm(hidden_channels * heads)
                                    for _ in range(num_layers - 1))

    def _fused_norm(self, layer: int, x: Tensor) -> bool:
        """The conv bias, LayerNorm and ELU can run as one pass over the
        attention output."""
        if layer >= self.num_layers - 1 or self.norms is None or not x.is_cuda:
            return False
        conv, norm = self.convs[layer], self.norms[layer]
        return (norm.elementwise_affine and norm.bias is not None
                and tuple(norm.normalized_shape) == (conv.out_channels * conv.heads,)
                and conv.concat)

    def _finish(self, layer: int, x: Tensor) -> Tensor:
        if layer < self.num_layers - 1:
            if self.norms is not None:
                x = self.norms[layer](x)
            x = F.elu(x)
        return x

    def forward_layer(self, layer: int, x: Tensor, adj) -> Tensor:
        return self.forward_gathered(layer, x, adj)

    def forward_gathered(self, layer: int, x: Tensor, adj, reuse=None, keep=None) -> Tensor:
        """forward_layer, with GATConv's projection of the (dropped-out) input
        rows appended to `keep`, or taken from `reuse` instead of recomputed
        (a recompute from the same rows, weights and dropout mask)."""
        x = F.dropout(x, p=self.dropout, training=self.training)
        num_dst = adj.sparse_sizes()[0]
        conv = self.convs[layer]
        if self._fused_norm(layer, x):
            norm = self.norms[layer]
            if conv._padded() == 0:
                hs = conv.project(x, reuse=reuse, keep=keep)
                return conv.attend_ln(hs, adj, norm)
            sink = RowDotSink()
            x = conv((x, x[:num_dst]), adj, add_bias=False, reuse=reuse, keep=keep,
                     rowdot_sink=sink)
            return bias_ln_act(x, conv.bias, norm.weight, norm.bias, norm.eps, "elu", sink)
        return self._finish(layer, conv((x, x[:num_dst]), adj, reuse=reuse, keep=keep))

    def input_projection(self, layer: int):
        """GATConv multiplies every source row by lin first; the dropout before
        it must be inactive."""
        if self.dropout != 0.0 and self.training:
            return None
        return self.convs[layer].lin.weight

    def projected_width(self, layer: int) -> int:
        """One head of C channels, C not a multiple of 4, is held C rounded up
        to 4 wide, the width its attention runs at (GATConv pads it): gathered
        rows need no padding copy, and dZ's 16-byte rows take the matrix-core
        dX product.  The pad columns of Z are zero."""
        conv = self.convs[layer]
        return conv.heads * conv.out_channels + conv._padded()

    def projected_sink_ok(self, layer: int) -> bool:
        """Z read in place for one head of 68..1024 channels (a multiple of
        4): the attention gathers each edge's source row of Z directly and
        its backward adds dZ in place, instead of a gather of the
        partition's rows before it and a scatter of their gradient after
        (at C5's 256-wide layer 0.44 ms of a partition's 1.6 ms).  Narrower
        layers gather: their rows are cheap to copy and stay in the caches."""
        conv = self.convs[layer]
        c = conv.out_channels
        return conv.heads == 1 and c % 4 == 0 and 64 < c <= 1024

    def forward_projected(self, layer: int, hs: Tensor, adj, sink=None,
                          scores=None, dest=None) -> Tensor:
        """The layer on hs = lin(x): the partition's gathered rows, or with
        `sink` the matrix of all partitions' rows read in place (then
        `scores` are the logit halves of all rows and of the partition's
        destination rows)."""
        if sink is not None and not self.projected_sink_ok(layer):
            raise ValueError(f"layer {layer} reads gathered rows; it takes no sink")
        conv = self.convs[layer]
        if self._fused_norm(layer, hs):
            return conv.attend_ln(hs, adj, self.norms[layer], scores=scores, sink=sink,
                                  dest=dest)
        return self._finish(layer, conv.attend(hs, adj, scores=scores, sink=sink))

    def projected_scores(self, layer: int, z: Tensor, whole: bool = False):
        """The attention logit halves of every row of the projected matrix z,
        formed once for all partitions (no autograd: the attention-vector
        gradients come from the attention's own backward).  whole: the
        attention reads all of z at once (a merged layer), so a narrow head
        also gets z's packed lines (GATConv.scores)."""
        with torch.no_grad():
            return self.convs[layer].scores(z, packed=whole)

    def layer_dims(self) -> List[int]:
        dims = [self.convs[0].in_channels]
        for i, conv in enumerate(self.convs):
            if i < len(self.convs) - 1:
                dims.append(conv.out_channels * conv.heads)
            else:
                dims.append(conv.out_channels)
        return dims
