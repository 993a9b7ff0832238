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

    def forward_projected(self, layer: int, hs: Tensor, adj, sink=None,
                          scores=None) -> Tensor:
        if sink is not None:
            raise ValueError("GAT layers read gathered rows; they take no sink")
        conv = self.convs[layer]
        if self._fused_norm(layer, hs):
            norm = self.norms[layer]
            sink = RowDotSink()
            x = conv.attend(hs, adj, add_bias=False, scores=scores, rowdot_sink=sink)
            return bias_ln_act(x, conv.bias, norm.weight, norm.bias, norm.eps, "elu", sink)
        return self._finish(layer, conv.attend(hs, adj, scores=scores))

    def projected_scores(self, layer: int, z: Tensor):
        """The attention logit halves of every row of the projected matrix z,
        formed once for all partitions (no autograd: the attention-vector
        gradients come from the attention's own backward)."""
        with torch.no_grad():
            return self.convs[layer].scores(z)

    def layer_dims(self) -> List[int]:
        dims = [self.convs[0].in_channels]
        for i, conv in enumerate(self.convs):
            if i < len(self.convs) - 1:
                dims.append(conv.out_channels * conv.heads)
            else:
                dims.append(conv.out_channels)
        return dims
