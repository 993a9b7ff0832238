"""GCN model (grinnder/nn/gcn.py:17-76) on the HIP GCNConv."""

from __future__ import annotations

from typing import List

import torch.nn.functional as F
from torch import Tensor
from torch.nn import LayerNorm, ModuleList

from grinnder_amd.aggregation import gcn_aggregate, gcn_aggregate_ln_relu
from grinnder_amd.dense import linear, linear_ln_act
from grinnder_amd.nn.base import GriNNderModel
from grinnder_amd.nn.conv import GCNConv


class GCN(GriNNderModel):
    """Graph Convolutional Network with full-graph symmetric normalisation.

    Layer l: conv -> (LayerNorm) -> (residual when shapes match) -> ReLU ->
    dropout, except the last layer which returns the conv output.
    """

    def __init__(self, in_channels: int, hidden_channels: int, out_channels: int,
                 num_layers: int, dropout: float = 0.5, norm: bool = False,
                 residual: bool = False):
        super().__init__(num_layers)
        self.dropout = dropout
        self.residual = residual
        self.convs = ModuleList()
        self.convs.append(GCNConv(in_channels, hidden_channels, normalize=False))
        for _ in range(num_layers - 2):
            self.convs.append(GCNConv(hidden_channels, hidden_channels, normalize=False))
        self.convs.append(GCNConv(hidden_channels, out_channels, normalize=False))
        self.norms = None
        if norm:
            self.norms = ModuleList(LayerNorm(hidden_channels) for _ in range(num_layers - 1))

    def _fusable(self, layer: int, x: Tensor, adj) -> bool:
        """conv -> LayerNorm -> ReLU runs as one fused kernel when nothing else
        sits between them: no residual add, no active dropout, affine LayerNorm
        over the full feature width."""
        if self.norms is None or layer >= self.num_layers - 1 or not x.is_cuda:
            return False
        norm = self.norms[layer]
        conv = self.convs[layer]
        out_shape = (adj.sparse_sizes()[0], conv.out_channels)
        return (norm.elementwise_affine and norm.bias is not None
                and tuple(norm.normalized_shape) == (conv.out_channels,)
                and not (self.residual and tuple(x.shape) == out_shape)
                and (self.dropout == 0.0 or not self.training))

    def forward_layer(self, layer: int, x: Tensor, adj) -> Tensor:
        if self._fusable(layer, x, adj):
            conv, norm = self.convs[layer], self.norms[layer]
            if conv.aggregate_first():
                return linear_ln_act(gcn_aggregate(x, adj), conv.lin.weight, conv.bias,
                                     norm.weight, norm.bias, norm.eps, "relu")
            return gcn_aggregate_ln_relu(linear(x, conv.lin.weight), adj, conv.bias,
                                         norm.weight, norm.bias, norm.eps)
        h = self.convs[layer](x, adj)
        if layer < self.num_layers - 1:
            if self.norms is not None:
                h = self.norms[layer](h)
            if self.residual and h.shape == x.shape:
                h = h + x
            h = F.relu(h)
            h = F.dropout(h, p=self.dropout, training=self.training)
        return h

    def layer_dims(self) -> List[int]:
        return [self.convs[0].in_channels] + [c.out_channels for c in self.convs]
