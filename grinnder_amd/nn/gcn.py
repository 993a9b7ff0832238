"""GCN model (grinnder/nn/gcn.py:17-76) on the HIP GCNConv."""

from __future__ import annotations

from typing import List

import torch.nn.functional as F
from torch import Tensor
from torch.nn import LayerNorm, ModuleList

from grinnder_amd.aggregation import ProjectedSink, gcn_aggregate, gcn_aggregate_ln_relu
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

    def _fusable_norm(self, layer: int, x: Tensor) -> bool:
        """conv -> LayerNorm -> ReLU can run as one fused kernel: affine
        LayerNorm over the full feature width, no active dropout after it."""
        if self.norms is None or layer >= self.num_layers - 1 or not x.is_cuda:
            return False
        norm = self.norms[layer]
        conv = self.convs[layer]
        return (norm.elementwise_affine and norm.bias is not None
                and tuple(norm.normalized_shape) == (conv.out_channels,)
                and (self.dropout == 0.0 or not self.training))

    def _fusable(self, layer: int, x: Tensor, adj) -> bool:
        """As _fusable_norm, and no residual add between the conv and the LayerNorm."""
        out_shape = (adj.sparse_sizes()[0], self.convs[layer].out_channels)
        return (self._fusable_norm(layer, x)
                and not (self.residual and tuple(x.shape) == out_shape))

    def input_projection(self, layer: int):
        """GCNConv computes A (x Wᵀ) + b (in the order PyG uses; an
        aggregate-first layer's (A x) Wᵀ + b is the same function), and
        dropout acts on layer outputs, so x enters only through x Wᵀ - unless
        the residual add needs x itself (in == out)."""
        conv = self.convs[layer]
        if self.residual and conv.in_channels == conv.out_channels:
            return None
        return conv.lin.weight

    def projected_width(self, layer: int) -> int:
        """Z rounded up to a multiple of 4 columns (16-byte rows; the pad
        columns are zero), so that gathered rows of Z need no padding copy."""
        d = self.convs[layer].out_channels
        return d + (-d) % 4

    def projected_sink_ok(self, layer: int) -> bool:
        """Z read in place for widths that are multiples of 4.  A narrower,
        padded layer gathers its rows: at C3 the 48-wide Z (470 MB) read in
        place over the whole graph cost more than gathering each partition's
        rows into a compact copy that stays in the caches."""
        return self.convs[layer].out_channels % 4 == 0

    def sink_writes_whole(self, layer: int) -> bool:
        """The aggregation's backward is the only write of dz."""
        return True

    def inplace_ok(self, layer: int) -> bool:
        """The first layer, when it aggregates first (it widens): (A x) Wᵀ
        aggregates the narrower input, and its input needs no gradient."""
        conv = self.convs[layer]
        return (layer == 0 and conv.aggregate_first()
                and not (self.residual and conv.in_channels == conv.out_channels))

    def forward_inplace(self, layer: int, x: Tensor, adj, gidx: Tensor, dest=None) -> Tensor:
        if not self.inplace_ok(layer):
            raise ValueError(f"layer {layer} has no in-place form")
        conv = self.convs[layer]
        h = gcn_aggregate(x, adj, sink=ProjectedSink(None, gidx))
        if self._fusable_norm(layer, x):
            norm = self.norms[layer]
            return linear_ln_act(h, conv.lin.weight, conv.bias, norm.weight, norm.bias,
                                 norm.eps, "relu", dest=dest)
        h = linear(h, conv.lin.weight, conv.bias)
        if layer < self.num_layers - 1:
            if self.norms is not None:
                h = self.norms[layer](h)
            h = F.relu(h)
            h = F.dropout(h, p=self.dropout, training=self.training)
        return h

    def draws_per_partition(self, layer: int) -> bool:
        # Dropout acts on the outputs of the layers below the last.
        return (self.training and self.dropout > 0.0
                and layer < self.num_layers - 1)

    def forward_projected(self, layer: int, z: Tensor, adj, sink=None, dest=None) -> Tensor:
        conv = self.convs[layer]
        d = conv.out_channels
        w = z.size(1)
        if w != d:
            # Z zero-padded to w columns (projected_width): aggregate all of
            # them (16-byte rows) with the bias padded alike; the pad columns
            # of the output are zero and are dropped.
            if w < d or w % 4 != 0:
                raise ValueError(f"layer {layer}: Z has {w} columns for a width of {d}")
            b = F.pad(conv.bias, (0, w - d)) if conv.bias is not None else None
            h = gcn_aggregate(z, adj, b, sink=sink)[:, :d]
        elif sink is not None and d % 4 != 0:
            raise ValueError(f"layer {layer}: a sink needs an output width divisible by 4")
        elif d % 4 != 0:
            # Widths that are not a multiple of 4 aggregate zero-padded rows
            # (16-byte vectors), as GCNConv does; the pad column stays zero.
            pad = (-d) % 4
            b = F.pad(conv.bias, (0, pad)) if conv.bias is not None else None
            h = gcn_aggregate(F.pad(z, (0, pad)), adj, b)[:, :d]
        elif self._fusable_norm(layer, z):
            norm = self.norms[layer]
            return gcn_aggregate_ln_relu(z, adj, conv.bias, norm.weight, norm.bias, norm.eps,
                                         sink=sink, dest=dest)
        else:
            h = gcn_aggregate(z, adj, conv.bias, sink=sink)
        if layer < self.num_layers - 1:
            if self.norms is not None:
                h = self.norms[layer](h)
            h = F.relu(h)
            h = F.dropout(h, p=self.dropout, training=self.training)
        return h

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
