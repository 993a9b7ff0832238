"""GriNNderModel: per-layer model interface (grinnder/nn/base.py:11-74)."""

from __future__ import annotations

from abc import abstractmethod
from typing import List, Optional

import torch
from torch import Tensor


class GriNNderModel(torch.nn.Module):
    """Base class of models trained layer-wise and partition-wise by the Trainer.

    Subclasses implement ``forward_layer(layer, x, adj)`` — x holds the E
    gathered source rows of one partition ([intra | halo]); the result holds
    its B destination rows — and ``layer_dims()`` ([in, hidden..., out],
    length num_layers + 1).
    """

    def __init__(self, num_layers: int):
        super().__init__()
        self._num_layers = num_layers

    @property
    def num_layers(self) -> int:
        return self._num_layers

    @abstractmethod
    def forward_layer(self, layer: int, x: Tensor, adj) -> Tensor:
        ...

    @abstractmethod
    def layer_dims(self) -> List[int]:
        ...

    def input_projection(self, layer: int) -> Optional[Tensor]:
        """The weight W [out, in] when ``forward_layer(layer, x, adj)`` starts
        by multiplying every gathered row of x by Wᵀ, with nothing applied to x
        before, so that it equals ``forward_projected(layer, x Wᵀ, adj)``.  A
        partitioned trainer may then project each partition's own rows once
        and gather projected rows (narrower when out < in).  None when the
        layer has no such form (the default)."""
        return None

    def forward_projected(self, layer: int, z: Tensor, adj, sink=None, dest=None) -> Tensor:
        """forward_layer(layer, x, adj) given z = x Wᵀ for the W of
        input_projection(layer).  With a sink (grinnder_amd.aggregation.
        ProjectedSink; only where projected_sink_ok(layer)), z is the whole
        projected matrix of all partitions, read in place through the sink's
        global ids, and the gradient of the partition's rows is added into
        the sink's dZ.  `dest` (grinnder_amd.dense.OutputRows): a block the
        layer may write its output into, returning a view of it, when its
        last step is a fused epilogue; a model may ignore it (the caller
        then copies the output)."""
        raise NotImplementedError(f"{type(self).__name__} has no projected form of layer {layer}")

    def projected_width(self, layer: int) -> int:
        """Columns of the projected matrix Z that forward_projected(layer, ...)
        reads: the rows of input_projection(layer)'s W (the default), or more
        when the model reads Z zero-padded (the trainer then keeps the columns
        past W's rows at zero)."""
        return self.input_projection(layer).size(0)

    def projected_sink_ok(self, layer: int) -> bool:
        """Whether forward_projected(layer, ...) accepts a sink."""
        return False

    def sink_writes_whole(self, layer: int) -> bool:
        """Whether the layer's backward, given a sink whose rows are every row
        of dz once and in order (a merged layer's), may write dz instead of
        adding into it: true when that sink is the backward's only write of
        dz."""
        return False

    def projected_scores(self, layer: int, z: Tensor, whole: bool = False):
        """Per-row quantities of the projected matrix z that
        forward_projected(layer, ...) can take precomputed for a partition's
        gathered rows (its `scores` argument), formed once for all rows; None
        when the layer has none (the default).  whole: the layer then reads
        all of z in one pass (a merged layer)."""
        return None

    def draws_per_partition(self, layer: int) -> bool:
        """Whether the layer's forward draws random numbers (an active
        dropout), so that one pass over all partitions would draw other masks
        than the partition-by-partition forwards (the reference's order) and
        a partitioned trainer must not merge it.  The default: in training,
        when the model has a nonzero `dropout` attribute."""
        return self.training and float(getattr(self, "dropout", 0.0) or 0.0) > 0.0

    def inplace_ok(self, layer: int) -> bool:
        """Whether forward_inplace(layer, ...) exists and is the cheaper form
        of the layer when all partitions' input rows are in device memory
        (the default: no)."""
        return False

    def forward_inplace(self, layer: int, x: Tensor, adj, gidx: Tensor, dest=None) -> Tensor:
        """forward_layer(layer, x[rows], adj) for the partition's gathered rows,
        with x the input rows of all partitions read in place through gidx
        (the global row of each CSR edge's source); x gets no gradient.
        `dest` as in forward_projected."""
        raise NotImplementedError(f"{type(self).__name__} has no in-place form of layer {layer}")

    def forward_gathered(self, layer: int, x: Tensor, adj, reuse=None, keep=None) -> Tensor:
        """forward_layer(layer, x, adj), for a partitioned trainer that
        recomputes the layer in its backward.  A model may append to the list
        `keep` one tensor the forward forms from x (detached; e.g. its first
        product), and take that tensor back as `reuse` in the recompute, which
        runs on the same rows with the same weights and dropout masks, instead
        of forming it again; the result must not change.  The default keeps
        nothing and ignores `reuse`."""
        return self.forward_layer(layer, x, adj)
