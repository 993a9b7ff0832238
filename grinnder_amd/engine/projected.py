"""Projected layers of the partitioned Trainer (grinnder_amd.engine.trainer).

Mixin of Trainer: planning (which layers run projected, in place or
gathered from HBM, which inputs and forward graphs stay in HBM, the layer-0
double buffer), the device buffers Z, dZ, resident inputs and their
gradients, the per-partition forward and backward of those layers, and the
layer-0 uploads.  The
trainer's module docstring describes the flow; the reference has no
counterpart (its trainer gathers every layer's input rows from the host,
grinnder/engine/trainer.py:477-1138).
"""

from __future__ import annotations

from typing import Dict, List, Optional, Set

import torch
from torch import Tensor

from grinnder_amd.aggregation import (KernelTimer, LNProductSink, ProjectedSink, dense_region,
                                      gather_rows, scatter_add_rows)
from grinnder_amd.dense import OutputRows, gemm_nt, gemm_tn
from grinnder_amd.loss import masked_cross_entropy
from grinnder_amd.utils import get_available_host_memory


class _GatherRows(torch.autograd.Function):
    """z = Z[rows] of an HBM-resident matrix Z (a projected layer's Z, or a
    gathered layer's input rows); the backward adds dL/dz into Z's gradient
    buffer dz at the same rows (distinct within a partition) instead of
    returning a gradient for Z.  `token` is a zero-element tensor that
    requires grad, so that autograd records the gather although Z does not."""

    @staticmethod
    def forward(ctx, token: Tensor, z: Tensor, rows: Tensor, dz: Tensor) -> Tensor:
        ctx.rows, ctx.dz = rows, dz
        return gather_rows(z, rows)

    @staticmethod
    def backward(ctx, grad: Tensor):
        d = grad.size(1)
        with KernelTimer.region("row_scatter_add", 3 * 4 * grad.size(0) * d, 0, d):
            scatter_add_rows(grad, ctx.rows, ctx.dz)
        return None, None, None, None


class _WholeRows(torch.autograd.Function):
    """Z itself as the source rows of a merged layer (every partition in one
    pass: the whole graph's adjacency indexes Z's global rows directly); the
    backward adds dL/dZ into Z's gradient buffer dz.  `token` as in
    _GatherRows."""

    @staticmethod
    def forward(ctx, token: Tensor, z: Tensor, dz: Tensor) -> Tensor:
        ctx.dz = dz
        return z.view_as(z)

    @staticmethod
    def backward(ctx, grad: Tensor):
        ctx.dz.add_(grad)
        return None, None, None


class ProjectedLayers:
    """Projected-layer machinery of Trainer (a mixin: it uses the trainer's
    graph, config, model, streams and host / device buffers)."""

    def _init_projected(self) -> None:
        # Projected layers: their W this epoch; Z, dZ per layer, two upload
        # buffers per input width and the HBM-resident inputs, kept across
        # epochs; the layers whose inputs stay in HBM this epoch; the device
        # row ids of each partition's gathered rows.
        self._proj: Dict[int, Tensor] = {}
        self._zbufs: Dict[int, Tensor] = {}
        self._dzbufs: Dict[int, Tensor] = {}
        self._xbufs: Dict[int, List[Tensor]] = {}
        self._xres: Dict[int, Tensor] = {}
        self._xin: Set[int] = set()
        self._grow: Dict[int, Tensor] = {}
        # Projected layers whose forward graphs are kept until their backward
        # this epoch (instead of being recomputed), the kept outputs, and the
        # RNG state each recomputed partition's forward started from.
        self._keep: Set[int] = set()
        self._graphs: Dict[int, Dict[int, Tensor]] = {}
        self._rng: Dict[tuple, Tensor] = {}
        self._token: Optional[Tensor] = None
        self._gsrc: Dict[int, tuple] = {}
        # Layers that read their resident input rows in place this epoch
        # (model.forward_inplace), in place of running projected.
        self._inplace: Set[int] = set()
        # Layer 0's resident input rows are double-buffered across epochs when
        # there is room: the next epoch's rows stream into the other buffer
        # (on streams of their own) while this epoch computes.
        self._x0bufs: List[Tensor] = []
        self._x0cur = 0
        self._x0double = False
        self._x0pending: Optional[tuple] = None
        # input_residency 'resident': the index of the buffer that holds the
        # layer-0 rows already (uploaded in an earlier epoch), else -1.
        self._x0loaded = -1
        self._pf_streams: List[torch.cuda.Stream] = []
        # Per-row quantities of each projected layer's Z formed once for all
        # partitions this epoch (GAT's attention scores), by layer.
        self._scores: Dict[int, tuple] = {}
        # W padded with zero rows to Z's width, per projected layer whose Z is
        # wider than W's rows (formed once per epoch: W changes between).
        self._wpad: Dict[int, Tensor] = {}
        self._wtdx: Dict[int, Tensor] = {}
        # HBM buffers of dL/dx for the gathered layers above layer 0 (layers
        # in self._xin that run neither projected nor in place), by layer.
        self._gxbufs: Dict[int, Tensor] = {}
        # Whether HBM has room this epoch for the logits of every partition
        # (self._xres[num_layers]); see _logits_on_device.
        self._out_room = False
        # What a gathered layer's forward kept for its recompute
        # (model.forward_gathered), by (layer, pid), and the bytes still free
        # for that this epoch.
        self._gkept: Dict[tuple, Tensor] = {}
        self._gkept_left = 0
        # Layers that run merged this epoch (every partition in one pass over
        # the whole graph's adjacency), whether HBM has room for that
        # adjacency's plan, the last layer's merged output (with its graph
        # when training) until the loss and backward take it, and the whole
        # adjacency's device row ids.
        self._merged: Set[int] = set()
        self._merge_room = False
        self._merged_out: Optional[Tensor] = None
        self._wids: Optional[tuple] = None

    @property
    def projected(self) -> bool:
        """Whether the current epoch runs any layer on projected rows."""
        return bool(self._proj)

    @property
    def projected_layers(self) -> List[int]:
        return sorted(self._proj)

    @property
    def resident_inputs(self) -> List[int]:
        """Layers whose input rows stay in HBM this epoch."""
        return sorted(self._xin)

    @property
    def gathered_layers(self) -> List[int]:
        """Layers that run the reference's per-partition forward this epoch
        (no input projection) on input rows gathered from HBM: their input
        rows stay there, and so does the gradient of those above layer 0."""
        return sorted(self._gathered())

    def _gathered(self) -> Set[int]:
        return {l for l in self._xin if l not in self._proj and l not in self._inplace}

    def _device_flow(self, layer: int) -> bool:
        """Whether layer `layer` runs this epoch without host buffers:
        projected, in place or gathered from HBM."""
        return layer in self._proj or layer in self._inplace or layer in self._xin

    def _grad_on_device(self, layer: int) -> bool:
        """Whether dL/d(x_layer) of every partition is in HBM once layer
        `layer`'s backward is done (projected: dZ W; gathered: its buffer)."""
        return layer in self._proj or (layer in self._xin and layer not in self._inplace)

    def _logits_on_device(self) -> bool:
        """Whether the last layer's outputs go to an HBM buffer for the loss
        this epoch instead of a D2H and an upload per partition: when that
        layer runs without host buffers and keeps no forward graphs (kept
        graphs hold the logits already).  Besides the two transfers, this
        keeps the forward off the copy engines while the next epoch's layer-0
        rows stream in: a D2H queued behind that upload waits for all of it."""
        last = self.model.num_layers - 1
        return self._out_room and self._device_flow(last) and last not in self._keep

    def _free_device_memory(self) -> int:
        """Bytes new tensors can take: the device's free memory plus the
        blocks torch's caching allocator holds unused (an earlier epoch's
        kept graphs and temporaries, which the allocator hands out again)."""
        free, _ = torch.cuda.mem_get_info(self.device)
        return free + torch.cuda.memory_reserved(self.device) - torch.cuda.memory_allocated(self.device)

    def _plan_projection(self) -> Dict[int, Tensor]:
        """Layers this epoch runs projected, with their input projection W:
        grinnder mode, every partition on this trainer, and room in HBM for
        Z, dZ and the upload buffers (plus 8 GiB for the per-partition
        working set).  A projected layer moves at most two N d_in uploads of
        its input rows over the host link (one, or none above layer 0, when
        they stay in HBM) instead of 2 E d_in of gathers and, above layer 0,
        an E d_in read-add-write scatter; when HBM is short, layers with the
        most input width per byte of Z go first.

        Also decides self._xin, with what room is left: the projected layers
        whose input rows x stay in HBM for the epoch.  Above layer 0, x is
        produced on the device by the layer below, so neither its D2H nor the
        upload for dW = sum_p dZ_pᵀ x_p crosses the host link; layer 0's rows
        are uploaded once per epoch, for the projection, and kept for dW
        instead of being uploaded a second time.  Layers above 0 go first
        (each of their bytes saves two crossings).  Then, with what room is
        still left, the gathered layers (added to self._xin): layers without
        an input projection whose input rows (and, above layer 0, their
        gradient) stay in HBM.  Then self._keep: the
        layers whose per-partition forward graphs are kept for the backward
        (training only)."""
        cfg, g = self.config, self.graph
        self._xin = set()
        self._keep = set()
        self._out_room = False
        self._merge_room = False
        self._wpad = {}
        self._wtdx = {}
        if (self._fast or cfg.mode != "grinnder" or cfg.project_first == "off"
                or self.cache is not None
                or (self._pid_start, self._pid_end) != (0, g.num_parts)):
            self._x0double = False
            self._drop_prefetch()
            return {}
        n, maxb = int(g.ptr[-1]), max(g.partition_sizes)
        cands = []
        for layer in range(self.model.num_layers):
            w = self.model.input_projection(layer)
            if w is not None:
                cands.append((w.size(1) / w.size(0), layer, w))
        free = None
        plan: Dict[int, Tensor] = {}
        for _, layer, w in sorted(cands, key=lambda c: (-c[0], c[1])):
            if layer not in self._zbufs:
                if free is None:
                    free = self._free_device_memory()
                need = 4 * (2 * n * self.model.projected_width(layer) + 2 * maxb * w.size(1))
                if need + (8 << 30) > free:
                    continue
                free -= need
            plan[layer] = w
        for layer in sorted(plan, key=lambda l: (l == 0, l)):
            if layer not in self._xres:
                if free is None:
                    free = self._free_device_memory()
                need = 4 * n * plan[layer].size(1)
                if need + (8 << 30) > free:
                    continue
                free -= need
            self._xin.add(layer)
        # Gathered layers: a layer with no input projection (GAT with active
        # input dropout, a model without one) runs the reference's
        # per-partition forward, but with its input rows kept in HBM when
        # there is room: each partition gathers its rows there, and the
        # backward adds dL/dx into an HBM buffer (above layer 0) instead of a
        # host read-add-write over the link.  Layers above 0 first (their
        # rows would cross the link four times, layer 0's twice).
        for layer in sorted((l for l in range(self.model.num_layers) if l not in plan),
                            key=lambda l: (l == 0, l)):
            din = self.host_features[layer].embedding_dim
            need = 0
            if layer not in self._xres:
                need += 4 * n * din
            if layer > 0 and layer not in self._gxbufs:
                need += 4 * n * din
            if need:
                if free is None:
                    free = self._free_device_memory()
                if need + (8 << 30) > free:
                    continue
                free -= need
            self._xin.add(layer)
        # Kept forward graphs (training only): a projected layer whose output
        # feeds a resident input, or the last layer, keeps each partition's
        # autograd graph until its backward, which then skips the recompute
        # (an aggregation pass and a gather of Z per partition); the last
        # layer's loss is then taken from the kept logits, which no longer
        # go through host memory.  What a graph holds is bounded by the
        # gathered rows, three [N, d_out] tensors and one float per edge.
        self._keep = set()
        if self.model.training:
            sum_e = sum(g.expanded_sizes)
            nnz = sum(int(a[1].numel()) for a in g.adj_csr)
            last = self.model.num_layers - 1
            for layer in sorted(plan):
                if layer + 1 not in self._xin and layer != last:
                    continue
                d = plan[layer].size(0)
                if free is None:
                    free = self._free_device_memory()
                need = 4 * (sum_e * d + 3 * n * d + nnz)
                if need + (8 << 30) > free:
                    continue
                free -= need
                self._keep.add(layer)
        # Room for the whole graph's adjacency, which merged layers run on
        # (_plan_merged): its device plan takes about 24 bytes an edge and 32
        # a node beside the partitions' plans, and its int32 edge and row ids
        # bound the graph to 2^31 - 1 edges.  A merged layer's graph holds no
        # more than the P kept graphs it replaces.
        self._merge_room = False
        nnz_all = sum(int(a[1].numel()) for a in g.adj_csr)
        if cfg.merge_partitions != "off" and nnz_all < 2 ** 31 - 1:
            whole = g._whole
            if whole is not None and whole.has_device_plan(self.device):
                self._merge_room = True
            else:
                need = 24 * nnz_all + 32 * n
                if free is None:
                    free = self._free_device_memory()
                # Host side: the whole adjacency keeps int64 row pointers and
                # column ids and fp32 values (20 bytes an edge) for the
                # graph's lifetime, and building its device plan briefly
                # needs about as much again for the transpose.
                host_need = 48 * nnz_all + 32 * n
                if (need + (8 << 30) <= free
                        and host_need + (4 << 30) <= get_available_host_memory()):
                    free -= need
                    self._merge_room = True
        # A second copy of layer 0's input rows for the next epoch's upload to
        # stream into while this epoch computes.
        self._x0double = False
        if 0 in self._xin and cfg.input_residency == "stream":
            if len(self._x0bufs) >= 2:
                self._x0double = True
            else:
                if free is None:
                    free = self._free_device_memory()
                need = 4 * n * self.host_features[0].embedding_dim
                if need + (8 << 30) <= free:
                    free -= need
                    self._x0double = True
        if not self._x0double:
            self._drop_prefetch()
        # Room for the logits of every partition (used when the last layer
        # runs without host buffers; see _logits_on_device).
        nl = self.model.num_layers
        self._out_room = nl in self._xres
        if not self._out_room:
            if free is None:
                free = self._free_device_memory()
            need = 4 * n * self.host_features[nl].embedding_dim
            self._out_room = need + (8 << 30) <= free
            if self._out_room:
                free -= need
        # What is left (training with gathered layers): what their forwards
        # keep for the recompute, partition by partition while it fits.
        self._gkept = {}
        self._gkept_left = 0
        if self.model.training and any(l not in plan for l in self._xin):
            if free is None:
                free = self._free_device_memory()
            self._gkept_left = max(0, free - (8 << 30))
        return dict(sorted(plan.items()))

    def _plan_inplace(self) -> None:
        """Moves a planned layer from projected to in place when its input
        rows stay in HBM this epoch and the model has a cheaper in-place form
        (GCN's widening first layer aggregates its narrower input, and the
        input needs no gradient): no Z, dZ or dW pass for it then."""
        self._inplace = set()
        for layer in sorted(self._proj):
            if layer in self._xin and self.model.inplace_ok(layer) \
                    and int(self.graph.ptr[-1]) < 2 ** 31:
                self._inplace.add(layer)
        for layer in self._inplace:
            del self._proj[layer]
        self._merged = self._plan_merged()

    def _plan_merged(self) -> Set[int]:
        """The layers that run merged this epoch (config.merge_partitions):
        projected or in place, with their graph kept when training (one
        backward, no recompute), drawing no random numbers (dropout masks
        stay those of the partition-by-partition order), and, below the last
        layer, with their output and its gradient in HBM (the next layer's
        input resident, its gradient dZ·W or an HBM buffer)."""
        mode = self.config.merge_partitions
        if not self._merge_room or mode == "off":
            return set()
        last = self.model.num_layers - 1
        merged = set()
        for layer in range(self.model.num_layers):
            if mode == "last" and layer != last:
                continue
            if layer not in self._proj and layer not in self._inplace:
                continue
            if self.model.training and layer not in self._keep:
                continue
            if self.model.draws_per_partition(layer):
                continue
            if layer != last and not (layer + 1 in self._xin
                                      and self._grad_on_device(layer + 1)):
                continue
            merged.add(layer)
        return merged

    @property
    def merged_layers(self) -> List[int]:
        """Layers that run merged this epoch (one pass over the whole graph)."""
        return sorted(self._merged)

    @property
    def inplace_layers(self) -> List[int]:
        """Layers that read their HBM-resident input rows in place this epoch."""
        return sorted(self._inplace)

    def _xres_buf(self, layer: int) -> Tensor:
        """HBM copy of layer `layer`'s input rows (all partitions, in order)."""
        x = self._xres.get(layer)
        if x is None:
            with torch.cuda.stream(self.streams.compute):
                x = torch.empty(int(self.graph.ptr[-1]), self.host_features[layer].embedding_dim,
                                device=self.device)
            self._xres[layer] = x
        return x

    def _gxbuf(self, layer: int) -> Tensor:
        """HBM buffer of dL/dx for a gathered layer's input rows."""
        gx = self._gxbufs.get(layer)
        if gx is None:
            with torch.cuda.stream(self.streams.compute):
                gx = torch.empty(int(self.graph.ptr[-1]), self.host_features[layer].embedding_dim,
                                 device=self.device)
            self._gxbufs[layer] = gx
        return gx

    def _zbuf(self, layer: int) -> Tensor:
        """Z of a projected layer, [N, model.projected_width(layer)]: the
        columns past W's rows (zero padding the model reads) stay zero."""
        z = self._zbufs.get(layer)
        if z is None:
            with torch.cuda.stream(self.streams.compute):
                z = torch.empty(int(self.graph.ptr[-1]), self.model.projected_width(layer),
                                device=self.device)
            self._zbufs[layer] = z
        return z

    def _dzbuf(self, layer: int) -> Tensor:
        dz = self._dzbufs.get(layer)
        if dz is None:
            with torch.cuda.stream(self.streams.compute):
                dz = torch.empty_like(self._zbuf(layer))
            self._dzbufs[layer] = dz
        return dz

    def _global_rows(self, pid: int) -> Tensor:
        """Device int64 ids (in partition order) of partition pid's gathered
        rows, laid out [intra | halo from p' = 0..P-1] like the host gather."""
        idx = self._grow.get(pid)
        if idx is None:
            idx = self.graph.gathered_rows(pid).to(self.device)
            self._grow[pid] = idx
        return idx

    def _gather_projected(self, layer: int, pid: int, grad: bool = False) -> Tensor:
        """Partition pid's gathered rows of Z_layer; with grad, the backward
        adds their gradient into dZ_layer."""
        return self._gather_rows("z_gather", pid, self._zbufs[layer],
                                 self._dzbuf(layer) if grad else None)

    def _gather_rows(self, name: str, pid: int, z: Tensor, dz: Optional[Tensor]) -> Tensor:
        """Partition pid's gathered rows of the HBM matrix z; with dz, the
        backward adds their gradient into dz."""
        rows = self._global_rows(pid)
        d = z.size(1)
        with KernelTimer.region(name, 2 * 4 * rows.numel() * d, 0, d):
            if dz is None:
                return gather_rows(z, rows)
            if self._token is None:
                self._token = torch.zeros(0, device=self.device, requires_grad=True)
            return _GatherRows.apply(self._token, z, rows, dz)

    def _gids(self, pid: int) -> tuple:
        """(global row of each CSR edge's source, global row of each gathered
        row) of partition pid, int32 on the device, cached."""
        ids = self._gsrc.get(pid)
        if ids is None:
            rows = self._global_rows(pid)
            plan = self.graph.adjacency(pid).device_plan(self.device)
            ids = (rows[plan.idx.long()].to(torch.int32), rows.to(torch.int32))
            self._gsrc[pid] = ids
        return ids

    def _sink(self, layer: int, pid: int):
        """A ProjectedSink for partition pid of a layer whose model reads Z in
        place (projected_sink_ok), or None: the global id of each CSR edge's
        source and of each gathered row, as int32 (cached per partition)."""
        if not self.model.projected_sink_ok(layer) or int(self.graph.ptr[-1]) >= 2 ** 31:
            return None
        ids = self._gids(pid)
        if self._token is None:
            self._token = torch.zeros(0, device=self.device, requires_grad=True)
        return ProjectedSink(self._dzbuf(layer), ids[0], ids[1], self._token,
                             self.graph._range(pid)[0])

    def _device_call(self, layer: int, pid: int, grad: bool,
                     dest: Optional[OutputRows] = None) -> Tensor:
        """forward_projected on partition pid: reading Z in place through a
        sink where the model allows it, else on gathered rows of Z (whose
        gradient the gather adds into dZ when grad).  `dest`: where the
        model may put the output (projected and in-place layers)."""
        adj = self.graph.adjacency(pid)
        if layer in self._inplace:
            return self.model.forward_inplace(layer, self._xres[layer], adj, self._gids(pid)[0],
                                              dest=dest)
        if layer not in self._proj:
            # A gathered layer: the reference's forward on the partition's
            # input rows, gathered from HBM (layer 0's get no gradient).  The
            # first forward keeps what the model offers for the recompute
            # (forward_gathered) while the epoch's budget allows; the
            # recompute takes it back.
            gx = self._gxbuf(layer) if grad and layer > 0 else None
            x = self._gather_rows("x_gather", pid, self._xres[layer], gx)
            if grad:
                return self.model.forward_gathered(layer, x, adj,
                                                   reuse=self._gkept.pop((layer, pid), None))
            if not self.model.training or self._gkept_left <= 0:
                return self.model.forward_layer(layer, x, adj)
            keep: List[Tensor] = []
            out = self.model.forward_gathered(layer, x, adj, keep=keep)
            if len(keep) == 1:
                nbytes = keep[0].numel() * keep[0].element_size()
                if nbytes <= self._gkept_left:
                    self._gkept[(layer, pid)] = keep[0]
                    self._gkept_left -= nbytes
            return out
        sink = self._sink(layer, pid)
        if sink is not None:
            sc = self._scores.get(layer)
            if sc is None:
                return self.model.forward_projected(layer, self._zbufs[layer], adj, sink=sink,
                                                    dest=dest)
            lo, hi = self.graph._range(pid)
            return self.model.forward_projected(layer, self._zbufs[layer], adj, sink=sink,
                                                scores=(sc[0], sc[1][lo:hi]), dest=dest)
        z = self._gather_projected(layer, pid, grad=grad)
        sc = self._scores.get(layer)
        if sc is None:
            return self.model.forward_projected(layer, z, adj, dest=dest)
        lo, hi = self.graph._range(pid)
        s_rows = gather_rows(sc[0], self._global_rows(pid))
        return self.model.forward_projected(layer, z, adj, scores=(s_rows, sc[1][lo:hi]),
                                            dest=dest)

    def _whole_ids(self) -> tuple:
        """(global source row of each edge, global row of each source row) of
        the whole graph's adjacency, int32 on the device: its own column ids
        and 0..N-1 (cached)."""
        if self._wids is None:
            plan = self.graph.whole_adjacency().device_plan(self.device)
            n = int(self.graph.ptr[-1])
            self._wids = (plan.idx, torch.arange(n, dtype=torch.int32, device=self.device))
        return self._wids

    def _whole_sink(self, layer: int) -> bool:
        """A merged layer reads Z in place through a sink over all rows."""
        return self.model.projected_sink_ok(layer) and int(self.graph.ptr[-1]) < 2 ** 31

    def _merged_call(self, layer: int, grad: bool,
                     dest: Optional[OutputRows] = None) -> Tensor:
        """The layer's forward for every partition at once, over the whole
        graph's adjacency: in place on its resident input, or on Z itself
        (read through a sink where the model takes one, else as a tensor
        whose gradient the backward adds into dZ), with the attention scores
        of all rows where the model takes them.  `dest`: where the model may
        put the output."""
        adj = self.graph.whole_adjacency()
        if layer in self._inplace:
            return self.model.forward_inplace(layer, self._xres[layer], adj,
                                              self._whole_ids()[0], dest=dest)
        sc = self._scores.get(layer)
        extra = {} if sc is None else {"scores": sc}
        if self._token is None:
            self._token = torch.zeros(0, device=self.device, requires_grad=True)
        if self._whole_sink(layer):
            gidx, rows = self._whole_ids()
            sink = ProjectedSink(self._dzbuf(layer), gidx, rows, self._token, 0,
                                 overwrite=self.model.sink_writes_whole(layer))
            return self.model.forward_projected(layer, self._zbufs[layer], adj, sink=sink,
                                                dest=dest, **extra)
        z = self._zbufs[layer]
        if grad:
            z = _WholeRows.apply(self._token, z, self._dzbuf(layer))
        return self.model.forward_projected(layer, z, adj, dest=dest, **extra)

    def _forward_merged(self, layer: int) -> None:
        """A merged layer's forward: every partition's output in one pass,
        with its graph when training.  The last layer's output waits for the
        one loss over all rows (_compute_losses) and its backward
        (_backward_device); a lower layer's goes to the next layer's resident
        input rows (and through W into Z when that layer runs projected)."""
        last = layer == self.model.num_layers - 1
        self._prepare_layer(layer)
        training = self.model.training
        with torch.cuda.stream(self.streams.compute):
            if last:
                with torch.set_grad_enabled(training):
                    self._merged_out = self._merged_call(layer, grad=training)
                # The one pass has taken its scores (the graph keeps what its
                # backward needs).
                self._scores.pop(layer, None)
                return
            n = int(self.graph.ptr[-1])
            x_next = self._xres_buf(layer + 1)[:n]
            with torch.set_grad_enabled(training):
                out = self._merged_call(layer, grad=training, dest=OutputRows(x_next))
            self._scores.pop(layer, None)
            if training:
                self._graphs.setdefault(layer, {})[-1] = out
            if (layer + 1) in self._proj:
                self._project_rows(layer + 1, out, 0, n)
            if out.data_ptr() != x_next.data_ptr():
                with torch.no_grad():
                    x_next.copy_(out)
            for pid in self._my_pids:
                self.activations[layer][pid] = None

    def _device_forward(self, layer: int, pid: int, keep: bool,
                        dest: Optional[Tensor] = None) -> Tensor:
        """The forward of a projected layer on partition pid: with its graph
        kept for the backward (keep), else without autograd, noting the RNG
        state so that the backward's recompute draws the same dropout masks
        (as torch.utils.checkpoint does in the reference's flow).  `dest`: a
        [B, D] block the output may be written into instead of a new tensor
        (the returned tensor is then a view of it)."""
        rows = OutputRows(dest) if dest is not None else None
        if keep:
            with torch.enable_grad():
                out = self._device_call(layer, pid, grad=True, dest=rows)
            self._graphs.setdefault(layer, {})[pid] = out
            return out
        if self.model.training:
            self._rng[(layer, pid)] = torch.cuda.get_rng_state(self._device_index())
        with torch.no_grad():
            return self._device_call(layer, pid, grad=False, dest=rows).contiguous()

    def _device_index(self) -> int:
        return self.device.index if self.device.index is not None else torch.cuda.current_device()

    def _device_recompute(self, layer: int, pid: int) -> Tensor:
        """The partition's forward again, with autograd, from the RNG state
        its first forward started from; the global RNG stream is left as it
        was."""
        state = self._rng.pop((layer, pid), None)
        dev = self._device_index()
        with torch.random.fork_rng(devices=[dev]), torch.enable_grad():
            if state is not None:
                torch.cuda.set_rng_state(state, dev)
            return self._device_call(layer, pid, grad=True)

    def _project_rows(self, layer: int, x: Tensor, lo: int, hi: int) -> None:
        """Z_layer[lo:hi] = x Wᵀ (no autograd); with Z wider than W's rows,
        through W padded with zero rows, which writes the pad columns' zeros."""
        z = self._zbuf(layer)
        w = self._padded_weight(layer, z.size(1))
        with torch.no_grad(), dense_region("fwd", hi - lo, w.size(1), w.size(0)):
            gemm_nt(x.detach(), w, out=z[lo:hi])

    def _each_input_partition(self, layer: int, fn, whole=None) -> None:
        """fn(pid, x_p, lo, hi) on the compute stream for every partition,
        x_p = the partition's rows of the host buffer of layer `layer`'s
        inputs, uploaded to HBM: into the layer's resident input buffer when
        it has one this epoch, else through two buffers, so that the next
        upload overlaps fn.  `whole(x)`, when given, does the same work for
        all rows at once; it runs instead when every row is already in HBM."""
        g, s, pids = self.graph, self.streams, self._my_pids
        host = self.host_features[layer]
        din = host.embedding_dim
        if layer in self._xin:
            self._upload_resident(layer, fn, whole)
            return
        bufs = self._xbufs.get(din)
        if bufs is None:
            with torch.cuda.stream(s.compute):
                bufs = [torch.empty(max(g.partition_sizes), din, device=self.device)
                        for _ in range(2)]
            self._xbufs[din] = bufs
        # The first upload into each buffer waits for the compute stream's
        # queued work: a buffer allocated just now may occupy memory that
        # queued compute kernels still read (the caching allocator reuses a
        # block as soon as its stream has queued the last use), and a cached
        # one may still be read by the previous call's last fn.
        entry = torch.cuda.Event()
        entry.record(s.compute)
        freed: List[torch.cuda.Event] = [entry, entry]

        def upload(i: int) -> torch.cuda.Event:
            k, pid = i % 2, pids[i]
            b = g.partition_sizes[pid]
            st = s.h2d[k % len(s.h2d)]
            st.wait_event(freed[k])
            with torch.cuda.stream(st):
                with KernelTimer.region("x_upload", 4 * b * din, 0, din):
                    bufs[k][:b].copy_(host[pid], non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(st)
            return ev

        ready = upload(0)
        for i, pid in enumerate(pids):
            k = i % 2
            nxt = upload(i + 1) if i + 1 < len(pids) else None
            s.compute.wait_event(ready)
            with torch.cuda.stream(s.compute):
                lo, hi = g._range(pid)
                fn(pid, bufs[k][:hi - lo], lo, hi)
                ev = torch.cuda.Event()
                ev.record(s.compute)
                freed[k] = ev
            ready = nxt

    def _upload_resident(self, layer: int, fn, whole=None) -> None:
        """_each_input_partition for layer 0's resident input buffer: every
        partition has its own rows there, so fn(p) waits only for partition
        p's upload.  The rows come from the upload the previous epoch started
        into this buffer when there is one, else from one started now; with
        two buffers, the next epoch's upload then starts into the other."""
        if layer != 0:
            raise ValueError("only layer 0's input rows are uploaded to a resident buffer")
        g, s, pids = self.graph, self.streams, self._my_pids
        resident = self.config.input_residency == "resident"
        if self._x0pending is not None:
            idx, ready = self._x0pending
            self._x0pending = None
        elif resident and self._x0loaded == self._x0cur:
            # Uploaded in an earlier epoch; compute work is ordered after it.
            idx, ready = self._x0cur, None
        else:
            idx = self._x0cur
            ready = self._issue_layer0_upload(idx)
        self._x0cur = idx
        if resident:
            self._x0loaded = idx
        x = self._xres[0] = self._x0bufs[idx]
        if ready is None and whole is not None and len(pids) == g.num_parts:
            # Every row is in HBM already: one call over all partitions'
            # rows (contiguous in partition order) instead of one per
            # partition, whose last partial wave of workgroups each launch
            # would pay.
            with torch.cuda.stream(s.compute):
                whole(x)
        else:
            self._each_resident_partition(x, ready, fn)
        if self._x0double:
            self._x0pending = (1 - idx, self._issue_layer0_upload(1 - idx))

    def _each_resident_partition(self, x: Tensor, ready, fn) -> None:
        g, s, pids = self.graph, self.streams, self._my_pids
        for i, pid in enumerate(pids):
            if ready is not None:
                s.compute.wait_event(ready[i])
            with torch.cuda.stream(s.compute):
                lo, hi = g._range(pid)
                fn(pid, x[lo:hi], lo, hi)

    def _issue_layer0_upload(self, idx: int) -> List[torch.cuda.Event]:
        """Starts uploading every partition's layer-0 input rows into buffer
        idx on the two prefetch streams; returns each partition's ready event.
        The uploads first wait for the compute stream's queued work: the
        buffer may be new (its memory just freed by queued compute work) or
        still read by an earlier epoch."""
        g, s, pids = self.graph, self.streams, self._my_pids
        host = self.host_features[0]
        n, din = int(g.ptr[-1]), host.embedding_dim
        while len(self._x0bufs) <= idx:
            with torch.cuda.stream(s.compute):
                self._x0bufs.append(torch.empty(n, din, device=self.device))
        x = self._x0bufs[idx]
        if not self._pf_streams:
            self._pf_streams = [torch.cuda.Stream(self.device) for _ in range(2)]
        entry = torch.cuda.Event()
        entry.record(s.compute)
        for st in self._pf_streams:
            st.wait_event(entry)
            x.record_stream(st)
        ready: List[torch.cuda.Event] = []
        for i, pid in enumerate(pids):
            lo, hi = g._range(pid)
            st = self._pf_streams[i % 2]
            with torch.cuda.stream(st):
                with KernelTimer.region("x_upload", 4 * (hi - lo) * din, 0, din):
                    x[lo:hi].copy_(host[pid], non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(st)
            ready.append(ev)
        return ready

    def _drop_prefetch(self) -> None:
        """Forgets an upload started for an epoch that will not use it; later
        compute work (and uploads, which wait for it) is ordered after it."""
        if self._x0pending is not None:
            for ev in self._x0pending[1]:
                self.streams.compute.wait_event(ev)
            self._x0pending = None

    def _device_grad(self, layer: int, pid: Optional[int],
                     consumer: Optional[Tensor] = None) -> Tensor:
        """dL/d(x_layer) of partition pid's rows (pid None: of all rows, for a
        merged layer below) when layer `layer` keeps that
        gradient in HBM: dZ_layer[rows] W when it runs projected, else (a
        gathered layer) its rows of the layer's dL/dx buffer.  The halo
        contributions of every partition are already summed in either.
        `consumer`: the layer output this gradient is for; when it is a fused
        LayerNorm output that accepts the gradient as a product (narrow W),
        dZ and W go to its backward (LNProductSink) and the returned tensor is
        the token that tells it so."""
        lo, hi = self.graph._range(pid) if pid is not None else (0, int(self.graph.ptr[-1]))
        if layer not in self._proj:
            return self._gxbufs[layer][lo:hi]
        w = self._proj[layer]
        dz = self._dzbufs[layer][lo:hi]
        if consumer is not None:
            wp = self._padded_weight(layer, dz.size(1))
            ln_sink = LNProductSink.accepts(consumer, wp)
            if ln_sink is not None:
                return ln_sink.hand_over(dz, wp, consumer.shape)
        with dense_region("dx", hi - lo, w.size(0), w.size(1)):
            return gemm_nt(dz, self._dx_weight(layer, dz.size(1)))

    def _padded_weight(self, layer: int, width: int) -> Tensor:
        """The layer's input projection W with zero rows up to `width` (Z's
        columns), formed once per epoch."""
        w = self._proj[layer].detach()
        if width == w.size(0):
            return w
        wp = self._wpad.get(layer)
        if wp is None:
            with torch.no_grad():
                wp = torch.nn.functional.pad(w, (0, 0, 0, width - w.size(0)))
            self._wpad[layer] = wp
        return wp

    def _dx_weight(self, layer: int, width: int) -> Tensor:
        """The B operand of dZ W for the layer's dZ rows of `width` columns:
        Wᵀ, with zero columns for Z's zero pad columns, formed once per epoch.
        Whole, 16-byte aligned dZ rows take the matrix-core product; the pad
        columns of dZ and rows of W are zero, so the sum gains only exact
        zero terms."""
        wt = self._wtdx.get(layer)
        if wt is None or wt.size(1) != width:
            w = self._proj[layer].detach()
            with torch.no_grad():
                if width != w.size(0):
                    w = torch.nn.functional.pad(w, (0, 0, 0, width - w.size(0)))
                wt = w.t().contiguous()
            self._wtdx[layer] = wt
        return wt

    def _backward_device(self, layer: int, losses: Optional[List[Tensor]] = None) -> None:
        """Backward of a projected layer: per partition, take the forward's
        kept graph or recompute the layer from its gathered rows of Z, and
        backpropagate into the layer's parameters and into dZ; then
        dW = sum_p dZ_pᵀ x_p.  An in-place layer backpropagates the same way
        into all its parameters (its input gets no gradient), with no dZ and
        no dW pass; so does a gathered layer, whose recompute regathers its
        input rows in HBM and adds their gradient into the layer's dL/dx
        buffer (above layer 0)."""
        g, pids, pool, s = self.graph, self._my_pids, self.config.pool_size, self.streams
        if not pids:
            return
        last = layer == self.model.num_layers - 1
        inplace = layer in self._inplace
        gathered = layer not in self._proj and not inplace
        if gathered:
            if layer > 0:
                with torch.cuda.stream(s.compute):
                    self._gxbuf(layer).zero_()
        elif not inplace:
            w = self._proj[layer]
            dz = self._dzbuf(layer)
            # A merged layer whose sink writes every row of dz (GCN) needs no
            # zeroed dz; otherwise the backward adds into it.
            if not (layer in self._merged and self._whole_sink(layer)
                    and self.model.sink_writes_whole(layer)):
                with torch.cuda.stream(s.compute):
                    dz.zero_()
        from_device = not last and self._grad_on_device(layer + 1)
        from_host = not last and not from_device
        gbuf = self.device_gradients[layer + 1] if not last else None
        merged = layer in self._merged
        if merged:
            # One backward for every partition.  The last layer's is that of
            # the one loss over all rows, formed from the merged logits; a
            # lower layer's takes the gradient of all its output rows.  Either
            # adds dL/dZ into dZ (a projected layer).
            with torch.cuda.stream(s.compute):
                if last:
                    if self._merged_out is None or len(losses) != 1:
                        raise RuntimeError("merged last layer: its forward did not run merged")
                    losses[0].backward()
                else:
                    out = self._graphs.get(layer, {}).pop(-1)
                    out.backward(self._device_grad(layer + 1, None, consumer=out))
                    del out
            self._merged_out = None
            for pid in pids:
                self.activations[layer][pid] = None
        if from_host:
            self._upload_grad(layer + 1, pids[0], s.h2d[0])
        for i, pid in enumerate(pids if not merged else []):
            k = i % pool
            if from_host:
                self.host_gradients[layer + 1].h2d_synchronize(s.h2d[k])
                s.compute.wait_stream(s.h2d[k])
            with torch.cuda.stream(s.compute):
                if from_host and i + 1 < len(pids) and pool > 1:
                    self._upload_grad(layer + 1, pids[i + 1], s.h2d[(i + 1) % pool])
                out = self._graphs.get(layer, {}).pop(pid, None)
                if last and out is not None:
                    # Kept logits: _compute_losses formed the loss from them.
                    losses[self._pid_to_loss_idx[pid]].backward()
                elif last:
                    out = self._device_recompute(layer, pid)
                    y, codes = self._labels_and_codes(pid)
                    with torch.enable_grad():
                        loss, _ = masked_cross_entropy(out, y, codes, "sum")
                    loss.backward()
                else:
                    if out is None:
                        out = self._device_recompute(layer, pid)
                    if from_device:
                        out.backward(self._device_grad(layer + 1, pid, consumer=out))
                    else:
                        out.backward(gbuf[pid])
                        gbuf.release(pid)
                # The gather's backward added dL/dz into dZ at the partition's
                # rows (distinct within one partition): each element of dZ
                # gets one addition per partition, in partition order.
                del out
                self.activations[layer][pid] = None
            if from_host and pool == 1 and i + 1 < len(pids):
                self._upload_grad(layer + 1, pids[i + 1], s.h2d[0])
        if inplace or gathered:
            s.compute.synchronize()
            return
        # dW over dZ's whole (16-byte) rows; the rows of dW for Z's zero pad
        # columns are zero and are dropped.
        with torch.cuda.stream(s.compute):
            dwp = torch.zeros(dz.size(1), w.size(1), dtype=w.dtype, device=w.device)
            dw = dwp[:w.size(0)]

        def accumulate(pid, xp, lo, hi):
            with dense_region("dw", hi - lo, w.size(0), w.size(1)):
                gemm_tn(dz[lo:hi], xp, out=dwp, beta=1.0)

        if layer in self._xin:
            x = self._xres[layer]
            with torch.cuda.stream(s.compute):
                if merged:
                    # One product over all rows, as the layer's forward: as
                    # fast as P products at C4/C5's 10M rows, 15% faster at
                    # C3's 2.45M x 256 x 256.
                    n = int(g.ptr[-1])
                    accumulate(None, x[:n], 0, n)
                else:
                    for pid in pids:
                        lo, hi = g._range(pid)
                        accumulate(pid, x[lo:hi], lo, hi)
        else:
            self._each_input_partition(layer, accumulate)
        with torch.cuda.stream(s.compute):
            if w.grad is None:
                w.grad = dw
            else:
                w.grad.add_(dw)
        s.compute.synchronize()


    def _prepare_layer(self, layer: int) -> None:
        """Before a layer's partition loop: the first layer's input rows
        uploaded into their HBM copy (in place, gathered) or projected into
        Z_0 as they arrive (projected); and, for a projected layer whose model
        takes per-row quantities of Z precomputed (GAT's attention scores),
        those formed once for all rows.  Nothing for the reference flow, which
        gathers per partition from the host."""
        if layer == 0:
            if layer in self._inplace or (layer in self._xin and layer not in self._proj):
                # Every partition reads halo rows of the others: all uploads
                # land before the compute stream goes on.
                self._upload_resident(0, lambda pid, x, lo, hi: None)
            elif layer in self._proj:
                self._each_input_partition(
                    0, lambda pid, x, lo, hi: self._project_rows(0, x, lo, hi),
                    whole=lambda x: self._project_rows(0, x, 0, x.size(0)))
        self._scores.pop(layer, None)
        if layer in self._proj:
            with torch.cuda.stream(self.streams.compute):
                sc = self.model.projected_scores(layer, self._zbufs[layer],
                                                 whole=layer in self._merged)
            if sc is not None:
                self._scores[layer] = sc

    def _forward_layer_resident(self, layer: int) -> None:
        """_forward_layer when the next layer's input rows stay in HBM: each
        partition's output goes to the resident copy of x_{layer+1} (and to
        Z_{layer+1} when that layer runs projected), and nothing crosses to
        the host."""
        if layer in self._merged:
            self._forward_merged(layer)
            return
        g, pids, pool, s = self.graph, self._my_pids, self.config.pool_size, self.streams
        projected = self._device_flow(layer)
        x_next = self._xres_buf(layer + 1)
        self._prepare_layer(layer)
        if not projected:
            self._gather(layer, pids[0], s.h2d[0])
        for i, pid in enumerate(pids):
            k = i % pool
            if not projected:
                self.device_features[layer].h2d_synchronize(s.h2d[k])
                s.compute.wait_stream(s.h2d[k])
            with torch.cuda.stream(s.compute):
                if not projected:
                    if i + 1 < len(pids) and pool > 1:
                        self._gather(layer, pids[i + 1], s.h2d[(i + 1) % pool])
                    out = self._checkpointed(layer, pid, k)
                lo, hi = g._range(pid)
                if projected:
                    # The model may write the output into x_next's rows itself.
                    out = self._device_forward(layer, pid, keep=layer in self._keep,
                                               dest=x_next[lo:hi])
                if (layer + 1) in self._proj:
                    self._project_rows(layer + 1, out, lo, hi)
                in_place = out.data_ptr() == x_next[lo:hi].data_ptr()
                if not in_place:
                    with torch.no_grad():
                        x_next[lo:hi].copy_(out)
                if in_place:
                    # The storage is x_next's: it is never freed here.
                    if layer not in self._keep:
                        self.activations[layer][pid] = None
                elif not (projected and layer in self._keep):
                    # The storage goes back to the allocator in stream order; a
                    # reference-flow layer keeps the tensor for its backward,
                    # which recomputes it.  A kept graph keeps its output.
                    self.activations[layer][pid] = out
                    self._free(out)
                if not projected:
                    self.device_features[layer].release(pid)
            if pool == 1 and not projected and i + 1 < len(pids):
                self._gather(layer, pids[i + 1], s.h2d[0])
