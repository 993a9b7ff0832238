"""Trainer: layer-wise, partition-wise full-graph training (grinnder/engine/trainer.py).

The algorithm is the reference's (Algorithm 1 of the GriNNder paper as
implemented in trainer.py:334-1138):

forward, per layer l, per partition p (double-buffered):
    gather x = [h_l[p] | halo rows from other partitions] host -> device,
    out = checkpoint(GradOffload(x) -> model.forward_layer(l, x, adj_p)),
    D2H out into the host buffer h_{l+1}[p], free device memory;
loss: upload each partition's logits, cross-entropy (sum) on its train rows;
backward, last layer first, per partition:
    re-gather x (grinnder mode) or restore its snapshot (hongtu mode),
    backpropagate (the checkpoint recomputes the layer), GradOffload
    scatter-adds dL/dx into the host gradient buffer of layer l (halo rows go
    to their owning partitions), and the next layer down uploads that buffer
    as the gradient of its outputs;
finally grads /= number of training nodes, optimizer step.

With one partition the reference's fast path is used (trainer.py:418-471):
plain full-graph forward/backward.  Here its inputs (features, labels, masks,
adjacency plans) stay resident in HBM across epochs.

Differences by design: host buffers are pinned so halo traffic moves by
device kernels; waits are per stream, not device-wide.  The storage tier
(grinnder mode, trainer.py:73-160) is set up only when the host buffers do
not fit the host-memory budget or a cache mode is asked for: then a
PartitionCache keeps layers (lru_layer) or dependency sets of partitions
(partition_lru) in host memory and the rest in files under
config.storage_dir, and the layers run with the reference's data movement.

Projected layers (config.project_first = 'auto', planned per epoch against
free HBM; 'off' keeps the reference's data movement):

- A layer whose input enters only through x Wᵀ (GCNConv; GATConv with
  inactive dropout) satisfies gather(x) Wᵀ = gather(x Wᵀ) row by row.  Z =
  x Wᵀ is formed once per partition from its own rows and stays in HBM with
  its gradient dZ, and partitions take their gathered rows from Z on the
  device instead of input rows from the host.  A GCN layer reads Z in place
  through global row ids (aggregation.ProjectedSink); a GAT layer gathers.
- The backward adds dL/dZ of a partition's rows into dZ (partitions in
  order, so sums are deterministic), hands dZ_p W to the layer below as the
  gradient of its outputs (no host scatter), and forms dL/dW = sum_p
  dZ_pᵀ x_p at the end.
- Layer inputs stay in HBM for the epoch when there is room
  (resident_inputs): layer 0's rows are uploaded once per epoch, those above
  come from the layer below and never reach the host.  Without room they are
  uploaded again for dW.
- The forward's autograd graphs are kept for the backward when there is
  room; otherwise the backward recomputes each partition from the RNG state
  its forward started from, as the reference's checkpoint does.
- A widening first GCN layer whose input rows stay in HBM runs in place
  instead (inplace_layers): it aggregates the narrower input first, reading
  it through global row ids, and needs no backward aggregation.
- A layer with no input projection (GATConv with active input dropout, a
  model without one) runs the reference's per-partition forward and
  recompute, but when there is room its input rows stay in HBM
  (gathered_layers): each partition gathers its rows there, and the
  backward adds dL/dx into an HBM buffer, partitions in order, in place of
  the host scatter.

Per layer this replaces two host gathers and a read-add-write scatter of
~E x d_in rows (plus the D2H of the output and the upload of its gradient)
with at most one N x d_in upload per epoch.
"""

from __future__ import annotations

from typing import Dict, List, Optional

import torch
from torch import Tensor
from torch.utils.checkpoint import checkpoint

from grinnder_amd.autograd.checkpoint import HongtuCheckpoint, ScatteredCheckpoint
from grinnder_amd.autograd.grad_offload import GradOffload
from grinnder_amd.buffer.device import DeviceBuffer
from grinnder_amd.buffer.host import HostBuffer
from grinnder_amd.config import GriNNderConfig
from grinnder_amd.data.graph import PartitionedGraph
from grinnder_amd.engine.projected import ProjectedLayers
from grinnder_amd.engine.streams import StreamManager
from grinnder_amd.nn.base import GriNNderModel
from grinnder_amd.loss import check_stats, mask_codes, masked_cross_entropy


class _EpochUploads:
    """Input features uploaded from pinned host memory once per epoch into
    two HBM buffers in turn: while an epoch computes on one buffer, the next
    epoch's upload runs on a side stream into the other.  An upload waits
    for the compute work queued before it, which includes the last epoch
    that read its buffer."""

    def __init__(self, host: Tensor, device: torch.device):
        self.host = host
        self.bufs = [torch.empty(host.shape, dtype=host.dtype, device=device) for _ in range(2)]
        self.stream = torch.cuda.Stream(device)
        self.pending: Optional[tuple] = None
        self.cur = 0

    def _issue(self, idx: int, compute: torch.cuda.Stream) -> torch.cuda.Event:
        entry = torch.cuda.Event()
        entry.record(compute)
        self.stream.wait_event(entry)
        with torch.cuda.stream(self.stream):
            from grinnder_amd.aggregation import KernelTimer
            with KernelTimer.region("x_upload", self.host.numel() * 4, 0, self.host.size(1)):
                self.bufs[idx].copy_(self.host, non_blocking=True)
            done = torch.cuda.Event()
            done.record(self.stream)
        return done

    def next(self, compute: torch.cuda.Stream) -> Tensor:
        if self.pending is None:
            idx, done = self.cur, self._issue(self.cur, compute)
        else:
            idx, done = self.pending
        compute.wait_event(done)
        self.cur = idx
        self.pending = (1 - idx, self._issue(1 - idx, compute))
        return self.bufs[idx]


class Trainer(ProjectedLayers):
    def __init__(self, model: GriNNderModel, graph: PartitionedGraph, config: GriNNderConfig,
                 partition_range: Optional[tuple] = None):
        if config.mode not in ("hongtu", "grinnder"):
            raise ValueError(f"unknown mode {config.mode!r}")
        if config.cache_mode not in ("auto", "lru_layer", "partition_lru"):
            raise ValueError(f"Unsupported cache mode {config.cache_mode!r}")
        if config.pool_size < 1:
            raise ValueError("pool_size must be >= 1")
        self.model = model
        self.graph = graph
        self.config = config
        self.device = torch.device(config.device)
        self.cache = None
        if partition_range is not None:
            self._pid_start, self._pid_end = partition_range
        else:
            self._pid_start, self._pid_end = 0, graph.num_parts
        # A partition with no nodes has no rows to gather, compute or
        # scatter (nor halo rows: it has no edges), and adds nothing to the
        # loss, its gradient or the metrics: the partition loops skip it.
        self._my_pids = [p for p in range(self._pid_start, self._pid_end)
                         if graph.partition_sizes[p] > 0]

        dims = model.layer_dims()
        if len(dims) != model.num_layers + 1:
            raise ValueError("layer_dims() must have num_layers + 1 entries")
        L, P = model.num_layers, graph.num_parts
        self.streams = StreamManager(pool_size=config.pool_size, device=config.device)
        # One partition runs the reference's full-graph fast path, except
        # under the partition-wise storage cache (trainer.py:148-160).
        self._fast = (graph.num_parts == 1 and partition_range is None
                      and not (config.mode == "grinnder"
                               and config.cache_mode == "partition_lru"))
        self.backend = None

        self.host_features: List[HostBuffer] = []
        self.host_gradients: List[Optional[HostBuffer]] = [None]
        self.device_features: List[DeviceBuffer] = []
        self.device_gradients: List[Optional[DeviceBuffer]] = [None]
        self.activations: List[List[Optional[Tensor]]] = [[None] * P for _ in range(L)]
        self._pid_to_loss_idx: Dict[int, int] = {}
        self._resident: Dict[str, Tensor] = {}
        self._uploads: Optional[_EpochUploads] = None
        self._label_cache: Dict[int, tuple] = {}
        self._init_projected()
        if not self._fast:
            for l in range(L + 1):
                self.host_features.append(HostBuffer(P, graph.partition_sizes, dims[l],
                                                     file_prefix=f"feat_l{l}", pin_memory=True))
            for l in range(1, L):
                self.host_gradients.append(HostBuffer(P, graph.partition_sizes, dims[l],
                                                      file_prefix=f"grad_l{l}",
                                                      pin_memory=True))
            for l in range(L):
                self.device_features.append(DeviceBuffer(P, graph.expanded_sizes, dims[l],
                                                         device=config.device))
            for l in range(1, L):
                self.device_gradients.append(DeviceBuffer(P, graph.partition_sizes, dims[l],
                                                          device=config.device))
            self._setup_storage()
            for pid in range(P):
                feats = graph.partition_features(pid)
                self.host_features[0][pid].copy_(feats)
                del feats
                if self._uses_partition_lru():
                    # Inputs wait in storage until a gather needs them.
                    self.host_features[0].cpu_to_storage(pid)
                    self.host_features[0].release(pid)

    # ------------------------------------------------------------ public API

    # ------------------------------------------------------- storage tier

    def _setup_storage(self) -> None:
        """The storage tier (grinnder mode): a StorageBackend under
        config.storage_dir and a PartitionCache over the host buffers.  With
        cache_mode 'auto' it is set up only when the host buffers of every
        layer do not fit the host-memory budget (host_memory_budget_gb, or the
        available memory), less the graph's resident metadata and the safety
        margin; when they fit, every layer stays in host memory, which is
        what the reference's lru_layer cache does without evicting."""
        from grinnder_amd.cache.partition_cache import PartitionCache, fixed_resident_bytes
        from grinnder_amd.utils import get_available_host_memory

        cfg, g = self.config, self.graph
        if cfg.mode != "grinnder":
            return
        fixed = fixed_resident_bytes(g)
        margin = int(cfg.runtime_safety_margin_gb * (1 << 30))
        if cfg.cache_mode == "auto":
            budget = (int(cfg.host_memory_budget_gb * (1 << 30)) if cfg.host_memory_budget_gb > 0
                      else get_available_host_memory())
            need = sum(b.total_nbytes for b in self.host_features)
            need += sum(b.total_nbytes for b in self.host_gradients if b is not None)
            if need <= budget - fixed - margin:
                return
        from grinnder_amd.storage.backend import StorageBackend

        self.backend = StorageBackend(cfg.storage_dir)
        for buf in self.host_features + [b for b in self.host_gradients if b is not None]:
            buf.attach_backend(self.backend)
        deps = [{p} | {q for q, b in enumerate(bnd) if q != p and b is not None and b.numel()}
                for p, bnd in enumerate(g.boundaries)]
        self.cache = PartitionCache(
            num_parts=g.num_parts, num_layers=self.model.num_layers,
            layer_dims=self.model.layer_dims(), num_nodes=g.num_nodes,
            host_buffers=self.host_features, grad_buffers=self.host_gradients,
            backend=self.backend, mode=cfg.cache_mode,
            host_memory_budget_gb=cfg.host_memory_budget_gb, fixed_resident_bytes=fixed,
            safety_margin_bytes=margin, dependency_sets=deps)

    def _uses_partition_lru(self) -> bool:
        return self.cache is not None and self.cache.mode == "partition_lru"

    def _cache_layer(self, layer: int) -> None:
        """lru_layer: the whole layer resident before its gathers."""
        if self.cache is not None and self.cache.mode == "lru_layer":
            self.cache.ensure_in_host(layer)

    def _spill_output(self, layer: int, pid: int) -> None:
        """partition_lru: a forward output partition goes to storage once its
        D2H is done (the reference writes it from the GPU directly,
        trainer.py:549-560), so host memory holds at most pool_size of them."""
        if self._uses_partition_lru():
            self.host_features[layer].cpu_to_storage(pid)
            self.host_features[layer].release(pid)

    def _gradient_partition_resident(self, layer: int, pid: int) -> None:
        """partition_lru: a gradient partition flushed by the layer above is
        loaded back for its upload, or zeroed if it has no copy (trainer.py:266-274)."""
        buf = self.host_gradients[layer]
        if buf is None or buf.is_allocated(pid) or not self._uses_partition_lru():
            return
        if buf.storage_exists(pid):
            buf.storage_to_cpu(pid)
        else:
            buf.zero_partition(pid)

    def reset_epoch(self) -> None:
        if self._uses_partition_lru():
            self.cache.reset()
            for buf in self.host_features[1:]:
                buf.release_all()
            for buf in self.host_gradients:
                if buf is not None:
                    buf.release_all()
        # Host activation buffers of layers >= 1 are fully overwritten by the
        # forward D2H fills and gradient buffers are zeroed before each
        # backward phase, so neither needs clearing here.
        for buf in self.device_features:
            buf.reset()
        for buf in self.device_gradients:
            if buf is not None:
                buf.reset()
        for acts in self.activations:
            for i in range(len(acts)):
                acts[i] = None
        self._graphs = {}
        self._rng = {}
        self._gkept = {}
        self._scores = {}
        self._merged_out = None

    def train_epoch(self, optimizer: torch.optim.Optimizer,
                    criterion: torch.nn.Module) -> Dict[str, float]:
        self.model.train()
        if self._fast:
            return self._train_fast(optimizer)
        self._proj = self._plan_projection()
        self._plan_inplace()
        self.reset_epoch()
        optimizer.zero_grad()
        # The layers run on the compute stream; the last optimizer step (and
        # anything else the caller queued) ran on the current one.
        self.streams.compute.wait_stream(torch.cuda.current_stream(self.device))
        for l in range(self.model.num_layers):
            self._forward_layer(l)
        losses, metrics = self._compute_losses()
        self._backward_last_layer(losses)
        for l in reversed(range(self.model.num_layers - 1)):
            self._backward_layer(l)
        n_train = metrics.get("_n_train", 1)
        if n_train > 0:
            for p in self.model.parameters():
                if p.grad is not None:
                    p.grad.div_(n_train)
        optimizer.step()
        return metrics

    @torch.no_grad()
    def evaluate(self, criterion: torch.nn.Module) -> Dict[str, float]:
        self.model.eval()
        if self._fast:
            out = self._fast_logits()
            _, metrics = self._fast_metrics(out)
            return metrics
        self._proj = self._plan_projection()
        self._plan_inplace()
        self.reset_epoch()
        self.streams.compute.wait_stream(torch.cuda.current_stream(self.device))
        for l in range(self.model.num_layers):
            self._forward_layer(l)
        _, metrics = self._compute_losses()
        return metrics

    # ------------------------------------------------ single-partition path

    def _res(self, name: str, make) -> Tensor:
        t = self._resident.get(name)
        if t is None:
            t = make()
            self._resident[name] = t
        return t

    def _fast_features(self) -> Tensor:
        """This epoch's input features in HBM.  'resident': uploaded once.
        'stream': uploaded from pinned host memory every epoch, as the
        reference does (trainer.py:421-428), the next epoch's upload queued
        on a side stream as soon as this epoch has its rows."""
        g = self.graph
        if self.config.input_residency == "resident":
            return self._res("x", lambda: g.partition_features(0).to(self.device))
        up = self._uploads
        if up is None:
            feats = g.partition_features(0)
            host = torch.empty(feats.shape, dtype=torch.float32, pin_memory=True)
            host.copy_(feats)
            del feats
            up = self._uploads = _EpochUploads(host, self.device)
        return up.next(torch.cuda.current_stream())

    def _fast_logits(self) -> Tensor:
        g = self.graph
        x = self._fast_features()
        adj = g.adjacency(0)
        out = x
        for l in range(self.model.num_layers):
            out = self.model.forward_layer(l, out, adj)
        return out

    def _fast_loss(self, out: Tensor):
        """(loss, stats) of the resident logits; no host synchronisation."""
        g = self.graph

        def labels():
            y = g.partition_labels(0)
            train = g.partition_train_mask(0)
            sel = train | g.partition_val_mask(0) | g.partition_test_mask(0)
            # The labels stay resident, so an out-of-range label among the
            # selected rows is reported once here, before any step is taken,
            # instead of by a host read of the statistics every epoch.
            bad = int((sel & ((y < 0) | (y >= out.size(1)))).sum())
            check_stats([0, 0, 0, 0, 0, bad])
            return y.to(self.device)

        y = self._res("y", labels)
        train = self._res("train", lambda: g.partition_train_mask(0).to(self.device))
        codes = self._res("codes", lambda: mask_codes(
            train, g.partition_val_mask(0), g.partition_test_mask(0)))
        return masked_cross_entropy(out, y, codes, "mean")

    @staticmethod
    def _fast_metrics_from(loss: Tensor, stats: Tensor) -> Dict[str, float]:
        st = stats.tolist()
        check_stats(st)
        n_train = st[0]
        return {
            "loss": float(loss.detach()) if n_train > 0 else 0.0,
            "val_acc": st[1] / st[2] if st[2] else 0.0,
            "test_acc": st[3] / st[4] if st[4] else 0.0,
            "_n_train": n_train,
        }

    def _fast_metrics(self, out: Tensor):
        loss, stats = self._fast_loss(out)
        return loss, self._fast_metrics_from(loss, stats)

    def _train_fast(self, optimizer) -> Dict[str, float]:
        optimizer.zero_grad()
        out = self._fast_logits()
        loss, stats = self._fast_loss(out)
        loss.backward()
        optimizer.step()
        # The statistics are read once the whole step is queued.
        return self._fast_metrics_from(loss, stats)

    # ------------------------------------------------- partitioned helpers

    def _gather(self, layer: int, pid: int, stream: torch.cuda.Stream) -> None:
        if self._uses_partition_lru():
            # The partitions this gather reads, made resident first (loaded
            # from storage; least recently used others evicted).  Earlier
            # gathers reading evicted partitions were waited for already.
            self.cache.ensure_dependencies_in_host(layer, pid,
                                                   boundaries=self.graph.boundaries[pid])
        with torch.cuda.stream(self.streams.compute):
            self.device_features[layer].async_gather(
                pid, self.host_features[layer], self.graph.boundaries[pid], stream)

    def _upload_grad(self, layer: int, pid: int, stream: torch.cuda.Stream) -> None:
        buf = self.device_gradients[layer]
        if buf is None or self.host_gradients[layer] is None:
            return
        self._gradient_partition_resident(layer, pid)
        with torch.cuda.stream(self.streams.compute):
            buf.allocate(pid)
            self.host_gradients[layer].async_upload(pid, buf[pid], stream)

    def _upoffload_wrapper(self, layer_id: int, pid: int, x: Tensor) -> Tensor:
        x = GradOffload.apply(
            x, layer_id, pid,
            self.host_gradients[layer_id] if layer_id > 0 else None,
            self.graph.boundaries[pid],
            self._scatter_stream(),
            self.streams.compute,
        )
        # Activations are stored, freed and re-uploaded as dense [B, D] blocks;
        # a layer may return a strided view (a padded product), made dense here.
        return self.model.forward_layer(layer_id, x, self.graph.adjacency(pid)).contiguous()

    def _scatter_stream(self) -> torch.cuda.Stream:
        """All halo-gradient scatters of a backward phase share one stream:
        partitions' halos overlap in the host write-back buffer, and the
        read-add-write of consecutive partitions must not interleave."""
        return self.streams.d2h[0]

    def _checkpointed(self, layer: int, pid: int, slot: int) -> Tensor:
        x = self.device_features[layer][pid]
        x.requires_grad_(True)
        if self.config.mode == "hongtu":
            hooks = HongtuCheckpoint(pid, self.device_features[layer])
        else:
            hooks = ScatteredCheckpoint(pid, self.device_features[layer],
                                        self.streams.act_h2d[slot])
        with hooks:
            return checkpoint(self._upoffload_wrapper, layer, pid, x, use_reentrant=True)

    @staticmethod
    def _free(t: Optional[Tensor]) -> None:
        if t is not None:
            t.untyped_storage().resize_(0)

    # ------------------------------------------------------------- forward

    def _forward_layer(self, layer: int) -> None:
        """Per partition: the layer's output from gathered input rows (the
        reference's flow) or from gathered rows of Z (a projected layer), D2H
        into the next layer's host buffer (or, when the next layer's input
        stays in HBM, a device copy into it), and, when the next layer runs
        projected, its rows of Z_{layer+1} = out Wᵀ formed right away."""
        g, pids, pool, s = self.graph, self._my_pids, self.config.pool_size, self.streams
        if not pids:
            return
        projected = self._device_flow(layer)
        w_next = self._proj.get(layer + 1)
        last = layer == self.model.num_layers - 1
        if last and layer in self._merged:
            self._forward_merged(layer)
            return
        if (layer + 1) in self._xin or (last and self._logits_on_device()):
            self._forward_layer_resident(layer)
            return
        self._prepare_layer(layer)
        if layer in self._keep and layer == self.model.num_layers - 1:
            # The last layer with its graphs kept: the loss reads the logits
            # from them (_compute_losses), so nothing goes to the host.
            for pid in pids:
                with torch.cuda.stream(s.compute):
                    self._device_forward(layer, pid, keep=True)
            return
        if not projected:
            self._cache_layer(layer)
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
                else:
                    out = self._device_forward(layer, pid, keep=False)
                if w_next is not None:
                    lo, hi = g._range(pid)
                    self._project_rows(layer + 1, out, lo, hi)
                self.activations[layer][pid] = out
                self.host_features[layer + 1].async_fill(pid, out, s.d2h[k])
                if not projected:
                    self.device_features[layer].release(pid)
                if i > 0 and pool > 1:
                    prev, pk = pids[i - 1], (i - 1) % pool
                    self.host_features[layer + 1].d2h_synchronize(s.d2h[pk])
                    self._free(self.activations[layer][prev])
                    self._spill_output(layer + 1, prev)
            if pool == 1:
                self.host_features[layer + 1].d2h_synchronize(s.d2h[0])
                self._free(self.activations[layer][pid])
                self._spill_output(layer + 1, pid)
                if not projected and i + 1 < len(pids):
                    self._gather(layer, pids[i + 1], s.h2d[0])
        if pool > 1:
            last = (len(pids) - 1) % pool
            self.host_features[layer + 1].d2h_synchronize(s.d2h[last])
            self._free(self.activations[layer][pids[-1]])
            self._spill_output(layer + 1, pids[-1])
        if self.cache is not None:
            self.cache.on_layer_complete(layer)

    # ---------------------------------------------------------------- loss

    def _compute_losses(self):
        pids, pool, s = self._my_pids, self.config.pool_size, self.streams
        last = self.model.num_layers - 1
        losses: List[Tensor] = []
        self._pid_to_loss_idx = {}
        if not pids:
            return losses, {"loss": 0.0, "val_acc": 0.0, "test_acc": 0.0, "_n_train": 0}

        if self._merged_out is not None:
            return self._merged_losses()

        loss_sums: List[Tensor] = []
        stat_rows: List[Tensor] = []

        def upload(pid: int, stream) -> None:
            act = self.activations[last][pid]
            if self._uses_partition_lru():
                self.host_features[-1].storage_to_cpu(pid)
            with torch.cuda.stream(s.compute):
                act.untyped_storage().resize_(act.numel() * act.element_size())
            self.host_features[-1].async_upload(pid, act, stream)

        if self.cache is not None and self.cache.mode == "lru_layer":
            self.cache.ensure_in_host(self.model.num_layers)

        kept = last in self._keep and last in self._graphs
        on_device = not kept and self._logits_on_device()
        with torch.cuda.stream(s.compute):
            if not kept and not on_device:
                upload(pids[0], s.h2d[0])
            for i, pid in enumerate(pids):
                k = i % pool
                if kept:
                    out = self._graphs[last][pid]
                elif on_device:
                    lo, hi = self.graph._range(pid)
                    out = self._xres[last + 1][lo:hi]
                else:
                    self.host_features[-1].h2d_synchronize(s.h2d[k])
                    s.compute.wait_stream(s.h2d[k])
                    if i + 1 < len(pids):
                        upload(pids[i + 1], s.h2d[(i + 1) % pool])
                    out = self.activations[last][pid]
                y, codes = self._labels_and_codes(pid)
                # Sum over the partition's train rows (zero, with a zero
                # gradient, when it has none); the accuracy counts ride along.
                loss, stats = masked_cross_entropy(out, y, codes, "sum")
                self._pid_to_loss_idx[pid] = len(losses)
                losses.append(loss)
                loss_sums.append(loss.detach())
                stat_rows.append(stats)
                if not kept and not on_device:
                    self._free(out)
            st = torch.stack(stat_rows).sum(0).tolist()
            total_loss = float(torch.stack(loss_sums).double().sum())
        check_stats(st)
        n_train = st[0]
        metrics = {
            "loss": total_loss / max(n_train, 1),
            "val_acc": st[1] / max(st[2], 1),
            "test_acc": st[3] / max(st[4], 1),
            "_n_train": n_train,
        }
        return losses, metrics

    def _merged_losses(self):
        """_compute_losses for a merged last layer: one loss, the sum over
        every train row of the graph (the sum of the per-partition sums), from
        the logits of all rows at once."""
        g = self.graph
        hit = self._label_cache.get(-1)
        if hit is None:
            n = int(g.ptr[-1])
            hit = (g.labels[:n].to(self.device),
                   mask_codes(g.train_mask[:n], g.val_mask[:n], g.test_mask[:n]).to(self.device))
            self._label_cache[-1] = hit
        y, codes = hit
        with torch.cuda.stream(self.streams.compute):
            loss, stats = masked_cross_entropy(self._merged_out, y, codes, "sum")
            if not self.model.training:
                self._merged_out = None
            st = stats.tolist()
            total_loss = float(loss.detach().double())
        check_stats(st)
        n_train = st[0]
        self._pid_to_loss_idx = {pid: 0 for pid in self._my_pids}
        metrics = {
            "loss": total_loss / max(n_train, 1),
            "val_acc": st[1] / max(st[2], 1),
            "test_acc": st[3] / max(st[4], 1),
            "_n_train": n_train,
        }
        return [loss], metrics

    def _labels_and_codes(self, pid: int):
        """Device labels and uint8 train/val/test codes of a partition (cached)."""
        hit = self._label_cache.get(pid)
        if hit is None:
            g = self.graph
            y = g.partition_labels(pid).to(self.device)
            codes = mask_codes(g.partition_train_mask(pid), g.partition_val_mask(pid),
                               g.partition_test_mask(pid)).to(self.device)
            hit = (y, codes)
            self._label_cache[pid] = hit
        return hit

    # ------------------------------------------------------------ backward

    def _regathers(self, layer: int) -> bool:
        return self.config.mode == "grinnder"

    def _backward_last_layer(self, losses: List[Tensor]) -> None:
        layer = self.model.num_layers - 1
        if self._device_flow(layer):
            self._backward_device(layer, losses)
        else:
            self._backward_pass(layer,
                                lambda pid: losses[self._pid_to_loss_idx[pid]].backward())
        for i in range(len(losses)):
            losses[i] = None

    def _backward_layer(self, layer: int) -> None:
        if self._device_flow(layer):
            self._backward_device(layer)
            return
        from_device = self._grad_on_device(layer + 1)

        def run(pid: int) -> None:
            act = self.activations[layer][pid]
            if act is None or act.grad_fn is None:
                return
            if from_device:
                act.backward(self._device_grad(layer + 1, pid))
                return
            gbuf = self.device_gradients[layer + 1]
            if gbuf is not None and gbuf.is_allocated(pid):
                act.backward(gbuf[pid])
            else:
                act.backward()
        self._backward_pass(layer, run, upload_grad=not from_device)

    def _backward_pass(self, layer: int, run, upload_grad: bool = False) -> None:
        """Per partition: re-gather x_layer, upload dL/d(out) if needed, backprop."""
        pids, pool, s = self._my_pids, self.config.pool_size, self.streams
        if not pids:
            return
        if self.host_gradients[layer] is not None:
            # partition_lru: partitions are zeroed when first touched.
            self.host_gradients[layer].initialize_zeros(lazy=self._uses_partition_lru())
        regather = self._regathers(layer)
        if regather:
            self._cache_layer(layer)
            self._gather(layer, pids[0], s.act_h2d[0])
        if upload_grad:
            self._upload_grad(layer + 1, pids[0], s.h2d[0])
        # The scatters of partition p are waited for after partition p+1's
        # backward ran, so they overlap that compute and the next gather; at
        # most two partitions' scatters are in flight (one stream, in order).
        hg = self.host_gradients[layer]
        for i, pid in enumerate(pids):
            k = i % pool
            if regather:
                self.device_features[layer].h2d_synchronize(s.act_h2d[k])
            if upload_grad and self.host_gradients[layer + 1] is not None:
                self.host_gradients[layer + 1].h2d_synchronize(s.h2d[k])
            s.compute.wait_stream(s.act_h2d[k])
            s.compute.wait_stream(s.h2d[k])
            with torch.cuda.stream(s.compute):
                if i + 1 < len(pids) and pool > 1:
                    if regather:
                        self._gather(layer, pids[i + 1], s.act_h2d[(i + 1) % pool])
                    if upload_grad:
                        self._upload_grad(layer + 1, pids[i + 1], s.h2d[(i + 1) % pool])
                queued_before = hg.d2h_queued if hg is not None else 0
                run(pid)
                s.compute.synchronize()
                act = self.activations[layer][pid]
                if act is not None:
                    self._free(act)
                    act.grad = None
                    self.activations[layer][pid] = None
                gbuf = self.device_gradients[layer + 1] if layer + 1 < len(
                    self.device_gradients) else None
                if gbuf is not None:
                    gbuf.release(pid)
                for _ in range(queued_before):
                    hg.d2h_wait_oldest()  # the previous partition's scatters
                self.device_features[layer].release(pid)
            if pool == 1 and i + 1 < len(pids):
                if regather:
                    self._gather(layer, pids[i + 1], s.act_h2d[0])
                if upload_grad:
                    self._upload_grad(layer + 1, pids[i + 1], s.h2d[0])
        if hg is not None:
            while hg.d2h_queued > 0:
                hg.d2h_wait_oldest()
            self._scatter_stream().synchronize()
        if self.cache is not None and (layer < self.model.num_layers - 1
                                       or self._uses_partition_lru()):
            # The layer's gradient write-back buffer goes to storage
            # (trainer.py:889-890, :1137-1138).
            self.cache.on_backward_layer_complete(layer)
