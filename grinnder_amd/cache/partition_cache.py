"""Which layers' host activations stay in RAM and which go to storage (the role
of grinnder/cache/partition_cache.py:38-446).

Two policies, chosen by `mode` or automatically from the host-memory budget:

- lru_layer: whole layers are resident or not.  A layer is loaded from
  storage when a gather needs it and is not resident; a layer produced by
  the forward stays resident.  When a layer does not fit the activation
  budget, least recently used layers are evicted (written to storage if
  their host rows changed, then released).
- partition_lru: (layer, partition) pairs.  Before a partition's gather, its
  dependency set (itself and every partition it reads halo rows from) is
  made resident; least recently used pairs outside that set are evicted.
  Forward outputs bypass host memory and go straight to storage; gradient
  partitions are flushed to storage after each backward layer.

Budget (the reference's accounting): host_memory_budget_gb, or the host's
available memory, minus the fixed resident bytes (graph metadata) and a
safety margin, is the cache's room.  lru_layer keeps one gradient layer's
bytes of that room free; 'auto' picks lru_layer when the largest activation
layer plus the largest gradient layer fit what is left, else partition_lru.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass
from typing import List, Literal, Optional, Set, Tuple

import torch

from grinnder_amd.utils import get_available_host_memory

MODES = ("auto", "lru_layer", "partition_lru")


@dataclass(frozen=True)
class CacheMemoryPlan:
    """Host-memory accounting behind the mode choice (bytes)."""

    total_budget_bytes: int
    fixed_resident_bytes: int
    safety_margin_bytes: int
    remaining_cache_bytes: int
    activation_layer_bytes: Tuple[int, ...]
    gradient_layer_bytes: Tuple[int, ...]
    all_layer_residency_bytes: int
    layer_working_set_bytes: int
    largest_partition_dependency_bytes: int


class PartitionCache:
    def __init__(self, num_parts: int, num_layers: int, layer_dims: List[int], num_nodes: int,
                 host_buffers, grad_buffers, backend,
                 mode: Literal["auto", "lru_layer", "partition_lru"] = "auto",
                 host_memory_budget_gb: float = 0, fixed_resident_bytes: int = 0,
                 safety_margin_bytes: int = 0,
                 dependency_sets: Optional[List[Set[int]]] = None):
        if mode not in MODES:
            raise ValueError(f"Unsupported cache mode {mode!r}; expected one of {sorted(MODES)}")
        self.num_parts = num_parts
        self.num_layers = num_layers
        self.layer_dims = layer_dims
        self.num_nodes = num_nodes
        self.host_buffers = host_buffers
        self.grad_buffers = grad_buffers
        self.backend = backend
        self.dependency_sets = dependency_sets

        budget = (int(host_memory_budget_gb * (1 << 30)) if host_memory_budget_gb > 0
                  else get_available_host_memory())
        self._memory_plan = self._plan(budget, max(0, int(fixed_resident_bytes)),
                                       max(0, int(safety_margin_bytes)))
        plan = self._memory_plan
        room = plan.remaining_cache_bytes
        layer_room = max(0, room - max(plan.gradient_layer_bytes or (0,)))
        if mode == "auto":
            mode = "lru_layer" if layer_room >= plan.layer_working_set_bytes else "partition_lru"
        self._mode = mode
        self._activation_cache_budget = layer_room if mode == "lru_layer" else room

        # Residency in least-recently-used order (oldest first).
        self._cached_layers: "OrderedDict[int, bool]" = OrderedDict()
        self._cached_partitions: "OrderedDict[Tuple[int, int], bool]" = OrderedDict()
        self._hits = 0
        self._misses = 0
        self._resident_activation_bytes = 0

    # ------------------------------------------------------------ properties

    @property
    def mode(self) -> str:
        return self._mode

    @property
    def hit_rate(self) -> float:
        n = self._hits + self._misses
        return self._hits / n if n else 0.0

    @property
    def memory_plan(self) -> CacheMemoryPlan:
        return self._memory_plan

    @property
    def remaining_cache_bytes(self) -> int:
        return self._memory_plan.remaining_cache_bytes

    @property
    def activation_cache_budget_bytes(self) -> int:
        return self._activation_cache_budget

    # -------------------------------------------------------------- accounting

    def _plan(self, budget: int, fixed: int, margin: int) -> CacheMemoryPlan:
        act = tuple(int(b.total_nbytes) for b in self.host_buffers)
        grad = tuple(0 if b is None else int(b.total_nbytes) for b in self.grad_buffers)
        biggest = max(range(len(act)), key=lambda i: act[i]) if act else 0
        dep_bytes = 0
        if self.host_buffers:
            buf = self.host_buffers[biggest]
            dep_bytes = max((sum(buf.partition_nbytes(q) for q in self._deps(p))
                             for p in range(self.num_parts)), default=0)
        return CacheMemoryPlan(
            total_budget_bytes=budget, fixed_resident_bytes=fixed, safety_margin_bytes=margin,
            remaining_cache_bytes=max(0, budget - fixed - margin),
            activation_layer_bytes=act, gradient_layer_bytes=grad,
            all_layer_residency_bytes=sum(act) + sum(grad),
            layer_working_set_bytes=max(act or (0,)) + max(grad or (0,)),
            largest_partition_dependency_bytes=dep_bytes)

    def _deps(self, pid: int, boundaries=None, dependencies=None) -> Set[int]:
        """The partitions `pid`'s gather reads: itself and every partition
        with a non-empty boundary towards it."""
        if dependencies is not None:
            return set(dependencies)
        if boundaries is not None:
            return {pid} | {q for q, b in enumerate(boundaries)
                            if q != pid and b is not None and b.numel() > 0}
        if self.dependency_sets is not None:
            return set(self.dependency_sets[pid])
        return {pid}

    def _layer_bytes(self, layer: int) -> int:
        return int(self.host_buffers[layer].total_nbytes)

    def _partition_bytes(self, layer: int, pid: int) -> int:
        return int(self.host_buffers[layer].partition_nbytes(pid))

    # ----------------------------------------------------------- whole layers

    def _make_room(self, need: int, what: str, evict_one) -> None:
        if need > self._activation_cache_budget:
            raise MemoryError(f"{what} requires {need} bytes, but only "
                              f"{self._activation_cache_budget} activation-cache bytes remain")
        while self._resident_activation_bytes + need > self._activation_cache_budget:
            if not evict_one():
                raise MemoryError(f"Cannot make room for {what} within "
                                  f"{self._activation_cache_budget} bytes")

    def _evict_oldest_layer(self) -> bool:
        if not self._cached_layers:
            return False
        layer, _ = self._cached_layers.popitem(last=False)
        self._evict_layer(layer)
        return True

    def ensure_in_host(self, layer_id: int) -> None:
        """Makes layer `layer_id` resident for its gathers / regathers."""
        if self._mode == "partition_lru":
            for pid in range(self.num_parts):
                self.ensure_partition_in_host(layer_id, pid)
            return
        if layer_id in self._cached_layers:
            self._cached_layers.move_to_end(layer_id)
            self._hits += 1
            return
        self._misses += 1
        need = self._layer_bytes(layer_id)
        self._make_room(need, f"Layer {layer_id}", self._evict_oldest_layer)
        buf = self.host_buffers[layer_id]
        missing = [p for p in range(self.num_parts) if not buf.is_allocated(p)]
        for pid in missing:
            buf.storage_to_cpu(pid=pid)
        self._cached_layers[layer_id] = True
        self._resident_activation_bytes += need

    def prepare_layer(self, layer_id: int) -> None:
        self.ensure_in_host(layer_id)

    def on_layer_complete(self, layer_id: int) -> None:
        """After layer `layer_id`'s forward: its output layer stays resident
        (lru_layer); partition_lru already sent the outputs to storage."""
        out = layer_id + 1
        if out >= len(self.host_buffers) or self._mode != "lru_layer":
            return
        if out in self._cached_layers:
            self._cached_layers.move_to_end(out)
            return
        need = self._layer_bytes(out)
        self._make_room(need, f"Layer {out}", self._evict_oldest_layer)
        self._cached_layers[out] = True
        self._resident_activation_bytes += need

    def on_backward_layer_complete(self, layer_id: int) -> None:
        """After layer `layer_id`'s backward: its gradient write-back buffer
        goes to storage (partition_lru: the resident partitions, which are
        then released)."""
        buf = self.grad_buffers[layer_id] if layer_id < len(self.grad_buffers) else None
        if buf is None:
            return
        if self._mode == "partition_lru":
            for pid in buf.allocated_pids():
                buf.cpu_to_storage(pid)
                buf.release(pid)
            return
        buf.cpu_to_storage()

    def _evict_layer(self, layer_id: int) -> None:
        buf = self.host_buffers[layer_id]
        for pid in range(self.num_parts):
            buf.ensure_storage_copy(pid)
            buf.release(pid)
        self._resident_activation_bytes = max(
            0, self._resident_activation_bytes - self._layer_bytes(layer_id))

    # ------------------------------------------------------------- partitions

    def ensure_partition_in_host(self, layer_id: int, pid: int) -> None:
        self.ensure_dependencies_in_host(layer_id, pid, dependencies={pid})

    def ensure_dependencies_in_host(self, layer_id: int, target_pid: int, boundaries=None,
                                    dependencies: Optional[Set[int]] = None) -> None:
        """Makes the dependency set of `target_pid` resident at layer
        `layer_id`, evicting least recently used pairs outside the set."""
        deps = self._deps(target_pid, boundaries, dependencies)
        protected = {(layer_id, p) for p in deps}
        demand = sum(self._partition_bytes(layer_id, p) for p in deps)
        if demand > self._activation_cache_budget:
            raise MemoryError(
                f"Layer {layer_id}, partition {target_pid} dependencies require {demand} "
                f"bytes, but only {self._activation_cache_budget} activation-cache bytes "
                "remain")
        missing = []
        for key in sorted(protected):
            if key in self._cached_partitions:
                self._cached_partitions.move_to_end(key)
                self._hits += 1
            else:
                missing.append(key)
                self._misses += 1
        need = sum(self._partition_bytes(layer_id, p) for _, p in missing)

        def evict_one() -> bool:
            for key in self._cached_partitions:
                if key not in protected:
                    self._evict_partition(*key)
                    return True
            return False

        self._make_room(need, f"layer {layer_id}, partition {target_pid} dependency set",
                        evict_one)
        buf = self.host_buffers[layer_id]
        for _, p in missing:
            buf.storage_to_cpu(pid=p)
            self._cached_partitions[(layer_id, p)] = True
            self._resident_activation_bytes += self._partition_bytes(layer_id, p)

    def _evict_partition(self, layer_id: int, pid: int) -> None:
        buf = self.host_buffers[layer_id]
        buf.ensure_storage_copy(pid)
        buf.release(pid)
        self._cached_partitions.pop((layer_id, pid), None)
        self._resident_activation_bytes = max(
            0, self._resident_activation_bytes - self._partition_bytes(layer_id, pid))

    # ------------------------------------------------------------------ epoch

    def reset(self) -> None:
        """Evicts everything the cache holds and clears its counters."""
        if self._mode == "lru_layer":
            for layer in list(self._cached_layers):
                self._evict_layer(layer)
        else:
            for layer, pid in list(self._cached_partitions):
                self._evict_partition(layer, pid)
        self._cached_layers.clear()
        self._cached_partitions.clear()
        self._hits = 0
        self._misses = 0
        self._resident_activation_bytes = 0


def fixed_resident_bytes(graph) -> int:
    """Host bytes of graph metadata that stay resident outside the cache:
    features, labels, masks, permutation, partition pointers, boundaries and
    the partitions' CSR (the reference's Trainer estimate)."""
    def nbytes(t) -> int:
        return int(t.numel() * t.element_size()) if isinstance(t, torch.Tensor) else 0

    total = sum(nbytes(t) for t in (graph.features, graph.labels, graph.train_mask,
                                    graph.val_mask, graph.test_mask, graph.perm, graph.ptr))
    total += 8 * len(graph.partition_sizes)
    total += sum(nbytes(b) for bnd in graph.boundaries for b in bnd if b is not None)
    total += sum(nbytes(t) for adj in graph.adj_csr for t in adj if t is not None)
    return total
