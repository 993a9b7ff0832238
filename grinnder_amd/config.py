"""GriNNderConfig: the reference's configuration dataclass (grinnder/config.py:17-67).

Same field names, defaults and environment override, so user code written for
the reference constructs it unchanged.  Fields that select subsystems outside
this package's scope (the NVMe storage tier and its partition-LRU cache) are
accepted and validated by the Trainer.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Any, Dict, Literal


def _default_threads() -> int:
    env_value = os.environ.get("GRINNDER_PARTITION_THREADS")
    if env_value:
        return max(1, int(env_value))
    return os.cpu_count() or 1


@dataclass
class GriNNderConfig:
    """Training configuration.

    mode: 'hongtu' keeps a CPU snapshot of each gathered input for the
        backward recompute; 'grinnder' re-gathers it from the host buffers
        (scattered checkpointing, no snapshot redundancy).
    num_parts / partitioner / partitioner_kwargs: graph partitioning.
    cache_mode: 'auto' | 'lru_layer' | 'partition_lru' (host cache policy of
        the storage tier; this package keeps every layer host-resident, which
        is what 'auto' resolves to when the working set fits).
    device: GPU device string; pool_size: transfer double-buffering depth.
    project_first: 'auto' lets the partitioned trainer (grinnder mode, all
        partitions) keep layer data in HBM where it fits, planned per epoch:
        a layer that starts with a bias-free input projection forms Z = x Wᵀ
        once per partition and gathers (or reads in place) rows of Z; any
        other layer gathers its input rows from an HBM copy and adds their
        gradient into one (same results up to fp32 summation order).  'off'
        gathers every layer's input rows from the host buffers as the
        reference does.  Not a field of the reference's config.
    merge_partitions: 'auto' runs each layer that needs no host buffers
        (projected or in place, its forward graph kept when training, its
        output and the gradient of that output resident in HBM; and the last
        layer on those terms) as one pass over the whole graph's adjacency,
        which indexes Z's (or the input's) global rows directly: the same
        edges and per-row orders as the P per-partition passes, without their
        launches, gathers and scatters (same results up to fp32 summation
        order in the backward's per-source sums and in dW).
        'last' merges only the last layer, 'off' none.  Not a field of the
        reference's config.
    input_residency: 'stream' (the reference's data movement) uploads the
        input features from pinned host memory every epoch, the next epoch's
        upload running on a side stream while this epoch computes (the
        single-partition path and the layer-0 rows of projected / in-place
        layers).  'resident' uploads them once and keeps them in HBM across
        epochs (the features are static).  Not a field of the reference's
        config.
    """

    mode: Literal["hongtu", "grinnder"] = "grinnder"

    num_parts: int = 8
    partitioner: Literal["grinnder", "spinner"] = "grinnder"
    partitioner_kwargs: Dict[str, Any] = field(
        default_factory=lambda: {
            "capacity": 1.1,
            "beta": 1.0,
            "max_iter": 50,
            "num_threads": _default_threads(),
        }
    )

    storage_dir: str = "/pci5_nvme/grinnder"

    cache_mode: Literal["auto", "lru_layer", "partition_lru"] = "auto"
    host_memory_budget_gb: float = 0
    runtime_safety_margin_gb: float = 0.0

    device: str = "cuda:0"
    pool_size: int = 2
    preprocess_workers: int = field(default_factory=_default_threads)

    num_gpus: int = 1

    project_first: Literal["auto", "off"] = "auto"
    merge_partitions: Literal["auto", "last", "off"] = "auto"
    input_residency: Literal["stream", "resident"] = "stream"
