"""grinnder_amd: MI355X-native partitioned GNN layer hot path of GriNNder.

Same public names as the reference package (grinnder/__init__.py:10-51),
resolved lazily so that ``from grinnder_amd.config import GriNNderConfig``
needs neither the HIP library nor a GPU.
"""

__version__ = "0.1.0"

_EXPORTS = {
    "GriNNderConfig": ("grinnder_amd.config", "GriNNderConfig"),
    "GriNNderModel": ("grinnder_amd.nn.base", "GriNNderModel"),
    "GCN": ("grinnder_amd.nn.gcn", "GCN"),
    "GAT": ("grinnder_amd.nn.gat", "GAT"),
    "Trainer": ("grinnder_amd.engine.trainer", "Trainer"),
    "PartitionedGraph": ("grinnder_amd.data.graph", "PartitionedGraph"),
    "build_partitioned_graph": ("grinnder_amd.data.partition", "build_partitioned_graph"),
}


def __getattr__(name):
    target = _EXPORTS.get(name)
    if target is None:
        raise AttributeError(f"module 'grinnder_amd' has no attribute {name!r}")
    import importlib

    return getattr(importlib.import_module(target[0]), target[1])


__all__ = list(_EXPORTS)
