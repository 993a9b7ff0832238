"""GNN models (grinnder/nn): GriNNderModel, GCN, GAT and their HIP-backed convs."""

from grinnder_amd.nn.base import GriNNderModel
from grinnder_amd.nn.conv import GATConv, GCNConv
from grinnder_amd.nn.gat import GAT
from grinnder_amd.nn.gcn import GCN

__all__ = ["GriNNderModel", "GCN", "GAT", "GCNConv", "GATConv"]
