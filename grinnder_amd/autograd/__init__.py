"""Autograd hooks: gradient offload and activation checkpoint policies."""

from grinnder_amd.autograd.checkpoint import HongtuCheckpoint, ScatteredCheckpoint
from grinnder_amd.autograd.grad_offload import GradOffload

__all__ = ["GradOffload", "HongtuCheckpoint", "ScatteredCheckpoint"]
