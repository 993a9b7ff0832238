"""Small helpers mirroring grinnder/utils.py:14-44."""

from __future__ import annotations

import random
from typing import Optional

import numpy as np
import torch
from torch import Tensor


def fix_seed(seed: int) -> None:
    """Seeds python, numpy and torch (CPU and GPU) generators."""
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)


def compute_micro_f1(pred: Tensor, target: Tensor, mask: Optional[Tensor] = None) -> float:
    """Micro-F1 (= accuracy) of argmax predictions over the masked rows."""
    if pred.dim() > 1:
        pred = pred.argmax(dim=-1)
    if mask is not None:
        mask = mask.to(pred.device)
        pred = pred[mask]
        target = target.to(pred.device)[mask]
    if target.numel() == 0:
        return 0.0
    return (pred == target.to(pred.device)).float().mean().item()


def ensure_dir(path: str) -> str:
    """Creates `path` (and parents) if missing; returns it."""
    import os

    os.makedirs(path, exist_ok=True)
    return path


def get_available_host_memory() -> int:
    """Bytes of host memory available to new allocations: MemAvailable from
    /proc/meminfo (grinnder/utils.py:47-64), else psutil, else 0."""
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except (OSError, ValueError):
        pass
    try:
        import psutil

        return int(psutil.virtual_memory().available)
    except ImportError:
        return 0
