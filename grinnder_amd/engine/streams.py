"""Streams of the double-buffered pipeline (grinnder/engine/streams.py:10-41).

All streams use the default priority.
"""

from __future__ import annotations

from typing import List

import torch


class StreamManager:
    """compute + pool_size streams each for h2d, d2h and act_h2d (backward re-gather)."""

    def __init__(self, pool_size: int = 2, device: str = "cuda:0"):
        self.pool_size = pool_size
        self.device = device
        self.compute = torch.cuda.Stream(device)
        self.h2d: List[torch.cuda.Stream] = [torch.cuda.Stream(device) for _ in range(pool_size)]
        self.d2h: List[torch.cuda.Stream] = [torch.cuda.Stream(device) for _ in range(pool_size)]
        self.act_h2d: List[torch.cuda.Stream] = [torch.cuda.Stream(device)
                                                  for _ in range(pool_size)]
