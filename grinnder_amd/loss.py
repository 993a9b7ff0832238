"""Masked cross-entropy and accuracy of a partition's logits on the GPU.

Replaces the loss and metric code of the reference trainer:
``F.cross_entropy(out[train], y[train], reduction="sum"|"mean")``
(grinnder/engine/trainer.py:709-721 per partition, :430-453 fast path) and
``compute_micro_f1`` (grinnder/utils.py:24-44) for the val / test rows.  One
HIP pass (``gr_xent_forward``) reads the logits once and produces the loss,
the accuracy counts and the gradient of the train-row nll sum; the backward
only scales that gradient, so the logits may be released after the forward
(the partitioned trainer frees the last layer's output right away).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from grinnder_amd import _lib

TRAIN, VAL, TEST = 1, 2, 4
_STATS = 7            # per-workgroup partial statistics of gr_xent_forward
_ROWS_PER_BLOCK = 256


def mask_codes(train: Optional[Tensor], val: Optional[Tensor] = None,
               test: Optional[Tensor] = None) -> Tensor:
    """uint8 row codes: bit 0 train, bit 1 val, bit 2 test (same device as `train`)."""
    code = train.to(torch.uint8) * TRAIN
    if val is not None:
        code = code | (val.to(code.device).to(torch.uint8) * VAL)
    if test is not None:
        code = code | (test.to(code.device).to(torch.uint8) * TEST)
    return code.contiguous()


class _MaskedCrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits: Tensor, labels: Tensor, codes: Tensor, mean: bool):
        if logits.stride(-1) != 1:
            logits = logits.contiguous()
        rows, classes = logits.shape
        dev = logits.device
        loss = torch.empty((), dtype=torch.float32, device=dev)
        stats = torch.empty(6, dtype=torch.int64, device=dev)
        nblk = max(1, (rows + _ROWS_PER_BLOCK - 1) // _ROWS_PER_BLOCK)
        ws = torch.empty(nblk * _STATS, dtype=torch.float64, device=dev)
        need_grad = ctx.needs_input_grad[0]
        grad = torch.empty((rows, classes), dtype=torch.float32, device=dev) if need_grad \
            else None
        _lib.call("gr_xent_forward", logits.data_ptr(), logits.stride(0), rows, classes,
                  labels.data_ptr(), codes.data_ptr(), int(mean), None, _lib.ptr(grad),
                  classes, loss.data_ptr(), stats.data_ptr(), ws.data_ptr(), ws.numel(),
                  _lib.stream_handle())
        if need_grad:
            ctx.save_for_backward(grad, stats)
        ctx.mean = mean
        ctx.mark_non_differentiable(stats)
        return loss, stats

    @staticmethod
    def backward(ctx, gloss: Tensor, _gstats):
        grad, stats = ctx.saved_tensors
        scale = gloss.to(torch.float32)
        if ctx.mean:
            scale = scale / stats[0].clamp(min=1).to(torch.float32)
        return grad * scale, None, None, None


def masked_cross_entropy(logits: Tensor, labels: Tensor, codes: Tensor,
                         reduction: str = "mean") -> Tuple[Tensor, Tensor]:
    """(loss, stats) over the rows of `logits` [rows, C] selected by `codes`.

    loss: 0-dim fp32 device tensor, sum or mean of the train-row nll (0 with
    no train rows, with a zero gradient, like the reference's ``out.sum() * 0``).
    stats: int64 device tensor [train rows, val correct, val rows,
    test correct, test rows, rows with an out-of-range label].
    """
    if reduction not in ("sum", "mean"):
        raise ValueError(f"reduction must be 'sum' or 'mean', got {reduction!r}")
    if not logits.is_cuda or logits.dtype != torch.float32 or logits.dim() != 2:
        raise RuntimeError("masked_cross_entropy: logits must be a 2-D fp32 GPU tensor")
    if labels.dtype != torch.int64 or codes.dtype != torch.uint8:
        raise RuntimeError("masked_cross_entropy: labels int64 and codes uint8 expected")
    if labels.numel() != logits.size(0) or codes.numel() != logits.size(0):
        raise ValueError("masked_cross_entropy: one label and one code per row expected")
    return _MaskedCrossEntropy.apply(logits, labels.contiguous(), codes.contiguous(),
                                     reduction == "mean")


def check_stats(stats: list) -> None:
    """Raises like torch's NLL for labels outside [0, C) on selected rows."""
    if stats[5]:
        raise IndexError(f"cross_entropy: {stats[5]} selected rows have a label outside "
                         "[0, num_classes)")
