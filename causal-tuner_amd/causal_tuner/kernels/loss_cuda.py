"""Fused weighted cross-entropy on gfx950 (the reference's kernels/loss_cuda.py:11-70).

`weighted_ce` keeps the reference's signature and contract: per-row weighted losses, and
with `gradient=True` the logits overwritten in place by the weighted softmax derivative.
It runs the HIP kernel ct_weighted_ce (one workgroup per row, fixed reduction order); the
`partials` workspace of the reference's split statistics is accepted and not needed.
"""

import torch

from . import _native


def weighted_ce(logits, targets, weights, *, gradient, loss=None, partials=None):
    """Write per-row weighted losses and optionally overwrite logits with derivatives."""
    rows, vocab = logits.shape
    if not logits.is_cuda:
        raise ValueError("weighted_ce expects device tensors")
    if logits.stride(1) != 1:
        raise ValueError("weighted_ce needs unit-stride logits rows")
    if loss is None:
        loss = torch.empty(rows, device=logits.device, dtype=torch.float32)
    targets = targets.to(torch.int64).contiguous()
    weights = weights.to(torch.float32).contiguous()
    if rows:
        with torch.cuda.device(logits.device):
            status = _native.library().ct_weighted_ce(
                _native.ptr(logits), _native.dtype_code(logits.dtype), rows, vocab, logits.stride(0),
                _native.ptr(targets), _native.ptr(weights), _native.ptr(loss), int(bool(gradient)),
                _native.stream_of(logits))
        _native.check(status, "ct_weighted_ce")
    return loss
