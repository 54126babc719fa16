"""Projection + weighted cross-entropy without ever holding the sequence's logits.

Interface of the reference's kernels/loss.py (`active_rows` 6-16, `row_count` 19-20,
`projection_loss` 23-66) and of its host autograd function `ProjectionLoss`
(kernels/reference.py:30-73). Device inputs take `loss_cuda.FusedProjectionLoss`; host
inputs take `ProjectionLoss` below. Both visit the supervised rows in tiles of at most
`token_budget` rows.
"""

import torch
import torch.nn.functional as F


def active_rows(weights, device=None):
    """The rows with weight > 0, chosen where the weights live. No supervised rows, or all
    of them, give a slice; host weights whose supervised rows form one interval give that
    slice (so the loss reads views and gathers nothing); otherwise the row indices, moved
    to `device` when given."""
    supervised = weights.flatten() > 0
    total = supervised.numel()
    count = int(supervised.sum())
    if count in (0, total):
        return slice(0, count)
    if weights.device.type == "cpu":
        first = int(supervised.to(torch.uint8).argmax())
        last = total - 1 - int(supervised.flip(0).to(torch.uint8).argmax())
        if last - first + 1 == count:
            return slice(first, last + 1)
    indices = supervised.nonzero().flatten()
    return indices if device is None else indices.to(device)


def row_count(rows):
    if isinstance(rows, slice):
        return rows.stop - rows.start
    return len(rows)


def _check_backend(implementation, cut_chunk_size, head):
    """The reference's backend options: 'fused' is the path here; 'cut' (the
    cut-cross-entropy package, not carried by this framework) is refused as it refuses it."""
    if implementation == "cut":
        if head.requires_grad:
            raise ValueError("cut cannot guarantee FP32 head-gradient accumulation; use fused")
        raise RuntimeError("The cut backend requires cut-cross-entropy")
    if implementation != "fused":
        raise ValueError("Unsupported projection-loss backend")
    if cut_chunk_size:
        raise ValueError("cut_chunk_size applies only to the cut backend")


def projection_loss(hidden, head, targets, weights, *, token_budget=128, compute_dtype=torch.bfloat16,
                    implementation="fused", cut_chunk_size=0, reuse_hidden=False, rows=None):
    """sum_i weights[i] * CE(hidden[i] head^T, targets[i]) over the supervised rows, with at
    most `token_budget` rows of logits at a time. `reuse_hidden` lets the gradient of
    `hidden` take over its storage (an exclusive contiguous non-leaf tensor). `rows` is a
    precomputed `active_rows` selection."""
    if token_budget <= 0:
        raise ValueError("loss_token_budget must be positive")
    selection = active_rows(weights, hidden.device) if rows is None else rows
    if hidden.is_cuda and head.requires_grad and head.dtype == torch.float32:
        # The logits GEMM is the BLAS library's: its bf16 reductions stay in fp32.
        torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    _check_backend(implementation, cut_chunk_size, head)
    if not hidden.is_cuda:
        return ProjectionLoss.apply(hidden, head, targets, weights, token_budget, compute_dtype, selection)
    if not torch.is_grad_enabled():
        hidden, head = hidden.detach(), head.detach()
    if reuse_hidden and hidden.requires_grad:
        shared = hidden.is_leaf or hidden._base is not None or not hidden.is_contiguous()
        if shared:
            raise ValueError("Hidden reuse requires an exclusive contiguous non-leaf tensor")
    from .loss_cuda import FusedProjectionLoss
    total, _ = FusedProjectionLoss.apply(hidden, head, targets, weights, token_budget, compute_dtype,
                                         reuse_hidden, selection)
    return total


def _host_tiles(selection, tile):
    """(row selector, size) of each tile of the supervised rows."""
    count = row_count(selection)
    for offset in range(0, count, tile):
        size = min(tile, count - offset)
        if isinstance(selection, slice):
            yield slice(selection.start + offset, selection.start + offset + size), size
        else:
            yield selection[offset:offset + size], size


class ProjectionLoss(torch.autograd.Function):
    """Host route. Per tile the logits are formed in the compute dtype and widened to fp32
    for the CE; the backward forms them again (nothing but the inputs is saved), rounds the
    weighted softmax derivative (scaled by the upstream value) to the compute dtype, and
    accumulates d head in fp32 for an fp32 head."""

    @staticmethod
    def forward(ctx, hidden, head, targets, weights, tile, compute_dtype, active):
        ctx.tile, ctx.compute_dtype = tile, compute_dtype
        ctx.interval = active if isinstance(active, slice) else None
        ctx.save_for_backward(hidden, head, targets, weights, None if ctx.interval is not None else active)
        h, labels, scale = hidden.reshape(-1, hidden.shape[-1]), targets.flatten(), weights.flatten()
        matrix = head.to(compute_dtype)
        total = torch.zeros((), device=hidden.device, dtype=torch.float32)
        for where, _ in _host_tiles(active, tile):
            logits = F.linear(h[where].to(compute_dtype), matrix).float()
            total += (F.cross_entropy(logits, labels[where], reduction="none") * scale[where]).sum()
        return total

    @staticmethod
    def backward(ctx, upstream):
        hidden, head, targets, weights, indices = ctx.saved_tensors
        active = ctx.interval if ctx.interval is not None else indices
        dtype = ctx.compute_dtype
        h, labels, scale = hidden.reshape(-1, hidden.shape[-1]), targets.flatten(), weights.flatten()
        matrix = head.to(dtype)
        d_hidden = torch.zeros_like(h) if ctx.needs_input_grad[0] else None
        d_head = torch.zeros_like(head) if ctx.needs_input_grad[1] else None
        for where, size in _host_tiles(active, ctx.tile):
            x = h[where].to(dtype)
            probabilities = F.linear(x, matrix).float().softmax(dim=-1)
            probabilities[torch.arange(size), labels[where]] -= 1
            derivative = (probabilities * (scale[where] * upstream)[:, None]).to(dtype)
            if d_hidden is not None:
                d_hidden[where] = (derivative @ matrix).to(d_hidden.dtype)
            if d_head is None:
                continue
            if head.dtype == torch.float32:
                d_head.addmm_(derivative.float().T, x.float())   # fp32 product, fp32 sums
            else:
                d_head += (derivative.T @ x).to(d_head.dtype)
        result = None if d_hidden is None else d_hidden.reshape_as(hidden)
        return result, d_head, None, None, None, None, None
