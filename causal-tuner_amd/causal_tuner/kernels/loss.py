"""Projection + weighted cross-entropy with bounded logits (the reference's kernels/loss.py).

`projection_loss` keeps the reference's signature, validation and dispatch (loss.py:23-66):
device tensors take `FusedProjectionLoss` (kernels/loss_cuda.py), whose weighted CE runs
in the HIP kernel ct_weighted_ce; host tensors take `ProjectionLoss` below, the
reference's host autograd function (kernels/reference.py:30-73) restated with the same
rounding points. `active_rows` / `row_count` select the supervised rows on the host
(loss.py:6-20).
"""

import torch
import torch.nn.functional as F


def active_rows(weights, device=None):
    """Rows with weight > 0: a slice when they are all rows, none, or (for host weights)
    one contiguous interval; otherwise an index tensor (moved to `device`). loss.py:6-16."""
    indices = torch.nonzero(weights.flatten() > 0, as_tuple=False).flatten()
    count = len(indices)
    if not count or count == weights.numel():
        return slice(0, count)
    if weights.device.type == "cpu":
        first, last = int(indices[0]), int(indices[-1])
        if last - first + 1 == count:
            return slice(first, last + 1)
    return indices.to(device) if device is not None else indices


def row_count(rows):
    return rows.stop - rows.start if isinstance(rows, slice) else len(rows)


def projection_loss(hidden, head, targets, weights, *, token_budget=128, compute_dtype=torch.bfloat16,
                    implementation="fused", cut_chunk_size=0, reuse_hidden=False, rows=None):
    """Sum over supervised rows of weight * CE(hidden @ head^T, target), never holding more
    than `token_budget` rows of logits. reuse_hidden lets the backward's dHidden take over
    `hidden`'s storage (an exclusive contiguous non-leaf output). loss.py:23-66."""
    if token_budget <= 0:
        raise ValueError("loss_token_budget must be positive")
    rows = active_rows(weights, hidden.device) if rows is None else rows
    if hidden.is_cuda and head.requires_grad and head.dtype == torch.float32:
        # The logits GEMM goes through the BLAS library: keep its bf16 reductions in fp32.
        torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    if implementation == "cut":
        if head.requires_grad:
            raise ValueError("cut cannot guarantee FP32 head-gradient accumulation; use fused")
        # The reference's cut backend is the cut-cross-entropy package, which this
        # framework does not carry.
        raise RuntimeError("The cut backend requires cut-cross-entropy")
    if implementation != "fused":
        raise ValueError("Unsupported projection-loss backend")
    if cut_chunk_size:
        raise ValueError("cut_chunk_size applies only to the cut backend")
    if hidden.is_cuda:
        from .loss_cuda import FusedProjectionLoss
        if not torch.is_grad_enabled():
            hidden, head = hidden.detach(), head.detach()
        if reuse_hidden and hidden.requires_grad and (hidden.is_leaf or hidden._base is not None
                                                      or not hidden.is_contiguous()):
            raise ValueError("Hidden reuse requires an exclusive contiguous non-leaf tensor")
        return FusedProjectionLoss.apply(hidden, head, targets, weights, token_budget, compute_dtype,
                                         reuse_hidden, rows)[0]
    return ProjectionLoss.apply(hidden, head, targets, weights, token_budget, compute_dtype, rows)


class ProjectionLoss(torch.autograd.Function):
    """Host route: per tile of rows, logits in the compute dtype widened to fp32, CE times
    weight; the backward recomputes the tile's logits (reference.py:30-73)."""

    @staticmethod
    def forward(ctx, hidden, head, targets, weights, tile, compute_dtype, active):
        ctx.tile, ctx.compute_dtype = tile, compute_dtype
        ctx.interval = active if isinstance(active, slice) else None
        ctx.save_for_backward(hidden, head, targets, weights, None if ctx.interval is not None else active)
        h, t, w = hidden.reshape(-1, hidden.shape[-1]), targets.flatten(), weights.flatten()
        matrix = head.to(compute_dtype)
        total = torch.zeros((), device=hidden.device, dtype=torch.float32)
        count = row_count(active)
        for start in range(0, count, tile):
            rows = (slice(active.start + start, active.start + min(start + tile, count))
                    if ctx.interval is not None else active[start:start + tile])
            logits = F.linear(h[rows].to(compute_dtype), matrix).float()
            total.add_((F.cross_entropy(logits, t[rows], reduction="none") * w[rows]).sum())
        return total

    @staticmethod
    def backward(ctx, upstream):
        hidden, head, targets, weights, active = ctx.saved_tensors
        active = ctx.interval if ctx.interval is not None else active
        h, t, w = hidden.reshape(-1, hidden.shape[-1]), targets.flatten(), weights.flatten()
        matrix = head.to(ctx.compute_dtype)
        dh = torch.zeros_like(h) if ctx.needs_input_grad[0] else None
        dw = torch.zeros_like(head) if ctx.needs_input_grad[1] else None
        count = row_count(active)
        for start in range(0, count, ctx.tile):
            size = min(ctx.tile, count - start)
            rows = (slice(active.start + start, active.start + start + size) if ctx.interval is not None
                    else active[start:start + size])
            x = h[rows].to(ctx.compute_dtype)
            logits = F.linear(x, matrix).float()
            derivative = logits.softmax(-1)
            derivative[torch.arange(size, device=h.device), t[rows]] -= 1
            derivative.mul_((w[rows] * upstream)[:, None])
            derivative = derivative.to(ctx.compute_dtype)
            if dh is not None:
                dh[rows] = (derivative @ matrix).to(dh.dtype)
            if dw is not None:
                if head.dtype == torch.float32:
                    dw.addmm_(derivative.float().T, x.float())  # fp32 product and fp32 tile sums
                else:
                    dw.add_((derivative.T @ x).to(dw.dtype))
        return None if dh is None else dh.reshape_as(hidden), dw, None, None, None, None, None
