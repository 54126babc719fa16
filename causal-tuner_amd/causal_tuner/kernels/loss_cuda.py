"""Fused weighted cross-entropy and the tiled projection loss on gfx950 (the reference's
kernels/loss_cuda.py).

`weighted_ce` (loss_cuda.py:11-70) keeps the reference's signature and contract: per-row
weighted losses, and with `gradient=True` the logits overwritten in place by the weighted
softmax derivative. It runs the HIP kernel ct_weighted_ce (4096-column splits per row as
the reference's _statistics/_finish, fixed reduction order) with its own workspace; the
reference's `partials` argument is accepted and not needed. `FusedProjectionLoss` (loss_cuda.py:81-162) drives it tile by tile.
"""

import torch

from . import _native

_CE_ROWS = 65535  # rows per ct_weighted_ce call


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
    lib = _native.library()
    for start in range(0, rows, _CE_ROWS):
        part = min(_CE_ROWS, rows - start)
        workspace = torch.empty(max(lib.ct_weighted_ce_workspace(part, vocab), 1), dtype=torch.uint8,
                                device=logits.device)
        with _native.device_of(logits):
            status = lib.ct_weighted_ce(
                _native.ptr(logits[start:start + part]), _native.dtype_code(logits.dtype), part, vocab,
                logits.stride(0), _native.ptr(targets[start:start + part]), _native.ptr(weights[start:start + part]),
                _native.ptr(loss[start:start + part]), int(bool(gradient)), _native.ptr(workspace), workspace.numel(),
                _native.stream_of(logits))
        _native.check(status, "ct_weighted_ce")
    return loss


class FusedProjectionLoss(torch.autograd.Function):
    """Projection + weighted CE over tiles of at most `tile` supervised rows, gradients
    computed once in the forward (the reference's kernels/loss_cuda.py:81-162).

    Per tile: logits = x head^T (the BLAS library's GEMM, as in the reference), then the
    HIP kernel ct_weighted_ce writes the weighted losses and overwrites the logits with the
    weighted softmax derivative; dHead += derivative^T x runs in `accumulate` (fp32 output;
    the HIP GEMM for bf16 operands); dHidden = derivative head goes to its rows. The
    backward only scales the cached gradients. One logits workspace serves every tile."""

    @staticmethod
    def forward(ctx, hidden, head, targets, weights, tile, dtype, reuse_hidden, active):
        from .linear import accumulate
        from .loss import row_count
        h = hidden.reshape(-1, hidden.shape[-1])
        t, w = targets.flatten(), weights.flatten()
        count = row_count(active)
        contiguous = isinstance(active, slice)
        reuse_hidden = reuse_hidden and ctx.needs_input_grad[0]
        allocate = torch.empty_like if contiguous else torch.zeros_like
        dh = (h if reuse_hidden else allocate(h)) if ctx.needs_input_grad[0] else None
        dw = (torch.empty_like(head) if count else torch.zeros_like(head)) if ctx.needs_input_grad[1] else None
        losses = torch.empty(count, device=hidden.device, dtype=torch.float32)
        rows = min(tile, count)
        # dHidden rows can be written straight into place when they form one interval and
        # the destination has the compute dtype.
        direct = contiguous and dh is not None and dh.dtype == dtype
        if rows:
            matrix = head.to(dtype)
            workspace = torch.empty((rows, len(matrix)), device=hidden.device, dtype=dtype)
            if not contiguous:
                inputs = h.new_empty((rows, h.shape[-1]))
                labels, factors = t.new_empty(rows), w.new_empty(rows)
            signals = (torch.empty((rows, h.shape[-1]), device=hidden.device, dtype=dtype)
                       if dh is not None and not direct else None)
            # The reference's split-statistics workspace, kept so that callers (and tests)
            # that inspect weighted_ce's arguments see the same contract.
            splits = -(-len(matrix) // 4096)
            partials = (torch.empty((rows, splits), device=hidden.device, dtype=torch.float32)
                        if splits > 1 else losses)
        for start in range(0, count, tile):
            size = min(tile, count - start)
            if contiguous:
                indices = slice(active.start + start, active.start + start + size)
                x, target, weight = h[indices].to(dtype), t[indices], w[indices]
            else:
                indices = active[start:start + size]
                torch.index_select(h, 0, indices, out=inputs[:size])
                torch.index_select(t, 0, indices, out=labels[:size])
                torch.index_select(w, 0, indices, out=factors[:size])
                x, target, weight = inputs[:size].to(dtype), labels[:size], factors[:size]
            logits = workspace[:size]
            torch.mm(x, matrix.T, out=logits)
            weighted_ce(logits, target, weight, gradient=dh is not None or dw is not None,
                        loss=losses[start:start + size], partials=partials[:size])
            # With reuse, dHidden's rows are x's storage: the head gradient reads x first.
            if dw is not None:
                accumulate(dw, logits.T, x, add=start > 0)
            if dh is not None:
                if direct:
                    torch.mm(logits, matrix, out=dh[indices])
                else:
                    torch.mm(logits, matrix, out=signals[:size])
                    if contiguous:
                        dh[indices].copy_(signals[:size])
                    else:
                        dh.index_copy_(0, indices, signals[:size].to(dh.dtype))
        if dh is not None and contiguous:
            if active.start:
                dh[:active.start].zero_()
            if active.stop < len(h):
                dh[active.stop:].zero_()
        if reuse_hidden:
            # Scattered supervision: active rows were gathered before their storage was
            # overwritten; the remaining (unsupervised) rows still hold hidden values.
            if not contiguous and count != len(h):
                dh.view(len(w), -1).masked_fill_(~(w > 0)[:, None], 0)
            ctx.mark_dirty(hidden)
            dh = hidden
        elif dh is not None:
            dh = dh.reshape_as(hidden)
        if dh is not None:
            ctx.mark_non_differentiable(dh)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(dh, dw)
        # Returning the consumed input lets autograd see its in-place change.
        return losses.sum(), dh

    @staticmethod
    def backward(ctx, upstream, unused):
        dh, dw = ctx.saved_tensors
        # Unit upstream (the training call) returns the cached gradients; any other scale
        # makes new tensors, so the cache stays valid for a repeated backward.
        scale = float(upstream)
        if scale != 1:
            dh = None if dh is None else dh * upstream
            dw = None if dw is None else dw * upstream
        return dh, dw, None, None, None, None, None, None
