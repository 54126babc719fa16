"""Weighted cross-entropy and the row-tiled projection loss on gfx950.

Interface of the reference's kernels/loss_cuda.py: `weighted_ce` (11-70) and
`FusedProjectionLoss` (81-162).

`weighted_ce` writes per-row weighted losses and, with `gradient=True`, overwrites the
logits with the weighted softmax derivative; it runs the HIP kernel ct_weighted_ce (two
launches over 4096-column splits, fixed reduction order). Its `partials` argument, the
reference's split-statistics buffer, is accepted for callers that pass it; the HIP kernel
keeps its statistics in its own workspace.

`FusedProjectionLoss` computes the loss and both gradients in its forward, tile by tile
over the supervised rows (`_SupervisedRows`), with one logits buffer for every tile:
logits = x head^T (the BLAS library's GEMM through torch.mm), the fused CE over them, then
d head += derivative^T x (`linear.accumulate`: fp32 output) and d hidden = derivative head
for the tile's rows. Its backward only scales the cached gradients.

d hidden reduces over the whole vocabulary into a [tile, d] output; for bf16 it runs
ct_gemm, which splits that reduction across the GPU (fixed-order fp32 partials): 1.6-3.4x
faster than hipBLASLt at 16-2048 rows of a 49152 x 2048 head on MI355X. The logits product
has a short reduction and a wide output, where hipBLASLt is as fast, and stays on torch.mm.
"""

import torch

from . import _native

_CE_ROWS = 65535  # rows per ct_weighted_ce call (the kernel's grid limit)


def weighted_ce(logits, targets, weights, *, gradient, loss=None, partials=None):
    rows, vocab = logits.shape
    if not logits.is_cuda:
        raise ValueError("weighted_ce expects device tensors")
    if logits.stride(1) != 1:
        raise ValueError("weighted_ce needs unit-stride logits rows")
    loss = torch.empty(rows, device=logits.device, dtype=torch.float32) if loss is None else loss
    labels = targets.to(torch.int64).contiguous()
    scale = weights.to(torch.float32).contiguous()
    lib = _native.library()
    code, pitch, stream = _native.dtype_code(logits.dtype), logits.stride(0), _native.stream_of(logits)
    for first in range(0, rows, _CE_ROWS):
        count = min(_CE_ROWS, rows - first)
        scratch = torch.empty(max(lib.ct_weighted_ce_workspace(count, vocab), 1), dtype=torch.uint8,
                              device=logits.device)
        window = slice(first, first + count)
        with _native.device_of(logits):
            status = lib.ct_weighted_ce(_native.ptr(logits[window]), code, count, vocab, pitch,
                                        _native.ptr(labels[window]), _native.ptr(scale[window]),
                                        _native.ptr(loss[window]), int(bool(gradient)), _native.ptr(scratch),
                                        scratch.numel(), stream)
        _native.check(status, "ct_weighted_ce")
    return loss


class _SupervisedRows:
    """The supervised rows of a flattened batch, visited in tiles of at most `tile` rows.

    An interval (a slice) is read through views and written in place; scattered rows (an
    index tensor) are gathered into staging buffers that every tile reuses and their
    gradients are scattered back with index_copy_."""

    def __init__(self, active, hidden, targets, weights, tile):
        self.active, self.tile = active, tile
        self.interval = isinstance(active, slice)
        self.count = (active.stop - active.start) if self.interval else len(active)
        self.hidden, self.targets, self.weights = hidden, targets, weights
        rows = min(tile, self.count)
        if not self.interval and rows:
            self.staged = (hidden.new_empty((rows, hidden.shape[-1])), targets.new_empty(rows),
                           weights.new_empty(rows))

    def __iter__(self):
        """(offset of the tile among the supervised rows, row selector, size)."""
        for offset in range(0, self.count, self.tile):
            size = min(self.tile, self.count - offset)
            if self.interval:
                first = self.active.start + offset
                yield offset, slice(first, first + size), size
            else:
                yield offset, self.active[offset:offset + size], size

    def gather(self, where, size):
        """(hidden rows, targets, weights) of one tile."""
        if self.interval:
            return self.hidden[where], self.targets[where], self.weights[where]
        rows, labels, scale = (buffer[:size] for buffer in self.staged)
        for source, buffer in ((self.hidden, rows), (self.targets, labels), (self.weights, scale)):
            torch.index_select(source, 0, where, out=buffer)
        return rows, labels, scale

    def clear_unsupervised(self, grad, holds_hidden):
        """Zero the gradient rows that no tile wrote. Rows outside an interval are always
        cleared; between scattered rows only when `grad` still holds the hidden values
        (fresh gradients of scattered rows start from zeros)."""
        if self.interval:
            grad[:self.active.start].zero_()
            grad[self.active.stop:].zero_()
        elif holds_hidden and self.count != len(grad):
            grad.masked_fill_(~(self.weights > 0)[:, None], 0)


class FusedProjectionLoss(torch.autograd.Function):
    """Sum over supervised rows of weight * CE(x head^T, target), gradients computed in the
    forward. `reuse` hands d hidden the storage of `hidden` (which must be an exclusive,
    contiguous non-leaf tensor): it is marked dirty and returned as the second output."""

    @staticmethod
    def forward(ctx, hidden, head, targets, weights, tile, dtype, reuse, active):
        from .linear import accumulate, product
        h = hidden.reshape(-1, hidden.shape[-1])
        rows = _SupervisedRows(active, h, targets.flatten(), weights.flatten(), tile)
        need_dh, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        reuse = reuse and need_dh
        if not need_dh:
            dh = None
        elif reuse:
            dh = h
        else:
            dh = torch.empty_like(h) if rows.interval else torch.zeros_like(h)
        dw = None if not need_dw else (torch.empty_like(head) if rows.count else torch.zeros_like(head))
        losses = torch.empty(rows.count, device=hidden.device, dtype=torch.float32)
        if rows.count:
            matrix = head.to(dtype)
            span = min(tile, rows.count)
            logits_buffer = torch.empty((span, len(matrix)), device=hidden.device, dtype=dtype)
            splits = -(-len(matrix) // 4096)
            statistics = (torch.empty((span, splits), device=hidden.device, dtype=torch.float32)
                          if splits > 1 else losses)
            # d hidden goes straight into its rows when they are an interval of the compute
            # dtype; otherwise through a staging buffer.
            in_place = rows.interval and dh is not None and dh.dtype == dtype
            staging = (torch.empty((span, h.shape[-1]), device=hidden.device, dtype=dtype)
                       if dh is not None and not in_place else None)
            for offset, where, size in rows:
                inputs, labels, scale = rows.gather(where, size)
                x = inputs.to(dtype)
                logits = logits_buffer[:size]
                torch.mm(x, matrix.T, out=logits)
                weighted_ce(logits, labels, scale, gradient=dh is not None or dw is not None,
                            loss=losses[offset:offset + size], partials=statistics[:size])
                # x may be a view of hidden's storage, which d hidden overwrites under reuse:
                # the head gradient reads it first.
                if dw is not None:
                    accumulate(dw, logits.T, x, add=offset > 0)
                if dh is None:
                    continue
                if in_place:
                    product(logits, matrix, dh[where])
                    continue
                tile_dh = staging[:size]
                product(logits, matrix, tile_dh)
                if rows.interval:
                    dh[where].copy_(tile_dh)
                else:
                    dh.index_copy_(0, where, tile_dh.to(dh.dtype))
        if dh is not None:
            rows.clear_unsupervised(dh, holds_hidden=reuse)
        if reuse:
            ctx.mark_dirty(hidden)
            dh = hidden
        elif dh is not None:
            dh = dh.reshape_as(hidden)
        if dh is not None:
            ctx.mark_non_differentiable(dh)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(dh, dw)
        return losses.sum(), dh

    @staticmethod
    def backward(ctx, upstream, _unused):
        dh, dw = ctx.saved_tensors
        # The training call's unit upstream returns the cached gradients themselves; any
        # other scale makes new tensors, so a repeated backward still finds them intact.
        if float(upstream) != 1:
            dh = None if dh is None else dh * upstream
            dw = None if dw is None else dw * upstream
        return dh, dw, None, None, None, None, None, None
