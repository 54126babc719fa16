"""The SwiGLU LoRA MLP as one autograd operator on gfx950.

Interface of the reference's kernels/mlp_cuda.py: `activation` (10-35, its Triton
`_activation`; here the HIP kernel `ct_silu_multiply`), `silu_multiply` (38-55),
`_forward_into` (58-81), `_TiledLoRAMLP` (84-143) and `tiled_lora_mlp` (146-161).

Design. One call builds an `_MLPProjections` view of the three projections: their frozen
bases as the HIP GEMMs consume them (`linear._Base`: packed NF4 is decoded inside the entry
points), their LoRA factors in the compute dtype (cast in one launch) and, when gate and up
share a rank, the stacked [a_gate; a_up] whose single GEMM gives both xa. Rows are processed
in tiles; per tile the forward is

    xa_gate | xa_up = x [a_gate; a_up]^T         (one GEMM, or one per projection)
    gate = x w_gate^T + xa_gate b_gate^T,  up = x w_up^T + xa_up b_up^T
    h = bf16(silu(gate)) * up                     (ct_silu_multiply)
    out = h w_down^T + (h a_down^T) b_down^T

and the backward runs the reference's analytic sequence without an autograd graph: the down
projection's input gradient dh, the SiLU backward in place of (gate, up, dh) giving (d gate,
d up, h), then dA/dB of down from h and of gate/up from x, and dx accumulated over gate and
up. In cache mode the forward keeps gate, up and their xa for every row and the backward
reads them instead of recomputing the two GEMMs; the activation backward then writes its
results into separate tile buffers so the kept values survive a repeated backward.
"""

import torch

from . import _native
from .linear import _Base, _low_rank, forward_linear, fusable, group_dx_ready, group_factors, group_input_gradient, \
    input_gradient, parameter_gradients, projection_parameters, stacked_rows


# ----------------------------------------------------------------------------- SiLU x up
def _silu_kernel(gate, up, hidden, d_gate, d_up, *, backward, reconstruct):
    """ct_silu_multiply over whole contiguous tensors of one device dtype."""
    operands = [t for t in (gate, up, hidden, d_gate, d_up) if t is not None]
    if any(not (t.is_cuda and t.is_contiguous() and t.dtype == gate.dtype) for t in operands):
        raise ValueError("activation expects contiguous device tensors of one dtype")
    code = _native.dtype_code(gate.dtype)
    if code == _native.CT_F16:
        raise NotImplementedError("activation: the HIP kernel takes bfloat16 or float32")
    with _native.device_of(gate):
        status = _native.library().ct_silu_multiply(
            _native.ptr(gate), _native.ptr(up), _native.ptr(hidden), _native.ptr(d_gate), _native.ptr(d_up),
            gate.numel(), int(backward), int(reconstruct), code, _native.stream_of(gate))
    _native.check(status, "ct_silu_multiply")


def activation(gate, up, gradient=None, *, out=None):
    """Forward: returns h = dtype(silu(gate)) * up (in `out` when given). With `gradient`
    (the upstream dh) the backward runs in place: gate becomes d gate, up becomes d up and
    `gradient` is overwritten with h, which is returned."""
    if gradient is None:
        hidden = torch.empty_like(gate) if out is None else out
        _silu_kernel(gate, up, hidden, None, None, backward=False, reconstruct=True)
        return hidden
    _silu_kernel(gate, up, gradient, gate, up, backward=True, reconstruct=True)
    return gradient


class _SiLUMultiply(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, up):
        operands = gate.contiguous(), up.contiguous()
        ctx.save_for_backward(*operands)
        return activation(*operands)

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        d_gate, d_up = torch.empty_like(gate), torch.empty_like(up)
        _silu_kernel(gate, up, grad.contiguous(), d_gate, d_up, backward=True, reconstruct=False)
        return d_gate, d_up


def silu_multiply(gate, up):
    return _SiLUMultiply.apply(gate, up)


# ----------------------------------------------------------------------------- projections
GATE, UP, DOWN = 0, 1, 2


class _MLPProjections:
    """Bases and compute-dtype factors of gate, up and down for one forward or backward."""

    def __init__(self, parameters, states, dtype, x):
        self.dtype, self.device = dtype, x.device
        self.bases = [_Base(parameters[4 * i], state, dtype) for i, state in enumerate(states)]
        factors, self.stacked = group_factors(parameters, 3, dtype, x, shared=2)
        self.a, self.b = factors[0::2], factors[1::2]
        self.rank = [len(a) for a in self.a]
        self.width = int(states[GATE].shape[0]) if states[GATE] is not None else len(parameters[0])

    def empty(self, *shape):
        return torch.empty(shape, device=self.device, dtype=self.dtype)

    def xa_buffer(self, rows):
        """Storage for xa_gate and xa_up over `rows` rows: the two column halves of one
        [rows, 2r] buffer when the stacked GEMM fills them, else two buffers."""
        if self.stacked is not None:
            pair = self.empty(rows, 2 * self.rank[GATE])
            return pair, (pair[:, :self.rank[GATE]], pair[:, self.rank[GATE]:])
        return None, (self.empty(rows, self.rank[GATE]), self.empty(rows, self.rank[UP]))

    def project(self, which, x, out, xa, epilogue=None):
        """out = x w^T + (x a^T) b^T for one projection, xa = x a^T written; `epilogue` an
        elementwise step fused into the GEMM's output."""
        if epilogue is None:
            forward_linear(x, self.bases[which], self.a[which], self.b[which], out=out, xa=xa)
        else:
            self.bases[which].forward(x, self.a[which], self.b[which], None, out, xa, epilogue=epilogue)

    def gate_up(self, x, gate, up, pair, xa, epilogue=None):
        """gate and up of one tile (`epilogue` applies to up's output, which gate precedes).
        With the stacked factors their xa come from one GEMM into `pair` (whose column
        halves are xa) and the projections read them."""
        if self.stacked is None or not len(x):
            self.project(GATE, x, gate, xa[GATE])
            self.project(UP, x, up, xa[UP], epilogue)
            return
        _low_rank(x, self.stacked, pair, transpose=True)
        for which, out in ((GATE, gate), (UP, up)):
            self.bases[which].forward(x, self.a[which], self.b[which], None, out, xa[which], xa_given=True,
                                      epilogue=epilogue if which == UP else None)

    def input_gradient(self, which, dy, dx, low, add, epilogue=None):
        if epilogue is None:
            input_gradient(dy, self.bases[which], self.a[which], self.b[which], dx, low, add=add)
        else:
            self.bases[which].input_gradient(dy, self.a[which], self.b[which], dx, low, add, epilogue)

    def low_product(self, which, dy, low):
        """low = dy b, when the input gradient is not needed."""
        _low_rank(dy, self.b[which], low, transpose=False)


def _tile_starts(rows, tile):
    return range(0, rows, tile)


# ----------------------------------------------------------------------------- forward
@torch.no_grad()
def _forward_into(output, x, dtype, tile, states, parameters, residual, *, save=False):
    """Fill `output` (the MLP's result, plus `residual`) tile by tile. With `save`, return
    (gate, up, xa_gate, xa_up) over all rows for the cached backward; else ()."""
    flat = x.reshape(-1, x.shape[-1]).to(dtype)
    rows = len(flat)
    mlp = _MLPProjections(parameters, states, dtype, flat)
    span = min(tile, rows)
    target = output.view(rows, -1)
    xa_down = mlp.empty(span, mlp.rank[DOWN])
    if save:
        gate_all, up_all = mlp.empty(rows, mlp.width), mlp.empty(rows, mlp.width)
        pair_all, xa_all = mlp.xa_buffer(rows)
        hidden_tile = mlp.empty(span, mlp.width)
    else:
        gate_tile, up_tile = mlp.empty(span, mlp.width), mlp.empty(span, mlp.width)
        pair_tile, xa_tile = mlp.xa_buffer(span)
    # SiLU x up runs in the up GEMM's epilogue (the raw up kept beside h in cache mode) and
    # the residual add in the down GEMM's, when the buffers allow it.
    fused = fusable(target, flat, *((gate_all, up_all, hidden_tile) if save else (gate_tile, up_tile)))
    residual_flat = None if residual is None else residual.reshape(rows, -1)
    residual_fused = residual_flat is not None and fused and fusable(residual_flat)
    for start in _tile_starts(rows, tile):
        part = flat[start:start + tile]
        n = len(part)
        window = slice(start, start + n)
        if save:
            gate, up = gate_all[window], up_all[window]
            pair = None if pair_all is None else pair_all[window]
            xa = tuple(value[window] for value in xa_all)
            hidden = hidden_tile[:n]
        else:
            gate, up = gate_tile[:n], up_tile[:n]
            pair = None if pair_tile is None else pair_tile[:n]
            xa = tuple(value[:n] for value in xa_tile)
            # h overwrites the tile's up (fused) or gate, neither needed after it
            hidden = up if fused else gate
        if fused:
            # up's GEMM writes h; in cache mode its raw output goes to the kept up
            silu = _native.epilogue(_native.CT_EPI_SILU, n, in0=gate, out0=up if save else None)
            mlp.gate_up(part, gate, hidden if save else up, pair, xa, silu)
        else:
            mlp.gate_up(part, gate, up, pair, xa)
            activation(gate, up, out=hidden)
        add = (_native.epilogue(_native.CT_EPI_RESIDUAL, n, in0=residual_flat[window]) if residual_fused
               else None)
        mlp.project(DOWN, hidden, target[window], xa_down[:n], add)
    if residual is not None and not residual_fused:
        output.add_(residual)
    return (gate_all, up_all, *xa_all) if save else ()


# ----------------------------------------------------------------------------- backward
def _backward(ctx, grad, x, kept, parameters):
    dtype, tile = ctx.dtype, ctx.tile
    flat = x.reshape(-1, x.shape[-1]).to(dtype)
    upstream = grad.reshape_as(flat).to(dtype)
    rows = len(flat)
    dx = torch.empty_like(flat) if ctx.needs_input_grad[0] else None
    mlp = _MLPProjections(parameters, ctx.states, dtype, flat)
    # fp32 adapter gradients; zeros when there are no rows (nothing accumulates into them)
    fresh = torch.empty_like if rows else torch.zeros_like
    grads = [(fresh(parameters[4 * i + 1]), fresh(parameters[4 * i + 2])) for i in range(3)]
    span = min(tile, rows)
    # From GROUP_DX_ROWS rows gate's and up's input gradients are one contraction over
    # [d gate | d up]: the two tile buffers are then the column halves of one matrix.
    grouped = (dx is not None and flat.is_cuda and dtype == torch.bfloat16
               and group_dx_ready(mlp.bases[:2], [mlp.width] * 2, mlp.rank[:2], span))
    # three [tile, width] buffers: (gate, up, dh) in, (d gate, d up, h) out
    if grouped:
        joined = mlp.empty(span, 2 * mlp.width)
        first, second = joined[:, :mlp.width], joined[:, mlp.width:]
        third = mlp.empty(span, mlp.width)
        low_pair = mlp.empty(span, mlp.rank[GATE] + mlp.rank[UP])
        a_stack = mlp.stacked if mlp.stacked is not None else stacked_rows(mlp.a[:2])
    else:
        first, second, third = (mlp.empty(span, mlp.width) for _ in range(3))
    low = mlp.empty(span, max(mlp.rank))
    xa_down = mlp.empty(span, mlp.rank[DOWN])
    pair_tile, xa_tile = (None, None) if kept else mlp.xa_buffer(span)
    # The SiLU backward runs in the epilogue of down's input-gradient GEMM when it can.
    fused = fusable(flat, first, *kept[:2])
    for start in _tile_starts(rows, tile):
        part, dy = flat[start:start + tile], upstream[start:start + tile]
        n = len(part)
        window = slice(start, start + n)
        d_gate, d_up, d_hidden = first[:n], second[:n], third[:n]
        if kept:
            xa = (kept[2][window], kept[3][window])
        else:
            xa = tuple(value[:n] for value in xa_tile)
            mlp.gate_up(part, d_gate, d_up, None if pair_tile is None else pair_tile[:n], xa)
        # dh, then (gate, up, dh) -> (d gate, d up, h): the tile buffers receive d gate and
        # d up (in place of the recomputed gate/up, or beside the kept ones) and h lands
        # over dh; fused into the dh GEMM's epilogue when the buffers allow it.
        gate, up = (kept[0][window], kept[1][window]) if kept else (d_gate, d_up)
        dsilu = (_native.epilogue(_native.CT_EPI_DSILU, n, in0=gate, in1=up, out0=d_gate, out1=d_up) if fused
                 else None)
        mlp.input_gradient(DOWN, dy, d_hidden, low[:n, :mlp.rank[DOWN]], False, dsilu)
        if not fused and grouped:
            # the separate kernel takes contiguous operands: column halves go through copies
            g, u = gate.contiguous(), up.contiguous()
            dg, du = torch.empty_like(g), torch.empty_like(u)
            _silu_kernel(g, u, d_hidden, dg, du, backward=True, reconstruct=True)
            d_gate.copy_(dg)
            d_up.copy_(du)
        elif not fused:
            _silu_kernel(gate, up, d_hidden, d_gate, d_up, backward=True, reconstruct=True)
        hidden = d_hidden
        _low_rank(hidden, mlp.a[DOWN], xa_down[:n], transpose=True)
        parameter_gradients(hidden, dy, *grads[DOWN], low[:n, :mlp.rank[DOWN]], xa_down[:n], add=start > 0)
        if grouped:
            group_input_gradient(mlp.bases[:2], joined[:n], [mlp.width] * 2, mlp.rank[:2], a_stack, mlp.b[:2],
                                 dx[window], low_pair[:n], False)
            for which, signal, columns in ((GATE, d_gate, slice(0, mlp.rank[GATE])),
                                           (UP, d_up, slice(mlp.rank[GATE], mlp.rank[GATE] + mlp.rank[UP]))):
                parameter_gradients(part, signal, *grads[which], low_pair[:n, columns], xa[which], add=start > 0)
            continue
        for which, signal in ((GATE, d_gate), (UP, d_up)):
            grad_low = low[:n, :mlp.rank[which]]
            if dx is not None:
                mlp.input_gradient(which, signal, dx[window], grad_low, which == UP)
            else:
                mlp.low_product(which, signal, grad_low)
            parameter_gradients(part, signal, *grads[which], grad_low, xa[which], add=start > 0)
    if dx is not None:
        dx = dx.reshape_as(x).to(x.dtype)
    return dx, [value for da, db in grads for value in (None, da, db, None)]


class _TiledLoRAMLP(torch.autograd.Function):
    """Saves the input and the parameters, plus (cache mode) gate, up and their xa. Outside
    cache mode the forward only registers what it saves and returns an empty output that
    `tiled_lora_mlp` fills with `_forward_into`, so a checkpoint replay that needs no
    output can stop before any GEMM (reference mlp_cuda.py:94-97)."""

    @staticmethod
    def forward(ctx, x, dtype, tile, states, residual, cache, *parameters):
        ctx.dtype, ctx.tile, ctx.states, ctx.cache = dtype, tile, states, cache
        output = torch.empty(x.shape, device=x.device, dtype=dtype)
        kept = _forward_into(output, x, dtype, tile, states, parameters, residual, save=True) if cache else ()
        ctx.save_for_backward(x, *kept, *parameters)
        return output

    @staticmethod
    def backward(ctx, grad):
        x, *rest = ctx.saved_tensors
        kept, parameters = (rest[:4], rest[4:]) if ctx.cache else ((), rest)
        dx, adapter_grads = _backward(ctx, grad, x, kept, parameters)
        residual_grad = grad if ctx.needs_input_grad[4] else None
        return (dx, None, None, None, residual_grad, None, *adapter_grads)


def tiled_lora_mlp(module, x, residual=None, *, tile=None, cache=None):
    """The MLP of `module` (gate_proj, up_proj, down_proj, tile, cache_intermediates; the
    reference's modeling/model.py:111-139) on x, plus `residual`."""
    projections = (module.gate_proj, module.up_proj, module.down_proj)
    dtype = projections[0].compute_dtype
    if residual is not None and (residual.dtype != dtype or residual.shape != x.shape):
        return tiled_lora_mlp(module, x, tile=tile, cache=cache) + residual
    parameters, states = [], []
    for projection in projections:
        values, state = projection_parameters(projection)
        parameters += values
        states.append(state)
    rows = x.numel() // x.shape[-1]
    tile = (tile if tile is not None else module.tile) or max(1, rows)
    cache = bool(module.cache_intermediates if cache is None else cache) and torch.is_grad_enabled()
    output = _TiledLoRAMLP.apply(x, dtype, tile, tuple(states), residual, cache, *parameters)
    if not cache:
        _forward_into(output, x, dtype, tile, states, parameters, residual)
    return output
