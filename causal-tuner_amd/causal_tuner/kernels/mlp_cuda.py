"""Tiled LoRA MLP with the SiLU-multiply and a graph-free analytic backward, on gfx950.

Same operator API as the reference's kernels/mlp_cuda.py: `activation` (10-35, the Triton
`_activation` kernel, here `ct_silu_multiply`), `_SiLUMultiply` / `silu_multiply` (38-55),
`_forward_into` (58-81), `_TiledLoRAMLP` (84-143) and `tiled_lora_mlp` (146-161). Gate, up and
down are NF4-LoRA projections on the helpers of kernels/linear.py; a packed NF4 base stays
packed below 512 rows (the GEMMs decode it in LDS) and is decoded once per call above.
"""

import torch

from . import _native
from .linear import _Base, group_factors, forward_linear, input_gradient, parameter_gradients, projection_parameters, _low_rank


def _silu(gate, up, h, dg, du, backward, reconstruct):
    tensors = [t for t in (gate, up, h, dg, du) if t is not None]
    if not all(t.is_cuda and t.is_contiguous() and t.dtype == gate.dtype for t in tensors):
        raise ValueError("activation expects contiguous device tensors of one dtype")
    code = _native.dtype_code(gate.dtype)
    if code == _native.CT_F16:
        raise NotImplementedError("activation: the HIP kernel takes bfloat16 or float32")
    with _native.device_of(gate):
        status = _native.library().ct_silu_multiply(
            _native.ptr(gate), _native.ptr(up), _native.ptr(h), _native.ptr(dg), _native.ptr(du), gate.numel(),
            int(backward), int(reconstruct), code, _native.stream_of(gate))
    _native.check(status, "ct_silu_multiply")


def activation(gate, up, gradient=None, *, out=None):
    """h = dtype(silu(gate)) * up (reference mlp_cuda.py:28-35). With `gradient`, the
    backward in place: gate <- d gate, up <- d up, gradient <- h."""
    if gradient is not None:
        out = gradient
    elif out is None:
        out = torch.empty_like(gate)
    if gradient is not None:
        _silu(gate, up, out, gate, up, True, True)
    else:
        _silu(gate, up, out, None, None, False, True)
    return out


class _SiLUMultiply(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, up):
        gate, up = gate.contiguous(), up.contiguous()
        ctx.save_for_backward(gate, up)
        return activation(gate, up)

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        dg, du = torch.empty_like(gate), torch.empty_like(up)
        _silu(gate, up, grad.contiguous(), dg, du, True, False)
        return dg, du


def silu_multiply(gate, up):
    return _SiLUMultiply.apply(gate, up)


def _bases(parameters, states, dtype):
    return [_Base(parameters[4*i], state, dtype) for i, state in enumerate(states)]


@torch.no_grad()
def _forward_into(output, x, dtype, tile, states, parameters, residual, *, save=False):
    flat = x.reshape(-1, x.shape[-1]).to(dtype)
    matrices = _bases(parameters, states, dtype)
    cast, stack = group_factors(parameters, 3, dtype, flat, shared=2)
    adapters = [(cast[2*i], cast[2*i+1]) for i in range(3)]
    rows = min(tile, len(flat))
    width = matrices[0].rows
    workspace = torch.empty((1 if save else 2, rows, width), device=x.device, dtype=dtype)
    low = torch.empty((rows, max(len(a) for a, _ in adapters)), device=x.device, dtype=dtype)
    r = len(adapters[0][0])
    # gate and up read the same rows: with a shared rank their xa come from one GEMM over
    # [a_gate; a_up] into the two column halves of one buffer.
    pair = None if stack is None or save else torch.empty((rows, 2 * r), device=x.device, dtype=dtype)
    if save:
        if stack is not None:
            both = torch.empty((len(flat), 2 * r), device=x.device, dtype=dtype)
            held = (both[:, :r], both[:, r:])
        else:
            held = tuple(torch.empty((len(flat), len(a)), device=x.device, dtype=dtype) for a, _ in adapters[:2])
    saved = (() if not save else (
        *(torch.empty((len(flat), width), device=x.device, dtype=dtype) for _ in range(2)), *held))
    destination = output.view_as(flat)
    for start in range(0, len(flat), tile):
        part = flat[start:start+tile]
        gate, up = ((buffer[start:start+len(part)] for buffer in saved[:2]) if save
                    else (buffer[:len(part)] for buffer in workspace))
        xa = [low[:len(part), :len(a)] for a, _ in adapters]
        if save:
            xa[:2] = [buffer[start:start+len(part)] for buffer in saved[2:]]
        elif pair is not None:
            xa[:2] = [pair[:len(part), :r], pair[:len(part), r:]]
        _gate_up(part, matrices, adapters, gate, up, xa, stack)
        hidden = activation(gate, up, out=workspace[0, :len(part)] if save else gate)
        forward_linear(hidden, matrices[2], *adapters[2], out=destination[start:start+tile], xa=xa[2])
    if residual is not None:
        output.add_(residual)
    return saved


def _gate_up(part, matrices, adapters, gate, up, xa, stack):
    """gate and up of one tile; with `stack` their xa (two column halves of one buffer)
    come from one GEMM first."""
    if stack is None or not len(part):
        forward_linear(part, matrices[0], *adapters[0], out=gate, xa=xa[0])
        forward_linear(part, matrices[1], *adapters[1], out=up, xa=xa[1])
        return
    r = len(adapters[0][0])
    both = xa[0].as_strided((len(part), 2 * r), xa[0].stride())
    _low_rank(part, stack, both, transpose=True)
    matrices[0].forward(part, *adapters[0], None, gate, xa[0], xa_given=True)
    matrices[1].forward(part, *adapters[1], None, up, xa[1], xa_given=True)


class _TiledLoRAMLP(torch.autograd.Function):
    """Saves only the input and the parameters (plus, in cache mode, gate/up and their xa);
    the backward recomputes gate/up per tile and never builds an autograd graph."""

    @staticmethod
    def forward(ctx, x, dtype, tile, states, residual, cache, *parameters):
        ctx.dtype, ctx.tile, ctx.states = dtype, tile, states
        ctx.cache = cache
        if cache:
            output = torch.empty(x.shape, device=x.device, dtype=dtype)
            saved = _forward_into(output, x, dtype, tile, states, parameters, residual, save=True)
            ctx.save_for_backward(x, *saved, *parameters)
            return output
        # Register the saved inputs before the wrapper fills this private output, so a
        # checkpoint replay can stop before the GEMMs (reference mlp_cuda.py:94-97).
        ctx.save_for_backward(x, *parameters)
        return torch.empty(x.shape, device=x.device, dtype=dtype)

    @staticmethod
    def backward(ctx, grad):
        x, *parameters = ctx.saved_tensors
        saved = parameters[:4] if ctx.cache else ()
        if ctx.cache:
            parameters = parameters[4:]
        residual_grad = grad if ctx.needs_input_grad[4] else None
        flat = x.reshape(-1, x.shape[-1]).to(ctx.dtype)
        grad = grad.reshape_as(flat).to(ctx.dtype)
        dx = torch.empty_like(flat) if ctx.needs_input_grad[0] else None
        matrices = _bases(parameters, ctx.states, ctx.dtype)
        cast, stack = group_factors(parameters, 3, ctx.dtype, flat, shared=2)
        adapters = [(cast[2*i], cast[2*i+1]) for i in range(3)]
        allocate = torch.empty_like if len(flat) else torch.zeros_like
        gradients = [(allocate(parameters[4*i+1]), allocate(parameters[4*i+2])) for i in range(3)]
        rows = min(ctx.tile, len(flat))
        workspace = torch.empty((3, rows, matrices[0].rows), device=x.device, dtype=ctx.dtype)
        if stack is not None and not ctx.cache:
            r = len(adapters[0][0])
            pair = torch.empty((rows, 2 * r), device=x.device, dtype=ctx.dtype)
            low_inputs = [pair[:, :r], pair[:, r:],
                          torch.empty((rows, len(adapters[2][0])), device=x.device, dtype=ctx.dtype)]
        else:
            low_inputs = [torch.empty((rows, len(a)), device=x.device, dtype=ctx.dtype) for a, _ in adapters]
        low_grad = torch.empty((rows, max(len(a) for a, _ in adapters)), device=x.device, dtype=ctx.dtype)
        for start in range(0, len(flat), ctx.tile):
            part, dy = flat[start:start+ctx.tile], grad[start:start+ctx.tile]
            gate, up, dh = (buffer[:len(part)] for buffer in workspace)
            xa = [buffer[:len(part)] for buffer in low_inputs]
            low = [low_grad[:len(part), :len(a)] for a, _ in adapters]
            if ctx.cache:
                xa[:2] = [value[start:start+len(part)] for value in saved[2:]]
            else:
                _gate_up(part, matrices, adapters, gate, up, xa, stack)
            input_gradient(dy, matrices[2], *adapters[2], dh, low[2])
            if ctx.cache:
                # The saved gate/up stay untouched (a repeated backward reads them again):
                # the activation backward reads them and writes d gate, d up into the tile
                # buffers and hidden over dh, where the reference copies the tile first.
                _silu(saved[0][start:start+len(part)], saved[1][start:start+len(part)], dh, gate, up, True, True)
                hidden = dh
            else:
                # Reuse the three wide tile buffers: (gate, up, dh) -> (d gate, d up, hidden).
                hidden = activation(gate, up, dh)
            _low_rank(hidden, adapters[2][0], xa[2], transpose=True)
            parameter_gradients(hidden, dy, *gradients[2], low[2], xa[2], add=start > 0)
            for index, signal in enumerate((gate, up)):
                if dx is not None:
                    input_gradient(signal, matrices[index], *adapters[index], dx[start:start+ctx.tile], low[index],
                                   add=index > 0)
                else:
                    _low_rank(signal, adapters[index][1], low[index], transpose=False)
                parameter_gradients(part, signal, *gradients[index], low[index], xa[index], add=start > 0)
        result = [value for da, db in gradients for value in (None, da, db, None)]
        return (None if dx is None else dx.reshape_as(x).to(x.dtype), None, None, None, residual_grad, None, *result)


def tiled_lora_mlp(module, x, residual=None, *, tile=None, cache=None):
    """`module` carries gate_proj, up_proj, down_proj (Projection), tile and
    cache_intermediates, as the reference's MLP (modeling/model.py:111-139) does."""
    modules = (module.gate_proj, module.up_proj, module.down_proj)
    dtype = modules[0].compute_dtype
    if residual is not None and (residual.shape != x.shape or residual.dtype != dtype):
        return tiled_lora_mlp(module, x, tile=tile, cache=cache)+residual
    parameters, states = [], []
    for projection in modules:
        values, state = projection_parameters(projection)
        parameters.extend(values)
        states.append(state)
    tile = (module.tile if tile is None else tile) or max(1, x.numel()//x.shape[-1])
    cache = (module.cache_intermediates if cache is None else cache) and torch.is_grad_enabled()
    output = _TiledLoRAMLP.apply(x, dtype, tile, tuple(states), residual, cache, *parameters)
    if not cache:
        _forward_into(output, x, dtype, tile, states, parameters, residual)
    return output
