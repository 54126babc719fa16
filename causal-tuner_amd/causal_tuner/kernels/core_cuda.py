"""Row-wise RMS normalization and partial GPT-J rotary embedding on gfx950 (the reference's
kernels/core_cuda.py).

`RMS` (core_cuda.py:96-130) is the autograd function behind the decoder's RMSNorm: the HIP
kernels ct_rms_forward / ct_rms_backward with the reference's rounding points, its
private-gradient reuse (the input gradient written over the incoming gradient) and its
output reconstruction mode (the backward reads the output and the weight instead of x).


Same operator API as the reference: `rotate_owned_qk` (core_cuda.py:192-200) rotates the
q and k outputs of a projection group in place, `inverse_rope_tile` (203-208) writes the
inverse rotation of an upstream gradient tile into a private buffer, and `PartialRoPE`
(211-229) is the autograd function behind `modeling.rotary.rotate`. All three run the HIP
kernel `ct_rope` with the reference's rounding (each product rounded to the tensor type,
then the sum or difference rounded again).
"""

import torch

from . import _native


class RMS(torch.autograd.Function):
    """y = T(T(x * rstd) * T(weight)) over the last dimension (reference core_cuda.py:96-130)."""

    @staticmethod
    def forward(ctx, x, weight, eps, reuse_grad=False, reconstruct=False):
        # Reconstruction and private-gradient reuse belong to frozen pre-norms.
        ctx.reuse_grad = reuse_grad and not weight.requires_grad
        ctx.reconstruct = reconstruct and not weight.requires_grad
        if not (x.is_cuda and weight.is_cuda):
            raise ValueError("RMS expects device tensors")
        x = x.contiguous()
        output = torch.empty_like(x)
        width = x.shape[-1]
        inverse = torch.empty(x.numel() // width if width else 0, device=x.device, dtype=torch.float32)
        with _native.device_of(x):
            status = _native.library().ct_rms_forward(
                _native.ptr(x), _native.dtype_code(x.dtype), _native.ptr(weight.contiguous()),
                _native.dtype_code(weight.dtype), _native.ptr(output), _native.ptr(inverse), len(inverse), width,
                float(eps), _native.stream_of(x))
        _native.check(status, "ct_rms_forward")
        ctx.save_for_backward(output if ctx.reconstruct else x, weight, inverse)
        return output

    @staticmethod
    def backward(ctx, grad):
        x, weight, inverse = ctx.saved_tensors
        grad = grad.contiguous()
        # Only decoder pre-norms followed by analytic projections opt in: those projections
        # hand back a private, freshly allocated input gradient.
        result = (grad if ctx.reuse_grad else torch.empty_like(x)) if ctx.needs_input_grad[0] else None
        dw = torch.empty_like(weight) if ctx.needs_input_grad[1] else None
        width, rows = x.shape[-1], len(inverse)
        lib = _native.library()
        ws_bytes = lib.ct_rms_backward_workspace(rows, width, int(dw is not None))
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        if result is not None or dw is not None:
            with _native.device_of(x):
                status = lib.ct_rms_backward(
                    _native.ptr(x), _native.dtype_code(x.dtype), _native.ptr(weight.contiguous()),
                    _native.dtype_code(weight.dtype), _native.ptr(inverse), _native.ptr(grad), _native.ptr(result),
                    _native.ptr(dw), rows, width, int(ctx.reconstruct), _native.ptr(workspace), ws_bytes,
                    _native.stream_of(x))
            _native.check(status, "ct_rms_backward")
        return (result, dw, None, None, None)[:len(ctx.needs_input_grad)]


def _token_pitch(t, tokens, width):
    """Elements between consecutive tokens of t viewed as [tokens, width] (contiguous within
    a token), or None when t has no such view."""
    if t.is_contiguous():
        return width
    if t.dim() == 2 and t.shape[0] == tokens and t.shape[1] == width and t.stride(1) == 1 and t.stride(0) >= width:
        return t.stride(0)
    return None


def _rope(x, y, cosine, sine, head_dim, *, inverse, rotated_only):
    """y <- RoPE(x) over [tokens, heads, head_dim] with cosine/sine [tokens, half]; x and y
    are contiguous, or [tokens, heads * head_dim] matrices with a row pitch (column ranges of
    wider matrices)."""
    if not (x.is_cuda and y.is_cuda and cosine.is_cuda and sine.is_cuda):
        raise ValueError("RoPE kernels expect device tensors")
    if not (cosine.is_contiguous() and sine.is_contiguous()):
        raise ValueError("RoPE kernels expect contiguous tensors")
    if x.dtype != y.dtype or cosine.dtype != sine.dtype:
        raise ValueError("RoPE: mismatched element types")
    if head_dim <= 0 or head_dim % 2 or x.numel() % head_dim or y.numel() != x.numel():
        raise ValueError(f"RoPE: {tuple(x.shape)} is not a whole number of heads of {head_dim}")
    half = cosine.shape[-1] if cosine.dim() else 0
    if half:
        tokens = cosine.numel() // half   # one row of the tables per token
        if sine.numel() != cosine.numel() or tokens == 0 or x.numel() % (tokens * head_dim):
            raise ValueError("RoPE: cosine/sine must hold [tokens, half] values for the tokens of x")
        heads = x.numel() // (tokens * head_dim)
    else:
        tokens, heads = 1, x.numel() // head_dim
    if x.numel() == 0:
        return y
    width = heads * head_dim
    ldx, ldy = _token_pitch(x, tokens, width), _token_pitch(y, tokens, width)
    if ldx is None or ldy is None:
        raise ValueError("RoPE kernels expect contiguous tensors")
    with _native.device_of(x):
        status = _native.library().ct_rope(
            _native.ptr(x), _native.ptr(y), _native.ptr(cosine), _native.ptr(sine), tokens, heads, head_dim, half,
            ldx, ldy, int(inverse), int(rotated_only), _native.dtype_code(x.dtype), _native.dtype_code(cosine.dtype),
            _native.stream_of(x))
    _native.check(status, "ct_rope")
    return y


def rotate_owned_qk(query, key, cosine, sine, head_dim):
    """Rotate newly allocated projection outputs before exposing them to autograd
    (reference core_cuda.py:192-200): q [..., q_heads*head_dim] and k [..., k_heads*head_dim]
    in place, positions from cosine/sine [tokens, half]."""
    for tensor in (query, key):
        _rope(tensor, tensor, cosine, sine, head_dim, inverse=False, rotated_only=True)


def inverse_rope_tile(grad, cosine, sine, head_dim, output):
    """Write an inverse rotation into a private tile, preserving caller gradients
    (reference core_cuda.py:203-208)."""
    return _rope(grad.contiguous(), output, cosine, sine, head_dim, inverse=True, rotated_only=False)


class PartialRoPE(torch.autograd.Function):
    """x [..., heads, head_dim] rotated on its first 2*half channels (reference
    core_cuda.py:211-229)."""

    @staticmethod
    def forward(ctx, x, cosine, sine):
        x = x.contiguous()
        output = torch.empty_like(x)
        ctx.head_dim = x.shape[-1]
        ctx.save_for_backward(cosine, sine)
        return _rope(x, output, cosine, sine, ctx.head_dim, inverse=False, rotated_only=False)

    @staticmethod
    def backward(ctx, grad):
        cosine, sine = ctx.saved_tensors
        grad = grad.contiguous()
        output = torch.empty_like(grad)
        return _rope(grad, output, cosine, sine, ctx.head_dim, inverse=True, rotated_only=False), None, None
