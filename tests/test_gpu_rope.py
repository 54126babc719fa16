"""Partial RoPE on the GPU (ct_rope) and the q/k/v projection group with rotary and
residual fusion (reference kernels/core_cuda.py:133-229, kernels/linear.py:59-148).

The kernels must equal the CPU oracle (oracle/rope.py) bit for bit: the rotation is
elementwise with fixed rounding points. The projection-group tests follow the reference's
tests/test_kernel_workspaces.py:17-63 (owned rotary preserves shared gradients),
:66-85 (beyond 512k rows) and :88-106 (NF4 base with rotary), bf16 compute dtype."""

import numpy as np
import pytest
import torch

from oracle import rope as orope

pytestmark = pytest.mark.gpu

NAMES = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def _tables(tokens, half, dtype, seed=0, scale=60000.0):
    g = torch.Generator().manual_seed(seed)
    angle = torch.rand(tokens, half, generator=g, dtype=torch.float64) * scale
    return angle.cos().to(dtype), angle.sin().to(dtype)


def _oracle(x, c, s, head_dim, dtype, inverse=False):
    tokens = c.shape[0]
    got = orope.rope(x.float().reshape(tokens, -1).numpy(), c.float().numpy(), s.float().numpy(), head_dim,
                     NAMES[dtype], inverse=inverse)
    return torch.from_numpy(got).reshape(x.shape)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("tokens,heads,head_dim,half", [(14, 3, 8, 2), (1000, 4, 128, 32), (37, 2, 64, 32),
                                                        (5, 1, 16, 0), (300, 1, 6, 1)])
def test_partial_rope_forward_and_backward_match_oracle(dtype, tokens, heads, head_dim, half):
    from causal_tuner.kernels.core_cuda import PartialRoPE
    g = torch.Generator().manual_seed(tokens + heads)
    x = torch.randn(tokens, heads, head_dim, generator=g).to(dtype)
    c, s = _tables(tokens, half, dtype, seed=1)
    xd = x.cuda().requires_grad_(True)
    y = PartialRoPE.apply(xd, c.cuda(), s.cuda())
    assert torch.equal(y.cpu().float(), _oracle(x, c, s, head_dim, dtype))
    grad = torch.randn(tokens, heads, head_dim, generator=g).to(dtype)
    y.backward(grad.cuda())
    assert torch.equal(xd.grad.cpu().float(), _oracle(grad, c, s, head_dim, dtype, inverse=True))


def test_trig_tables_in_float32_with_bf16_activations():
    from causal_tuner.kernels.core_cuda import PartialRoPE
    x = torch.randn(9, 2, 16).to(torch.bfloat16)
    c, s = _tables(9, 4, torch.float32, seed=2)
    y = PartialRoPE.apply(x.cuda(), c.cuda(), s.cuda())
    assert torch.equal(y.cpu().float(), _oracle(x, c, s, 16, torch.bfloat16))


def test_rotate_owned_qk_in_place_touches_only_rotated_channels():
    from causal_tuner.kernels.core_cuda import rotate_owned_qk
    rows, head_dim, half = 4099, 128, 32
    q = torch.randn(rows, 3 * head_dim).to(torch.bfloat16)
    k = torch.randn(rows, head_dim).to(torch.bfloat16)
    c, s = _tables(rows, half, torch.bfloat16, seed=3)
    qd, kd = q.cuda(), k.cuda()
    rotate_owned_qk(qd, kd, c.cuda(), s.cuda(), head_dim)
    for got, raw in ((qd, q), (kd, k)):
        assert torch.equal(got.cpu().float(), _oracle(raw, c, s, head_dim, torch.bfloat16))


def test_owned_rotary_beyond_512k():
    """tests/test_kernel_workspaces.py:66-85: 524289 tokens (a masked tail after 65,536
    position tiles), checked against the oracle on bounded token windows."""
    from causal_tuner.kernels.core_cuda import rotate_owned_qk
    rows, head_dim, half = 524289, 128, 32
    g = torch.Generator(device="cuda").manual_seed(4)
    query = torch.randn(rows, 3 * head_dim, device="cuda", generator=g).to(torch.bfloat16)
    key = torch.randn(rows, head_dim, device="cuda", generator=g).to(torch.bfloat16)
    original = (query.clone(), key.clone())
    angles = torch.randn(rows, half, device="cuda", generator=g)
    cosine, sine = angles.cos().bfloat16(), angles.sin().bfloat16()
    rotate_owned_qk(query, key, cosine, sine, head_dim)
    for start in (0, 65536 * 4 - 2048, rows - 4097):
        window = slice(start, start + 4097)
        c, s = cosine[window].cpu(), sine[window].cpu()
        for actual, raw in zip((query, key), original):
            want = _oracle(raw[window].cpu(), c, s, head_dim, torch.bfloat16)
            assert torch.equal(actual[window].cpu().float(), want)


def _group(width, head_dim, dtype=torch.bfloat16, nf4=False, seed=0):
    from causal_tuner.modeling.lora import Projection
    torch.manual_seed(seed)
    modules = [Projection(width, out, bias=True, rank=rank, base_dtype=dtype, compute_dtype=dtype, device="cuda")
               for out, rank in zip((width, head_dim, head_dim), (3, 5, 7))]
    for module in modules:
        if nf4:
            module.install_nf4(module.weight.detach().clone(), "cuda")
        torch.nn.init.normal_(module.lora_B, std=.03)
        torch.nn.init.normal_(module.bias, std=.1)
    return modules


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tile", [0, 5])
@pytest.mark.parametrize("head_dim,rotary_dim", [(8, 4), (128, 64)])
def test_projection_owned_rotary_preserves_shared_gradients(dtype, tile, head_dim, rotary_dim, monkeypatch):
    """tests/test_kernel_workspaces.py:17-63 with its tolerances: bit-exact in bf16,
    2e-6 in float32 (the float32 products run on ct_gemm_f32)."""
    import causal_tuner.kernels.core_cuda as core
    from causal_tuner.kernels.linear import project_group
    from causal_tuner.modeling.rotary import rotate
    width = head_dim * 4
    modules = _group(width, head_dim, dtype)
    x = torch.randn(2, 7, width, device="cuda", dtype=dtype, requires_grad=True)
    original_input = x.detach().clone()
    angles = torch.arange(14, device="cuda").reshape(2, 7, 1) * 60000 * torch.rand(rotary_dim // 2, device="cuda")
    cosine, sine = angles.cos().to(dtype), angles.sin().to(dtype)
    actual = project_group(modules, x, tile, rotary=(cosine, sine, head_dim))
    raw = project_group(modules, x, tile)
    expected = tuple(rotate(t.reshape(2, 7, -1, head_dim), cosine, sine).reshape_as(t) if i < 2 else t
                     for i, t in enumerate(raw))
    tolerance = dict(rtol=0, atol=0) if dtype == torch.bfloat16 else dict(rtol=2e-6, atol=2e-6)
    for a, e in zip(actual, expected):
        torch.testing.assert_close(a, e, **tolerance)
    for a, r in zip(actual[:2], raw[:2]):
        assert torch.equal(a.reshape(2, 7, -1, head_dim)[..., rotary_dim:],
                           r.reshape(2, 7, -1, head_dim)[..., rotary_dim:])
    shared = torch.randn_like(actual[0])
    signals = (shared, shared[..., :head_dim], shared[..., :head_dim])
    saved_signal = shared.clone()
    parameters = (x, *(p for module in modules for p in module.parameters() if p.requires_grad))
    largest_tile = 0
    original_inverse = core.inverse_rope_tile

    def bounded_inverse(grad, *args):
        nonlocal largest_tile
        largest_tile = max(largest_tile, len(grad))
        return original_inverse(grad, *args)
    monkeypatch.setattr(core, "inverse_rope_tile", bounded_inverse)
    ag = torch.autograd.grad(actual, parameters, signals, retain_graph=True)
    eg = torch.autograd.grad(expected, parameters, signals)
    repeated = torch.autograd.grad(actual, parameters, signals)
    assert 0 < largest_tile <= (tile or 4096)
    for a, e, r in zip(ag, eg, repeated):
        torch.testing.assert_close(a, e, **tolerance)
        assert torch.equal(a, r)
    assert torch.equal(shared, saved_signal)
    assert torch.equal(x, original_input)


def test_nf4_projection_rotary_input_gradient():
    """tests/test_kernel_workspaces.py:88-106."""
    from causal_tuner.kernels.linear import project_group
    from causal_tuner.modeling.rotary import rotate
    modules = _group(32, 8, nf4=True, seed=5)
    x = torch.randn(2, 7, 32, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    angles = torch.randn(2, 7, 2, device="cuda")
    cosine, sine = angles.cos().bfloat16(), angles.sin().bfloat16()
    actual = project_group(modules, x, 5, rotary=(cosine, sine, 8))
    raw = project_group(modules, x, 5)
    expected = tuple(rotate(t.reshape(2, 7, -1, 8), cosine, sine).reshape_as(t) if i < 2 else t
                     for i, t in enumerate(raw))
    signal = tuple(torch.randn_like(t) for t in actual)
    parameters = (x, *(p for m in modules for p in m.parameters() if p.requires_grad))
    for a, e in zip(torch.autograd.grad(actual, parameters, signal),
                    torch.autograd.grad(expected, parameters, signal)):
        assert torch.equal(a, e)


@pytest.mark.parametrize("tile", [0, 3])
def test_output_projection_residual_is_added_after_rounding(tile):
    """o-proj residual (linear.py:90-91, 129, 135-139): out = bf16(out) + residual, the
    residual gradient is the upstream gradient, and a mismatched residual falls back to an
    unfused add."""
    from causal_tuner.kernels.linear import project_group
    from causal_tuner.modeling.lora import Projection
    torch.manual_seed(6)
    module = Projection(48, 40, rank=4, device="cuda")
    torch.nn.init.normal_(module.lora_B, std=.05)
    x = torch.randn(3, 5, 48, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    residual = torch.randn(3, 5, 40, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    saved = residual.detach().clone()
    fused = project_group((module,), x, tile, residual=residual)[0]
    plain = project_group((module,), x, tile)[0] + residual
    assert torch.equal(fused, plain)
    assert torch.equal(residual, saved)
    grad = torch.randn_like(fused)
    fused_grads = torch.autograd.grad(fused, (x, residual, module.lora_A, module.lora_B), grad)
    plain_grads = torch.autograd.grad(plain, (x, residual, module.lora_A, module.lora_B), grad)
    for a, b in zip(fused_grads, plain_grads):
        assert torch.equal(a, b)
    wide = torch.randn(3, 5, 40, device="cuda", dtype=torch.float32)
    out = project_group((module,), x, tile, residual=wide)[0]
    assert out.dtype == torch.float32
    with pytest.raises(ValueError):
        project_group((module, module), x, tile, residual=residual)
