"""Tiled LoRA MLP on the MI355X through the reference's operator API (kernels/mlp_cuda.py).

Restates the reference's MLP tests: saved tensors (tests/test_fast_training.py:143-158),
cache mode against recompute mode (tests/test_mlp_cache.py:15-49), and the NF4 tiny MLP
against an independent autograd formulation (tests/test_fast_training.py:237-253); plus
the SiLU-multiply kernel and a C3-sized MLP against the float64 oracle (oracle/mlp.py)."""

import pytest
import torch
from torch.nn import functional as F

from oracle import mlp as omlp

pytestmark = pytest.mark.gpu


def _mlp(h, i, r, *, nf4, tile=None, seed=0, std=.05, dtype=torch.bfloat16):
    from causal_tuner.modeling.mlp import MLP
    torch.manual_seed(seed)
    module = MLP(h, i, rank=r, base_dtype=dtype, compute_dtype=dtype, device="cuda", tile=tile)
    for projection in (module.gate_proj, module.up_proj, module.down_proj):
        torch.nn.init.normal_(projection.lora_B, std=std)
        if nf4:
            projection.install_nf4(projection.weight.detach().clone(), "cuda")
    return module


def _params(module, x):
    return (x, *(p for p in module.parameters() if p.requires_grad))


def test_silu_multiply_kernel_against_float64():
    from causal_tuner.kernels.mlp_cuda import activation
    torch.manual_seed(0)
    for n in (4099, 8192 * 3):
        gate = (torch.randn(n, device="cuda") * 3).to(torch.bfloat16)
        up = torch.randn(n, device="cuda").to(torch.bfloat16)
        grad = torch.randn(n, device="cuda").to(torch.bfloat16)
        hidden = activation(gate, up)
        want = omlp.activation_forward(gate.cpu().double(), up.cpu().double())
        # one bf16 ulp at most: the exponential differs from the reference's by float rounding
        assert ((hidden.cpu().double() - want).abs() <= want.abs() * 2 ** -7 + 1e-30).all()
        g, u, d = gate.clone(), up.clone(), grad.clone()
        activation(g, u, d)   # in place: g <- d gate, u <- d up, d <- hidden
        wg, wu, wh = omlp.activation_backward(gate.cpu().double(), up.cpu().double(), grad.cpu().double())
        for got, w in ((g, wg), (u, wu), (d, wh)):
            err = (got.cpu().double() - w).abs()
            assert (err <= w.abs() * 2 ** -6 + 1e-6).all()


def test_silu_multiply_autograd_matches_torch():
    from causal_tuner.kernels.mlp_cuda import silu_multiply
    torch.manual_seed(1)
    gate = torch.randn(33, 70, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    up = torch.randn(33, 70, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    out = silu_multiply(gate, up)
    dy = torch.randn_like(out)
    dg, du = torch.autograd.grad(out, (gate, up), dy)
    g, u = gate.detach().float().requires_grad_(), up.detach().float().requires_grad_()
    ref = F.silu(g) * u
    rg, ru = torch.autograd.grad(ref, (g, u), dy.float())
    for got, want in ((out, ref), (dg, rg), (du, ru)):
        assert ((got.float() - want).norm() / want.norm()) < 1e-2


@pytest.mark.parametrize("nf4", [False, True])
def test_fused_mlp_saves_only_boundary_and_weights(nf4, monkeypatch):
    module = _mlp(32, 68, 4, nf4=nf4, tile=5)
    x = torch.randn(2, 13, 32, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    saved = []

    def pack(tensor):
        saved.append(tensor)
        return tensor
    with torch.autograd.graph.saved_tensors_hooks(pack, lambda tensor: tensor):
        output = module(x)
    allowed = {x.data_ptr(), *(parameter.data_ptr() for parameter in module.parameters())}
    assert all(tensor.data_ptr() in allowed for tensor in saved)

    def forbidden(*args, **kwargs):
        raise AssertionError("The fused MLP backward must not build per-tile autograd graphs")
    monkeypatch.setattr(torch.autograd, "grad", forbidden)
    output.sum().backward()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tile", [0, 5])
@pytest.mark.parametrize("nf4", [False, True])
def test_saved_mlp_matches_recompute_and_preserves_repeated_backward(tile, nf4, dtype, monkeypatch):
    """tests/test_mlp_cache.py:15-49 (float32 and bf16; plus NF4 bases)."""
    from causal_tuner.kernels import mlp_cuda
    module = _mlp(32, 68, 4, nf4=nf4, tile=tile, dtype=dtype)
    x = torch.randn(2, 7, 32, device="cuda", dtype=dtype, requires_grad=True)
    original = x.detach().clone()
    signal = torch.randn_like(x)
    params = _params(module, x)
    expected = module(x, residual=x)
    reference = torch.autograd.grad(expected, params, signal)
    module.cache_intermediates = True
    saved = []
    with torch.autograd.graph.saved_tensors_hooks(lambda t: saved.append(t) or t, lambda t: t):
        actual = module(x, residual=x)
    allowed = {x.data_ptr(), *(p.data_ptr() for p in module.parameters())}
    retained = [t for t in saved if t.data_ptr() not in allowed]
    assert sum(t.numel() * t.element_size() for t in retained) == module.cache_bytes(14)
    snapshots = [t.clone() for t in retained]

    def forbidden(*a, **kw):
        raise AssertionError("Cached backward must not recompute gate/up projections")
    monkeypatch.setattr(mlp_cuda, "forward_linear", forbidden)
    monkeypatch.setattr(mlp_cuda._MLPProjections, "gate_up", forbidden)
    gradients = torch.autograd.grad(actual, params, signal, retain_graph=True)
    repeated = torch.autograd.grad(actual, params, signal)
    torch.testing.assert_close(actual, expected, rtol=0, atol=0)
    for value, expected_grad, repeat in zip(gradients, reference, repeated):
        torch.testing.assert_close(value, expected_grad, rtol=0, atol=0)
        torch.testing.assert_close(value, repeat, rtol=0, atol=0)
    assert all(g.dtype == torch.float32 for g in gradients[1:])
    for value, snapshot in zip(retained, snapshots):
        torch.testing.assert_close(value, snapshot, rtol=0, atol=0)
    torch.testing.assert_close(x, original, rtol=0, atol=0)


def _plain_linear(module, x):
    """tests/test_fast_training.py:18-23: the projection as plain torch ops."""
    dtype = module.compute_dtype
    x = x.to(dtype)
    weight = module.base_weight().to(dtype)
    bias = None if module.bias is None else module.bias.to(dtype)
    return F.linear(x, weight, bias) + F.linear(F.linear(x, module.lora_A.to(dtype)), module.lora_B.to(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("train_input", [False, True])
@pytest.mark.parametrize("mixed_ranks", [False, True])
@pytest.mark.parametrize("cache", [False, True])
def test_fused_tiled_mlp_independent_gradients(dtype, train_input, mixed_ranks, cache):
    """tests/test_fast_training.py:26-57 with its tolerances (float32: rtol 3e-5, atol 2e-6
    against torch's float32 products with TF32 off): the tiny config's MLP (32 -> 68,
    rank 4, tile 5), mixed ranks 3/5/7, cache on and off."""
    import copy
    from causal_tuner.modeling.lora import Projection
    from causal_tuner.modeling.mlp import MLP
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.manual_seed(4)
    module = MLP(32, 68, rank=4, base_dtype=dtype, compute_dtype=dtype, device="cuda", tile=5)
    module.cache_intermediates = cache
    if mixed_ranks:
        for name, rank in (("gate_proj", 3), ("up_proj", 5), ("down_proj", 7)):
            original = getattr(module, name)
            setattr(module, name, Projection(original.weight.shape[1], original.weight.shape[0], rank=rank,
                                             base_dtype=dtype, compute_dtype=dtype, device="cuda"))
    for name, parameter in module.named_parameters():
        if "lora_B" in name:
            torch.nn.init.normal_(parameter, std=.1)
    reference = copy.deepcopy(module)
    x = torch.randn(2, 7, 32, device="cuda", dtype=dtype, requires_grad=train_input)
    y = x.detach().clone().requires_grad_(train_input)
    actual = module(x)
    expected = _plain_linear(reference.down_proj, F.silu(_plain_linear(reference.gate_proj, y)) *
                             _plain_linear(reference.up_proj, y))
    tolerance = dict(rtol=.04, atol=.003) if dtype == torch.bfloat16 else dict(rtol=3e-5, atol=2e-6)
    torch.testing.assert_close(actual, expected, **tolerance)
    signal = torch.randn_like(actual)
    actual.backward(signal)
    expected.backward(signal)
    if train_input:
        torch.testing.assert_close(x.grad, y.grad, **tolerance)
    for (name, a), (_, b) in zip(module.named_parameters(), reference.named_parameters()):
        if a.requires_grad:
            assert a.grad.dtype == torch.float32, name
            torch.testing.assert_close(a.grad, b.grad, **tolerance)


def test_nf4_fused_tiled_mlp_gradients():
    """tests/test_fast_training.py:237-253: tiny NF4 MLP, tile 5, 13 tokens, against the
    independent autograd formulation on the decoded bases, at the reference's tolerances."""
    module = _mlp(32, 68, 4, nf4=True, tile=5, seed=3)
    x = torch.randn(13, 32, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    out = module(x)
    dy = torch.randn_like(out)
    params = _params(module, x)
    got = torch.autograd.grad(out, params, dy)
    xr = x.detach().clone().requires_grad_()
    lin = [lambda t, p=p: F.linear(t, p.base_weight().to(t.dtype)) + F.linear(F.linear(t, p.lora_A.to(t.dtype)),
                                                                               p.lora_B.to(t.dtype))
           for p in (module.gate_proj, module.up_proj, module.down_proj)]
    ref = lin[2](F.silu(lin[0](xr)) * lin[1](xr))
    want = torch.autograd.grad(ref, (xr, *params[1:]), dy)
    torch.testing.assert_close(out, ref, rtol=.04, atol=.003)
    for g, w in zip(got, want):
        torch.testing.assert_close(g.float(), w.float(), rtol=.05, atol=.003)


@pytest.mark.parametrize("tokens,hidden,inter,rank,tile", [(300, 256, 704, 16, 0), (1024, 1024, 2752, 64, 384),
                                                            (40, 512, 1408, 32, 0)])
def test_mlp_against_float64_oracle(tokens, hidden, inter, rank, tile):
    module = _mlp(hidden, inter, rank, nf4=True, tile=tile or None, seed=5, std=.02)
    x = torch.randn(tokens, hidden, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    out = module(x)
    dy = torch.randn_like(out)
    params = _params(module, x)
    grads = torch.autograd.grad(out, params, dy)
    projections = (module.gate_proj, module.up_proj, module.down_proj)
    weights = [p.base_weight().cpu() for p in projections]
    adapters = [(p.lora_A.detach().cpu(), p.lora_B.detach().cpu()) for p in projections]
    oout, odx, ograds = omlp.oracle_mlp(x.detach().cpu(), weights, adapters, dy.cpu())

    def rel(a, b):
        return float((a.detach().cpu().double() - b).norm() / b.norm())
    # bf16 rounding of gate/up/dh feeds the SiLU; single-rounding differences propagate
    assert rel(out, oout) < 5e-3
    assert rel(grads[0], odx) < 5e-3
    for k in range(3):
        assert rel(grads[1 + 2 * k], ograds[k][0]) < 5e-3, ("dA", k)
        assert rel(grads[2 + 2 * k], ograds[k][1]) < 5e-3, ("dB", k)
