"""Pins oracle/mlp.py (the float64 LoRA MLP restatement) by mathematics, not by retyping it:
the SiLU derivative against central differences, and the whole forward/backward against
float64 autograd of the unrounded MLP (bf16 rounding points bound the gap)."""

import torch
from torch.nn import functional as F

from oracle import mlp as omlp


def test_silu_derivative_formula_matches_central_differences():
    g = torch.linspace(-8, 8, 401, dtype=torch.float64)
    h = 1e-6
    numeric = (F.silu(g + h) - F.silu(g - h)) / (2 * h)
    sig = torch.sigmoid(g)
    closed = sig * (1 + g * (1 - sig))  # the factor in reference mlp_cuda.py:21
    assert torch.allclose(numeric, closed, rtol=1e-7, atol=1e-9)


def test_activation_backward_is_the_product_rule():
    torch.manual_seed(0)
    gate = torch.randn(257, dtype=torch.float64).to(torch.bfloat16).double()
    up = torch.randn(257, dtype=torch.float64).to(torch.bfloat16).double()
    grad = torch.randn(257, dtype=torch.float64).to(torch.bfloat16).double()
    dgate, dup, hidden = omlp.activation_backward(gate, up, grad)
    g, u = gate.clone().requires_grad_(), up.clone().requires_grad_()
    (F.silu(g) * u).backward(grad)
    for got, want in ((dgate, g.grad), (dup, u.grad), (hidden, F.silu(gate) * up)):
        assert ((got - want).norm() / want.norm()) < 8e-3   # bf16 rounding points only


def test_oracle_mlp_against_unrounded_autograd():
    torch.manual_seed(1)
    m, h, i, r = 11, 32, 68, 4
    x = torch.randn(m, h, dtype=torch.float64)
    weights = [torch.randn(i, h, dtype=torch.float64) * .1, torch.randn(i, h, dtype=torch.float64) * .1,
               torch.randn(h, i, dtype=torch.float64) * .1]
    adapters = [(torch.randn(r, w.shape[1], dtype=torch.float64) * .2, torch.randn(w.shape[0], r, dtype=torch.float64) * .2)
                for w in weights]
    dy = torch.randn(m, h, dtype=torch.float64)
    out, dx, grads = omlp.oracle_mlp(x, weights, adapters, dy)
    rx = x.to(torch.bfloat16).double().requires_grad_()
    W = [w.to(torch.bfloat16).double() for w in weights]
    AB = [(a.to(torch.bfloat16).double().requires_grad_(), b.to(torch.bfloat16).double().requires_grad_())
          for a, b in adapters]
    lin = [lambda t, k=k: t @ W[k].T + (t @ AB[k][0].T) @ AB[k][1].T for k in range(3)]
    ref = lin[2](F.silu(lin[0](rx)) * lin[1](rx))
    params = [rx] + [p for ab in AB for p in ab]
    got = torch.autograd.grad(ref, params, dy.to(torch.bfloat16).double())
    assert ((out - ref.detach()).norm() / ref.norm()) < 1e-2
    assert ((dx - got[0]).norm() / got[0].norm()) < 1e-2
    for k in range(3):
        for j in range(2):
            want = got[1 + 2 * k + j]
            assert ((grads[k][j] - want).norm() / want.norm()) < 2e-2, (k, j)
