"""The RMS-normalization oracle (oracle/rmsnorm.py), pinned on the CPU.

It restates _rms_forward / _rms_gradient_row (reference kernels/core_cuda.py:29-75). What
pins it: in float32 (no rounding) its forward equals the textbook formula and its
gradients equal float64 autograd of that formula; with bf16 rounding points it equals the
package's host RMSNorm (the reference's torch formula) to one bf16 rounding; the
reconstruction mode (normalized values recovered from the output) agrees with the
gradient from x; scaling x leaves y unchanged (homogeneity)."""

import numpy as np
import torch

from oracle import rmsnorm


def test_forward_is_the_textbook_formula_in_float32():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 33)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 33).astype(np.float32)
    y, rstd = rmsnorm.forward(x, w, 1e-6, "float32")
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(y, want, rtol=2e-7, atol=1e-7)
    np.testing.assert_allclose(rstd, 1 / np.sqrt((x64 ** 2).mean(-1) + 1e-6), rtol=1e-15)


def test_gradients_match_float64_autograd():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((7, 64)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    go = rng.standard_normal((7, 64)).astype(np.float32)
    _, rstd = rmsnorm.forward(x, w, 1e-6, "float32")
    gx, dw = rmsnorm.backward(x, w, rstd, go, "float32")
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    yt = xt * torch.rsqrt((xt ** 2).mean(-1, keepdim=True) + 1e-6) * wt
    ex, ew = torch.autograd.grad(yt, (xt, wt), torch.tensor(go, dtype=torch.float64))
    np.testing.assert_allclose(gx, ex.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dw, ew.numpy(), rtol=1e-5, atol=1e-5)


def test_bf16_forward_matches_the_host_formula():
    from causal_tuner.modeling.norm import RMSNorm
    g = torch.Generator().manual_seed(2)
    x = torch.randn(9, 96, generator=g).to(torch.bfloat16)
    norm = RMSNorm(96, 1e-6, torch.bfloat16, "cpu")
    with torch.no_grad():
        norm.weight.uniform_(0.5, 1.5, generator=g)
    host = norm(x).detach().float().numpy()
    y, _ = rmsnorm.forward(x.float().numpy(), norm.weight.detach().float().numpy(), 1e-6, "bfloat16")
    # the host formula rounds x * rstd from float32 arithmetic, the oracle from float64:
    # at most one bf16 step apart before the final product
    np.testing.assert_allclose(y, host, rtol=2 ** -7, atol=0)


def test_reconstruction_matches_the_gradient_from_x():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 128)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    go = rng.standard_normal((6, 128)).astype(np.float32)
    y, rstd = rmsnorm.forward(x, w, 1e-6, "float32")
    from_x, _ = rmsnorm.backward(x, w, rstd, go, "float32")
    from_y, dw = rmsnorm.backward(y, w, rstd, go, "float32", from_output=True)
    assert dw is None
    np.testing.assert_allclose(from_y, from_x, rtol=1e-4, atol=1e-5)


def test_scaling_x_leaves_y_unchanged():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 40)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 40).astype(np.float32)
    y1, _ = rmsnorm.forward(x, w, 0.0, "float32")
    y2, _ = rmsnorm.forward(x * 8, w, 0.0, "float32")   # a power of two: exact scaling
    np.testing.assert_array_equal(y1, y2)
