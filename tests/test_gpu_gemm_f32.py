"""ct_gemm_f32, the float32 products of the projection operators' float32 compute dtype
(the reference's torch.mm / addmm with float32 operands, kernels/linear.py:16-44, TF32 off
as in train.py:80-82 and tests/conftest.py:10).

Checked against a float64 product of the same float32 operands: a full-precision fp32
GEMM stays within a few fp32 ulps times sqrt(k) of it, so the bar is relative 1e-5 of the
operands' scale. Every layout (A and B stored either way), odd tails in m, n and k,
strided views, bias, accumulation into an existing output (beta = 1), beta = 0 over NaN
(tests/test_kernel_workspaces.py:269-279) and k = 0 are covered; a second call gives
bit-identical results."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(left, right, out=None, bias=None):
    want = left.double() @ right.double()
    if bias is not None:
        want = want + bias.double()
    if out is not None:
        want = want + out.double()
    return want


def _close(got, want, k):
    scale = max(1.0, float(want.abs().max()))
    err = float((got.double() - want).abs().max())
    assert err <= 1e-6 * scale * max(1.0, k ** 0.5) + 1e-6, (err, scale)


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 13, 5), (128, 128, 16), (130, 257, 67), (300, 96, 1000),
                                   (2048, 512, 256)])
@pytest.mark.parametrize("trans_l", [False, True])
@pytest.mark.parametrize("trans_r", [False, True])
def test_layouts_against_float64(m, n, k, trans_l, trans_r):
    from causal_tuner.kernels.linear import mm_f32
    g = torch.Generator(device="cuda").manual_seed(m * 31 + n * 7 + k)
    left = torch.randn(k, m, device="cuda", generator=g).T if trans_l else torch.randn(m, k, device="cuda", generator=g)
    right = torch.randn(n, k, device="cuda", generator=g).T if trans_r else torch.randn(k, n, device="cuda", generator=g)
    out = torch.empty(m, n, device="cuda")
    mm_f32(left, right, out)
    _close(out, _ref(left, right), k)
    again = torch.empty_like(out)
    mm_f32(left, right, again)
    assert torch.equal(out, again)


def test_bias_accumulate_and_strided_views():
    from causal_tuner.kernels.linear import mm_f32
    g = torch.Generator(device="cuda").manual_seed(3)
    big = torch.randn(200, 300, device="cuda", generator=g)
    left = big[3:150, 5:98]            # row pitch 300, unaligned start
    right = torch.randn(120, 93, device="cuda", generator=g)[:, :].T[:, 7:101]   # column-major view
    bias = torch.randn(94, device="cuda", generator=g)
    out = torch.randn(147, 94, device="cuda", generator=g)
    start = out.clone()
    mm_f32(left, right, out, add=True)
    _close(out, _ref(left, right, start), 93)
    mm_f32(left, right, out, bias=bias)
    _close(out, _ref(left, right, bias=bias), 93)
    wide = torch.full((147, 200), float("nan"), device="cuda")
    mm_f32(left, right, wide[:, 50:144])   # beta = 0 ignores NaN in a strided destination
    _close(wide[:, 50:144], _ref(left, right), 93)
    assert torch.isnan(wide[:, :50]).all() and torch.isnan(wide[:, 144:]).all()


def test_empty_reduction_and_empty_output():
    from causal_tuner.kernels.linear import mm_f32
    left, right = torch.empty(5, 0, device="cuda"), torch.empty(0, 9, device="cuda")
    out = torch.full((5, 9), float("nan"), device="cuda")
    mm_f32(left, right, out)
    assert torch.equal(out, torch.zeros(5, 9, device="cuda"))
    out = torch.ones(5, 9, device="cuda")
    mm_f32(left, right, out, add=True)
    assert torch.equal(out, torch.ones(5, 9, device="cuda"))
    mm_f32(torch.empty(0, 4, device="cuda"), torch.empty(4, 3, device="cuda"), torch.empty(0, 3, device="cuda"))


def test_float32_projection_matches_torch_float32():
    """The float32 device route of forward_linear / input_gradient / parameter_gradients
    (kernels/linear.py:27-44) against torch's own float32 products with TF32 off."""
    from causal_tuner.kernels.linear import forward_linear, input_gradient, parameter_gradients
    torch.backends.cuda.matmul.allow_tf32 = False
    g = torch.Generator(device="cuda").manual_seed(5)
    m, k, n, r = 77, 96, 40, 8
    x, w = torch.randn(m, k, device="cuda", generator=g), torch.randn(n, k, device="cuda", generator=g) * .1
    a, b = torch.randn(r, k, device="cuda", generator=g) * .1, torch.randn(n, r, device="cuda", generator=g)
    bias, dy = torch.randn(n, device="cuda", generator=g), torch.randn(m, n, device="cuda", generator=g)
    out, xa = torch.empty(m, n, device="cuda"), torch.empty(m, r, device="cuda")
    forward_linear(x, w, a, b, out=out, xa=xa, bias=bias)
    want_xa = x @ a.T
    want = torch.addmm(bias, x, w.T).addmm_(want_xa, b.T)
    torch.testing.assert_close(xa, want_xa, rtol=2e-6, atol=2e-6)
    torch.testing.assert_close(out, want, rtol=2e-6, atol=2e-6)
    dx, low = torch.full((m, k), float("nan"), device="cuda"), torch.empty(m, r, device="cuda")
    input_gradient(dy, w, a, b, dx, low)
    torch.testing.assert_close(low, dy @ b, rtol=2e-6, atol=2e-6)
    torch.testing.assert_close(dx, (dy @ w).addmm_(dy @ b, a), rtol=2e-6, atol=2e-6)
    da, db = torch.full((r, k), float("nan"), device="cuda"), torch.empty(n, r, device="cuda")
    parameter_gradients(x, dy, da, db, low, xa, add=False)
    torch.testing.assert_close(da, low.T @ x, rtol=2e-6, atol=2e-6)
    torch.testing.assert_close(db, dy.T @ xa, rtol=2e-6, atol=2e-6)
