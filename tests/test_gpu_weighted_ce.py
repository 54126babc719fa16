"""Fused weighted cross-entropy on the GPU (ct_weighted_ce behind weighted_ce; reference
kernels/loss_cuda.py:11-70).

Mirrors the reference's tests/test_kernel_workspaces.py:282-300 (target boundaries at the
4096-column split edges, a row of weight 0, logits untouched without gradient and
overwritten with the derivative with it), with its tolerances, against torch's float32
cross-entropy and autograd; plus a float64 check of the loss and determinism."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("vocab", [97, 4096, 4097, 185600])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_ce_target_boundaries_and_logit_ownership(vocab, dtype):
    from causal_tuner.kernels.loss_cuda import weighted_ce
    logits = (torch.randn(5, vocab, device="cuda") * 4).to(dtype)
    targets = torch.tensor([0, min(4095, vocab - 1), min(4096, vocab - 1), vocab // 2, vocab - 1], device="cuda")
    weights = torch.tensor([0, .125, 1, 2, .5], device="cuda")
    reference = logits.float().requires_grad_(True)
    loss = (torch.nn.functional.cross_entropy(reference, targets, reduction="none") * weights).sum()
    expected_grad, = torch.autograd.grad(loss, reference)
    for gradient in (False, True):
        workspace = logits.clone()
        actual = weighted_ce(workspace, targets, weights, gradient=gradient).sum()
        torch.testing.assert_close(actual, loss, rtol=2e-6, atol=1e-5)
        if gradient:
            tolerance = .008 if dtype == torch.bfloat16 else 2e-6
            torch.testing.assert_close(workspace, expected_grad.to(dtype), rtol=tolerance, atol=1e-7)
        else:
            torch.testing.assert_close(workspace, logits, rtol=0, atol=0)


def test_weighted_ce_against_float64_and_repeatable():
    """Large rows (C4's vocab, 49152), per-row losses against float64 log-sum-exp, a target
    outside the vocabulary (its term is 0), and bit-identical repeats."""
    from causal_tuner.kernels.loss_cuda import weighted_ce
    g = torch.Generator(device="cuda").manual_seed(5)
    rows, vocab = 64, 49152
    logits = (torch.randn(rows, vocab, device="cuda", generator=g) * 3).to(torch.bfloat16)
    targets = torch.randint(vocab, (rows,), device="cuda", generator=g)
    targets[3] = -100
    weights = torch.rand(rows, device="cuda", generator=g)
    loss = weighted_ce(logits.clone(), targets, weights, gradient=False)
    again = weighted_ce(logits.clone(), targets, weights, gradient=False)
    assert torch.equal(loss, again)
    l64 = logits.double()
    lse = torch.logsumexp(l64, dim=1)
    picked = torch.where((targets >= 0) & (targets < vocab), l64.gather(1, targets.clamp(0, vocab - 1)[:, None])[:, 0],
                         torch.zeros_like(lse))
    expected = weights.double() * (lse - picked)
    torch.testing.assert_close(loss.double(), expected, rtol=1e-6, atol=1e-5)
    grad = logits.clone()
    weighted_ce(grad, targets, weights, gradient=True)
    grad2 = logits.clone()
    weighted_ce(grad2, targets, weights, gradient=True)
    assert torch.equal(grad, grad2)
    # each row's derivative sums to 0 (softmax sums to 1, minus the one-hot), or to the
    # row's weight when the target lies outside the vocabulary
    sums = grad.float().sum(1)
    want = torch.zeros_like(sums)
    want[3] = weights[3]
    torch.testing.assert_close(sums, want, rtol=0, atol=3e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("pad", [0, 3])
def test_weighted_ce_row_pitch_and_split_edges(dtype, pad):
    """Rows with a pitch past the vocabulary (pad 3: rows not 16-byte aligned, so the
    per-element path) and a vocabulary just past two 4096-column splits, against float64;
    the columns past the vocabulary are never written."""
    from causal_tuner.kernels.loss_cuda import weighted_ce
    rows, vocab = 9, 8192 + 5
    g = torch.Generator(device="cuda").manual_seed(8)
    storage = (torch.randn(rows, vocab + pad, device="cuda", generator=g) * 2).to(dtype)
    logits = storage[:, :vocab]
    targets = torch.tensor([0, 4095, 4096, 8191, 8192, vocab - 1, 17, -1, vocab], device="cuda")
    weights = torch.rand(rows, device="cuda", generator=g) + 0.5
    l64 = logits.double()
    lse = torch.logsumexp(l64, dim=1)
    inside = (targets >= 0) & (targets < vocab)
    picked = torch.where(inside, l64.gather(1, targets.clamp(0, vocab - 1)[:, None])[:, 0], torch.zeros_like(lse))
    want_loss = weights.double() * (lse - picked)
    soft = torch.softmax(l64, dim=1)
    onehot = torch.zeros_like(soft)
    onehot[inside.nonzero()[:, 0], targets[inside]] = 1
    want_grad = (soft - onehot) * weights.double()[:, None]
    before = storage.clone()
    loss = weighted_ce(logits, targets, weights, gradient=True)
    torch.testing.assert_close(loss.double(), want_loss, rtol=1e-5, atol=1e-5)
    tol = {torch.float32: 1e-6, torch.bfloat16: 8e-3, torch.float16: 1e-3}[dtype]
    torch.testing.assert_close(logits.double(), want_grad.to(dtype).double(), rtol=tol, atol=1e-6)
    if pad:
        assert torch.equal(storage[:, vocab:], before[:, vocab:])


@pytest.mark.parametrize("column", [3, 5000])
def test_nan_logit_gives_nan_loss(column):
    """A NaN logit in a non-target column makes that row's loss NaN, as sum(exp(values -
    max)) does in the reference's kernel, so a diverging step does not report a finite
    loss; the other rows are unaffected."""
    from causal_tuner.kernels.loss_cuda import weighted_ce
    logits = torch.randn(3, 8192, device="cuda").to(torch.bfloat16)
    logits[1, column] = float("nan")
    targets = torch.tensor([7, 7, 7], device="cuda")
    weights = torch.ones(3, device="cuda")
    loss = weighted_ce(logits.clone(), targets, weights, gradient=False)
    assert torch.isnan(loss[1])
    assert bool(torch.isfinite(loss[[0, 2]]).all())
    want = torch.nn.functional.cross_entropy(logits[[0, 2]].float(), targets[[0, 2]], reduction="none")
    torch.testing.assert_close(loss[[0, 2]], want, rtol=2e-6, atol=1e-5)
    grad = logits.clone()
    weighted_ce(grad, targets, weights, gradient=True)
    assert bool(torch.isnan(grad[1].float()).all()) and bool(torch.isfinite(grad[[0, 2]].float()).all())
