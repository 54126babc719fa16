"""projection_loss on host tensors and the host-side row selection (reference
kernels/loss.py, kernels/reference.py:30-73).

Mirrors the reference's tests/test_operators.py:72-108 (full-logit CE with and without a
trainable head, fp32 accumulation of a bf16 head gradient) and checks `active_rows`'
slice/index contract (loss.py:6-16) and the argument validation (loss.py:25-52)."""

import pytest
import torch
import torch.nn.functional as F

from causal_tuner.kernels.loss import active_rows, projection_loss, row_count


@pytest.mark.parametrize("train_head", [False, True])
@pytest.mark.parametrize("weight", [0.0, .2, 1.0])
def test_projection_loss_against_full_logits(train_head, weight):
    hidden = torch.randn(2, 5, 7, requires_grad=True)
    head = torch.randn(13, 7, requires_grad=train_head)
    targets = torch.randint(0, 13, (2, 5))
    weights = torch.zeros(2, 5)
    weights[0, 1] = weight
    weights[1, 3] = weight * 2
    actual = projection_loss(hidden, head, targets, weights, token_budget=1, compute_dtype=torch.float32)
    logits = F.linear(hidden, head).flatten(0, 1)
    expected = (F.cross_entropy(logits, targets.flatten(), reduction="none") * weights.flatten()).sum()
    params = [hidden] + ([head] if train_head else [])
    expected_grads = torch.autograd.grad(expected, params)
    actual_grads = torch.autograd.grad(actual, params)
    torch.testing.assert_close(actual, expected)
    for a, b in zip(actual_grads, expected_grads):
        torch.testing.assert_close(a, b, atol=2e-6, rtol=2e-6)


def test_bf16_head_gradient_uses_fp32_accumulation_on_host():
    hidden = torch.randn(2, 7, 8, dtype=torch.bfloat16, requires_grad=True)
    head = torch.randn(19, 8, dtype=torch.float32, requires_grad=True)
    targets = torch.randint(0, 19, (2, 7))
    weights = torch.rand(2, 7)
    actual = projection_loss(hidden, head, targets, weights, token_budget=2, compute_dtype=torch.bfloat16)
    actual.backward()
    x = hidden.detach().flatten(0, 1)
    logits = F.linear(x, head.detach().bfloat16()).float()
    derivative = logits.softmax(-1)
    derivative[torch.arange(len(x)), targets.flatten()] -= 1
    derivative = (derivative * weights.flatten()[:, None]).bfloat16()
    expected = derivative.float().T @ x.float()
    torch.testing.assert_close(head.grad, expected, rtol=1e-6, atol=1e-6)
    assert not torch.equal(head.grad, expected.bfloat16().float())


def test_active_rows_slices_and_indices():
    weights = torch.tensor([0., 1., 2., 0., 3.])
    rows = active_rows(weights)
    assert torch.equal(rows, torch.tensor([1, 2, 4])) and row_count(rows) == 3
    assert active_rows(torch.tensor([0., 1., 1., 0.])) == slice(1, 3)
    assert active_rows(torch.ones(4)) == slice(0, 4)
    assert active_rows(torch.zeros(4)) == slice(0, 0) and row_count(slice(0, 0)) == 0
    assert active_rows(torch.tensor([float("nan"), -1., 0.])) == slice(0, 0)


def test_projection_loss_argument_errors():
    hidden, head = torch.randn(1, 3, 4), torch.randn(5, 4)
    targets, weights = torch.zeros(1, 3, dtype=torch.long), torch.ones(1, 3)
    with pytest.raises(ValueError, match="positive"):
        projection_loss(hidden, head, targets, weights, token_budget=0)
    with pytest.raises(ValueError, match="Unsupported"):
        projection_loss(hidden, head, targets, weights, implementation="other")
    with pytest.raises(ValueError, match="cut backend"):
        projection_loss(hidden, head, targets, weights, cut_chunk_size=2)
    with pytest.raises(ValueError, match="use fused"):
        projection_loss(hidden, head.requires_grad_(True), targets, weights, implementation="cut")
    with pytest.raises(RuntimeError, match="cut-cross-entropy"):
        projection_loss(hidden, head.detach(), targets, weights, implementation="cut")
