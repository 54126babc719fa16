"""projection_loss on the device: FusedProjectionLoss driving the HIP weighted CE
(reference kernels/loss_cuda.py:81-162, kernels/loss.py:23-66).

Mirrors the reference's tests with their tolerances: tests/test_fast_training.py:120-140
(large vocabulary, fp32 and bf16, scaled backward) and :255-268 (cached gradients reused
by a repeated backward); tests/test_kernel_workspaces.py:125-150 (one logits workspace for
every tile, no gradients in evaluation), :185-220 (hidden reuse by a final norm's output,
rejected for leaves and views), :366-380 (unsupervised batch projects nothing), :383-418
(host row selection: intervals avoid gathers, scattered rows gather, weighted gradients);
tests/test_operators.py:92-108 (bf16 head gradient accumulated in fp32)."""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _full(x, head, labels, weights, dtype):
    logits = F.linear(x.detach(), head.detach().to(dtype)).float().flatten(0, 1)
    return (F.cross_entropy(logits, labels.flatten(), reduction="none") * weights.flatten()).sum(), logits


@pytest.mark.parametrize("vocab", [97, 185600])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_loss_large_vocabulary_and_scaled_gradient(vocab, dtype):
    from causal_tuner.kernels.loss import projection_loss
    x = torch.randn(1, 7, 32, device="cuda", dtype=dtype, requires_grad=True)
    head = torch.randn(vocab, 32, device="cuda", dtype=torch.float32, requires_grad=True) * .1
    head.retain_grad()
    labels = torch.randint(vocab, (1, 7), device="cuda")
    weights = torch.tensor([[0, .1, 1, .5, 0, 2, .2]], device="cuda")
    actual = projection_loss(x, head, labels, weights, token_budget=3, compute_dtype=dtype)
    expected, logits = _full(x, head, labels, weights, dtype)
    torch.testing.assert_close(actual, expected, rtol=2e-6, atol=1e-5)
    actual.mul(2.5).backward()
    derivative = logits.softmax(-1)
    derivative[torch.arange(7, device="cuda"), labels.flatten()] -= 1
    derivative = (derivative * weights.flatten()[:, None]).to(dtype)
    expected_head = (derivative.float().T @ x.detach().flatten(0, 1).float()) * 2.5
    torch.testing.assert_close(head.grad, expected_head, rtol=.01, atol=1e-4)


@pytest.mark.parametrize("vocab", [97, 4099])
def test_fused_loss_float16_compute_with_float32_head(vocab):
    """A float16 compute dtype with a float32 trainable head: the head gradient accumulates
    d^T x with fp16 operands into fp32, which the reference does with addmm on operands cast
    to the output dtype (kernels/linear.py:22-23, called from loss_cuda.py:145)."""
    from causal_tuner.kernels.loss import projection_loss
    dtype = torch.float16
    x = torch.randn(1, 7, 32, device="cuda", dtype=dtype, requires_grad=True)
    head = (torch.randn(vocab, 32, device="cuda", dtype=torch.float32) * .1).requires_grad_()
    labels = torch.randint(vocab, (1, 7), device="cuda")
    weights = torch.tensor([[0, .1, 1, .5, 0, 2, .2]], device="cuda")
    actual = projection_loss(x, head, labels, weights, token_budget=3, compute_dtype=dtype)
    expected, logits = _full(x, head, labels, weights, dtype)
    torch.testing.assert_close(actual, expected, rtol=1e-3, atol=1e-3)
    actual.backward()
    derivative = logits.softmax(-1)
    derivative[torch.arange(7, device="cuda"), labels.flatten()] -= 1
    derivative = (derivative * weights.flatten()[:, None]).to(dtype)
    expected_head = derivative.float().T @ x.detach().flatten(0, 1).float()
    assert head.grad.dtype == torch.float32
    torch.testing.assert_close(head.grad, expected_head, rtol=.01, atol=1e-4)
    expected_x = (derivative.float() @ head.detach().to(dtype).float()).to(dtype).view_as(x)
    torch.testing.assert_close(x.grad, expected_x, rtol=.01, atol=1e-3)


@pytest.mark.parametrize("supervised", [False, True])
def test_fused_loss_cached_gradients_can_be_reused(supervised):
    from causal_tuner.kernels.loss import projection_loss
    x = torch.randn(2, 5, 32, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    head = torch.randn(97, 32, device="cuda", dtype=torch.float32, requires_grad=True)
    labels = torch.randint(97, (2, 5), device="cuda")
    weights = torch.full((2, 5), .1 if supervised else 0, device="cuda")
    loss = projection_loss(x, head, labels, weights, token_budget=3)
    first = torch.autograd.grad(loss, (x, head), retain_graph=True)
    second = torch.autograd.grad(loss * 4, (x, head))
    for initial, repeated in zip(first, second):
        torch.testing.assert_close(repeated, initial * 4, rtol=0, atol=0)
        if not supervised:
            assert not initial.any()


@pytest.mark.parametrize("grad_enabled", [False, True])
def test_loss_reuses_logits_and_skips_evaluation_gradients(grad_enabled, monkeypatch):
    import causal_tuner.kernels.loss_cuda as loss_kernel
    from causal_tuner.kernels.loss import projection_loss
    x = torch.randn(2, 7, 32, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    head = torch.randn(4099, 32, device="cuda", requires_grad=True)
    targets = torch.randint(4099, (2, 7), device="cuda")
    weights = torch.rand(2, 7, device="cuda")
    weights[0, 1] = 0
    pointers, statistics, labels, factors = [], [], [], []
    original = loss_kernel.weighted_ce

    def checked(logits, targets, weights, *, gradient, **workspace):
        assert gradient == grad_enabled
        pointers.append(logits.data_ptr())
        statistics.append(workspace["partials"].data_ptr())
        labels.append(targets.data_ptr())
        factors.append(weights.data_ptr())
        return original(logits, targets, weights, gradient=gradient, **workspace)
    monkeypatch.setattr(loss_kernel, "weighted_ce", checked)
    with torch.set_grad_enabled(grad_enabled):
        output = projection_loss(x, head, targets, weights, token_budget=5)
    assert len(pointers) == 3 and len(set(pointers)) == 1
    assert all(len(set(values)) == 1 for values in (statistics, labels, factors))
    assert output.requires_grad == grad_enabled
    expected, _ = _full(x, head, targets, weights, torch.bfloat16)
    torch.testing.assert_close(output, expected, rtol=2e-6, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("train_head", [False, True])
@pytest.mark.parametrize("supervision", ["all", "mixed", "none"])
def test_loss_consumes_only_owned_final_norm_output(dtype, train_head, supervision):
    from causal_tuner.kernels.loss import projection_loss
    from causal_tuner.modeling.norm import RMSNorm
    norm = RMSNorm(32, 1e-6, dtype, "cuda")
    norm.weight.requires_grad_(False)
    x = torch.randn(2, 7, 32, device="cuda", dtype=dtype, requires_grad=True)
    other = x.detach().clone().requires_grad_(True)
    head = torch.randn(4099, 32, device="cuda", requires_grad=train_head)
    other_head = head.detach().clone().requires_grad_(train_head)
    targets = torch.randint(4099, (2, 7), device="cuda")
    weights = torch.rand(2, 7, device="cuda")
    if supervision == "mixed":
        weights[:, ::2] = 0
    elif supervision == "none":
        weights.zero_()
    hidden = norm(x)
    original = hidden.detach().clone()
    actual = projection_loss(hidden, head, targets, weights, token_budget=3, compute_dtype=dtype, reuse_hidden=True)
    cached = actual.grad_fn.saved_tensors[0]
    assert cached.data_ptr() == hidden.data_ptr()
    assert not cached[weights == 0].any()
    expected = projection_loss(norm(other), other_head, targets, weights, token_budget=3, compute_dtype=dtype)
    torch.testing.assert_close(actual, expected, rtol=0, atol=0)
    cached_before_backward = cached.clone()
    parameters = (x, head) if train_head else (x,)
    other_parameters = (other, other_head) if train_head else (other,)
    for a, e in zip(torch.autograd.grad(actual, parameters, retain_graph=True),
                    torch.autograd.grad(expected, other_parameters)):
        torch.testing.assert_close(a, e, rtol=0, atol=0)
    torch.testing.assert_close(cached, cached_before_backward, rtol=0, atol=0)
    scaled = torch.autograd.grad(actual * 2, x)[0]
    torch.testing.assert_close(scaled, torch.autograd.grad(norm(x), x, cached_before_backward * 2)[0],
                               rtol=0, atol=0)
    with torch.no_grad():
        torch.testing.assert_close(norm(x), original, rtol=0, atol=0)


def test_loss_rejects_consuming_leaf_or_view():
    from causal_tuner.kernels.loss import projection_loss
    x = torch.randn(2, 7, 32, device="cuda", requires_grad=True)
    head = torch.randn(17, 32, device="cuda")
    targets = torch.randint(17, (2, 7), device="cuda")
    weights = torch.ones(2, 7, device="cuda")
    for value in (x, (x * 2).view_as(x), (x * 2).transpose(0, 1)):
        with pytest.raises(ValueError, match="exclusive contiguous non-leaf"):
            projection_loss(value, head, targets, weights, reuse_hidden=True)


def test_zero_supervision_skips_head_cast_and_projection(monkeypatch):
    from causal_tuner.kernels.loss import projection_loss
    hidden = torch.randn(2, 7, 32, device="cuda", requires_grad=True)
    head = torch.randn(97, 32, device="cuda", requires_grad=True)
    original_to = torch.Tensor.to

    def checked_to(tensor, *args, **kwargs):
        assert tensor is not head, "An unsupervised batch must not materialize the head"
        return original_to(tensor, *args, **kwargs)

    def forbidden(*args, **kwargs):
        raise AssertionError("An unsupervised batch must not project logits")
    monkeypatch.setattr(torch.Tensor, "to", checked_to)
    monkeypatch.setattr(torch, "mm", forbidden)
    loss = projection_loss(hidden, head, torch.full((2, 7), -100, device="cuda"), torch.zeros(2, 7, device="cuda"))
    gradients = torch.autograd.grad(loss, (hidden, head))
    assert loss == 0 and all(torch.count_nonzero(gradient) == 0 for gradient in gradients)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("reuse", [False, True])
@pytest.mark.parametrize("layout", ["all", "interval", "gaps", "empty"])
def test_host_loss_rows_preserve_weighted_gradients_and_avoid_dense_gathers(dtype, reuse, layout, monkeypatch):
    from causal_tuner.kernels.loss import active_rows, projection_loss
    values = torch.randn(17, 32, device="cuda", dtype=dtype)
    leaf = values.clone().requires_grad_(True)
    hidden = leaf + 0 if reuse else leaf
    head = torch.randn(259, 32, device="cuda", dtype=torch.float32, requires_grad=True)
    weights = torch.rand(17)
    if layout == "interval":
        weights[:3] = weights[-2:] = 0
    elif layout == "gaps":
        weights[::3] = 0
    elif layout == "empty":
        weights.zero_()
    selection = active_rows(weights, "cuda")
    assert isinstance(selection, slice) == (layout != "gaps")
    targets = torch.randint(259, (17,), device="cuda")
    weights = weights.cuda()
    oracle_input = values.clone().requires_grad_(True)
    oracle_head = head.detach().clone().requires_grad_(True)
    logits = F.linear(oracle_input, oracle_head.to(dtype)).float()
    expected = (F.cross_entropy(logits, targets, reduction="none") * weights).sum()

    def forbidden(*a, **kw):
        raise AssertionError("Host selection and contiguous views must avoid CUDA selection/gather")
    monkeypatch.setattr(torch, "nonzero", forbidden)
    if layout != "gaps":
        monkeypatch.setattr(torch, "index_select", forbidden)
        monkeypatch.setattr(torch.Tensor, "index_copy_", forbidden)
    actual = projection_loss(hidden, head, targets, weights, token_budget=5, compute_dtype=dtype,
                             reuse_hidden=reuse, rows=selection)
    torch.testing.assert_close(actual, expected, rtol=2e-5, atol=2e-5)
    gradients = torch.autograd.grad(actual, (leaf, head), retain_graph=True)
    for result, oracle in zip(gradients, torch.autograd.grad(expected, (oracle_input, oracle_head))):
        tol = .03 if dtype == torch.bfloat16 else 3e-5
        torch.testing.assert_close(result, oracle, rtol=tol, atol=tol)
    for result, repeat in zip(gradients, torch.autograd.grad(actual, (leaf, head))):
        torch.testing.assert_close(result, repeat, rtol=0, atol=0)
    torch.testing.assert_close(leaf, values, rtol=0, atol=0)


def test_bf16_head_gradient_uses_fp32_accumulation():
    from causal_tuner.kernels.loss import projection_loss
    hidden = torch.randn(2, 7, 8, dtype=torch.bfloat16, device="cuda", requires_grad=True)
    head = torch.randn(19, 8, dtype=torch.float32, device="cuda", requires_grad=True)
    targets = torch.randint(0, 19, (2, 7), device="cuda")
    weights = torch.rand(2, 7, device="cuda")
    actual = projection_loss(hidden, head, targets, weights, token_budget=2, compute_dtype=torch.bfloat16)
    actual.backward()
    x = hidden.detach().flatten(0, 1)
    logits = F.linear(x, head.detach().bfloat16()).float()
    derivative = logits.softmax(-1)
    derivative[torch.arange(len(x), device="cuda"), targets.flatten()] -= 1
    derivative = (derivative * weights.flatten()[:, None]).bfloat16()
    expected = derivative.float().T @ x.float()
    torch.testing.assert_close(head.grad, expected, rtol=1e-6, atol=1e-6)
    assert not torch.equal(head.grad, expected.bfloat16().float())


def test_projection_loss_device_matches_host_route():
    """The device route against the host autograd function on the same inputs (fp32)."""
    from causal_tuner.kernels.loss import projection_loss
    hidden = torch.randn(3, 11, 24, requires_grad=True)
    head = torch.randn(301, 24, requires_grad=True)
    targets = torch.randint(0, 301, (3, 11))
    weights = torch.rand(3, 11)
    weights[1, ::2] = 0
    host = projection_loss(hidden, head, targets, weights, token_budget=4, compute_dtype=torch.float32)
    host_grads = torch.autograd.grad(host, (hidden, head))
    dh = hidden.detach().cuda().requires_grad_(True)
    dw = head.detach().cuda().requires_grad_(True)
    device = projection_loss(dh, dw, targets.cuda(), weights.cuda(), token_budget=4, compute_dtype=torch.float32)
    device_grads = torch.autograd.grad(device, (dh, dw))
    torch.testing.assert_close(device.cpu(), host, rtol=2e-5, atol=2e-5)
    for a, b in zip(device_grads, host_grads):
        torch.testing.assert_close(a.cpu(), b, rtol=3e-5, atol=3e-5)
