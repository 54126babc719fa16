"""RMS normalization on the GPU (ct_rms_forward / ct_rms_backward behind RMS and RMSNorm;
reference kernels/core_cuda.py:29-130, modeling/model.py:38-64).

Follows the reference's tests/test_fused_core.py:7-74 (forward/backward against the torch
formula, trainable weight with fp32 reduction, empty input) and
tests/test_kernel_workspaces.py:108-124, 220-253 (gradient ownership, reconstruction), with
their tolerances, plus the float64 oracle (oracle/rmsnorm.py): results within one rounding
of the stored dtype (the row sums' order and the reciprocal square root differ from the
reference's Triton kernel, so bit-exactness is not the bar here; repeated calls are
bit-identical)."""

import numpy as np
import pytest
import torch

from oracle import rmsnorm as orms

pytestmark = pytest.mark.gpu
NAMES = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("width", [32, 4096])
def test_fused_rms_matches_torch_forward_backward(dtype, width):
    """tests/test_fused_core.py:7-25."""
    from causal_tuner.modeling.norm import RMSNorm
    x = torch.randn(2, 17, width, device="cuda", dtype=dtype, requires_grad=True)
    reference = x.detach().clone().requires_grad_(True)
    norm = RMSNorm(width, 1e-6, dtype, "cuda")
    torch.nn.init.uniform_(norm.weight, .5, 1.5)
    norm.weight.requires_grad_(False)
    expected = ((reference.float() * torch.rsqrt(reference.float().square().mean(-1, keepdim=True) + 1e-6)).to(dtype)
                * norm.weight)
    actual = norm(x)
    tolerance = .02 if dtype == torch.bfloat16 else 2e-6
    torch.testing.assert_close(actual, expected, rtol=tolerance, atol=tolerance)
    go = torch.randn_like(x)
    torch.testing.assert_close(torch.autograd.grad(actual, x, go)[0], torch.autograd.grad(expected, reference, go)[0],
                               rtol=tolerance, atol=tolerance)


@pytest.mark.parametrize("dtype,weight_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                               (torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("width", [33, 4096])
@pytest.mark.parametrize("train_input", [False, True])
def test_trainable_rms_bounded_fp32_weight_reduction(dtype, weight_dtype, width, train_input):
    """tests/test_fused_core.py:28-65: trainable weight (zero and negative entries), fp32
    weight reduction over at most 4 x CUs row groups, repeated gradients bit-identical,
    upstream gradient not mutated."""
    from causal_tuner.kernels import _native
    from causal_tuner.modeling.norm import RMSNorm
    x = torch.randn(257, width, device="cuda", dtype=dtype, requires_grad=train_input)
    oracle_x = x.detach().clone().requires_grad_(train_input)
    norm = RMSNorm(width, 1e-6, weight_dtype, "cuda")
    with torch.no_grad():
        norm.weight.uniform_(.5, 1.5)
        norm.weight[:3] = torch.tensor([0., -1., 2.], device="cuda")
    oracle_w = norm.weight.detach().float().requires_grad_(True)
    rounded_w = oracle_w + (oracle_w.to(dtype).float() - oracle_w).detach()
    normalized = (oracle_x.float() * torch.rsqrt(oracle_x.float().square().mean(-1, keepdim=True) + 1e-6)).to(dtype)
    expected = (normalized.float() * rounded_w).to(dtype)
    actual = norm(x, reuse_grad=True)
    upstream = torch.randn_like(actual.T).contiguous().T
    original = upstream.clone()
    tolerance = dict(rtol=.02, atol=.04) if dtype == torch.bfloat16 else dict(rtol=3e-5, atol=2e-5)
    torch.testing.assert_close(actual, expected, **tolerance)
    inputs = (x, norm.weight) if train_input else (norm.weight,)
    reference = (oracle_x, oracle_w) if train_input else (oracle_w,)
    gradients = torch.autograd.grad(actual, inputs, upstream, retain_graph=True)
    oracles = torch.autograd.grad(expected, reference, upstream)
    for result, oracle in zip(gradients, oracles):
        torch.testing.assert_close(result, oracle.to(result.dtype), **tolerance)
    for result, repeat in zip(gradients, torch.autograd.grad(actual, inputs, upstream)):
        torch.testing.assert_close(result, repeat, rtol=0, atol=0)
    torch.testing.assert_close(upstream, original, rtol=0, atol=0)
    maximum = 4 * torch.cuda.get_device_properties(x.device).multi_processor_count
    assert 0 < _native.library().ct_rms_backward_workspace(257, width, 1) <= maximum * width * 4


def test_trainable_rms_empty_input_has_zero_weight_gradient():
    """tests/test_fused_core.py:68-74."""
    from causal_tuner.modeling.norm import RMSNorm
    norm = RMSNorm(33, 1e-6, torch.float32, "cuda")
    x = torch.empty(0, 33, device="cuda", requires_grad=True)
    dx, dw = torch.autograd.grad(norm(x).sum(), (x, norm.weight))
    assert dx.shape == x.shape and torch.count_nonzero(dw) == 0


@pytest.mark.parametrize("reuse", [False, True])
def test_rms_gradient_ownership_and_zero_weights(reuse):
    """tests/test_kernel_workspaces.py:108-124."""
    from causal_tuner.kernels.core_cuda import RMS
    x = torch.randn(3, 4096, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    weight = torch.randn(4096, device="cuda", dtype=torch.bfloat16)
    weight[:64] = 0
    signal = torch.randn_like(x)
    original = signal.clone()
    expected = torch.autograd.grad(RMS.apply(x, weight, 1e-6), x, original)[0]
    result = torch.autograd.grad(RMS.apply(x, weight, 1e-6, reuse), x, signal)[0]
    torch.testing.assert_close(result, expected, rtol=0, atol=0)
    assert (result.data_ptr() == signal.data_ptr()) == reuse
    if not reuse:
        torch.testing.assert_close(signal, original, rtol=0, atol=0)


@pytest.mark.parametrize("width", [32, 4096, 4100])
def test_reconstructed_rms_shares_output_and_bounds_gradient_error(width):
    """tests/test_kernel_workspaces.py:220-238."""
    from causal_tuner.modeling.norm import RMSNorm
    norm = RMSNorm(width, 1e-6, torch.bfloat16, "cuda")
    norm.weight.requires_grad_(False)
    torch.nn.init.uniform_(norm.weight, .5, 1.5)
    x = torch.randn(2, 7, width, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    saved = []
    with torch.autograd.graph.saved_tensors_hooks(lambda tensor: saved.append(tensor) or tensor, lambda tensor: tensor):
        output = norm(x, reuse_grad=True)
    assert saved[0].data_ptr() == output.data_ptr() and saved[0].data_ptr() != x.data_ptr()
    exact = norm(x)
    torch.testing.assert_close(output, exact, rtol=0, atol=0)
    signal = torch.randn_like(output)
    expected = torch.autograd.grad(exact, x, signal)[0].float()
    actual = torch.autograd.grad(output, x, signal.clone())[0].float()
    assert (actual - expected).norm() / expected.norm() < .003
    assert (actual - expected).abs().max() < .05


@pytest.mark.parametrize("bad_weight", [0., 1e-9, 1e9, float("inf"), float("nan")])
def test_reconstructed_rms_invalidates_cache_and_falls_back(bad_weight):
    """tests/test_kernel_workspaces.py:241-253."""
    from causal_tuner.modeling.norm import RMSNorm
    norm = RMSNorm(32, 1e-6, torch.bfloat16, "cuda")
    norm.weight.requires_grad_(False)
    x = torch.randn(2, 7, 32, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    assert norm._can_reconstruct(x.dtype)
    norm.weight[0] = bad_weight
    saved = []
    with torch.autograd.graph.saved_tensors_hooks(lambda tensor: saved.append(tensor) or tensor, lambda tensor: tensor):
        norm(x, reuse_grad=True)
    assert not norm._can_reconstruct(x.dtype)
    assert saved[0].data_ptr() == x.data_ptr()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,width", [(4096, 2048), (37, 4100), (5, 33)])
def test_rms_matches_oracle(dtype, rows, width):
    """Against the float64 oracle with the reference's rounding points: the output within
    two steps of the dtype (x * rstd may round to the neighbouring value, and the product
    with the weight is rounded again), gradients to the dtype's precision; trainable fp32
    weight."""
    from causal_tuner.kernels.core_cuda import RMS
    g = torch.Generator().manual_seed(rows + width)
    x = torch.randn(rows, width, generator=g).to(dtype)
    w = (torch.rand(width, generator=g) + 0.5).float()
    go = torch.randn(rows, width, generator=g).to(dtype)
    xd = x.cuda().requires_grad_(True)
    wd = w.cuda().requires_grad_(True)
    y = RMS.apply(xd, wd, 1e-6)
    gx, dw = torch.autograd.grad(y, (xd, wd), go.cuda())
    want_y, rstd = orms.forward(x.float().numpy(), w.numpy(), 1e-6, NAMES[dtype])
    want_gx, want_dw = orms.backward(x.float().numpy(), w.numpy(), rstd, go.float().numpy(), NAMES[dtype])
    step = {torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10, torch.float32: 2 ** -22}[dtype]
    got = y.detach().float().cpu().numpy()
    assert np.all(np.abs(got - want_y) <= 2 * step * np.abs(want_y) + 1e-30)
    if dtype != torch.float32:   # (in fp32 the float32 rstd alone moves most last bits)
        assert np.mean(got == want_y) > 0.99   # almost every element exactly the oracle's
    gx_err = np.abs(gx.float().cpu().numpy() - want_gx).max() / np.abs(want_gx).max()
    assert gx_err <= 4 * step, gx_err
    dw_err = np.abs(dw.cpu().numpy() - want_dw).max() / np.abs(want_dw).max()
    assert dw_err <= 1e-5 + 2 * step, dw_err
