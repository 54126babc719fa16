"""FusedAdamW (ct_adamw_step) against the optimizer the reference builds: torch.optim.AdamW
with fused=True (training/engine.py:10-16), on the same parameters and gradients.

Two groups with and without weight decay as make_optimizer builds them, fp32 parameters
(the LoRA factors) and bf16 parameters with bf16 states (the reference's reference_bf16
recipe, tests/test_fast_training.py:272-298), tensors below and above one chunk, maximize,
and a state dict that round-trips into torch's optimizer."""

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu


def _params(dtype, sizes):
    g = torch.Generator(device="cpu").manual_seed(7)
    return [torch.randn(*s, generator=g).to("cuda", dtype) for s in sizes]


def _run(cls, params, grads, steps, maximize, **extra):
    mats = [p.clone().requires_grad_(True) for p in params]
    groups = [{"params": [p for p in mats if p.ndim > 1], "weight_decay": 0.1},
              {"params": [p for p in mats if p.ndim <= 1], "weight_decay": 0.0}]
    opt = cls(groups, lr=3e-3, betas=(0.9, 0.95), eps=1e-6, weight_decay=0.1, maximize=maximize, **extra)
    for step in range(steps):
        for p, g in zip(mats, grads[step]):
            p.grad = g.clone()
        opt.step()
    return mats, opt


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("maximize", [False, True])
def test_adamw_matches_torch_fused(dtype, maximize):
    from causal_tuner.optim import FusedAdamW
    sizes = [(256, 4096), (4096, 256), (17,), (3, 5), (70001,), (129, 1023)]
    params = _params(dtype, sizes)
    g = torch.Generator(device="cpu").manual_seed(11)
    grads = [[(torch.randn(*s, generator=g) * 0.1).to("cuda", dtype) for s in sizes] for _ in range(4)]
    ours, opt = _run(FusedAdamW, params, grads, 4, maximize)
    want, ref = _run(torch.optim.AdamW, params, grads, 4, maximize, foreach=False, fused=True)
    for a, b in zip(ours, want):
        if dtype == torch.float32:
            torch.testing.assert_close(a, b, rtol=2e-6, atol=1e-7)
        else:  # one bf16 rounding step of slack
            torch.testing.assert_close(a.float(), b.float(), rtol=8e-3, atol=1e-5)
    for p, q in zip(ours, want):
        s, t = opt.state[p], ref.state[q]
        assert set(s) == set(t) == {"step", "exp_avg", "exp_avg_sq"}
        assert s["step"].is_cuda and s["step"].dtype == torch.float32 and float(s["step"]) == 4.0
        assert s["exp_avg"].dtype == dtype
        tol = dict(rtol=2e-6, atol=1e-8) if dtype == torch.float32 else dict(rtol=8e-3, atol=1e-6)
        torch.testing.assert_close(s["exp_avg"].float(), t["exp_avg"].float(), **tol)
        torch.testing.assert_close(s["exp_avg_sq"].float(), t["exp_avg_sq"].float(), **tol)


def test_adamw_state_dict_round_trip_and_skipped_parameters():
    from causal_tuner.optim import FusedAdamW
    params = _params(torch.float32, [(64, 32), (32,), (8, 8)])
    mats = [p.clone().requires_grad_(True) for p in params]
    opt = FusedAdamW(mats, lr=1e-2, weight_decay=0.05)
    for step in range(2):
        mats[0].grad = torch.randn_like(mats[0])
        mats[1].grad = torch.randn_like(mats[1])  # mats[2] never gets a gradient
        opt.step()
    assert mats[2] not in opt.state or not opt.state[mats[2]]
    torch.testing.assert_close(mats[2], params[2], rtol=0, atol=0)
    clone = [m.detach().clone().requires_grad_(True) for m in mats]
    ref = torch.optim.AdamW(clone, lr=1e-2, weight_decay=0.05, fused=True)
    # (load_state_dict may keep the given state tensors, so each optimizer gets its own copy)
    ref.load_state_dict(copy.deepcopy(opt.state_dict()))
    mine = FusedAdamW([m.detach().clone().requires_grad_(True) for m in mats], lr=1e-2, weight_decay=0.05)
    mine.load_state_dict(copy.deepcopy(opt.state_dict()))
    grad = torch.randn_like(mats[0])
    for group in (ref.param_groups[0]["params"], mine.param_groups[0]["params"]):
        group[0].grad = grad.clone()
        group[1].grad = None
    ref.step()
    mine.step()
    torch.testing.assert_close(mine.param_groups[0]["params"][0], ref.param_groups[0]["params"][0],
                               rtol=2e-6, atol=1e-7)
    assert float(mine.state[mine.param_groups[0]["params"][0]]["step"]) == 3.0
