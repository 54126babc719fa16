"""FusedAdamW's host-side contract (no device needed): argument validation as in
torch.optim.AdamW, the fused-state flag the reference's checkpoint loader reads
(checkpointing/io.py:214), and loud refusal of host parameters."""

import pytest
import torch


def test_adamw_arguments_and_defaults():
    from causal_tuner.optim import FusedAdamW
    p = torch.nn.Parameter(torch.zeros(3))
    opt = FusedAdamW([p], lr=1e-3)
    assert opt.defaults["fused"] and not opt.defaults["amsgrad"]
    for kwargs in ({"lr": -1.0}, {"eps": -1.0}, {"betas": (1.0, 0.9)}, {"weight_decay": -0.1}):
        with pytest.raises(ValueError):
            FusedAdamW([p], **kwargs)
    with pytest.raises(NotImplementedError):
        FusedAdamW([p], amsgrad=True)


def test_adamw_refuses_host_parameters():
    from causal_tuner.optim import FusedAdamW
    p = torch.nn.Parameter(torch.zeros(3))
    p.grad = torch.ones(3)
    with pytest.raises(NotImplementedError, match="device"):
        FusedAdamW([p]).step()
