"""FusedAdam's host side without a GPU: argument checks as torch.optim.Adam
makes them, and no CPU fallback (a CPU parameter raises)."""
from __future__ import annotations

import pytest
import torch

from tropnn_amd import FusedAdam, FusedAdamW


@pytest.mark.parametrize(
    "kwargs",
    [dict(lr=-1.0), dict(eps=-1.0), dict(betas=(1.0, 0.999)), dict(betas=(0.9, -0.1)), dict(weight_decay=-1.0)],
)
def test_rejects_bad_hyperparameters(kwargs):
    with pytest.raises(ValueError):
        FusedAdam([torch.nn.Parameter(torch.zeros(3))], **kwargs)


def test_rejects_unsupported_modes():
    p = [torch.nn.Parameter(torch.zeros(3))]
    with pytest.raises(NotImplementedError):
        FusedAdam(p, amsgrad=True)
    with pytest.raises(NotImplementedError):
        FusedAdam(p, maximize=True)
    with pytest.raises(TypeError):
        FusedAdam(p, lr=torch.tensor(1e-3))


def test_adamw_defaults_follow_torch():
    p = [torch.nn.Parameter(torch.zeros(3))]
    ours, ref = FusedAdamW(p).defaults, torch.optim.AdamW(p).defaults
    assert ours["decoupled_weight_decay"] is True
    for key in ("lr", "betas", "eps", "weight_decay"):
        assert ours[key] == ref[key], key


def test_cpu_parameter_raises():
    p = torch.nn.Parameter(torch.zeros(3))
    p.grad = torch.ones(3)
    with pytest.raises(TypeError, match="GPU"):
        FusedAdam([p]).step()


def test_no_grad_is_a_no_op():
    p = torch.nn.Parameter(torch.zeros(3))
    opt = FusedAdam([p])
    opt.step()
    assert len(opt.state) == 0 and torch.equal(p.detach(), torch.zeros(3))
