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


def test_loaded_amsgrad_group_raises():
    """A torch.optim.Adam state dict carries its group flags; FusedAdam
    refuses a loaded amsgrad group instead of ignoring it."""
    p = torch.nn.Parameter(torch.zeros(3))
    src = torch.optim.Adam([p], amsgrad=True)
    opt = FusedAdam([p])
    opt.load_state_dict(src.state_dict())
    with pytest.raises(NotImplementedError, match="amsgrad"):
        opt.step()


def test_loaded_step_becomes_f32_on_the_parameter_device():
    """torch's loader keeps "step" as saved unless the group is capturable or
    fused; FusedAdam converts it to a 0-dim f32 tensor on the parameter's
    device (here the CPU, the only device without a GPU)."""
    p = torch.nn.Parameter(torch.zeros(3))
    src = torch.optim.Adam([p])
    p.grad = torch.ones(3)
    src.step()
    sd = src.state_dict()
    sd["state"][0]["step"] = torch.tensor(1.0, dtype=torch.float64)
    opt = FusedAdam([p])
    opt.load_state_dict(sd)
    step = opt.state[p]["step"]
    assert step.dtype == torch.float32 and step.dim() == 0 and float(step) == 1.0
