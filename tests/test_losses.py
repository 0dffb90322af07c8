"""cross_entropy's host side without a GPU: no CPU fallback, and the argument
checks (device, dtype, shape) that run before any launch."""
from __future__ import annotations

import pytest
import torch

from tropnn_amd import cross_entropy
from tropnn_amd.losses import cross_entropy_hip


def test_cpu_logits_raise():
    with pytest.raises(ValueError, match="GPU"):
        cross_entropy(torch.zeros(4, 3), torch.zeros(4, dtype=torch.int64))


def test_bad_shapes_and_dtypes_raise_before_launch(monkeypatch):
    # pretend the tensors are on a GPU: the dtype and shape checks come first
    class Fake:
        def __init__(self, shape, dtype):
            self.shape, self.dtype, self.ndim = torch.Size(shape), dtype, len(shape)
            self.device = torch.device("cuda:0")

    with pytest.raises(TypeError, match="f32"):
        cross_entropy_hip(Fake((4, 3), torch.float16), Fake((4,), torch.int64))
    with pytest.raises(TypeError, match="int64"):
        cross_entropy_hip(Fake((4, 3), torch.float32), Fake((4,), torch.int32))
    with pytest.raises(ValueError, match="rows"):
        cross_entropy_hip(Fake((4, 3), torch.float32), Fake((5,), torch.int64))
    with pytest.raises(ValueError, match="rows"):
        cross_entropy_hip(Fake((4, 3, 2), torch.float32), Fake((4,), torch.int64))


def test_unit_gradient_is_kept_and_replaced_after_a_write():
    from tropnn_amd import unit_gradient
    from tropnn_amd.losses import _is_unit

    loss = torch.tensor(2.5)
    u = unit_gradient(loss)
    assert u.shape == () and u.dtype == torch.float32 and float(u) == 1.0
    assert unit_gradient(torch.tensor(0.0)) is u  # one per device and dtype
    assert _is_unit(u) and not _is_unit(torch.ones(()))
    assert unit_gradient(torch.tensor(1.0, dtype=torch.float64)) is not u
    u.mul_(3.0)  # a write: no longer the unit
    assert not _is_unit(u)
    fresh = unit_gradient(loss)
    assert fresh is not u and float(fresh) == 1.0 and _is_unit(fresh)
