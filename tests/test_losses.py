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
