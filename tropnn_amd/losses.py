"""Cross entropy whose forward and gradient run as one HIP launch.

The reference's training step calls F.cross_entropy(logits, y) with the
defaults (mean over rows, ignore_index -100; examples/emnist.py:221).
cross_entropy(logits, target) computes that loss and, in the same kernel
(tropnn_hip_cross_entropy), d loss / d logits, which backward scales by the
incoming gradient, or returns as it is when the incoming gradient is the kept
unit_gradient(loss) (then a training step launches nothing for the loss
between the kernel and the last layer's backward). Only f32 logits [rows,
classes] on a GPU with int64 targets [rows] are supported; anything else
raises (no CPU fallback). Class weights and label smoothing are not supported
(the reference uses neither).

The kernel is one workgroup of 1024 threads, sized for the classifier's step
(512 rows of 10 logits: ~5 us): its time grows linearly with rows * classes
beyond a few thousand rows, where F.cross_entropy's multi-workgroup kernels
are the better choice. An empty batch gives a NaN loss and an empty gradient
without a launch, as F.cross_entropy's mean over no rows does.
"""
from __future__ import annotations

import torch
from torch import Tensor

from .backends.pairwise_hip import _check, _stream, load_library


def cross_entropy_hip(logits: Tensor, target: Tensor, ignore_index: int = -100) -> tuple[Tensor, Tensor]:
    """(loss, grad_logits): the mean cross entropy as a 0-dim tensor and its
    gradient with respect to logits, from one launch on the current stream."""
    if logits.device.type != "cuda" or target.device != logits.device:
        raise ValueError(f"cross_entropy needs logits and target on one GPU, got {logits.device} and {target.device}")
    if logits.dtype != torch.float32:
        raise TypeError(f"cross_entropy needs f32 logits, got {logits.dtype}")
    if target.dtype != torch.int64:
        raise TypeError(f"cross_entropy needs int64 targets, got {target.dtype}")
    if logits.ndim != 2 or target.shape != (logits.shape[0],):
        raise ValueError(f"cross_entropy needs logits [rows, classes] and target [rows], got "
                         f"{tuple(logits.shape)} and {tuple(target.shape)}")
    logits = logits.contiguous()
    target = target.contiguous()
    if logits.shape[0] == 0:
        # the mean over no rows, as F.cross_entropy returns it
        return torch.full((), float("nan"), dtype=torch.float32, device=logits.device), torch.empty_like(logits)
    loss = torch.empty((), dtype=torch.float32, device=logits.device)
    grad = torch.empty_like(logits)
    rc = load_library().tropnn_hip_cross_entropy(
        logits.shape[0], logits.shape[1], logits.data_ptr(), target.data_ptr(), int(ignore_index), loss.data_ptr(),
        grad.data_ptr(), _stream(logits.device))
    _check(rc, "tropnn_hip_cross_entropy")
    return loss, grad


_UNITS: dict[tuple[torch.device, torch.dtype], Tensor] = {}


def unit_gradient(loss: Tensor) -> Tensor:
    """The 0-dim one to start a scalar loss's backward with:
    loss.backward(unit_gradient(loss)) computes what loss.backward() does.
    One tensor per device and dtype, made on first use and kept, so autograd
    launches no fill for the implicit d loss / d loss of each step, and
    cross_entropy's backward, handed this tensor, returns its saved logits
    gradient as it is instead of launching a multiplication by one. Make the
    first call outside graph capture (a training loop's eager warmup step
    does). A tensor that was written to in place (its version moved) is
    replaced by a fresh one."""
    key = (loss.device, loss.dtype)
    unit = _UNITS.get(key)
    if unit is None or unit._version != 0:
        unit = torch.ones((), dtype=loss.dtype, device=loss.device)
        _UNITS[key] = unit
    return unit


def _is_unit(grad_out: Tensor) -> bool:
    """Whether grad_out is (a view of) the kept unit gradient, unchanged: a
    host-side check of its address and version, no device read."""
    unit = _UNITS.get((grad_out.device, grad_out.dtype))
    return unit is not None and unit._version == 0 and grad_out.data_ptr() == unit.data_ptr() and grad_out.ndim == 0


class _CrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits: Tensor, target: Tensor, ignore_index: int) -> Tensor:
        loss, grad = cross_entropy_hip(logits.detach(), target, ignore_index)
        ctx.save_for_backward(grad)
        return loss

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        (grad,) = ctx.saved_tensors
        if _is_unit(grad_out):
            return grad, None, None  # d loss / d logits as the kernel wrote it: no scaling launch
        return grad * grad_out, None, None


def cross_entropy(logits: Tensor, target: Tensor, ignore_index: int = -100) -> Tensor:
    """F.cross_entropy(logits, target, ignore_index=ignore_index) with mean
    reduction, on the HIP kernel."""
    return _CrossEntropy.apply(logits, target, ignore_index)
