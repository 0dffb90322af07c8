"""Cross entropy whose forward and gradient run as one HIP launch.

The reference's training step calls F.cross_entropy(logits, y) with the
defaults (mean over rows, ignore_index -100; examples/emnist.py:221).
cross_entropy(logits, target) computes that loss and, in the same kernel
(tropnn_hip_cross_entropy), d loss / d logits, which backward scales by the
incoming gradient. Only f32 logits [rows, classes] on a GPU with int64
targets [rows] are supported; anything else raises (no CPU fallback). Class
weights and label smoothing are not supported (the reference uses neither).

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


class _CrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits: Tensor, target: Tensor, ignore_index: int) -> Tensor:
        loss, grad = cross_entropy_hip(logits.detach(), target, ignore_index)
        ctx.save_for_backward(grad)
        return loss

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        (grad,) = ctx.saved_tensors
        return grad * grad_out, None, None


def cross_entropy(logits: Tensor, target: Tensor, ignore_index: int = -100) -> Tensor:
    """F.cross_entropy(logits, target, ignore_index=ignore_index) with mean
    reduction, on the HIP kernel."""
    return _CrossEntropy.apply(logits, target, ignore_index)
