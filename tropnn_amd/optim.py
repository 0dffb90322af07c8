"""Adam / AdamW whose update runs as one HIP launch over all parameters.

The reference trains its classifiers with torch.optim.AdamW(weight_decay=0)
(examples/emnist.py:310). FusedAdam is a drop-in torch.optim.Optimizer for
that role: the same update as torch's Adam (non-amsgrad, op order of its
single-tensor path), the same per-parameter state ("step", "exp_avg",
"exp_avg_sq", so state dicts move between the two in both directions),
computed by tropnn_hip_adam_step in libtropnn_hip.so. The step counters live
on the device, so a training step captured in a HIP graph replays with the
current count; lr and the other hyperparameters are read when step() runs (a
captured graph keeps the values it was captured with).

The kernel writes the tensors through raw device pointers, so step() bumps
the autograd version counter of every tensor it updates, as torch's in-place
optimizers do: caches keyed by a parameter's version (PairwiseLinear's f16
LUT copy, the lazy route-debug guard) see the update. A replayed HIP graph
runs no Python and bumps nothing; PairwiseLinear re-casts its f16 copy inside
a captured forward for that reason.

Only dense f32 parameters on a GPU are supported; anything else raises (there
is no CPU fallback).
"""
from __future__ import annotations

import ctypes
from collections import defaultdict

import torch

from .backends.pairwise_hip import _check, _stream, load_library


def adam_step_hip(params, grads, exp_avgs, exp_avg_sqs, steps, *, lr: float, beta1: float, beta2: float,
                  eps: float, weight_decay: float, decoupled_weight_decay: bool) -> None:
    """One Adam / AdamW update of equal-length lists of contiguous f32 tensors
    on one GPU (steps: 0-dim f32 tensors, one per parameter), on the current
    stream of that GPU."""
    n = len(params)
    if not (len(grads) == len(exp_avgs) == len(exp_avg_sqs) == len(steps) == n):
        raise ValueError("params, grads, exp_avgs, exp_avg_sqs and steps must have equal lengths")
    if n == 0:
        return
    dev = params[0].device
    for name, ts in (("params", params), ("grads", grads), ("exp_avgs", exp_avgs), ("exp_avg_sqs", exp_avg_sqs),
                     ("steps", steps)):
        for k, t in enumerate(ts):
            if t.device != dev or t.device.type != "cuda":
                raise ValueError(f"{name}[{k}] is on {t.device}, expected {dev} (a GPU)")
            if t.dtype != torch.float32:
                raise TypeError(f"{name}[{k}] has dtype {t.dtype}, expected torch.float32")
            if not t.is_contiguous():
                raise ValueError(f"{name}[{k}] is not contiguous")
    for k in range(n):
        numel = params[k].numel()
        if grads[k].numel() != numel or exp_avgs[k].numel() != numel or exp_avg_sqs[k].numel() != numel:
            raise ValueError(f"tensor {k}: grad / exp_avg / exp_avg_sq sizes differ from the parameter's {numel}")
        if steps[k].numel() != 1:
            raise ValueError(f"steps[{k}] must hold one element")
    ptrs = ctypes.c_void_p * n
    lib = load_library()
    rc = lib.tropnn_hip_adam_step(
        n,
        ptrs(*[t.data_ptr() for t in params]),
        ptrs(*[t.data_ptr() for t in grads]),
        ptrs(*[t.data_ptr() for t in exp_avgs]),
        ptrs(*[t.data_ptr() for t in exp_avg_sqs]),
        (ctypes.c_int64 * n)(*[t.numel() for t in params]),
        ptrs(*[t.data_ptr() for t in steps]),
        float(lr), float(beta1), float(beta2), float(eps), float(weight_decay), int(bool(decoupled_weight_decay)),
        _stream(dev),
    )
    _check(rc, "tropnn_hip_adam_step")
    # the launch wrote these through raw pointers: tell autograd and the
    # version-keyed caches, as an in-place torch op would
    torch.autograd.graph.increment_version(params + exp_avgs + exp_avg_sqs + steps)


class FusedAdam(torch.optim.Optimizer):
    """torch.optim.Adam's update (amsgrad=False, maximize=False) on the GPU in
    one launch per parameter group and device. decoupled_weight_decay=True
    gives AdamW."""

    def __init__(self, params, lr: float = 1e-3, betas: tuple[float, float] = (0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.0, decoupled_weight_decay: bool = False, *, amsgrad: bool = False,
                 maximize: bool = False) -> None:
        if isinstance(lr, torch.Tensor):
            raise TypeError("FusedAdam takes lr as a float")
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        if amsgrad or maximize:
            raise NotImplementedError("FusedAdam supports amsgrad=False and maximize=False only")
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                        decoupled_weight_decay=decoupled_weight_decay)
        super().__init__(params, defaults)

    def load_state_dict(self, state_dict) -> None:
        """torch's loader leaves "step" where it was saved unless the group is
        capturable or fused (Optimizer._process_value_according_to_param_policy),
        e.g. on the CPU for a torch.optim.Adam state dict or a checkpoint
        loaded with map_location="cpu"; the kernel reads it from the
        parameter's device as f32."""
        super().load_state_dict(state_dict)
        for p, state in self.state.items():
            step = state.get("step")
            if step is None:
                continue
            if not isinstance(step, torch.Tensor):
                step = torch.tensor(float(step))
            if step.device != p.device or step.dtype != torch.float32 or step.dim() != 0:
                state["step"] = step.detach().reshape(()).to(device=p.device, dtype=torch.float32)

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            if group.get("amsgrad") or group.get("maximize"):
                # a loaded torch.optim.Adam state dict can carry these flags
                raise NotImplementedError("FusedAdam supports amsgrad=False and maximize=False only")
            by_device: dict[torch.device, list] = defaultdict(lambda: ([], [], [], [], []))
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("FusedAdam does not support sparse gradients")
                if p.device.type != "cuda" or p.dtype != torch.float32:
                    raise TypeError(f"FusedAdam needs f32 parameters on a GPU, got {p.dtype} on {p.device}")
                state = self.state[p]
                if len(state) == 0:
                    state["step"] = torch.zeros((), dtype=torch.float32, device=p.device)
                    state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                lists = by_device[p.device]
                lists[0].append(p)
                lists[1].append(p.grad)
                lists[2].append(state["exp_avg"])
                lists[3].append(state["exp_avg_sq"])
                lists[4].append(state["step"])
            beta1, beta2 = group["betas"]
            for dev, (ps, gs, ms, vs, ss) in by_device.items():
                with torch.cuda.device(dev):
                    adam_step_hip(ps, gs, ms, vs, ss, lr=group["lr"], beta1=beta1, beta2=beta2, eps=group["eps"],
                                  weight_decay=group["weight_decay"],
                                  decoupled_weight_decay=group["decoupled_weight_decay"])
        return loss


class FusedAdamW(FusedAdam):
    """torch.optim.AdamW's update: FusedAdam with decoupled weight decay
    (default 1e-2, as torch.optim.AdamW)."""

    def __init__(self, params, lr: float = 1e-3, betas: tuple[float, float] = (0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2, *, amsgrad: bool = False, maximize: bool = False) -> None:
        super().__init__(params, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, decoupled_weight_decay=True,
                         amsgrad=amsgrad, maximize=maximize)
