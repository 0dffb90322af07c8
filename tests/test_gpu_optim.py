"""FusedAdam (tropnn_hip_adam_step) against torch.optim.Adam / AdamW's
single-tensor path on the CPU, over several steps, with tensor counts above
one launch's group of 16, sizes that are not multiples of four, parameters
without gradients, gradients small enough that eps dominates the update, and
a training step captured in a HIP graph.

Tolerance, per tensor: |ours - torch| <= 1e-6 |torch| + 1e-6 max|torch|
(each op is rounded to f32 on both sides, from the same f64 bias
corrections; the GPU's f64 pow and the host's may differ in the last place,
and where m or v cancel to near zero one rounding step of the inputs'
magnitude shows). A wrong sign, a dropped bias correction or a dropped eps
(at the small-gradient case) moves the result by far more.
"""
from __future__ import annotations

import copy

import pytest
import torch

from tropnn_amd import FusedAdam, FusedAdamW

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

SHAPES = [(136, 64, 128), (136, 6), (7,), (1,), (3, 5), (0,), (1025,)] + [(k + 2,) for k in range(14)]


def make_params(seed: int):
    gen = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=gen) for s in SHAPES]


def grads_for(step: int, seed: int, scale: float = 1.0):
    gen = torch.Generator().manual_seed(1000 * seed + step)
    return [torch.randn(s, generator=gen) * (0.1 + k % 3) * scale for k, s in enumerate(SHAPES)]


def close(ours: torch.Tensor, ref: torch.Tensor, rtol: float = 1e-6, frac: float = 1e-6) -> None:
    ours = ours.detach().cpu()
    ref = ref.detach().cpu()
    if ref.numel() == 0:
        return
    bad = (ours - ref).abs() > rtol * ref.abs() + frac * float(ref.abs().max())
    assert not bad.any(), f"{int(bad.sum())} of {ref.numel()} differ, max {float((ours - ref).abs().max()):.3e}"


@pytest.mark.parametrize(
    "cls,ref_cls,kwargs,gscale",
    [
        (FusedAdam, torch.optim.Adam, dict(lr=1e-3), 1.0),
        (FusedAdam, torch.optim.Adam, dict(lr=3e-2, betas=(0.8, 0.99), eps=1e-6, weight_decay=0.1), 1.0),
        (FusedAdamW, torch.optim.AdamW, dict(lr=1e-2, weight_decay=0.05), 1.0),
        (FusedAdam, torch.optim.Adam, dict(lr=1e-3, betas=(0.3, 0.9)), 1.0),  # 1 - beta1 >= 0.5: lerp's other form
        (FusedAdam, torch.optim.Adam, dict(lr=1e-1, eps=1e-6), 1e-6),  # eps comparable to sqrt(v)
    ],
)
def test_matches_torch_adam(cls, ref_cls, kwargs, gscale):
    seed = 7
    ref = [torch.nn.Parameter(t.clone()) for t in make_params(seed)]
    ours = [torch.nn.Parameter(t.clone().to(DEV)) for t in make_params(seed)]
    opt_ref = ref_cls(ref, foreach=False, **kwargs)
    opt = cls(ours, **kwargs)
    skip = {3, 9}  # parameters without a gradient on even steps
    for step in range(5):
        for k, g in enumerate(grads_for(step, seed, gscale)):
            has = not (step % 2 == 0 and k in skip)
            ref[k].grad = g.clone() if has else None
            ours[k].grad = g.to(DEV) if has else None
        opt_ref.step()
        opt.step()
    torch.cuda.synchronize()
    for k in range(len(SHAPES)):
        close(ours[k], ref[k])
        st, st_ref = opt.state[ours[k]], opt_ref.state[ref[k]]
        assert float(st["step"]) == float(st_ref["step"]), k
        close(st["exp_avg"], st_ref["exp_avg"])
        close(st["exp_avg_sq"], st_ref["exp_avg_sq"])


def test_state_dict_moves_to_torch_adam():
    """The state layout is torch's: a FusedAdam state dict loads into
    torch.optim.Adam, which then continues the same trajectory."""
    seed = 3
    ours = [torch.nn.Parameter(t.clone().to(DEV)) for t in make_params(seed)[:3]]
    opt = FusedAdam(ours, lr=1e-3)
    for step in range(3):
        for p, g in zip(ours, grads_for(step, seed)):
            p.grad = g.to(DEV)
        opt.step()
    twin = [torch.nn.Parameter(p.detach().clone()) for p in ours]
    opt_t = torch.optim.Adam(twin, lr=1e-3, capturable=True)
    opt_t.load_state_dict(copy.deepcopy(opt.state_dict()))  # load_state_dict would share the state tensors
    for p, q, g in zip(ours, twin, grads_for(3, seed)):
        p.grad, q.grad = g.to(DEV), g.to(DEV)
    opt.step()
    opt_t.step()
    for p, q in zip(ours, twin):
        close(p, q, 1e-5, 1e-6)  # torch's capturable path forms the bias corrections in f32


def test_graph_replays_match_eager():
    """A captured optimizer step replays with the device step counter: every
    replay equals an eager FusedAdam step on a twin, with eager work and
    synchronisations between the replays."""
    seed = 11
    cap = [torch.nn.Parameter(t.clone().to(DEV)) for t in make_params(seed)]
    eag = [torch.nn.Parameter(t.clone().to(DEV)) for t in make_params(seed)]
    opt_c, opt_e = FusedAdam(cap, lr=1e-2, weight_decay=0.01), FusedAdam(eag, lr=1e-2, weight_decay=0.01)
    grads = [g.to(DEV) for g in grads_for(0, seed)]
    for p, g in zip(cap, grads):
        p.grad = g.clone()
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):
        opt_c.step()  # warm-up step outside the graph creates the state
    torch.cuda.current_stream(DEV).wait_stream(side)
    for p, g in zip(eag, grads):
        p.grad = g.clone()
    opt_e.step()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opt_c.step()
    torch.cuda.synchronize()
    for rep in range(4):
        new = [g.to(DEV) for g in grads_for(rep + 1, seed)]
        for p, q, g in zip(cap, eag, new):
            p.grad.copy_(g)
            q.grad = g.clone()
        graph.replay()
        opt_e.step()
        _ = torch.ones(1024, device=DEV).sum().item()  # eager work between replays
        torch.cuda.synchronize()
        for p, q in zip(cap, eag):
            assert torch.equal(p.detach(), q.detach()), rep
        for p, q in zip(cap, eag):
            assert float(opt_c.state[p]["step"]) == float(opt_e.state[q]["step"]) == rep + 2
