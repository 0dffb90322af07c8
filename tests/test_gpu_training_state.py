"""Training state that lives outside the kernels, on the GPU:

  * the f16 LUT read copy (device_lut_dtype="f16") stays in step with the f32
    LUT that FusedAdam updates through raw pointers, in eager steps and in
    replays of a captured training step (forward + backward + FusedAdam),
    against the f32-LUT oracle trained by torch.optim.Adam on the CPU;
  * the lazy route-debug guard raises once FusedAdam has moved the
    thresholds;
  * optimizer state dicts move from torch.optim.Adam, and from a checkpoint
    mapped to the CPU, into FusedAdam;
  * f16 / bf16 inputs through the module shell (layers/base.py:34-35, 84 of
    the reference): computed in f32, output and input gradient cast back.

Bars: outputs and gradients with f16 LUT reads within 1e-3 relative
(max|hip - oracle| / max|oracle|) of the f32-LUT oracle; route codes
bit-exact. A stale f16 copy after one step of lr 5e-2 misses the output by
0.72 relative (the oracle's output with the pre-step LUT against the
post-step one, on these inputs).
"""
from __future__ import annotations

import copy
import io

import pytest
import torch

from oracle import pairwise_torch as orc
from tropnn_amd import FusedAdam, PairwiseLinear

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
F16_TOL = 1e-3
LR = 5e-2
SHAPE = dict(i=48, o=40, t=12, c=5)
BATCH = 64


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    yield
    torch.cuda.synchronize()


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    assert a.shape == b.shape, (a.shape, b.shape)
    scale = float(b.abs().max())
    diff = float((a - b).abs().max())
    return diff / scale if scale > 0 else diff


def make_pair(lut_dtype: str = "f16", seed: int = 4):
    i, o, t, c = SHAPE["i"], SHAPE["o"], SHAPE["t"], SHAPE["c"]
    ref = orc.OraclePairwiseLinear(i, o, tables=t, comparisons=c, seed=seed).train()
    hip = PairwiseLinear(i, o, tables=t, comparisons=c, seed=seed, device_lut_dtype=lut_dtype)
    with torch.no_grad():
        hip.anchors.copy_(ref.anchors)
        hip.thresholds.copy_(ref.thresholds)
        hip.lut.copy_(ref.lut)
    # frozen thresholds keep the route independent of the optimizer's
    # rounding (codes compared bit-exactly); the STE gradient goes to x
    ref.thresholds.requires_grad_(False)
    hip.thresholds.requires_grad_(False)
    return ref, hip.to(DEV).train()


def batches(n: int):
    gen = torch.Generator().manual_seed(99)
    return [
        (torch.randn(BATCH, SHAPE["i"], generator=gen), torch.randn(BATCH, 1, SHAPE["o"], generator=gen))
        for _ in range(n)
    ]


def ref_step(ref, opt_ref, x, g):
    opt_ref.zero_grad(set_to_none=True)
    xr = x.clone().requires_grad_(True)
    y = ref(xr)
    y.backward(g)
    grads = (xr.grad.clone(), ref.lut.grad.clone())
    opt_ref.step()
    return y.detach(), grads


def check(tag, y, gx, glut, y_ref, grads_ref, hip, ref):
    errs = {
        "output": rel_err(y, y_ref),
        "grad_x": rel_err(gx, grads_ref[0]),
        "grad_lut": rel_err(glut, grads_ref[1]),
        "lut_after_step": rel_err(hip.lut, ref.lut),
    }
    bad = {k: v for k, v in errs.items() if not v <= F16_TOL}
    assert not bad, f"{tag}: beyond {F16_TOL}: {bad} (all {errs})"


def test_f16_lut_fused_adam_eager_steps():
    ref, hip = make_pair()
    opt_ref = torch.optim.Adam(ref.parameters(), lr=LR, foreach=False)
    opt = FusedAdam(hip.parameters(), lr=LR)
    for k, (x, g) in enumerate(batches(3)):
        y_ref, grads_ref = ref_step(ref, opt_ref, x, g)
        opt.zero_grad(set_to_none=True)
        xh = x.to(DEV).requires_grad_(True)
        y = hip(xh)
        assert torch.equal(hip._last_indices.cpu(), ref._last_indices), f"step {k}: route codes differ"
        y.backward(g.to(DEV))
        gx, glut = xh.grad.clone(), hip.lut.grad.clone()
        v0 = hip.lut._version
        opt.step()
        assert hip.lut._version > v0, "FusedAdam did not bump the LUT's version counter"
        torch.cuda.synchronize()
        check(f"eager step {k}", y, gx, glut, y_ref, grads_ref, hip, ref)
    # an eval forward after training reads the refreshed copy too
    x = batches(4)[3][0]
    with torch.no_grad():
        y_ref = ref.eval()(x)
        y = hip.eval()(x.to(DEV))
    assert rel_err(y, y_ref) <= F16_TOL


def test_f16_lut_fused_adam_graph_replays():
    """One training step (forward, backward, FusedAdam) captured in a HIP
    graph; each replay must read the f16 copy of the LUT as the previous
    replay's optimizer step left it. Step 0 runs eagerly on a side stream
    (it creates the optimizer state), then three replays with eager work and
    synchronisations between them."""
    ref, hip = make_pair()
    hip.cache_route_debug = False
    opt_ref = torch.optim.Adam(ref.parameters(), lr=LR, foreach=False)
    opt = FusedAdam(hip.parameters(), lr=LR)
    data = batches(4)
    static_x = torch.empty(BATCH, SHAPE["i"], device=DEV).requires_grad_(True)
    static_g = torch.empty(BATCH, 1, SHAPE["o"], device=DEV)

    def hip_step():
        y = hip(static_x)
        y.backward(static_g)
        opt.step()
        return y.detach()  # keeps no autograd node of the step alive

    with torch.no_grad():
        static_x.copy_(data[0][0])
        static_g.copy_(data[0][1])
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):
        opt.zero_grad(set_to_none=True)
        y0 = hip_step()
        gx0, glut0 = static_x.grad.clone(), hip.lut.grad.clone()
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()
    y_ref, grads_ref = ref_step(ref, opt_ref, *data[0])
    check("eager step 0", y0, gx0, glut0, y_ref, grads_ref, hip, ref)

    opt.zero_grad(set_to_none=True)
    static_x.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_y = hip_step()
    torch.cuda.synchronize()
    for k in (1, 2, 3):
        x, g = data[k]
        with torch.no_grad():
            static_x.copy_(x)
            static_g.copy_(g)
        graph.replay()
        _ = torch.ones(1024, device=DEV).sum().item()  # eager work between replays
        torch.cuda.synchronize()
        y_ref, grads_ref = ref_step(ref, opt_ref, x, g)
        check(f"replay {k}", static_y, static_x.grad, hip.lut.grad, y_ref, grads_ref, hip, ref)
    # an eager forward after the replays must not reuse the graph's copy
    x = batches(5)[4][0]
    with torch.no_grad():
        y_ref = ref.eval()(x)
        y = hip.eval()(x.to(DEV))
    assert rel_err(y, y_ref) <= F16_TOL


def test_lazy_margins_raise_after_fused_adam_step():
    i, o, t, c = SHAPE["i"], SHAPE["o"], SHAPE["t"], SHAPE["c"]
    hip = PairwiseLinear(i, o, tables=t, comparisons=c, seed=1).to(DEV).train()
    hip.cache_route_debug = "lazy"
    opt = FusedAdam(hip.parameters(), lr=1e-2)
    x = torch.randn(BATCH, i, device=DEV)
    hip(x).square().mean().backward()
    before = hip._route_debug  # the call's lazy record, margins not yet read
    opt.step()
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="modified in place"):
        _ = before.margins
    # the next call's margins are available again
    hip(x)
    assert hip._last_margins.shape == (BATCH, 1, t, c)


def _train_params(seed: int):
    gen = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=gen) for s in ((12, 32, 40), (12, 5), (7,))]


def _grads(step: int, n: int):
    gen = torch.Generator().manual_seed(500 + step)
    return [torch.randn(s, generator=gen) for s in ((12, 32, 40), (12, 5), (7,))][:n]


def test_torch_adam_state_dict_loads_into_fused_adam():
    """torch.optim.Adam (not capturable) keeps "step" on the CPU; FusedAdam
    moves it to the parameter's device when loading, then continues the
    same trajectory as torch's Adam."""
    ref = [torch.nn.Parameter(t.clone()) for t in _train_params(2)]
    opt_ref = torch.optim.Adam(ref, lr=1e-2, foreach=False)
    for step in range(3):
        for p, g in zip(ref, _grads(step, 3)):
            p.grad = g.clone()
        opt_ref.step()
    ours = [torch.nn.Parameter(p.detach().clone().to(DEV)) for p in ref]
    opt = FusedAdam(ours, lr=1e-2)
    opt.load_state_dict(copy.deepcopy(opt_ref.state_dict()))
    for p in ours:
        st = opt.state[p]
        assert st["step"].device == p.device and st["step"].dtype == torch.float32
        assert st["exp_avg"].device == p.device
    for p, q, g in zip(ref, ours, _grads(3, 3)):
        p.grad, q.grad = g.clone(), g.to(DEV)
    opt_ref.step()
    opt.step()
    torch.cuda.synchronize()
    for p, q in zip(ref, ours):
        assert rel_err(q, p) <= 1e-6
        assert float(opt.state[q]["step"]) == 4.0


def test_fused_adam_checkpoint_mapped_to_cpu_round_trip():
    """A FusedAdam checkpoint saved and loaded with map_location="cpu" (as a
    host-side checkpoint loader does) resumes on the GPU exactly where an
    uninterrupted run goes."""
    base = _train_params(5)
    run = [torch.nn.Parameter(t.clone().to(DEV)) for t in base]
    opt = FusedAdam(run, lr=3e-3, weight_decay=0.01)
    for step in range(2):
        for p, g in zip(run, _grads(step, 3)):
            p.grad = g.to(DEV)
        opt.step()
    buf = io.BytesIO()
    torch.save({"params": [p.detach() for p in run], "opt": opt.state_dict()}, buf)
    buf.seek(0)
    ckpt = torch.load(buf, map_location="cpu", weights_only=True)
    resumed = [torch.nn.Parameter(t.to(DEV)) for t in ckpt["params"]]
    opt2 = FusedAdam(resumed, lr=3e-3, weight_decay=0.01)
    opt2.load_state_dict(ckpt["opt"])
    for step in (2, 3):
        for p, q, g in zip(run, resumed, _grads(step, 3)):
            p.grad, q.grad = g.to(DEV), g.to(DEV)
        opt.step()
        opt2.step()
    torch.cuda.synchronize()
    for p, q in zip(run, resumed):
        assert torch.equal(p.detach(), q.detach())
        assert float(opt2.state[q]["step"]) == 4.0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_half_inputs_through_the_module(dtype):
    """f16 / bf16 inputs are computed in f32 and the output and the input
    gradient come back in the input's dtype, as the reference shell does
    (layers/base.py:34-35, 84). Both sides round the same f32 values (within
    1e-5 relative of each other) to the half type, so they agree to one unit
    in the last place of that type."""
    i, o, t, c = SHAPE["i"], SHAPE["o"], SHAPE["t"], SHAPE["c"]
    ref = orc.OraclePairwiseLinear(i, o, tables=t, comparisons=c, seed=8).train()
    hip = PairwiseLinear(i, o, tables=t, comparisons=c, seed=8)
    gen = torch.Generator().manual_seed(3)
    with torch.no_grad():
        ref.thresholds.copy_(0.2 * torch.randn(ref.thresholds.shape, generator=gen))
        hip.anchors.copy_(ref.anchors)
        hip.thresholds.copy_(ref.thresholds)
        hip.lut.copy_(ref.lut)
    hip = hip.to(DEV).train()
    x = torch.randn(BATCH, i, generator=gen).to(dtype)
    g = torch.randn(BATCH, 1, o, generator=gen).to(dtype)
    xr = x.clone().requires_grad_(True)
    xh = x.to(DEV).requires_grad_(True)
    y_ref = ref(xr)
    y = hip(xh)
    y_ref.backward(g)
    y.backward(g.to(DEV))
    torch.cuda.synchronize()
    assert y.dtype == dtype and xh.grad.dtype == dtype
    assert torch.equal(hip._last_indices.cpu(), ref._last_indices)
    ulp = torch.finfo(dtype).eps
    for name, a, b in (("output", y, y_ref), ("grad_x", xh.grad, xr.grad)):
        a32, b32 = a.detach().float().cpu(), b.detach().float().cpu()
        bound = ulp * b32.abs() + 1e-5 * float(b32.abs().max())
        assert bool(((a32 - b32).abs() <= bound).all()), f"{name}: max diff {float((a32 - b32).abs().max()):.3e}"
    assert rel_err(hip.lut.grad, ref.lut.grad) <= 1e-5
    assert rel_err(hip.thresholds.grad, ref.thresholds.grad) <= 1e-5
