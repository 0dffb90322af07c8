"""tropnn_amd.cross_entropy (tropnn_hip_cross_entropy) against F.cross_entropy
in f64 on the CPU: loss and logits gradient, with ignored rows, every row
ignored, large logits, one class, many classes (several LDS tiles, rows wider
than a tile), a non-unit incoming gradient and graph replays.

Tolerance: loss |Δ| <= 2e-6 |ref| + 1e-6, gradient |Δ| <= 1e-5 |ref| + 1e-8
(f32 exp / log per element and a fixed-order f32 sum over rows)."""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from tropnn_amd import cross_entropy

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def reference(logits: torch.Tensor, target: torch.Tensor, scale: float = 1.0):
    x = logits.detach().double().requires_grad_(True)
    loss = F.cross_entropy(x, target)
    (loss * scale).backward()
    return loss.detach(), x.grad


@pytest.mark.parametrize(
    "rows,classes,shift,ignored",
    [
        (512, 10, 0.0, 0),
        (3, 1, 0.0, 0),
        (2000, 37, 0.0, 300),  # LDS tiles of 332 rows
        (7, 1000, 0.0, 2),  # tiles of 12 rows
        (64, 10, 1e4, 5),
        (1030, 5, -50.0, 0),  # tiles of 1024 rows
        (3, 13000, 0.0, 0),  # rows wider than a tile: read from global memory
    ],
)
def test_matches_torch(rows, classes, shift, ignored):
    gen = torch.Generator().manual_seed(rows + classes)
    logits = torch.randn(rows, classes, generator=gen) * 3 + shift
    target = torch.randint(0, classes, (rows,), generator=gen)
    if ignored:
        target[torch.randperm(rows, generator=gen)[:ignored]] = -100
    want_loss, want_grad = reference(logits, target, scale=2.5)
    x = logits.to(DEV).requires_grad_(True)
    loss = cross_entropy(x, target.to(DEV))
    (loss * 2.5).backward()
    got_loss, got_grad = loss.detach().cpu().double(), x.grad.cpu().double()
    assert abs(float(got_loss - want_loss)) <= 2e-6 * abs(float(want_loss)) + 1e-6, (float(got_loss), float(want_loss))
    bad = (got_grad - want_grad).abs() > 1e-5 * want_grad.abs() + 1e-8
    assert not bad.any(), float((got_grad - want_grad).abs().max())
    if ignored:
        assert torch.all(got_grad[target == -100] == 0)


def test_every_row_ignored_is_nan():
    x = torch.randn(6, 4, device=DEV, requires_grad=True)
    loss = cross_entropy(x, torch.full((6,), -100, dtype=torch.int64, device=DEV))
    assert math.isnan(float(loss.detach())) and math.isnan(float(F.cross_entropy(x.detach().cpu(), torch.full((6,), -100))))
    loss.backward()
    assert torch.all(x.grad == 0)


def test_graph_replays_match_eager():
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(512, 10, generator=gen).to(DEV)
    y = torch.randint(0, 10, (512,), generator=gen).to(DEV)
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):
        cross_entropy(x, y)
    torch.cuda.current_stream(DEV).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = cross_entropy(x, y)
    for rep in range(3):
        x.copy_(torch.randn(512, 10, generator=gen).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        want = cross_entropy(x, y)
        _ = torch.ones(64, device=DEV).sum().item()
        assert torch.equal(out, want), rep


def test_empty_batch_gives_nan_loss():
    """No rows: the mean over nothing is NaN, as F.cross_entropy returns, and
    the gradient is empty; no kernel is launched."""
    logits = torch.empty(0, 10, device=DEV, requires_grad=True)
    target = torch.empty(0, dtype=torch.int64, device=DEV)
    loss = cross_entropy(logits, target)
    ref = F.cross_entropy(logits.detach().cpu().double(), target.cpu())
    assert math.isnan(loss.detach().item()) and math.isnan(float(ref))
    loss.backward()
    assert logits.grad is not None and logits.grad.shape == (0, 10)


def test_unit_gradient_backward_matches_plain_backward():
    """loss.backward(unit_gradient(loss)) returns the kernel's logits gradient
    unscaled (no multiplication launch) and equals loss.backward(); a scaled
    incoming gradient still scales it."""
    from tropnn_amd import unit_gradient

    gen = torch.Generator().manual_seed(3)
    logits = torch.randn(512, 10, generator=gen)
    target = torch.randint(0, 10, (512,), generator=gen)
    want_loss, want_grad = reference(logits, target)
    grads = []
    for how in ("plain", "unit", "unit again", "scaled"):
        x = logits.to(DEV).requires_grad_(True)
        loss = cross_entropy(x, target.to(DEV))
        if how == "plain":
            loss.backward()
        elif how == "scaled":
            loss.backward(torch.tensor(3.0, device=DEV))
        else:
            loss.backward(unit_gradient(loss))
        grads.append(x.grad.detach().cpu())
    assert torch.equal(grads[0], grads[1]) and torch.equal(grads[1], grads[2])
    bad = (grads[1].double() - want_grad).abs() > 1e-5 * want_grad.abs() + 1e-8
    assert not bad.any()
    assert torch.allclose(grads[3], 3.0 * grads[0], rtol=1e-6, atol=0)
