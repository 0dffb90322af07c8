"""c5: the pairwise EMNIST classifier
784 -> 128 -> 128 -> 10 (three PairwiseLinear layers, T = 136, C = 6, seeds
0, 1, 2), batch 512 of sparse inputs, cross entropy, Adam lr 1e-3
(examples/emnist.py:121-175, 194-214, 310), against the oracle stack on the
CPU; the HIP side runs tropnn_amd.cross_entropy and FusedAdam, the oracle
F.cross_entropy and torch.optim.Adam. Sparse inputs give exact-zero margins (argmin ties, u = 0) in layer 1,
and layer 3 has O = 10."""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import pairwise_torch as orc
from tropnn_amd import FusedAdam, cross_entropy
from tropnn_amd.examples import EmnistPairwiseClassifier, make_c5_batch, train_step

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 1e-5


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    yield
    torch.cuda.synchronize()


class OracleClassifier(nn.Module):
    """The oracle's layers in the classifier's order and seeds."""

    def __init__(self, dims, tables, comparisons, seed=0):
        super().__init__()
        self.layers = nn.ModuleList(
            [
                orc.OraclePairwiseLinear(d_in, d_out, tables=tables, comparisons=comparisons, seed=seed + idx)
                for idx, (d_in, d_out) in enumerate(zip(dims[:-1], dims[1:]))
            ]
        )

    def forward(self, x):
        x = x.unsqueeze(1)
        for layer in self.layers:
            x = layer(x)
        return x.squeeze(1)


def rel(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    scale = float(b.abs().max())
    return float((a - b).abs().max()) / scale if scale > 0 else float((a - b).abs().max())


def check_step(ref, hip, loss_ref, loss_hip):
    lr_f, lh_f = float(loss_ref.detach()), float(loss_hip.detach())
    assert abs(lr_f - lh_f) <= TOL * abs(lr_f)
    for k, (lr_, lh) in enumerate(zip(ref.layers, hip.layers)):
        assert torch.equal(lh._last_indices.cpu(), lr_._last_indices), f"layer {k}: route codes differ"
        for name in ("thresholds", "lut"):
            gr, gh = getattr(lr_, name).grad, getattr(lh, name).grad
            assert rel(gh, gr) <= TOL, (k, name, rel(gh, gr))


def test_c5_training_steps_match_oracle():
    dims = [784, 128, 128, 10]
    ref = OracleClassifier(dims, tables=136, comparisons=6)
    hip = EmnistPairwiseClassifier(input_dim=784, hidden_dim=128, num_classes=10, depth=3).to(DEV)
    for lr_, lh in zip(ref.layers, hip.layers):  # same seeded init, layer by layer
        assert torch.equal(lh.anchors.cpu(), lr_.anchors)
        assert torch.equal(lh.lut.detach().cpu(), lr_.lut.detach())
    x, y = make_c5_batch(512, seed=0)
    assert float((x == 0).float().mean()) > 0.75

    # step 1 from the same init: loss, every layer's codes and gradients, then
    # the Adam update (its first step is ~lr * sign(g), so entries whose
    # gradient is at rounding level are left out of the comparison)
    opt_ref = torch.optim.Adam(ref.parameters(), lr=1e-3)
    opt_hip = FusedAdam(hip.parameters(), lr=1e-3)  # the library's Adam kernel, as in the c5 benchmark
    before = [p.detach().clone() for p in ref.parameters()]
    loss_ref = train_step(ref, opt_ref, x, y)
    loss_hip = train_step(hip, opt_hip, x.to(DEV), y.to(DEV), loss_fn=cross_entropy)  # as the c5 benchmark
    check_step(ref, hip, loss_ref, loss_hip)
    for p0, pr, ph in zip(before, ref.parameters(), hip.parameters()):
        g = pr.grad.abs()
        clear = g > 1e-3 * float(g.max())
        assert torch.allclose(ph.detach().cpu()[clear], pr.detach()[clear], atol=1e-7, rtol=0)
        assert not torch.equal(pr.detach(), p0)  # the step moved the parameters

    # step 2 from the HIP model's parameters (copied into the oracle), fresh
    # plain gradients: the second forward and backward of the stack
    with torch.no_grad():
        for pr, ph in zip(ref.parameters(), hip.parameters()):
            pr.copy_(ph.detach().cpu())
    for m in (ref, hip):
        m.zero_grad(set_to_none=True)
    loss_ref = F.cross_entropy(ref(x), y)
    loss_hip = F.cross_entropy(hip(x.to(DEV)), y.to(DEV))
    loss_ref.backward()
    loss_hip.backward()
    check_step(ref, hip, loss_ref, loss_hip)


def test_c5_ten_training_steps_track_the_oracle():
    """Ten steps of the c5 training loop, each on a fresh batch
    (make_c5_batch seed 1000 + step), HIP (tropnn_amd.cross_entropy from the
    kept unit gradient, FusedAdam) beside the oracle stack (F.cross_entropy,
    torch.optim.Adam), each from its own updated parameters: every layer's
    route codes agree bit for bit at every step and the losses within 1e-5
    relative, so the trajectories stay together through ten Adam updates
    (the benchmark's 100-step curve reports where they part, at a margin
    within rounding of zero)."""
    dims = [784, 128, 128, 10]
    ref = OracleClassifier(dims, tables=136, comparisons=6).train()
    hip = EmnistPairwiseClassifier(input_dim=784, hidden_dim=128, num_classes=10, depth=3).to(DEV).train()
    opt_ref = torch.optim.Adam(ref.parameters(), lr=1e-3, foreach=False)
    opt_hip = FusedAdam(hip.parameters(), lr=1e-3)
    losses = []
    for step in range(10):
        x, y = make_c5_batch(512, seed=1000 + step)
        loss_ref = train_step(ref, opt_ref, x, y)
        loss_hip = train_step(hip, opt_hip, x.to(DEV), y.to(DEV), loss_fn=cross_entropy)
        lr_f, lh_f = float(loss_ref.detach()), float(loss_hip.detach())
        losses.append((lh_f, lr_f))
        for k, (lr_, lh) in enumerate(zip(ref.layers, hip.layers)):
            assert torch.equal(lh._last_indices.cpu(), lr_._last_indices), f"step {step}, layer {k}: codes differ"
        assert abs(lr_f - lh_f) <= TOL * abs(lr_f), (step, lh_f, lr_f)
    print("c5 losses (hip, oracle):", losses)
