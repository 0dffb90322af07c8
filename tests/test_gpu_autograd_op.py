"""The autograd operator behind pairwise_hip (torch.ops.tropnn_hip.pairwise):
gradient selection, saved-tensor semantics and error mapping. The values
themselves are pinned against the oracle in test_gpu_parity.py; here every
check is against the operator's own full backward, bit for bit (the kernels
and their summation order do not depend on which gradients are asked for)."""
from __future__ import annotations

import pytest
import torch

from tropnn_amd.backends.pairwise_hip import pairwise_hip

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(batch, steps, in_f, out_f, tables, comps, seed):
    gen = torch.Generator().manual_seed(seed)
    latent = torch.randn(batch, steps, in_f, generator=gen).to(DEV).requires_grad_(True)
    anchors = torch.randint(0, in_f, (tables, comps, 2), generator=gen).to(DEV)
    thr = (0.3 * torch.randn(tables, comps, generator=gen)).to(DEV).requires_grad_(True)
    lut = torch.randn(tables, 1 << comps, out_f, generator=gen).to(DEV).requires_grad_(True)
    grad = torch.randn(batch, steps, out_f, generator=gen).to(DEV)
    return latent, anchors, thr, lut, grad


@pytest.mark.parametrize("min_margin", [True, False])
@pytest.mark.parametrize("surrogate", ["fast_sigmoid_odd", "izhikevich"])
def test_partial_gradients_equal_the_full_backward(min_margin, surrogate):
    """autograd.grad over any subset of (latent, thresholds, lut) gives the
    full backward's gradients for that subset: the backward computes only
    what the pass asks for."""
    latent, anchors, thr, lut, grad = _inputs(96, 2, 48, 40, 20, 6, seed=1)
    named = {"latent": latent, "thresholds": thr, "lut": lut}

    def grads(names):
        out, _, _ = pairwise_hip(
            latent, anchors, thr, lut, use_min_margin_ste=min_margin, surrogate=surrogate,
            output_scale=0.5, return_route=False,
        )
        return dict(zip(names, torch.autograd.grad(out, [named[n] for n in names], grad)))

    full = grads(("latent", "thresholds", "lut"))
    assert all(bool(t.abs().sum() > 0) for t in full.values())
    for names in (("lut",), ("latent",), ("thresholds",), ("latent", "thresholds"), ("thresholds", "lut")):
        for n, t in grads(names).items():
            assert torch.equal(t, full[n]), (names, n)


def test_forward_under_no_grad_and_with_grad_agree():
    latent, anchors, thr, lut, _ = _inputs(64, 1, 32, 24, 12, 5, seed=2)
    with torch.no_grad():
        out0, idx0, mar0 = pairwise_hip(latent, anchors, thr, lut, output_scale=0.25)
    out1, idx1, mar1 = pairwise_hip(latent, anchors, thr, lut, output_scale=0.25)
    assert out0.grad_fn is None and out1.grad_fn is not None
    assert not idx1.requires_grad and not mar1.requires_grad
    assert torch.equal(out0, out1) and torch.equal(idx0, idx1) and torch.equal(mar0, mar1)
    # a call that records nothing because no input needs a gradient (the
    # operator then launches without its autograd function), in every route
    # mode, against the recorded call
    frozen = (latent.detach(), anchors, thr.detach(), lut.detach())
    for mode in (True, "codes", False):
        out2, idx2, mar2 = pairwise_hip(*frozen, output_scale=0.25, return_route=mode)
        out3, idx3, mar3 = pairwise_hip(latent, anchors, thr, lut, output_scale=0.25, return_route=mode)
        assert out2.grad_fn is None and not out2.requires_grad and out3.grad_fn is not None
        assert torch.equal(out2, out3) and torch.equal(idx2, idx3) and torch.equal(mar2, mar3)
        assert idx2.dtype == idx3.dtype and idx2.shape == idx3.shape and mar2.shape == mar3.shape


def test_only_lut_gradient_when_latent_and_thresholds_are_frozen():
    latent, anchors, thr, lut, grad = _inputs(64, 1, 32, 24, 12, 5, seed=3)
    out, _, _ = pairwise_hip(latent, anchors, thr, lut, return_route=False)
    (full_lut,) = torch.autograd.grad(out, [lut], grad)
    out, _, _ = pairwise_hip(latent.detach(), anchors, thr.detach(), lut, return_route=False)
    out.backward(grad)
    assert torch.equal(lut.grad, full_lut)


def test_retain_graph_and_freed_saved_tensors():
    latent, anchors, thr, lut, grad = _inputs(64, 1, 32, 24, 12, 5, seed=4)
    out, _, _ = pairwise_hip(latent, anchors, thr, lut, return_route=False)
    first = torch.autograd.grad(out, [latent, thr, lut], grad, retain_graph=True)
    second = torch.autograd.grad(out, [latent, thr, lut], grad)
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    with pytest.raises(RuntimeError, match="second time|freed"):
        torch.autograd.grad(out, [lut], grad)


def test_in_place_change_of_a_saved_lut_is_detected():
    """The LUT the kernels read is saved for the backward with its version."""
    latent, anchors, thr, lut, grad = _inputs(32, 1, 16, 8, 6, 4, seed=5)
    out, _, _ = pairwise_hip(latent, anchors, thr, lut, return_route=False)
    with torch.no_grad():
        lut.add_(1.0)
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        out.backward(grad)


def test_library_errors_keep_their_python_exception_types():
    """Status codes of the C ABI raise as the ctypes bindings raise them:
    unsupported -> NotImplementedError, invalid argument -> ValueError."""
    latent = torch.randn(2, 1, 40, device=DEV)
    anchors = torch.zeros(3, 2, 2, dtype=torch.int64, device=DEV)
    thr = torch.zeros(3, 2, device=DEV)
    with pytest.raises(NotImplementedError, match="comparisons <= 8"):  # the operator's own check
        pairwise_hip(latent, torch.zeros(3, 9, 2, dtype=torch.int64, device=DEV), torch.zeros(3, 9, device=DEV),
                     torch.zeros(3, 512, 5, device=DEV))
    # the library's TROPNN_ERR_UNSUPPORTED: two million one-comparison tables
    # give the forward's waves code lists past a workgroup's LDS
    many = 2_000_000
    with pytest.raises(NotImplementedError, match="tables too many"):
        pairwise_hip(latent[:1], torch.zeros(many, 1, 2, dtype=torch.int64, device=DEV),
                     torch.zeros(many, 1, device=DEV), torch.zeros(many, 2, 1, device=DEV))
    with pytest.raises(ValueError, match="out_features"):
        pairwise_hip(latent[:, :, :16].contiguous(), anchors, thr, torch.zeros(3, 4, 0, device=DEV))
    with pytest.raises(TypeError, match="float32"):
        pairwise_hip(latent.double(), anchors, thr, torch.zeros(3, 4, 5, device=DEV))
    with pytest.raises(ValueError, match="thresholds must have shape"):
        pairwise_hip(latent, anchors, torch.zeros(3, 3, device=DEV), torch.zeros(3, 4, 5, device=DEV))
