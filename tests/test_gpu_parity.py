"""GPU parity: the HIP path (through libtropnn_hip.so's C ABI) against the CPU
oracle on the same seeded inputs and parameters.

Bars:
  * route codes and margins: bit-exact (torch.equal on int64 codes and on the
    f32 margin bit patterns);
  * f32 LUT: forward output and every gradient within 1e-5 relative error,
    measured norm-wise as max|hip - oracle| / max|oracle|, and (training,
    f32 eval forward, views, c4's sampled rows) also element by element
    within 2e-4 of |oracle| + 1e-3 max|oracle|;
  * f16 LUT reads: within 1e-3 relative of the f32-LUT oracle.
The reference's own parity tests (test_backend_parity.py:348-369) use
allclose(atol=1e-6); test_reference_case repeats that case and bar.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pairwise_torch as orc
from oracle import routing_np
from tropnn_amd import PairwiseLinear, pairwise_hip_forward

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
F32_TOL = 1e-5
F16_TOL = 1e-3


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    yield
    torch.cuda.synchronize()


ELEM_RTOL = 2e-4
ELEM_FLOOR = 1e-3


def elem_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max over elements of |a - b| / (|b| + ELEM_FLOOR max|b|), in float64."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    if b.numel() == 0:
        return 0.0
    scale = b.abs().max()
    if scale == 0:
        return (a - b).abs().max().item()
    return ((a - b).abs() / (b.abs() + ELEM_FLOOR * scale)).max().item()


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    assert a.shape == b.shape, (a.shape, b.shape)
    if b.numel() == 0:
        return 0.0
    scale = float(b.abs().max())
    diff = float((a - b).abs().max())
    return diff / scale if scale > 0 else diff


def make_pair(i, o, t, c, *, seed=0, thr_std=0.0, lut_dtype="f32", gen_seed=1234, **ste):
    ref = orc.OraclePairwiseLinear(i, o, tables=t, comparisons=c, seed=seed, **ste)
    hip = PairwiseLinear(i, o, tables=t, comparisons=c, seed=seed, device_lut_dtype=lut_dtype, **ste)
    with torch.no_grad():
        if thr_std:
            g = torch.Generator().manual_seed(gen_seed)
            ref.thresholds.copy_(thr_std * torch.randn(ref.thresholds.shape, generator=g))
        hip.anchors.copy_(ref.anchors)
        hip.thresholds.copy_(ref.thresholds)
        hip.lut.copy_(ref.lut)
    return ref, hip.to(DEV)


def seeded(shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


def train_step(ref, hip, x, g, *, x_grad=True):
    ref.train()
    hip.train()
    x_ref = x.clone().requires_grad_(x_grad)
    x_hip = x.to(DEV).requires_grad_(x_grad)
    y_ref = ref(x_ref)
    y_hip = hip(x_hip)
    y_ref.backward(g)
    y_hip.backward(g.to(DEV))
    torch.cuda.synchronize()
    return (y_ref, x_ref), (y_hip, x_hip)


def assert_train_parity(ref, hip, yx_ref, yx_hip, tol=F32_TOL, x_grad=True, elem_rtol=ELEM_RTOL):
    (y_ref, x_ref), (y_hip, x_hip) = yx_ref, yx_hip
    assert torch.equal(hip._last_indices.cpu(), ref._last_indices), "route codes differ"
    errs = {
        "output": rel_err(y_hip, y_ref),
        "grad_thresholds": rel_err(hip.thresholds.grad, ref.thresholds.grad),
        "grad_lut": rel_err(hip.lut.grad, ref.lut.grad),
    }
    if x_grad:
        errs["grad_x"] = rel_err(x_hip.grad, x_ref.grad)
    else:
        assert x_hip.grad is None and x_ref.grad is None
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, f"beyond {tol}: {bad} (all: {errs})"
    if tol == F32_TOL:
        # and element by element: |hip - ref| <= ELEM_RTOL (|ref| + ELEM_FLOOR
        # max|ref|). Far stricter than the norm-wise bar on small elements;
        # the floor covers sums that cancel, where any change of summation
        # order in f32 moves the result (seen: 9.4e-5 at most)
        pairs = {"output": (y_hip, y_ref), "grad_thresholds": (hip.thresholds.grad, ref.thresholds.grad),
                 "grad_lut": (hip.lut.grad, ref.lut.grad)}
        if x_grad:
            pairs["grad_x"] = (x_hip.grad, x_ref.grad)
        elem = {k: elem_err(h, r) for k, (h, r) in pairs.items()}
        bad = {k: v for k, v in elem.items() if not v <= elem_rtol}
        assert not bad, f"element-wise beyond {elem_rtol}: {bad} (all: {elem})"
    return errs


# ---------------------------------------------------------------- route codes
@pytest.mark.parametrize(
    "i,t,c,b",
    [(8, 3, 3, 4), (16, 1, 1, 7), (33, 5, 2, 9), (128, 136, 6, 512), (64, 17, 8, 40), (300, 70, 7, 33), (1024, 64, 5, 3)],
)
def test_codes_and_margins_bit_exact(i, t, c, b):
    ref, hip = make_pair(i, 4, t, c, seed=t + c, thr_std=0.5)
    x = seeded((b, i), seed=i + b)
    with torch.no_grad():
        hip.eval()(x.to(DEV))
    torch.cuda.synchronize()
    codes = routing_np.route_codes(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    margins = routing_np.margins_f32(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    got_codes = hip._last_indices.cpu().reshape(b, t).numpy()
    got_margins = hip._last_margins.cpu().reshape(b, t, c).numpy()
    np.testing.assert_array_equal(got_codes, codes)
    np.testing.assert_array_equal(got_margins.view(np.uint32), margins.view(np.uint32))


def test_codes_edge_values():
    """Subnormal, signed-zero, NaN and infinite margins: bit c is set iff the
    f32 margin is > 0, with no denormal flushing."""
    tiny = np.float32(1.4e-45)  # smallest positive subnormal
    x = np.array(
        [
            [tiny, 0.0, -tiny, np.nan, np.inf, -np.inf, 1.0, 1.0],
            [0.0, tiny, 0.0, -0.0, 2.0, np.nan, np.inf, np.inf],
        ],
        dtype=np.float32,
    )
    anchors = torch.tensor(
        [[[0, 1], [1, 0], [2, 1], [3, 0]], [[4, 5], [5, 4], [6, 7], [7, 6]], [[4, 6], [6, 4], [3, 3], [0, 2]]],
        dtype=torch.long,
    )
    thr = torch.zeros(3, 4)
    ref, hip = make_pair(8, 3, 3, 4, seed=0)
    with torch.no_grad():
        hip.anchors.copy_(anchors.to(DEV))
        hip.thresholds.copy_(thr.to(DEV))
        hip.eval()(torch.from_numpy(x).to(DEV))
    torch.cuda.synchronize()
    expect = routing_np.route_codes(x, anchors.numpy(), thr.numpy())
    np.testing.assert_array_equal(hip._last_indices.cpu().reshape(2, 3).numpy(), expect)
    # the subnormal margin sets bit 0 of table 0 for item 0
    assert expect[0, 0] & 1 == 1


# ---------------------------------------------------------------- eval forward
@pytest.mark.parametrize(
    "i,o,t,c,b",
    [(256, 512, 16, 6, 8), (128, 128, 136, 6, 512), (128, 128, 136, 6, 1), (8, 5, 3, 3, 4), (784, 128, 136, 6, 64), (128, 10, 136, 6, 33), (32, 3, 9, 8, 17)],
)
def test_eval_forward_f32(i, o, t, c, b):
    ref, hip = make_pair(i, o, t, c, seed=0, thr_std=0.1)
    x = seeded((b, i), seed=0)
    with torch.no_grad():
        y_ref = ref.eval()(x)
        y_hip = hip.eval()(x.to(DEV))
    assert torch.equal(hip._last_indices.cpu(), ref._last_indices)
    assert rel_err(y_hip, y_ref) <= F32_TOL
    assert elem_err(y_hip, y_ref) <= ELEM_RTOL


@pytest.mark.parametrize(
    "i,o,t,c,b",
    # f16 row loads of 1, 2, 4 and 8 halves per lane, and several output tiles
    [(64, 9, 20, 5, 33), (64, 128, 20, 5, 33), (64, 256, 37, 4, 17), (64, 1000, 12, 8, 5), (96, 2048, 40, 7, 3)],
)
def test_eval_forward_f16_shapes(i, o, t, c, b):
    ref, hip = make_pair(i, o, t, c, seed=1, thr_std=0.1, lut_dtype="f16")
    x = seeded((b, i), seed=2)
    with torch.no_grad():
        y_ref = ref.eval()(x)
        y_hip = hip.eval()(x.to(DEV))
    assert torch.equal(hip._last_indices.cpu(), ref._last_indices)
    assert rel_err(y_hip, y_ref) <= F16_TOL


@pytest.mark.parametrize("b", [1, 64, 8192])
def test_eval_forward_f16_lut(b):
    """c3: same layer, LUT read as an RNE f16 copy, against the f32 oracle."""
    ref, hip = make_pair(128, 128, 136, 6, seed=0, lut_dtype="f16")
    x = seeded((b, 128), seed=0)
    with torch.no_grad():
        y_ref = ref.eval()(x)
        y_hip = hip.eval()(x.to(DEV))
        y_fn = pairwise_hip_forward(
            x.to(DEV).unsqueeze(1), hip.anchors, hip.thresholds, hip.lut, lut_dtype="f16", output_scale=hip.output_scale
        )
    assert rel_err(y_hip, y_ref) <= F16_TOL
    assert rel_err(y_fn, y_ref) <= F16_TOL


def test_pairwise_hip_forward_matches_zig_restatement():
    """The Zig-ABI-shaped entry points against the C restatement of the Zig
    forward (f32: atol 1e-6, f16: 5e-3 as test_backend_parity.py:232, 246)."""
    from oracle import lut_cpu

    lut_cpu.build()
    ref, hip = make_pair(8, 5, 4, 3, seed=2, thr_std=0.2)
    x = seeded((7, 1, 8), seed=5)
    for dt, atol in (("f32", 1e-6), ("f16", 5e-3)):
        want = lut_cpu.forward(x, ref.anchors, ref.thresholds.detach(), ref.lut.detach(), lut_dtype=dt, threads=1)
        got = pairwise_hip_forward(x.to(DEV), hip.anchors, hip.thresholds, hip.lut, lut_dtype=dt)
        assert torch.allclose(got.cpu(), want, atol=atol), dt


# ---------------------------------------------------------------- train fwd + bwd
@pytest.mark.parametrize(
    "min_margin,surrogate,seed",
    [(True, "fast_sigmoid_odd", 1), (False, "fast_sigmoid_odd", 1), (True, "izhikevich", 2)],
)
def test_reference_case_square_mean(min_margin, surrogate, seed):
    """test_backend_parity.py:348-392: PairwiseLinear(8, 5, tables=3,
    comparisons=3), min-margin and full STE (seed 1) and the izhikevich
    surrogate (seed 2), x = randn(4, 8), loss = square().mean(), at the
    reference's atol 1e-6 (x is drawn on the CPU: the reference draws it from
    the CUDA generator)."""
    torch.manual_seed(0)
    ref, hip = make_pair(8, 5, 3, 3, seed=seed, use_min_margin_ste=min_margin, surrogate=surrogate)
    x = torch.randn(4, 8)
    x_ref = x.clone().requires_grad_(True)
    x_hip = x.to(DEV).requires_grad_(True)
    ref.train()(x_ref).square().mean().backward()
    hip.train()(x_hip).square().mean().backward()
    with torch.no_grad():
        assert torch.allclose(ref(x), hip(x.to(DEV)).cpu(), atol=1e-6)
    assert torch.allclose(x_ref.grad, x_hip.grad.cpu(), atol=1e-6)
    assert torch.allclose(ref.thresholds.grad, hip.thresholds.grad.cpu(), atol=1e-6)
    assert torch.allclose(ref.lut.grad, hip.lut.grad.cpu(), atol=1e-6)


def test_c2_north_star_config():
    """c2: PairwiseLinear(128->128, T=136, C=6), B=512, x seed 0, G seed 1."""
    ref, hip = make_pair(128, 128, 136, 6, seed=0)
    x = seeded((512, 128), seed=0)
    g = seeded((512, 1, 128), seed=1)
    errs = assert_train_parity(ref, hip, *train_step(ref, hip, x, g))
    print("c2 errors", errs)


@pytest.mark.parametrize(
    "i,o,t,c,b,thr_std",
    [
        (8, 5, 3, 3, 4, 0.0),
        (128, 128, 136, 6, 1, 0.2),
        (784, 128, 136, 6, 64, 0.0),
        (128, 10, 136, 6, 37, 0.3),
        (64, 64, 20, 8, 50, 0.3),
        (16, 7, 5, 1, 19, 0.1),
        (40, 3, 33, 4, 70, 0.5),
        (256, 512, 16, 6, 8, 0.0),
        (100, 96, 7, 2, 300, 0.2),
        (32, 64, 10, 5, 2500, 0.2),
        (48, 128, 12, 6, 2100, 0.1),
        (24, 200, 9, 6, 1500, 0.3),
        (20, 100, 6, 4, 40, 0.2),
        (64, 300, 8, 5, 9000, 0.2),  # general path past 8192 items: the reduce kernel's direct record stores
    ],
)
def test_train_parity(i, o, t, c, b, thr_std):
    ref, hip = make_pair(i, o, t, c, seed=i + t, thr_std=thr_std)
    x = seeded((b, i), seed=b)
    g = seeded((b, 1, o), seed=b + 1)
    assert_train_parity(ref, hip, *train_step(ref, hip, x, g))


@pytest.mark.parametrize(
    "i,o,t,c,b,min_margin,surrogate,lut_dtype",
    [
        (128, 128, 136, 6, 512, True, "izhikevich", "f32"),  # fused path
        (40, 10, 33, 4, 70, True, "izhikevich", "f32"),  # fused path, 2 columns per lane
        (40, 34, 33, 4, 70, True, "izhikevich", "f32"),  # general path (O % 4 != 0, O > 32)
        (64, 30, 40, 8, 2100, True, "fast_sigmoid_odd", "f16"),  # fused, 2 columns per lane, R = 256, 3 tiles
        (16, 2, 9, 2, 33, True, "fast_sigmoid_odd", "f32"),  # fused, one lane per row
        (128, 128, 136, 6, 256, False, "fast_sigmoid_odd", "f32"),  # full STE
        (64, 96, 20, 8, 50, False, "izhikevich", "f32"),
        (16, 7, 5, 1, 19, False, "fast_sigmoid_odd", "f32"),
        (48, 128, 12, 6, 2100, False, "izhikevich", "f32"),  # several table-kernel tiles
        (128, 256, 40, 5, 64, False, "fast_sigmoid_odd", "f32"),  # 4 columns per lane
        (128, 128, 136, 6, 256, False, "izhikevich", "f16"),
        (100, 1000, 12, 7, 40, False, "fast_sigmoid_odd", "f16"),  # 8 f16 columns per lane
        (100, 1000, 12, 7, 300, True, "fast_sigmoid_odd", "f16"),  # general path, 16 column chunks
        (64, 300, 20, 8, 2100, True, "izhikevich", "f32"),  # general path, 5 chunks, 3 sort tiles
        (40, 3, 50, 3, 500, True, "izhikevich", "f32"),  # general path, 4-lane row groups
        (40, 6, 50, 3, 500, True, "izhikevich", "f32"),  # fused path, 2 columns per lane
        # general path, rows of whole 64-column chunks: 8 columns per lane in
        # 4-slot batches; f16: the LUT chunk as f16 in LDS in
        # 512-thread workgroups; f32: neighbour rows by byte permute
        (48, 320, 20, 6, 700, True, "izhikevich", "f16"),
        (48, 320, 20, 6, 700, True, "fast_sigmoid_odd", "f32"),
        (32, 320, 4, 6, 6000, True, "izhikevich", "f32"),  # ~12 batches of 4 slots per row group: two slot-offset windows, the second partial
    ],
)
def test_train_parity_ste_variants(i, o, t, c, b, min_margin, surrogate, lut_dtype):
    """Full STE (use_min_margin_ste=False, layers/pairwise.py:168-200) and the
    izhikevich surrogate (layers/surrogate.py:9-13), against the oracle."""
    ref, hip = make_pair(
        i, o, t, c, seed=i + t, thr_std=0.2, lut_dtype=lut_dtype, use_min_margin_ste=min_margin, surrogate=surrogate
    )
    x = seeded((b, i), seed=b)
    g = seeded((b, 1, o), seed=b + 1)
    tol = F16_TOL if lut_dtype == "f16" else F32_TOL
    assert_train_parity(ref, hip, *train_step(ref, hip, x, g), tol=tol)


@pytest.mark.parametrize("i,o,t,c,b", [(128, 128, 136, 6, 64), (48, 320, 20, 6, 300)])
@pytest.mark.parametrize("case", ["transposed_x_sum", "strided_grad", "sliced_3d_x"])
def test_noncontiguous_inputs_and_grads(i, o, t, c, b, case):
    """Views as inputs and upstream gradients (fused and general backward):
    a transposed x with y.sum().backward() (the upstream gradient is an
    expanded ones tensor with zero strides), a step-2 slice as the upstream
    gradient, and a [B, S, I] slice with S = 2. Codes bit-exact, output and
    gradients at the f32 bars, against the oracle fed the same views."""
    ref, hip = make_pair(i, o, t, c, seed=7, thr_std=0.3)

    def run(mod, dev):
        mod.train()
        if case == "transposed_x_sum":
            leaf = seeded((i, b), seed=5).to(dev).requires_grad_(True)
            x = leaf.t()
            y = mod(x)
            y.sum().backward()
        elif case == "strided_grad":
            leaf = seeded((b, i), seed=5).to(dev).requires_grad_(True)
            x = leaf
            y = mod(x)
            g = seeded((b, 1, 2 * o), seed=6).to(dev)[..., ::2]
            y.backward(g)
        else:
            leaf = seeded((b, 4, i), seed=5).to(dev).requires_grad_(True)
            x = leaf[:, ::2, :]
            y = mod(x)
            y.backward(seeded(tuple(y.shape), seed=6).to(dev))
        assert not x.is_contiguous() or case == "strided_grad"
        return y, leaf

    y_ref, leaf_ref = run(ref, torch.device("cpu"))
    y_hip, leaf_hip = run(hip, DEV)
    torch.cuda.synchronize()
    assert y_hip.shape == y_ref.shape
    assert torch.equal(hip._last_indices.cpu(), ref._last_indices), "route codes differ"
    pairs = {"output": (y_hip, y_ref), "grad_x": (leaf_hip.grad, leaf_ref.grad),
             "grad_thresholds": (hip.thresholds.grad, ref.thresholds.grad), "grad_lut": (hip.lut.grad, ref.lut.grad)}
    errs = {k: (rel_err(h, r), elem_err(h, r)) for k, (h, r) in pairs.items()}
    bad = {k: v for k, v in errs.items() if not (v[0] <= F32_TOL and v[1] <= ELEM_RTOL)}
    assert not bad, f"beyond the f32 bars: {bad} (all: {errs})"


def test_full_ste_without_route_debug():
    """With the route debug cache off the forward still keeps the margins the
    full STE needs."""
    ref, hip = make_pair(32, 16, 9, 5, seed=3, thr_std=0.2, use_min_margin_ste=False)
    hip.cache_route_debug = False
    x = seeded((40, 32), seed=5)
    g = seeded((40, 1, 16), seed=6)
    x_ref = x.clone().requires_grad_(True)
    x_hip = x.to(DEV).requires_grad_(True)
    ref.train()(x_ref).backward(g)
    hip.train()(x_hip).backward(g.to(DEV))
    assert rel_err(x_hip.grad, x_ref.grad) <= F32_TOL
    assert rel_err(hip.thresholds.grad, ref.thresholds.grad) <= F32_TOL
    assert rel_err(hip.lut.grad, ref.lut.grad) <= F32_TOL


def test_train_without_input_grad():
    """The reference harness trains with an x that needs no grad
    (tools/benchmarking/benchmark.py:105-118): thresholds and LUT grads only."""
    ref, hip = make_pair(128, 128, 136, 6, seed=0, thr_std=0.1)
    x = seeded((96, 128), seed=3)
    g = seeded((96, 1, 128), seed=4)
    assert_train_parity(ref, hip, *train_step(ref, hip, x, g, x_grad=False), x_grad=False)


def test_sequence_input_3d():
    """[B,S,I] input flattens to B*S items (pairwise_tilelang.py:438-441)."""
    ref, hip = make_pair(24, 12, 10, 5, seed=4, thr_std=0.2)
    x = seeded((6, 5, 24), seed=9)
    g = seeded((6, 5, 12), seed=10)
    assert_train_parity(ref, hip, *train_step(ref, hip, x, g))


def test_eval_mode_has_no_ste_gradient():
    """Eval mode: no STE, so x and thresholds get no gradient while the LUT
    still does (layers/pairwise.py:245-247)."""
    ref, hip = make_pair(32, 16, 12, 6, seed=1, thr_std=0.2)
    x = seeded((20, 32), seed=2)
    g = seeded((20, 1, 16), seed=3)
    x_ref = x.clone().requires_grad_(True)
    x_hip = x.to(DEV).requires_grad_(True)
    ref.eval()(x_ref).backward(g)
    hip.eval()(x_hip).backward(g.to(DEV))
    assert x_ref.grad is None and x_hip.grad is None
    assert ref.thresholds.grad is None and hip.thresholds.grad is None
    assert rel_err(hip.lut.grad, ref.lut.grad) <= F32_TOL


def test_ties_zero_margins_and_duplicate_anchors():
    """Sparse inputs (many exact zeros) give |m| ties, resolved to the first
    comparison, and u = 0, whose surrogate gradient is 0; an anchor pair with
    a == b gives zero net input gradient."""
    ref, hip = make_pair(20, 8, 6, 4, seed=7)
    with torch.no_grad():
        ref.anchors[0, 1] = torch.tensor([3, 3])
        hip.anchors.copy_(ref.anchors)
    gen = torch.Generator().manual_seed(0)
    x = torch.rand(30, 20, generator=gen) * (torch.rand(30, 20, generator=gen) >= 0.8)
    g = seeded((30, 1, 8), seed=2)
    assert_train_parity(ref, hip, *train_step(ref, hip, x, g))


@pytest.mark.parametrize(
    "i,o,t,c,b,min_margin,surrogate",
    [
        (128, 128, 136, 6, 512, True, "izhikevich"),  # fused backward (c2's shape)
        (784, 128, 136, 6, 512, True, "izhikevich"),  # fused backward (c5's first layer)
        (128, 10, 136, 6, 512, True, "izhikevich"),  # fused backward, 2 columns per lane (c5's last layer)
        (40, 34, 33, 4, 70, True, "izhikevich"),  # general backward (O % 4 != 0, O > 32)
        (48, 320, 20, 6, 700, True, "izhikevich"),  # general backward, 64-column chunks
        (64, 24, 17, 6, 2053, True, "izhikevich"),  # multi-item forward, 3 sort tiles
        (128, 128, 136, 6, 256, False, "izhikevich"),  # full STE
        (64, 96, 20, 8, 50, False, "izhikevich"),
        (128, 128, 136, 6, 256, False, "fast_sigmoid_odd"),
        (48, 24, 17, 6, 2053, False, "fast_sigmoid_odd"),
    ],
)
def test_sparse_inputs_exact_zero_margins(i, o, t, c, b, min_margin, surrogate):
    """Sparse inputs as c5's (x = rand * (rand >= 0.8)) with zero thresholds
    give many margins of exactly 0: the surrogate's u = 0 branch, +0.5 for
    izhikevich (where(u > 0, -1, +1) takes +1, layers/surrogate.py:9-13) and
    0 for fast_sigmoid_odd, plus |m| ties resolved to the first comparison,
    on every backward path, against the oracle at the f32 bars."""
    ref, hip = make_pair(i, o, t, c, seed=i + t + b, use_min_margin_ste=min_margin, surrogate=surrogate)
    gen = torch.Generator().manual_seed(b)
    x = torch.rand(b, i, generator=gen) * (torch.rand(b, i, generator=gen) >= 0.8)
    g = seeded((b, 1, o), seed=b + 3)
    yx_ref, yx_hip = train_step(ref, hip, x, g)
    margins = ref._last_margins.reshape(b, t, c)
    zero = margins == 0
    if min_margin:  # the selected comparison has margin 0 wherever any does
        assert zero.any(-1).float().mean() > 0.3
    else:
        assert zero.float().mean() > 0.3
    assert_train_parity(ref, hip, yx_ref, yx_hip)


@pytest.mark.parametrize(
    "i,o,t,c,b,lut_dtype",
    [
        (128, 10, 136, 6, 8192, "f32"),  # 69 items per item workgroup: three LDS chunks; 8 table-role tiles
        (128, 96, 136, 6, 512, "f32"),  # 384-byte rows, the widest f32 rows the item role takes at 136 tables
        (128, 128, 136, 6, 700, "f16"),  # f16 rows of 256 bytes
        (64, 8, 192, 4, 300, "f32"),  # 192 tables: the most the item role takes, 64 item workgroups
        (32, 24, 5, 3, 3, "f32"),  # 3 items: one per item workgroup
    ],
)
def test_fused_item_role(i, o, t, c, b, lut_dtype):
    """Shapes whose fused backward forms the input gradient in the fused
    launch's item role (no scatter kernel, no workspace): every gradient
    against the oracle, at the f32 bars on the LUT the kernels read."""
    lib = __import__("tropnn_amd.backends.pairwise_hip", fromlist=["load_library"])
    ws = lib.load_library().tropnn_hip_pairwise_backward_workspace_size(
        b, i, o, t, c, lib.LUT_F16 if lut_dtype == "f16" else lib.LUT_F32, lib.STE_MIN_MARGIN)
    assert ws == 0  # the item role's plan
    ref, hip = make_pair(i, o, t, c, seed=i + o + t, thr_std=0.3, lut_dtype=lut_dtype)
    if lut_dtype == "f16":
        with torch.no_grad():
            ref.lut.copy_(ref.lut.half().float())  # the values the kernels read
    x = seeded((b, i), seed=b + 5)
    g = seeded((b, 1, o), seed=b + 6)
    assert_train_parity(ref, hip, *train_step(ref, hip, x, g))


@pytest.mark.parametrize(
    "i,o,t,c,b,lut_dtype",
    [
        (128, 128, 136, 6, 512, "f32"),  # c2: scatter kernel by the row-width rule
        (128, 10, 136, 6, 512, "f32"),  # c5's last layer: item role by the rule
        (128, 128, 136, 6, 700, "f16"),
        (64, 8, 193, 4, 300, "f32"),  # past the item role's table limit: "fused" keeps the scatter kernel
    ],
)
def test_input_grad_forms_are_bit_identical(i, o, t, c, b, lut_dtype):
    """PairwiseLinear(input_grad=...): the fused launch's item role and the
    scatter kernel give the same bits for every gradient (same dots, same
    feature walk), so the caller's choice moves only the time; c2's shape on
    the item role against the oracle at the f32 bars."""
    results = {}
    for form in ("auto", "fused", "scatter"):
        ref, hip = make_pair(i, o, t, c, seed=i + o + t, thr_std=0.3, lut_dtype=lut_dtype)
        hip.input_grad = form
        if lut_dtype == "f16":
            with torch.no_grad():
                ref.lut.copy_(ref.lut.half().float())
        x = seeded((b, i), seed=b + 15)
        g = seeded((b, 1, o), seed=b + 16)
        yx_ref, yx_hip = train_step(ref, hip, x, g)
        assert_train_parity(ref, hip, yx_ref, yx_hip)
        results[form] = [t_.detach().cpu() for t_ in (yx_hip[0], yx_hip[1].grad, hip.thresholds.grad, hip.lut.grad)]
    for form in ("fused", "scatter"):
        for k, (a, r) in enumerate(zip(results[form], results["auto"])):
            assert torch.equal(a, r), (form, k)


def test_input_grad_option_is_validated():
    with pytest.raises(ValueError, match="input_grad"):
        PairwiseLinear(8, 8, tables=2, comparisons=2, input_grad="sideways")


@pytest.mark.parametrize("min_margin", [True, False])
def test_long_rows_lut_gradient_against_float64(min_margin):
    """Sparse input with three comparisons: most items share a few codes
    (rows of up to ~370 of 513 items), so each LUT-gradient element is a long
    sum that cancels. There the f32 oracle's own rounding is above the
    element-wise bar (1.7e-4 of it, found by a randomized sweep), so the LUT
    gradient is held to a float64 sum over the same codes: element-wise
    within 1e-4 (|exact| + 1e-3 max|exact|), norm-wise within 1e-6; and to
    the oracle at the norm-wise bar."""
    i, o, t, c, b = 16, 320, 40, 3, 513
    ref, hip = make_pair(i, o, t, c, seed=i + o + t, thr_std=0.3, use_min_margin_ste=min_margin,
                         surrogate="izhikevich")
    gen = torch.Generator().manual_seed(75)
    x = torch.rand(b, i, generator=gen) * (torch.rand(b, i, generator=gen) >= 0.8)
    g = seeded((b, 1, o), seed=b + c + 76)
    (y_ref, x_ref), (y_hip, x_hip) = train_step(ref, hip, x, g)
    codes = ref._last_indices.reshape(b, t)
    assert torch.equal(hip._last_indices.cpu().reshape(b, t), codes)
    counts = torch.stack([torch.bincount(codes[:, k], minlength=1 << c) for k in range(t)])
    assert int(counts.max()) > 300  # the long rows this case is about
    exact = torch.zeros(t, 1 << c, o, dtype=torch.float64)
    g64 = g.reshape(b, o).double()
    for k in range(t):
        exact[k].index_add_(0, codes[:, k], g64)
    exact /= t ** 0.5
    got = hip.lut.grad.detach().cpu().double()
    assert elem_err(got, exact) <= 1e-4
    assert rel_err(got, exact) <= 1e-6
    assert rel_err(hip.lut.grad, ref.lut.grad) <= F32_TOL
    for name, (h, r) in {"output": (y_hip, y_ref), "grad_x": (x_hip.grad, x_ref.grad),
                         "grad_thresholds": (hip.thresholds.grad, ref.thresholds.grad)}.items():
        assert rel_err(h, r) <= F32_TOL, name


def test_fused_item_role_input_gradient_only():
    """Parameters frozen, only the input gradient asked for: the fused launch
    is item workgroups alone (no table role), and grad_latent matches the
    oracle."""
    ref, hip = make_pair(128, 32, 136, 6, seed=3, thr_std=0.3)
    for p in list(ref.parameters()) + list(hip.parameters()):
        p.requires_grad_(False)
    x = seeded((512, 128), seed=8)
    g = seeded((512, 1, 32), seed=9)
    (y_ref, x_ref), (y_hip, x_hip) = train_step(ref, hip, x, g)
    assert torch.equal(hip._last_indices.cpu(), ref._last_indices)
    assert hip.lut.grad is None and hip.thresholds.grad is None
    assert rel_err(x_hip.grad, x_ref.grad) <= F32_TOL
    assert elem_err(x_hip.grad, x_ref.grad) <= ELEM_RTOL


def test_f16_lut_training():
    """f16 LUT reads in training: forward and gradients within 1e-3 of the f32 oracle."""
    ref, hip = make_pair(128, 128, 136, 6, seed=0, lut_dtype="f16", thr_std=0.1)
    x = seeded((256, 128), seed=0)
    g = seeded((256, 1, 128), seed=1)
    assert_train_parity(ref, hip, *train_step(ref, hip, x, g), tol=F16_TOL)


@pytest.mark.parametrize(
    "i,o,t,c,b,mode",
    [
        (128, 128, 136, 6, 512, "train"),  # fused path (the c2 layer)
        (48, 320, 20, 6, 700, "train"),  # general path, 8 columns per lane, the LUT chunk f16 in LDS
        (100, 1000, 12, 7, 300, "train"),  # general path, a partial last column chunk
        (32, 320, 4, 6, 6000, "train"),  # general path, f16: ~24 batches per row group, three slot-offset windows
        (128, 128, 136, 6, 4100, "eval"),  # wave-item forward
        (256, 512, 16, 6, 8, "eval"),  # one-item forward (the c1 layer)
    ],
)
def test_f16_reads_match_the_oracle_on_the_f16_lut(i, o, t, c, b, mode):
    """The f16-LUT paths widen each f16 element exactly and compute in f32, so
    against the oracle run on the same RNE f16 copy of the LUT they agree to
    the f32 tolerance (against the f32 oracle only to the LUT's own rounding,
    F16_TOL): a kernel error of a few 1e-4 would pass the F16_TOL tests but
    not this one."""
    ref, hip = make_pair(i, o, t, c, seed=i + o, thr_std=0.3, lut_dtype="f16")
    with torch.no_grad():
        ref.lut.copy_(ref.lut.half().float())  # the values the kernels read
    x = seeded((b, i), seed=b + 3)
    if mode == "train":
        g = seeded((b, 1, o), seed=b + 4)
        assert_train_parity(ref, hip, *train_step(ref, hip, x, g), tol=F32_TOL)
    else:
        hip.eval()
        with torch.no_grad():
            y = hip(x.to(DEV))
            y_ref = ref.eval()(x)
        assert torch.equal(hip._last_indices.cpu().reshape(b, t), ref._last_indices.reshape(b, t))
        assert rel_err(y, y_ref) <= F32_TOL


def test_f16_cache_follows_lut_updates():
    _, hip = make_pair(16, 8, 4, 3, seed=0, lut_dtype="f16")
    first = hip._lut_for_reading()
    assert first.dtype == torch.float16
    with torch.no_grad():
        hip.lut.add_(1.0)
    second = hip._lut_for_reading()
    assert second is not first
    assert torch.equal(second, hip.lut.detach().half())


def test_empty_batch():
    ref, hip = make_pair(16, 8, 4, 3, seed=0)
    x = torch.zeros(0, 16, device=DEV, requires_grad=True)
    y = hip.train()(x)
    assert y.shape == (0, 1, 8)
    y.sum().backward()
    assert torch.count_nonzero(hip.lut.grad) == 0


def test_route_debug_cache_off():
    _, hip = make_pair(16, 8, 4, 3, seed=0)
    hip.cache_route_debug = False
    with torch.no_grad():
        hip(seeded((5, 16), 0).to(DEV))
    assert hip._last_indices is None and hip._last_margins is None


# ---------------------------------------------------------------- large batches
@pytest.mark.parametrize("lut_dtype", ["f32", "f16"])
def test_large_batch_forward_multi_item(lut_dtype):
    """From 2048 items a forward workgroup takes 8 items. At 2053 items (a
    partial last workgroup): codes and margins bit-exact against the oracle,
    the output within tolerance, and bit-identical to the one-item kernel's
    (the same items run as two calls below the threshold)."""
    i, o, t, c, b = 128, 128, 136, 6, 2053
    ref, hip = make_pair(i, o, t, c, seed=4, thr_std=0.3, lut_dtype=lut_dtype)
    x = seeded((b, i), seed=21)
    xd = x.to(DEV)
    hip.eval()
    with torch.no_grad():
        y_full = hip(xd)
        idx, mar = hip._last_indices.clone(), hip._last_margins.clone()
        y_parts = torch.cat([hip(xd[:1024]), hip(xd[1024:])])
    torch.cuda.synchronize()
    assert torch.equal(y_full, y_parts)
    codes = routing_np.route_codes(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    margins = routing_np.margins_f32(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    np.testing.assert_array_equal(idx.cpu().reshape(b, t).numpy(), codes)
    np.testing.assert_array_equal(mar.cpu().reshape(b, t, c).numpy().view(np.uint32), margins.view(np.uint32))
    with torch.no_grad():
        y_ref = ref.eval()(x)
    assert rel_err(y_full, y_ref) <= (F16_TOL if lut_dtype == "f16" else F32_TOL)


@pytest.mark.parametrize(
    "i,o,t,c,min_margin,surrogate",
    [
        (64, 32, 20, 5, True, "fast_sigmoid_odd"),
        (64, 10, 20, 5, True, "fast_sigmoid_odd"),  # fused backward, 2 columns per lane, 3 tiles
        (64, 34, 20, 5, True, "fast_sigmoid_odd"),  # general backward path (O % 4 != 0, O > 32)
        (48, 24, 17, 6, False, "izhikevich"),  # full STE
    ],
)
def test_large_batch_training_multi_item(i, o, t, c, min_margin, surrogate):
    """Training at 2053 items: the multi-item forward, and the backward's
    sort over several 1024-item tiles."""
    ref, hip = make_pair(i, o, t, c, seed=6, thr_std=0.4, use_min_margin_ste=min_margin, surrogate=surrogate)
    x = seeded((2053, i), seed=22)
    g = seeded((2053, 1, o), seed=23)
    yx_ref, yx_hip = train_step(ref, hip, x, g)
    assert_train_parity(ref, hip, yx_ref, yx_hip)


# ---------------------------------------------------------------- route-debug codes format
@pytest.mark.parametrize(
    "i,o,t,c,b",
    [(16, 8, 4, 3, 5), (128, 128, 136, 6, 512), (64, 300, 17, 8, 40), (300, 4, 70, 1, 33), (1024, 1100, 64, 5, 3)],
)
def test_lazy_route_debug_codes(i, o, t, c, b):
    """cache_route_debug='lazy': the forward writes uint8 codes only; int64
    codes and margins materialise on first access, bit-identical to the
    eager cache and to the oracle's route. Output widths of 300 and 1100
    span several column tiles, of which only the first writes."""
    ref, hip = make_pair(i, o, t, c, seed=t + c, thr_std=0.5)
    x = seeded((b, i), seed=i + b)
    xd = x.to(DEV)
    hip.eval()
    with torch.no_grad():
        y_eager = hip(xd)
        eager_idx, eager_mar = hip._last_indices.clone(), hip._last_margins.clone()
        hip.cache_route_debug = "lazy"
        y_lazy = hip(xd)
    assert torch.equal(y_lazy, y_eager)
    codes = hip._last_codes
    assert codes.dtype == torch.uint8 and codes.shape == (b, 1, t)
    expect = routing_np.route_codes(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    np.testing.assert_array_equal(codes.cpu().reshape(b, t).numpy(), expect)
    assert torch.equal(hip._last_indices, eager_idx)
    assert hip._last_margins.shape == (b, 1, t, c)
    assert torch.equal(hip._last_margins.view(torch.int32), eager_mar.view(torch.int32))


def test_route_only_entry_point():
    """pairwise_hip_route against the oracle's codes and margins, at an item x
    table count that is not a multiple of the launch's 256 threads."""
    from tropnn_amd import pairwise_hip_route

    ref, hip = make_pair(40, 4, 13, 7, seed=5, thr_std=0.4)
    x = seeded((3, 7, 40), seed=11)
    codes, idx, mar = pairwise_hip_route(x.to(DEV), hip.anchors, hip.thresholds, codes=True)
    torch.cuda.synchronize()
    xs = x.reshape(21, 40).numpy()
    expect = routing_np.route_codes(xs, ref.anchors.numpy(), ref.thresholds.detach().numpy())
    margins = routing_np.margins_f32(xs, ref.anchors.numpy(), ref.thresholds.detach().numpy())
    assert codes.shape == (3, 7, 13) and idx.shape == (3, 7, 13) and mar.shape == (3, 7, 13, 7)
    np.testing.assert_array_equal(codes.cpu().reshape(21, 13).numpy(), expect)
    np.testing.assert_array_equal(idx.cpu().reshape(21, 13).numpy(), expect)
    np.testing.assert_array_equal(mar.cpu().reshape(21, 13, 7).numpy().view(np.uint32), margins.view(np.uint32))
    c0, i0, m0 = pairwise_hip_route(torch.zeros(0, 1, 40, device=DEV), hip.anchors, hip.thresholds, codes=True)
    assert c0.shape == (0, 1, 13) and i0.shape == (0, 1, 13) and m0.shape == (0, 1, 13, 7)


def test_module_compute_indices():
    """PairwiseLinear._compute_indices, the reference's route method
    (layers/pairwise.py:127-135), on a [B, S, I] latent: int64 indices and f32
    margins equal to the oracle's compute_route bit for bit, and to the
    module's own forward debug cache."""
    ref, hip = make_pair(40, 4, 13, 7, seed=6, thr_std=0.4)
    x = seeded((3, 7, 40), seed=12)
    idx, mar = hip._compute_indices(x.to(DEV))
    want_idx, want_mar = orc.compute_route(x, ref.anchors, ref.thresholds.detach())
    assert idx.dtype == torch.int64 and mar.dtype == torch.float32
    assert torch.equal(idx.cpu(), want_idx)
    assert torch.equal(mar.cpu().view(torch.int32), want_mar.view(torch.int32))
    hip.eval()
    with torch.no_grad():
        hip(x.to(DEV))
    assert torch.equal(hip._last_indices, idx) and torch.equal(hip._last_margins, mar)


@pytest.mark.parametrize("min_margin", [True, False])
def test_lazy_route_debug_training(min_margin):
    """Training with the lazy codes format gives the eager path's gradients;
    its margins are refused once an in-place update has touched the
    thresholds they were computed from."""
    ref, hip = make_pair(32, 16, 9, 5, seed=3, thr_std=0.3, use_min_margin_ste=min_margin)
    hip.cache_route_debug = "lazy"
    x = seeded((20, 32), 7)
    g = seeded((20, 1, 16), 8)
    yx_ref, yx_hip = train_step(ref, hip, x, g)
    assert_train_parity(ref, hip, yx_ref, yx_hip)
    margins = routing_np.margins_f32(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    got = hip._last_margins.cpu().reshape(20, 9, 5).numpy()
    np.testing.assert_array_equal(got.view(np.uint32), margins.view(np.uint32))
    hip(x.to(DEV))
    with torch.no_grad():
        hip.thresholds.add_(0.1)
    with pytest.raises(RuntimeError, match="lazy"):
        _ = hip._last_margins
    assert hip._last_codes.shape == (20, 1, 9)


def test_single_hip_runtime_in_process():
    """libtropnn_hip.so must bind the HIP runtime torch already loaded."""
    from tropnn_amd.backends.pairwise_hip import load_library

    load_library()
    maps = open("/proc/self/maps").read().splitlines()
    paths = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(paths) == 1, paths


# ---------------------------------------------------------------- c4 (full size)
def test_c4_large_layer_properties():
    """c4: PairwiseLinear(1024->4096, T=512, C=8), f16 LUT reads, B=8192.

    The full-size oracle is out of reach on the CPU, so parity is checked
    against the closed forms of the backward (layers/pairwise.py:137-166 with
    the autograd of the gather) and on properties that do not depend on size:
      * every one of the 8192 x 512 route codes against the numpy route;
      * for six tables (both ends, the middle and three seeded picks), over
        all 8192 items, in float64 from the HIP codes, the numpy margins and
        the f16 values the kernels read:
          grad_lut[t, r, :] = s * sum_{b: code[b,t] = r} G[b, :],
          D[b] = s * sum_o G[b, o] * (L[t, nb, o] - L[t, code, o]),
          nb = code ^ 2^r*, r* = first argmin_c |m[b, t, c]|, u = m[b, t, r*],
          grad_thresholds[t, c] = -sum_{b: r* = c} D[b] * fast_sigmoid_odd'(u)
        (an item placed in the wrong row of a later sort tile, or a wrong
        sign or comparison in the threshold gradient, fails these);
      * forward and input gradient of a row depend on that row only: a random
        subset of rows is compared with the oracle run on those rows alone
        (at the f16 bar with the f32 LUT, and at the f32 bars with the LUT
        rounded to f16 as the kernels read it);
      * every item adds its scaled grad row to exactly one row per table, so
        sum_r grad_lut[t, r, :] = s * sum_b G[b, :] for every table t;
      * gradients are linear in G: grad(G1 + G2) = grad(G1) + grad(G2).
    """
    i, o, t, c, b = 1024, 4096, 512, 8, 8192
    ref = orc.OraclePairwiseLinear(i, o, tables=t, comparisons=c, seed=0)
    hip = PairwiseLinear(i, o, tables=t, comparisons=c, seed=0, device_lut_dtype="f16").to(DEV)
    assert torch.equal(hip.anchors.cpu(), ref.anchors)
    x = seeded((b, i), seed=0).to(DEV)
    gfull = seeded((b, 1, o), seed=1).to(DEV)
    sub = torch.randperm(b, generator=torch.Generator().manual_seed(0))[:32]

    def run(g):
        hip.zero_grad(set_to_none=True)
        xg = x.clone().requires_grad_(True)
        y = hip.train()(xg)
        y.backward(g)
        return y.detach(), xg.grad.detach(), hip.thresholds.grad.detach().clone(), hip.lut.grad.detach().clone()

    y, gx, gthr, glut = run(gfull)
    codes = hip._last_indices.view(b, t).cpu().numpy()
    x_np = x.cpu().numpy()
    margins = routing_np.margins_f32(x_np, ref.anchors.numpy(), ref.thresholds.detach().numpy())
    np.testing.assert_array_equal(codes, routing_np.codes_from_margins(margins))

    s = hip.output_scale
    lut16 = hip._lut_f16.cpu().double()  # the f16 read copy the kernels used
    g64 = gfull.view(b, o).cpu().double()
    picks = torch.randperm(t - 2, generator=torch.Generator().manual_seed(5))[:3] + 1
    tables = [0, t // 2, t - 1] + [int(v) for v in picks]
    gthr_cpu, glut_t = gthr.cpu(), None
    for tt in tables:
        code_t = torch.from_numpy(codes[:, tt])
        want_lut = torch.zeros(1 << c, o, dtype=torch.float64).index_add_(0, code_t, g64) * s
        glut_t = glut[tt].cpu()
        assert rel_err(glut_t, want_lut) <= F32_TOL, f"grad_lut of table {tt}"
        m = margins[:, tt, :]
        r_star = torch.from_numpy(routing_np.min_margin_index(m))
        u = torch.from_numpy(m).double().gather(1, r_star.view(-1, 1)).view(-1)
        nb = code_t ^ (1 << r_star)
        d = s * ((lut16[tt][nb] - lut16[tt][code_t]) * g64).sum(1)
        gu = d * (-0.5 * torch.sign(u) / (1.0 + u.abs()).square())
        want_thr = -torch.zeros(c, dtype=torch.float64).index_add_(0, r_star, gu)
        assert rel_err(gthr_cpu[tt], want_thr) <= 1e-4, f"grad_thresholds of table {tt}"

    x_sub = x[sub.to(DEV)].cpu().requires_grad_(True)
    y_sub = ref.train()(x_sub)
    y_sub.backward(gfull[sub.to(DEV)].cpu())
    assert rel_err(y[sub.to(DEV)], y_sub) <= F16_TOL
    assert rel_err(gx[sub.to(DEV)], x_sub.grad) <= F16_TOL
    # and at the f32 bar (norm-wise and element-wise) against the oracle
    # reading the same f16-rounded LUT: what is left is summation order
    with torch.no_grad():
        ref.lut.copy_(ref.lut.half().float())
    ref.zero_grad(set_to_none=True)
    x_sub = x[sub.to(DEV)].cpu().requires_grad_(True)
    y_sub = ref.train()(x_sub)
    y_sub.backward(gfull[sub.to(DEV)].cpu())
    for name, (h, r) in {"output": (y[sub.to(DEV)], y_sub), "grad_x": (gx[sub.to(DEV)], x_sub.grad)}.items():
        assert rel_err(h, r) <= F32_TOL and elem_err(h, r) <= ELEM_RTOL, (name, rel_err(h, r), elem_err(h, r))

    row_sums = glut.sum(dim=1)  # [T, O]
    want = (gfull.view(b, o).double().sum(0) * s).float()
    assert rel_err(row_sums, want.expand(t, o)) <= 1e-4

    mask = torch.zeros(b, 1, 1, device=DEV)
    mask[: b // 2] = 1.0
    _, gx1, gthr1, glut1 = run(gfull * mask)
    _, gx2, gthr2, glut2 = run(gfull * (1 - mask))
    assert rel_err(gx1 + gx2, gx) <= 1e-5
    assert rel_err(gthr1 + gthr2, gthr) <= 1e-4
    assert rel_err(glut1 + glut2, glut) <= 1e-5


# ---------------------------------------------------------------- determinism and the anchor index
def test_backward_is_deterministic():
    """Every backward sum runs in a fixed order (no atomics): two runs on the
    same inputs give bit-identical gradients."""
    _, hip = make_pair(128, 128, 136, 6, seed=0, thr_std=0.1)
    x = seeded((512, 128), seed=0).to(DEV)
    g = seeded((512, 1, 128), seed=1).to(DEV)
    grads = []
    for _ in range(2):
        hip.zero_grad(set_to_none=True)
        xg = x.clone().requires_grad_(True)
        hip.train()(xg).backward(g)
        grads.append((xg.grad.clone(), hip.thresholds.grad.clone(), hip.lut.grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize(
    "i,t,c",
    [(37, 29, 5), (2000, 300, 8), (8192, 600, 8), (1, 70, 3), (3, 700, 8), (8193, 5, 2), (16384, 300, 8),
     (20000, 40, 6)],
)
def test_anchor_index_matches_numpy(i, t, c):
    """The inverse anchor index (a stable counting sort over windows of 8192
    features) against numpy: one chunk of 1024 anchors, several chunks,
    in_features = 8192 (one whole window), one feature (no feature bits to
    compare), three features shared by 11,200 anchors (long runs of equal
    features inside every wave and across chunks), and two or three windows
    (the last one of a single feature, two whole ones, a partial third)."""
    from tropnn_amd.backends.pairwise_hip import anchor_index

    gen = torch.Generator().manual_seed(3)
    anchors = torch.randint(0, i, (t, c, 2), generator=gen)
    offsets, entries = anchor_index(anchors.to(DEV), i)
    offsets, entries = offsets.cpu().numpy(), entries.cpu().numpy()
    flat = anchors.reshape(-1).numpy()
    want_entries = []
    want_offsets = [0]
    for f in range(i):
        for k in np.nonzero(flat == f)[0]:
            tt, cc, side = (k // 2) // c, (k // 2) % c, k % 2
            want_entries.append(((tt * c + cc) << 1) | side)
        want_offsets.append(len(want_entries))
    np.testing.assert_array_equal(offsets, np.array(want_offsets))
    np.testing.assert_array_equal(entries[: len(want_entries)], np.array(want_entries))


def test_no_grad_inference_writes_no_route_record():
    """Under torch.no_grad() the forward runs without the autograd Function
    and without a route record; outputs and debug tensors equal a forward
    with grad enabled."""
    _, hip = make_pair(16, 8, 5, 3, seed=1, thr_std=0.3)
    x = seeded((9, 16), 3).to(DEV)
    hip.eval()
    y_grad = hip(x)
    idx_grad, mar_grad = hip._last_indices.clone(), hip._last_margins.clone()
    with torch.no_grad():
        y_nog = hip(x)
    assert not y_nog.requires_grad and y_grad.requires_grad
    assert torch.equal(y_nog, y_grad.detach())
    assert torch.equal(hip._last_indices, idx_grad) and torch.equal(hip._last_margins, mar_grad)


def test_retain_graph_backward_twice():
    """Two backward passes over one forward (retain_graph=True) through the
    module: the second accumulates the same gradients again."""
    ref, hip = make_pair(64, 32, 20, 5, seed=2, thr_std=0.2)
    x = seeded((77, 64), 4)
    g = seeded((77, 1, 32), 5)
    x_hip = x.to(DEV).requires_grad_(True)
    y = hip.train()(x_hip)
    y.backward(g.to(DEV), retain_graph=True)
    first = (x_hip.grad.clone(), hip.thresholds.grad.clone(), hip.lut.grad.clone())
    y.backward(g.to(DEV))
    torch.cuda.synchronize()
    for a, total in zip(first, (x_hip.grad, hip.thresholds.grad, hip.lut.grad)):
        assert torch.equal(total, a + a)
    x_ref = x.clone().requires_grad_(True)
    ref.train()(x_ref).backward(g)
    assert rel_err(first[0], x_ref.grad) <= F32_TOL


@pytest.mark.parametrize(
    "lut_dtype,t,o,c,i",
    [
        ("f32", 64, 512, 8, 64),
        ("f16", 128, 512, 8, 64),
        ("f32", 256, 512, 6, 64),
        ("f32", 1100, 128, 6, 64),
        ("f16", 128, 512, 8, 37),  # input rows off 16-byte boundaries: the route kernel's 4-byte staging
        ("f32", 64, 512, 8, 3000),  # 12 KB rows: 4 items per route workgroup
    ],
)
def test_streamed_training_forward(lut_dtype, t, o, c, i):
    """Large training shapes (>= 4096 items, rows of whole 64-byte chunks,
    a LUT of >= 32 MiB: here 32 MiB, 1100 tables 34 MiB) take the streamed forward: a
    route-record kernel, then per (item block, column chunk) workgroups that
    walk the tables with each table's LUT chunk in LDS. Its route debug
    tensors are bit-identical to the eval forward's (a kernel that routes and
    gathers in one launch); its output, a sum over the tables in table order,
    equals the eval forward's to f32 rounding (that kernel sums blocks of
    tables, then the blocks) and repeats bit for bit; the training step (4100
    items: a partial last item block) matches the oracle. With 64-row tables
    (C = 6) the staged chunks' rows past the table repeat its last row and no
    code reads them. The route kernel gathers a block's records in LDS when
    they fit beside its input rows (T * 8 items * 8 bytes); 1100 tables
    (70 KB of records) take its direct stores."""
    b = 4100
    ref, hip = make_pair(i, o, t, c, seed=1, thr_std=0.2, lut_dtype=lut_dtype)
    x = seeded((b, i), seed=3)
    g = seeded((b, 1, o), seed=4)
    with torch.no_grad():
        y_eval = hip.eval()(x.to(DEV)).clone()
        idx_eval, mar_eval = hip._last_indices.clone(), hip._last_margins.clone()
    yx_ref, yx_hip = train_step(ref, hip, x, g)
    y_train = yx_hip[0].detach()
    # two f32 summation orders of t terms: the norm-wise gap grows as sqrt(t) eps,
    # an element's worst case (cancellation) as t eps
    assert rel_err(y_train, y_eval) <= max(1e-6, 4 * 2.0**-24 * t**0.5)
    elem_rtol = ELEM_RTOL * max(1.0, t / 256)
    assert elem_err(y_train, y_eval) <= elem_rtol
    assert torch.equal(hip._last_indices, idx_eval)
    assert torch.equal(hip._last_margins.view(torch.int32), mar_eval.view(torch.int32))
    assert_train_parity(ref, hip, yx_ref, yx_hip, tol=F16_TOL if lut_dtype == "f16" else F32_TOL, elem_rtol=elem_rtol)
    # a second training forward (grad mode: the streamed path) repeats the sum bit for bit
    assert torch.equal(hip.train()(x.to(DEV).requires_grad_(True)).detach(), y_train)


@pytest.mark.parametrize(
    "i,o,t,c,b,min_margin",
    [
        (64, 16, 1100, 8, 37, True),  # general path: the scatter kernel stages 106 KB
        (64, 16, 1100, 8, 37, False),  # full STE: the per-item kernel stages 106 KB
        (64, 32, 3000, 4, 40, True),  # fused path: the scatter kernel stages 144 KB
    ],
)
def test_large_tables_times_comparisons(i, o, t, c, b, min_margin):
    """Shapes whose per-item gu slots [T * C] and inverse anchor index need
    more than the default 64 KB of LDS (up to the workgroup's 160 KB)."""
    ref, hip = make_pair(i, o, t, c, seed=7, thr_std=0.3, use_min_margin_ste=min_margin)
    x = seeded((b, i), seed=8)
    g = seeded((b, 1, o), seed=9)
    assert_train_parity(ref, hip, *train_step(ref, hip, x, g))


# ---------------------------------------------------------------- fused backward over table counts and code skews
@pytest.mark.parametrize(
    "i,o,t,c,b,thr_std",
    [
        (96, 64, 40, 6, 512, 0.3),
        (128, 128, 150, 6, 512, 0.3),
        (128, 128, 136, 6, 512, 4.0),  # skewed: most items in a few rows
        (64, 96, 200, 5, 300, 0.3),
        (64, 32, 300, 4, 512, 0.3),  # more tables than compute units
        (80, 10, 136, 6, 511, 0.3),  # O = 10, two columns per lane
        (48, 128, 7, 6, 1, 0.3),  # one item
    ],
)
def test_fused_backward_table_counts(i, o, t, c, b, thr_std):
    """The fused backward (one workgroup per table) from 7 to 300 tables,
    with large thresholds that put most items into a few rows of each table
    (long rows crossing many row-group ranges, many empty rows), and a
    single item."""
    ref, hip = make_pair(i, o, t, c, seed=t + b, thr_std=thr_std, gen_seed=b)
    x = seeded((b, i), seed=i + t)
    g = seeded((b, 1, o), seed=o + b)
    yx_ref, yx_hip = train_step(ref, hip, x, g)
    assert_train_parity(ref, hip, yx_ref, yx_hip)
