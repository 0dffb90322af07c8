"""Seeded random shapes over every forward kernel (one-item, multi-item,
wave-item) and both backward paths (fused, general; min-margin and full STE,
both surrogates), f32 and f16 LUTs, against the CPU oracle: route codes
exact, outputs and every gradient within the f32 tolerance (f16 LUT reads
against the oracle run on the same RNE f16 copy of the LUT), and the
gradients also within it of the float64 closed forms (oracle/closed_form.py).
A regression guard beside the hand-picked cases of test_gpu_parity."""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle import routing_np
from oracle.closed_form import gradients_f64
from test_gpu_parity import DEV, F32_TOL, assert_train_parity, make_pair, rel_err, seeded, train_step

pytestmark = pytest.mark.gpu


def _cases(seed: int, n: int):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        kind = rng.choice(["eval", "train", "train"])
        c = rng.choice([1, 2, 3, 4, 5, 6, 7, 8])
        t = rng.choice([1, 3, 9, 17, 40, 136])
        i = rng.choice([4, 16, 33, 64, 128, 300])
        o = rng.choice([2, 6, 10, 32, 64, 96, 128, 136, 256, 320, 512, 1000])
        b = rng.choice([1, 7, 64, 513, 2100, 4100] if kind == "eval" else [1, 5, 33, 512, 1100, 2100])
        if t * (2**c) * o * 4 > (256 << 20) or b * t * o > 60_000_000:
            continue  # keep the CPU oracle within seconds
        out.append(
            (kind, i, o, t, c, b, rng.choice(["f32", "f16"]), rng.random() < 0.7,
             rng.choice(["fast_sigmoid_odd", "izhikevich"]), rng.choice([0.0, 0.3]))
        )
    return out


def _wide_cases(seed: int, n: int):
    """Inputs past the kernels' LDS copies (12,000 to 45,000 features) and
    many tables (2,000 to 3,500): the forward's global-memory input row, the
    windowed anchor index and the wide scatter kernel."""
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        kind = rng.choice(["eval", "train", "train", "train"])
        if rng.random() < 0.5:
            i, t = rng.choice([12000, 20000, 45000]), rng.choice([1, 9, 40])
        else:
            i, t = rng.choice([16, 64, 300]), rng.choice([2000, 3500])
        c = rng.choice([1, 3, 5, 6, 8])
        o = rng.choice([2, 10, 32, 64, 96, 300])
        b = rng.choice([1, 5, 33, 300])
        if t * (2**c) * o * 4 > (256 << 20) or b * t * o > 20_000_000 or b * i > 4_000_000:
            continue  # keep the CPU oracle within seconds
        out.append(
            (kind, i, o, t, c, b, rng.choice(["f32", "f16"]), rng.random() < 0.7,
             rng.choice(["fast_sigmoid_odd", "izhikevich"]), rng.choice([0.0, 0.3]))
        )
    return out


@pytest.mark.parametrize("case", _cases(2024, 36), ids=lambda c: "-".join(str(v) for v in c))
def test_random_shape(case):
    _run(case)


@pytest.mark.parametrize("case", _wide_cases(77, 16), ids=lambda c: "-".join(str(v) for v in c))
def test_random_wide_shape(case):
    _run(case)


def _run(case):
    kind, i, o, t, c, b, lut_dtype, min_margin, surrogate, thr = case
    print(f"[random shape] {case}", flush=True)
    ref, hip = make_pair(
        i, o, t, c, seed=i + o + t, thr_std=thr, lut_dtype=lut_dtype, use_min_margin_ste=min_margin,
        surrogate=surrogate,
    )
    if lut_dtype == "f16":
        with torch.no_grad():
            ref.lut.copy_(ref.lut.half().float())  # the values the kernels read
    x = seeded((b, i), seed=b + c)
    if kind == "train":
        g = seeded((b, 1, o), seed=b + c + 1)
        yx_ref, yx_hip = train_step(ref, hip, x, g)
        assert_train_parity(ref, hip, yx_ref, yx_hip, tol=F32_TOL)
        # and against the float64 closed forms on the same codes: the HIP
        # gradients within 1e-5 of exact arithmetic, norm-wise
        gx, gt, gl = gradients_f64(x, ref.anchors, ref.thresholds, ref.lut, g.reshape(b, o), min_margin=min_margin,
                                   surrogate=surrogate, output_scale=1.0 / t ** 0.5)
        for got, exact in ((yx_hip[1].grad, gx), (hip.thresholds.grad, gt), (hip.lut.grad, gl)):
            assert rel_err(got.double(), exact) <= F32_TOL
        return
    hip.eval()
    with torch.no_grad():
        y = hip(x.to(DEV))
        idx = hip._last_indices
        y_ref = ref.eval()(x)
    codes = routing_np.route_codes(x.numpy(), ref.anchors.numpy(), ref.thresholds.detach().numpy())
    np.testing.assert_array_equal(idx.cpu().reshape(b, t).numpy(), codes)
    assert rel_err(y, y_ref) <= F32_TOL
