"""Pins for the oracle's forward and STE backward (CPU only).

What fixes each value, independently of the oracle's vectorised code:
  * seeded init: golden fixtures written from the reference itself
    (tests/golden/make_golden.py), for the oracle and for the product module;
  * route-chunk sizes: the hand-computed values of the c2 / c4 / c5 plans;
  * forward: a float64 loop over (item, table) that sums the selected LUT rows;
  * backward: central finite differences, in float64, of the smooth function
    whose exact gradient the STE defines -- the Heaviside step replaced by the
    antiderivative S of the surrogate (S(u) = 0.5 / (1 + |u|) for
    fast_sigmoid_odd, -2 sigmoid(|u|) for izhikevich), with the selected
    comparison, code and neighbour frozen. A dropped term, a sign error or a
    wrong anchor index changes these derivatives;
  * the LUT gradient: finite differences of the (linear) forward;
  * the surrogate signs of the reference test (test_pairwise.py:9-15).
"""
from __future__ import annotations

import hashlib
import math
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import pairwise_torch as orc

GOLDEN = Path(__file__).resolve().parent / "golden"


def _fixtures():
    meta = json.loads((GOLDEN / "init_fixtures.json").read_text())
    arrays = np.load(GOLDEN / "init_fixtures.npz")
    return meta, arrays


def _check_init(key, meta, arrays, anchors, thresholds, lut, next_randn, output_scale, powers):
    m = meta[key]
    np.testing.assert_array_equal(anchors.numpy(), arrays[f"{key}__anchors"].astype(np.int64))
    flat = lut.detach().contiguous().numpy().reshape(-1)
    assert list(lut.shape) == m["lut_shape"]
    assert hashlib.sha256(flat.tobytes()).hexdigest() == m["lut_sha256"]
    assert [float(flat[p]) for p in m["lut_sample_pos"]] == m["lut_sample_val"]
    if f"{key}__lut" in arrays:
        np.testing.assert_array_equal(lut.detach().numpy(), arrays[f"{key}__lut"])
    assert bool((thresholds == 0).all()) == m["thresholds_all_zero"]
    assert powers.tolist() == m["powers"]
    assert output_scale == m["output_scale"]
    assert next_randn == m["next_randn"]


SMALL_CASES = ["i8_o5_t3_c3_s1", "i8_o5_t4_c3_s2", "i256_o512_t16_c6_s0", "i128_o128_t136_c6_s0",
               "i784_o128_t136_c6_s0", "i128_o128_t136_c6_s1", "i128_o10_t136_c6_s2"]


@pytest.mark.parametrize("key", SMALL_CASES)
def test_init_matches_reference_fixture(key):
    from tropnn_amd import PairwiseLinear

    meta, arrays = _fixtures()
    m = meta[key]
    args = (m["in_features"], m["out_features"])
    kw = dict(tables=m["tables"], comparisons=m["comparisons"], seed=m["seed"])
    ref = orc.OraclePairwiseLinear(*args, **kw)
    nxt = float(torch.randn(()).item())
    _check_init(key, meta, arrays, ref.anchors, ref.thresholds, ref.lut, nxt, ref.output_scale, ref.powers)
    prod = PairwiseLinear(*args, **kw)
    nxt = float(torch.randn(()).item())
    _check_init(key, meta, arrays, prod.anchors, prod.thresholds, prod.lut, nxt, prod.output_scale, prod.powers)


def test_init_matches_reference_fixture_c4():
    """c4's 2 GiB LUT (1024->4096, T=512, C=8): product module init only."""
    from tropnn_amd import PairwiseLinear

    meta, arrays = _fixtures()
    key = "i1024_o4096_t512_c8_s0"
    prod = PairwiseLinear(1024, 4096, tables=512, comparisons=8, seed=0)
    nxt = float(torch.randn(()).item())
    _check_init(key, meta, arrays, prod.anchors, prod.thresholds, prod.lut, nxt, prod.output_scale, prod.powers)


def test_route_chunk_sizes():
    # c2: 16 MiB / (512 * 128 * 4 B) = 64 tables per chunk
    assert orc.route_chunk_size(512, 128, torch.float32, 136) == 64
    # c4: 8192 * 4096 * 4 B = 128 MiB per table > 16 MiB -> 1
    assert orc.route_chunk_size(8192, 4096, torch.float32, 512) == 1
    # c5 last layer: 512 * 10 * 4 B = 20 KB per table -> all 136 at once
    assert orc.route_chunk_size(512, 10, torch.float32, 136) == 136
    # full STE payload O * (C + 1) with an 8 MiB target: 8 MiB / (512 * 896 * 4 B) = 4
    assert orc.route_chunk_size(512, 128 * 7, torch.float32, 136, target_bytes=8 * 1024 * 1024) == 4


def test_surrogate_signs():
    u = torch.tensor([-2.0, 0.0, 2.0])
    for name in orc.SURROGATES:
        g = orc.surrogate_gradient(u, name)
        assert g[0] > 0 and g[2] < 0
    assert orc.surrogate_gradient(u, "fast_sigmoid_odd")[1] == 0
    with pytest.raises(ValueError, match="unsupported surrogate"):
        orc.surrogate_gradient(u, "nope")


def _random_layer(i, o, t, c, seed, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    anchors = torch.stack([torch.randperm(i, generator=gen)[:2] for _ in range(t * c)]).view(t, c, 2)
    thr = (torch.randn(t, c, generator=gen) * 0.3).to(dtype)
    lut = (torch.randn(t, 1 << c, o, generator=gen) * 0.5).to(dtype)
    x = torch.randn(5, 2, i, generator=gen).to(dtype)
    g = torch.randn(5, 2, o, generator=gen).to(dtype)
    return anchors, thr, lut, x, g


def _codes_loop(x, anchors, thr):
    """Per item and table, the code by explicit loops in f32 arithmetic."""
    xs = x.reshape(-1, x.shape[-1]).to(torch.float32).numpy()
    th = thr.to(torch.float32).numpy()
    an = anchors.numpy()
    items, tables, comps = xs.shape[0], an.shape[0], an.shape[1]
    codes = np.zeros((items, tables), dtype=np.int64)
    for b in range(items):
        for t in range(tables):
            code = 0
            for c in range(comps):
                m = np.float32(np.float32(xs[b, an[t, c, 0]] - xs[b, an[t, c, 1]]) - th[t, c])
                if m > 0:
                    code |= 1 << c
            codes[b, t] = code
    return codes


@pytest.mark.parametrize("case", [(6, 4, 3, 3), (9, 7, 5, 1), (12, 3, 4, 6)])
def test_forward_matches_float64_loop(case):
    i, o, t, c = case
    anchors, thr, lut, x, _ = _random_layer(i, o, t, c, seed=sum(case), dtype=torch.float32)
    out, idx, _ = orc.route_output(x, anchors, thr, lut, training=False)
    codes = _codes_loop(x, anchors, thr)
    np.testing.assert_array_equal(idx.reshape(-1, t).numpy(), codes)
    want = np.zeros((codes.shape[0], o))
    L = lut.double().numpy()
    for b in range(codes.shape[0]):
        for tt in range(t):
            want[b] += L[tt, codes[b, tt]]
    np.testing.assert_allclose(out.reshape(-1, o).double().numpy(), want, rtol=1e-6, atol=1e-6)


def _S(u, surrogate):
    if surrogate == "fast_sigmoid_odd":
        return 0.5 / (1.0 + np.abs(u))
    return -2.0 / (1.0 + np.exp(-np.abs(u)))  # -2 * sigmoid(|u|)


def _smoothed_objective(x, thr, lut, anchors, g, frozen, surrogate, full):
    """sum_b <g_b, y~_b> where the STE value (H_ste(u) - [u>0]) is replaced
    by S(u) - S(u0) and the selection, codes and neighbours stay frozen."""
    codes, sel, u0 = frozen
    xs = x.reshape(-1, x.shape[-1])
    gs = g.reshape(-1, g.shape[-1])
    total = 0.0
    items, tables = codes.shape
    comps = anchors.shape[1]
    for b in range(items):
        for t in range(tables):
            cur = codes[b, t]
            total += gs[b] @ lut[t, cur]
            cs = range(comps) if full else [sel[b, t]]
            for c in cs:
                a0, a1 = anchors[t, c]
                u = xs[b, a0] - xs[b, a1] - thr[t, c]
                nb = cur ^ (1 << c)
                total += (_S(u, surrogate) - _S(u0[b, t, c], surrogate)) * (gs[b] @ (lut[t, nb] - lut[t, cur]))
    return total


@pytest.mark.parametrize("surrogate", ["fast_sigmoid_odd", "izhikevich"])
@pytest.mark.parametrize("full", [False, True])
def test_ste_backward_matches_finite_differences(surrogate, full):
    i, o, t, c = 7, 4, 3, 3
    anchors, thr, lut, x, g = _random_layer(i, o, t, c, seed=11 if full else 5)
    xr = x.clone().requires_grad_(True)
    thr_r = thr.clone().requires_grad_(True)
    lut_r = lut.clone().requires_grad_(True)
    out, idx, margins = orc.route_output(
        xr, anchors, thr_r, lut_r, training=True, use_min_margin_ste=not full, surrogate=surrogate
    )
    out.backward(g)
    m = margins.detach().reshape(-1, t, c).numpy()
    assert np.abs(m).min() > 1e-3  # away from the surrogate's kink at 0
    codes = idx.reshape(-1, t).numpy()
    sel = np.abs(m).argmin(-1)
    frozen = (codes, sel, m)
    an = anchors.numpy()
    xn, thn, ln, gn = x.numpy(), thr.numpy(), lut.numpy(), g.numpy()

    def f(xv, tv, lv):
        return _smoothed_objective(xv, tv, lv, an, gn, frozen, surrogate, full)

    h = 1e-6
    gx = np.zeros_like(xn)
    for k in np.ndindex(xn.shape):
        xp, xm = xn.copy(), xn.copy()
        xp[k] += h
        xm[k] -= h
        gx[k] = (f(xp, thn, ln) - f(xm, thn, ln)) / (2 * h)
    gt = np.zeros_like(thn)
    for k in np.ndindex(thn.shape):
        tp, tm = thn.copy(), thn.copy()
        tp[k] += h
        tm[k] -= h
        gt[k] = (f(xn, tp, ln) - f(xn, tm, ln)) / (2 * h)
    rng = np.random.default_rng(0)
    for _ in range(12):
        k = tuple(int(rng.integers(0, s)) for s in ln.shape)
        lp, lm = ln.copy(), ln.copy()
        lp[k] += h
        lm[k] -= h
        fd = (f(xn, thn, lp) - f(xn, thn, lm)) / (2 * h)
        assert lut_r.grad[k].item() == pytest.approx(fd, rel=1e-6, abs=1e-8)
    # the reference computes the STE branch in float32 (layers/pairwise.py:145, 148)
    np.testing.assert_allclose(xr.grad.numpy(), gx, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(thr_r.grad.numpy(), gt, rtol=1e-5, atol=1e-6)


def test_zero_margin_and_duplicate_anchor_give_no_input_gradient():
    """u = 0 has surrogate 0 (no gradient through that table); a == b gives
    +gu - gu = 0 on the shared feature."""
    anchors = torch.tensor([[[0, 1], [2, 2]]])
    thr = torch.zeros(1, 2, dtype=torch.float64)
    lut = torch.randn(1, 4, 3, dtype=torch.float64)
    x = torch.tensor([[[0.5, 0.5, 1.0]]], dtype=torch.float64, requires_grad=True)  # m0 = 0 -> r* = 0, u = 0
    out, _, _ = orc.route_output(x, anchors, thr, lut, training=True)
    out.sum().backward()
    assert torch.count_nonzero(x.grad) == 0
    thr2 = torch.tensor([[0.0, -0.2]], dtype=torch.float64)  # a == b: m1 = 0.2 is the min, u != 0
    x2 = torch.tensor([[[1.0, 0.0, 3.0]]], dtype=torch.float64, requires_grad=True)
    out, _, margins = orc.route_output(x2, anchors, thr2, lut, training=True)
    assert margins[0, 0, 0].tolist() == [1.0, 0.2]
    out.sum().backward()
    assert x2.grad[0, 0, 2] == 0 and torch.count_nonzero(x2.grad) == 0


def test_surrogates_at_zero():
    """The reference's surrogates at u = 0 (layers/surrogate.py:9-17).
    izhikevich takes the +1 branch of where(u > 0, -1, +1) at u = 0 (and at
    -0.0, which is not > 0), so izhikevich(0) = 2 sigmoid(0) (1 - sigmoid(0))
    = +0.5, while its limit from above is -0.5; fast_sigmoid_odd has
    sign(0) = 0, so 0. A sign(u) slip in izhikevich gives 0 at u = 0 and
    fails here; a > / >= slip gives -0.5 and fails here."""
    u = torch.tensor([0.0, -0.0], dtype=torch.float32)
    assert orc.surrogate_gradient(u, "izhikevich").tolist() == [0.5, 0.5]
    fso = orc.surrogate_gradient(u, "fast_sigmoid_odd")
    assert fso.tolist() == [0.0, 0.0]
    eps = torch.tensor([1e-30, -1e-30], dtype=torch.float32)  # either side of the kink
    assert orc.surrogate_gradient(eps, "izhikevich").tolist() == [-0.5, 0.5]
    assert orc.surrogate_gradient(eps, "fast_sigmoid_odd").tolist() == [-0.5, 0.5]


def _sigma_prime(u: float, surrogate: str) -> float:
    """The surrogate derivative from its formula, in float64: fast_sigmoid_odd
    -0.5 sign(u) / (1 + |u|)^2; izhikevich s' 2 s (1 - s), s = 1 / (1 +
    exp(-|u|)), s' = -1 for u > 0 else +1."""
    if surrogate == "fast_sigmoid_odd":
        sgn = (u > 0) - (u < 0)
        return -0.5 * sgn / (1.0 + abs(u)) ** 2
    s = 1.0 / (1.0 + math.exp(-abs(u)))
    return (-1.0 if u > 0 else 1.0) * 2.0 * s * (1.0 - s)


@pytest.mark.parametrize("surrogate,sigma0", [("izhikevich", 0.5), ("fast_sigmoid_odd", 0.0)])
@pytest.mark.parametrize("full", [False, True])
def test_exact_zero_margin_gradient_closed_form(surrogate, sigma0, full):
    """One item, one table, C = 2 with disjoint anchors (0, 1) and (2, 3),
    thresholds 0, x = [0.7, 0.7, 2.0, 0.5]: m0 = 0 exactly, m1 = 1.5, code
    = 0b10 = 2. With D_c = G . (L[code ^ 2^c] - L[code]) and
    gu_c = D_c sigma'(m_c), the STE gives x.grad[a_c] += gu_c,
    x.grad[b_c] -= gu_c, thr.grad[c] = -gu_c (layers/pairwise.py:137-200
    through autograd), and lut.grad[code] = G. The min-margin STE selects
    c = 0 (|m0| = 0 is the smallest), so only gu_0 = D_0 sigma'(0) flows:
    0.5 D_0 for izhikevich, 0 for fast_sigmoid_odd; the full STE adds gu_1."""
    anchors = torch.tensor([[[0, 1], [2, 3]]])
    thr = torch.zeros(1, 2, dtype=torch.float64, requires_grad=True)
    lut_vals = np.array([[[1.0, -2.0, 0.5], [0.25, 3.0, -1.0], [-0.5, 1.5, 2.0], [4.0, -0.75, 1.25]]])
    lut = torch.tensor(lut_vals, requires_grad=True)
    x = torch.tensor([[[0.7, 0.7, 2.0, 0.5]]], dtype=torch.float64, requires_grad=True)
    g = np.array([0.3, -1.1, 0.8])
    out, idx, margins = orc.route_output(x, anchors, thr, lut, training=True, use_min_margin_ste=not full,
                                         surrogate=surrogate)
    assert margins[0, 0, 0].tolist() == [0.0, 1.5] and int(idx[0, 0, 0]) == 2
    out.backward(torch.tensor(g).view(1, 1, 3))
    d0 = float(g @ (lut_vals[0, 3] - lut_vals[0, 2]))
    d1 = float(g @ (lut_vals[0, 0] - lut_vals[0, 2]))
    gu0 = d0 * sigma0
    assert _sigma_prime(0.0, surrogate) == sigma0
    gu1 = d1 * _sigma_prime(1.5, surrogate) if full else 0.0
    want_x = np.array([gu0, -gu0, gu1, -gu1])
    # the reference runs the STE branch in float32 (layers/pairwise.py:145, 148)
    np.testing.assert_allclose(x.grad.view(-1).numpy(), want_x, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(thr.grad.view(-1).numpy(), [-gu0, -gu1], rtol=1e-6, atol=1e-7)
    want_lut = np.zeros_like(lut_vals)
    want_lut[0, 2] = g
    np.testing.assert_allclose(lut.grad.numpy(), want_lut, rtol=0, atol=0)
    if surrogate == "izhikevich":
        assert gu0 != 0.0  # the u = 0 branch carries a gradient


@pytest.mark.parametrize("min_margin", [True, False])
@pytest.mark.parametrize("surrogate", ["fast_sigmoid_odd", "izhikevich"])
@pytest.mark.parametrize("sparse", [False, True])
def test_closed_form_gradients_match_the_oracle_autograd(min_margin, surrogate, sparse):
    """oracle/closed_form.py (float64 sums of the gradients' closed forms on
    the forward's own codes) against the autograd of the torch restatement,
    on shapes with ties and exact-zero margins (sparse input): two separate
    statements of the same backward agree to f32 rounding, so neither drops
    a term, a sign or an index the other keeps."""
    from oracle.closed_form import gradients_f64

    i, o, t, c, b = 20, 24, 9, 4, 64
    ref = orc.OraclePairwiseLinear(i, o, tables=t, comparisons=c, seed=3, use_min_margin_ste=min_margin,
                                   surrogate=surrogate).train()
    gen = torch.Generator().manual_seed(21)
    with torch.no_grad():
        ref.thresholds.copy_(0.0 if sparse else 0.3 * torch.randn(t, c, generator=gen))
    if sparse:
        x = torch.rand(b, i, generator=gen) * (torch.rand(b, i, generator=gen) >= 0.8)
    else:
        x = torch.randn(b, i, generator=gen)
    g = torch.randn(b, 1, o, generator=gen)
    xr = x.clone().requires_grad_(True)
    ref(xr).backward(g)
    gx, gt, gl = gradients_f64(x, ref.anchors, ref.thresholds, ref.lut, g.reshape(b, o), min_margin=min_margin,
                               surrogate=surrogate, output_scale=1.0 / math.sqrt(t))
    for got, exact in ((xr.grad, gx), (ref.thresholds.grad, gt), (ref.lut.grad, gl)):
        scale = float(exact.abs().max())
        assert scale > 0
        assert float((got.double() - exact).abs().max()) <= 1e-5 * scale
    if sparse:
        assert (torch.from_numpy(np.abs(ref._last_margins.numpy())) == 0).any()  # exact-zero margins ran
