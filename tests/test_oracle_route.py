"""Pins for the oracle's comparator route (CPU only).

Each check is independent of the oracle's own formula:
  * the Zig known-answer test (kernels/src/lut.zig:320-325);
  * hand-built inputs whose codes are worked out bit by bit;
  * brute force over every sign pattern of a small table;
  * torch.argmin's documented tie / NaN behaviour for the min-margin pick
    (layers/pairwise.py:138), checked on crafted rows;
  * the numpy restatement against the torch restatement on random inputs
    (two independent formulations of layers/pairwise.py:127-135).
"""
from __future__ import annotations

import itertools

import numpy as np
import torch

from oracle import pairwise_torch as orc
from oracle import routing_np


def test_zig_known_answer():
    # lut.zig:320-325: x = [3, 1, -1], anchors (0,1), (1,2), offsets [1.5, 3.0] -> code 1
    x = np.array([[3.0, 1.0, -1.0]], dtype=np.float32)
    anchors = np.array([[[0, 1], [1, 2]]])
    thr = np.array([[1.5, 3.0]], dtype=np.float32)
    assert routing_np.route_codes(x, anchors, thr).tolist() == [[1]]
    idx, margins = orc.compute_route(torch.from_numpy(x).unsqueeze(1), torch.from_numpy(anchors), torch.from_numpy(thr))
    assert idx.tolist() == [[[1]]]
    assert margins.flatten().tolist() == [0.5, -1.0]


def test_every_sign_pattern_of_a_table():
    """C = 4 comparisons on disjoint anchor pairs: for each of the 16 sign
    patterns the code must be the pattern read as binary, bit c = comparison c."""
    comps = 4
    anchors = np.array([[[2 * c, 2 * c + 1] for c in range(comps)]])
    thr = np.zeros((1, comps), dtype=np.float32)
    for bits in itertools.product([0, 1], repeat=comps):
        x = np.zeros((1, 2 * comps), dtype=np.float32)
        for c, bit in enumerate(bits):
            x[0, 2 * c] = 1.0 if bit else -1.0
        want = sum(bit << c for c, bit in enumerate(bits))
        assert routing_np.route_codes(x, anchors, thr)[0, 0] == want
        idx, _ = orc.compute_route(torch.from_numpy(x).unsqueeze(1), torch.from_numpy(anchors), torch.from_numpy(thr))
        assert int(idx) == want


def test_margin_rounding_order_and_edge_values():
    """margin = (x[a] - x[b]) - thr in f32, left to right: with x[a] = 1e8,
    x[b] = -1 and thr = 1e8 the exact value is +1 but f32 gives 0 (no bit);
    subnormal positive margins set the bit; NaN and +-0 do not."""
    x = np.array([[1e8, -1.0, 1.4e-45, 0.0, np.nan]], dtype=np.float32)
    anchors = np.array([[[0, 1], [2, 3], [3, 2], [4, 0], [3, 3]]])
    thr = np.array([[1e8, 0.0, 0.0, 0.0, 0.0]], dtype=np.float32)
    m = routing_np.margins_f32(x, anchors, thr)[0, 0]
    assert m[0] == np.float32(0.0)  # (1e8 - -1) rounds to 1e8 in f32
    assert m[1] > 0 and m[1] < 1e-44  # subnormal kept
    assert routing_np.route_codes(x, anchors, thr)[0, 0] == 0b00010
    _, tm = orc.compute_route(torch.from_numpy(x).unsqueeze(1), torch.from_numpy(anchors), torch.from_numpy(thr))
    np.testing.assert_array_equal(tm.numpy().reshape(-1).view(np.uint32), m.view(np.uint32))


def test_min_margin_pick_follows_torch_argmin_semantics():
    rows = np.array(
        [
            [0.5, -0.5, 0.25, -0.25],  # tie between 0.25 and -0.25: first wins -> 2
            [1.0, np.nan, 0.0, np.nan],  # NaN propagates: first NaN -> 1
            [3.0, 2.0, -1.0, np.inf],  # plain minimum -> 2
            [np.inf, -np.inf, np.inf, 7.0],  # finite beats inf -> 3
            [0.0, -0.0, 0.0, 0.0],  # all zero: first -> 0
        ],
        dtype=np.float32,
    )
    assert routing_np.min_margin_index(rows).tolist() == [2, 1, 2, 3, 0]
    assert torch.from_numpy(rows).abs().argmin(-1).tolist() == [2, 1, 2, 3, 0]


def test_numpy_and_torch_restatements_agree():
    gen = torch.Generator().manual_seed(7)
    for i, t, c in [(16, 5, 3), (128, 136, 6), (40, 9, 8), (7, 3, 1)]:
        anchors = torch.randint(0, i, (t, c, 2), generator=gen)
        thr = torch.randn(t, c, generator=gen) * 0.3
        x = torch.randn(33, i, generator=gen)
        idx, margins = orc.compute_route(x.unsqueeze(1), anchors, thr)
        np_codes = routing_np.route_codes(x.numpy(), anchors.numpy(), thr.numpy())
        np_margins = routing_np.margins_f32(x.numpy(), anchors.numpy(), thr.numpy())
        np.testing.assert_array_equal(idx.squeeze(1).numpy(), np_codes)
        np.testing.assert_array_equal(margins.squeeze(1).numpy().view(np.uint32), np_margins.view(np.uint32))
        r_star, _, _ = orc.min_margin_select(idx, margins)
        np.testing.assert_array_equal(r_star.squeeze(1).numpy(), routing_np.min_margin_index(np_margins))
