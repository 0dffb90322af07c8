"""numpy restatement of the comparator route. TEST INFRASTRUCTURE ONLY.

Integer/bit work, restated in plain numpy so the codes the HIP route produces
can be compared bit for bit without going through torch:
  * margin m[b,t,c] = fl32(fl32(x[b,a] - x[b,b']) - thr[t,c])
        layers/pairwise.py:131-133, kernels/src/lut.zig:38-42
  * code[b,t]      = sum_c [m > 0] << c   (NaN margins give 0)
        layers/pairwise.py:134, kernels/src/lut.zig:40-41
  * r*[b,t]        = first argmin_c |m|, a NaN |m| counting as smallest
        (torch.argmin semantics, layers/pairwise.py:138)
"""
from __future__ import annotations

import numpy as np


def margins_f32(x: np.ndarray, anchors: np.ndarray, thresholds: np.ndarray) -> np.ndarray:
    """x [B,I] f32, anchors [T,C,2] int, thresholds [T,C] f32 -> margins [B,T,C] f32."""
    x = np.asarray(x, dtype=np.float32)
    thr = np.asarray(thresholds, dtype=np.float32)
    first = x[:, anchors[..., 0]]
    second = x[:, anchors[..., 1]]
    with np.errstate(invalid="ignore", over="ignore"):
        diff = (first - second).astype(np.float32)
        return (diff - thr[None]).astype(np.float32)


def codes_from_margins(margins: np.ndarray) -> np.ndarray:
    """[B,T,C] f32 -> [B,T] int64 codes, bit c set iff margin > 0."""
    comps = margins.shape[-1]
    with np.errstate(invalid="ignore"):
        bits = (margins > 0).astype(np.int64)
    return (bits << np.arange(comps, dtype=np.int64)).sum(axis=-1)


def route_codes(x: np.ndarray, anchors: np.ndarray, thresholds: np.ndarray) -> np.ndarray:
    return codes_from_margins(margins_f32(x, anchors, thresholds))


def min_margin_index(margins: np.ndarray) -> np.ndarray:
    """First index of the smallest |margin| along the last axis; the first NaN
    wins over any number (torch.argmin propagates NaN)."""
    mag = np.abs(margins)
    nan = np.isnan(mag)
    has_nan = nan.any(axis=-1)
    first_nan = np.argmax(nan, axis=-1)
    filled = np.where(nan, np.inf, mag)
    first_min = np.argmin(filled, axis=-1)  # numpy argmin also keeps the first of ties
    return np.where(has_nan, first_nan, first_min).astype(np.int64)
