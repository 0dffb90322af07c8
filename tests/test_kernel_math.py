"""CPU checks of arithmetic shortcuts inside the HIP kernels, in float32 as
the GPU computes them (round-to-nearest-even products and sums, truncating
float -> int conversion)."""
from __future__ import annotations

import numpy as np


def test_small_div_is_exact():
    """device.hpp small_div: floor(x / d) == int((float(x) + 0.5f) * (1.0f / d))
    for every 0 <= x < 2^21, at the divisors the kernels use (row-group
    range lengths) and a spread of larger ones."""
    x = np.arange(1 << 21, dtype=np.int64)
    xf = x.astype(np.float32) + np.float32(0.5)
    for d in list(range(1, 65)) + [97, 127, 128, 255, 256, 1000, 1023, 1024, 4095, 65535]:
        inv = np.float32(1.0) / np.float32(d)
        q = (xf * inv).astype(np.int64)  # truncation, as v_cvt_i32_f32
        np.testing.assert_array_equal(q, x // d, err_msg=f"d={d}")
