"""Wide inputs and many tables: shapes whose input row, or whose gu slots and
inverse anchor index, do not fit one workgroup's LDS.

* An input row past the forward's LDS budget (in_features above ~16,000 at
  these table counts): the one-item forward reads it from global memory.
* An item's gu slots plus the inverse anchor index past 160 KB
  ((3 T C + in_features) words): the input gradient comes from the wide
  scatter kernel, which reads the index and the {gu, r} records (full STE:
  the gu of every comparison) from global memory.
* In between (in_features 20,000 here), the LDS paths with more than the
  default 64 KB of LDS.

Parity against the oracle at the f32 bars of test_gpu_parity (codes bit-exact,
outputs and gradients norm-wise and element-wise), every backward path: the
fused table kernel with its item role or the scatter kernel, the general
path (sort, row, reduce), and the full STE. The reference takes any
in_features (layers/pairwise.py:55-68 draws anchors from [0, in_features)).
"""
from __future__ import annotations

import pytest
import torch

from test_gpu_parity import DEV, F16_TOL, F32_TOL, assert_train_parity, make_pair, rel_err, seeded, train_step

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    yield
    torch.cuda.synchronize()


CASES = [
    # (in, out, tables, comps, batch, lut dtype, ste, input_grad)
    (20000, 64, 24, 6, 300, "f32", {}, "auto"),  # x in global memory; item role with an 80 KB index in LDS
    (20000, 64, 24, 6, 300, "f32", {}, "scatter"),  # the LDS scatter kernel with an 80 KB index
    (50000, 64, 24, 6, 200, "f32", {}, "auto"),  # index past the LDS: fused table kernel + wide scatter
    (50000, 300, 20, 5, 257, "f32", {}, "auto"),  # general path + wide scatter
    (50000, 300, 20, 5, 257, "f16", {}, "auto"),
    (50000, 48, 20, 5, 150, "f32", {"use_min_margin_ste": False}, "auto"),  # full STE + wide scatter (gu of every comparison)
    (64, 32, 3000, 6, 64, "f32", {}, "auto"),  # 18,000 (table, comparison) pairs: wide scatter at a narrow input
    # 13,000 pairs: the full-STE item kernel's own walk with 156 KB of LDS, just inside a workgroup's
    (96, 40, 2600, 5, 48, "f32", {"use_min_margin_ste": False, "surrogate": "izhikevich"}, "auto"),
]


@pytest.mark.parametrize("i,o,t,c,b,lut_dtype,ste,input_grad", CASES)
def test_wide_training_parity(i, o, t, c, b, lut_dtype, ste, input_grad):
    print(f"[wide] i={i} o={o} t={t} c={c} b={b} {lut_dtype} {ste} input_grad={input_grad}", flush=True)
    ref, hip = make_pair(i, o, t, c, seed=7, thr_std=0.25, lut_dtype=lut_dtype, **ste)
    hip.input_grad = input_grad
    x = seeded((b, i), 11)
    g = seeded((b, 1, o), 12)
    if lut_dtype == "f16":
        with torch.no_grad():
            ref.lut.copy_(ref.lut.half().float())  # the values the kernels read
    yx_ref, yx_hip = train_step(ref, hip, x, g)
    assert_train_parity(ref, hip, yx_ref, yx_hip, tol=F32_TOL)
    # every input feature that no anchor names has a zero gradient
    named = torch.zeros(i, dtype=torch.bool)
    named[ref.anchors.reshape(-1)] = True
    assert torch.count_nonzero(yx_hip[1].grad.cpu()[:, ~named]) == 0


@pytest.mark.parametrize("i,b", [(40000, 5), (100000, 3)])
def test_wide_eval_forward(i, b):
    """Eval forward of a wide input (x read from global memory), f32 and f16
    LUT reads, against the oracle; codes bit-exact."""
    print(f"[wide eval] i={i} b={b}", flush=True)
    for lut_dtype, tol in (("f32", F32_TOL), ("f16", F16_TOL)):
        ref, hip = make_pair(i, 96, 40, 6, seed=3, thr_std=0.2, lut_dtype=lut_dtype)
        x = seeded((b, i), 5)
        ref.eval()
        hip.eval()
        with torch.no_grad():
            y_ref = ref(x)
            y_hip = hip(x.to(DEV))
        assert torch.equal(hip._last_indices.cpu(), ref._last_indices)
        assert rel_err(y_hip, y_ref) <= tol
