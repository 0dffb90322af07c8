"""The oracle's C restatement of the Zig CPU forward (oracle/lut_cpu.c),
pinned by the Zig sources' own known-answer tests and by the torch oracle.

  * simd.zig:178-218   grouped accumulators handle a length-19 tail (f32, f16)
  * parallel.zig:65-73 worker count for a configured thread count
  * lut.zig:320-325    comparison-hash code
  * exhaustive f16 -> f32 conversion against numpy
  * forward vs the torch oracle: atol 1e-6 (f32), 5e-3 (f16), the bars of
    test_backend_parity.py:221-246; thread counts give identical bits
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import lut_cpu
from oracle import pairwise_torch as orc


@pytest.fixture(scope="module")
def lib():
    lut_cpu.build()
    return lut_cpu.load()


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def test_grouped_accumulate_tails(lib):
    n = 19
    dest = np.ones(n, dtype=np.float32)
    srcs = [np.full(n, v, dtype=np.float32) for v in (2, 3, 4, 5)]
    lib.lut_cpu_test_add4_f32(_ptr(dest), *[_ptr(s) for s in srcs], n)
    assert (dest == 15).all()
    dest = np.ones(n, dtype=np.float32)
    hs = [np.full(n, v, dtype=np.float16).view(np.uint16) for v in (2, 3, 4, 5)]
    lib.lut_cpu_test_add4_f16(_ptr(dest), *[_ptr(s) for s in hs], n)
    assert (dest == 15).all()


def test_worker_count(lib):
    lib.tropnn_set_num_threads(1)
    assert lib.lut_cpu_worker_count(1024, 64) == 1
    lib.tropnn_set_num_threads(4)
    assert lib.lut_cpu_worker_count(1024, 64) == 4
    assert lib.lut_cpu_worker_count(8, 64) == 1
    assert lib.lut_cpu_worker_count(128, 64) == 2
    lib.tropnn_set_num_threads(0)


def test_comparison_code(lib):
    x = np.array([3.0, 1.0, -1.0], dtype=np.float32)
    anchors = np.array([0, 1, 1, 2], dtype=np.uint64)
    offsets = np.array([1.5, 3.0], dtype=np.float32)
    assert lib.lut_cpu_test_code(_ptr(x), _ptr(anchors), _ptr(offsets), 0, 2) == 1


def test_half_conversion_exhaustive(lib):
    bits = np.arange(65536, dtype=np.uint32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([lib.lut_cpu_test_half_to_float(ctypes.c_uint16(int(b))) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype,atol", [("f32", 1e-6), ("f16", 5e-3)])
def test_forward_matches_torch_oracle(lib, dtype, atol):
    for i, o, t, c, seed in [(8, 5, 3, 3, 1), (8, 5, 4, 3, 2), (64, 19, 13, 6, 3), (32, 40, 7, 8, 4)]:
        ref = orc.OraclePairwiseLinear(i, o, tables=t, comparisons=c, seed=seed).eval()
        with torch.no_grad():
            ref.thresholds.copy_(torch.randn(t, c, generator=torch.Generator().manual_seed(seed)) * 0.2)
            x = torch.randn(70, 2, i, generator=torch.Generator().manual_seed(seed + 9))
            want = ref(x) / ref.output_scale
        got = lut_cpu.forward(x, ref.anchors, ref.thresholds.detach(), ref.lut.detach(), lut_dtype=dtype)
        assert torch.allclose(got, want, atol=atol)


def test_thread_counts_are_bit_identical(lib):
    ref = orc.OraclePairwiseLinear(48, 37, tables=22, comparisons=6, seed=5)
    x = torch.randn(300, 1, 48, generator=torch.Generator().manual_seed(1))
    outs = [lut_cpu.forward(x, ref.anchors, ref.thresholds.detach(), ref.lut.detach(), threads=n) for n in (1, 2, 5)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_restatement_is_clean_under_sanitizers(tmp_path):
    """oracle/sanitize_check.c drives both forwards over every loop of the
    restatement (row- and table-major, remainders after the table groups and
    the vector steps, 1 to 8 comparisons, 1 to 8 threads) built with
    AddressSanitizer + UndefinedBehaviorSanitizer, then with
    ThreadSanitizer: any report aborts the run."""
    import shutil
    import subprocess
    from pathlib import Path

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    here = Path(lut_cpu.__file__).resolve().parent
    out = subprocess.run(["make", "-s", "-C", str(here), "sanitize", f"SAN_DIR={tmp_path}"], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.count("sanitize_check ok") == 2
