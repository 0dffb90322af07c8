"""Host-side behaviour of the module and the backend wrapper without a GPU:
constructor validation and state layout as the reference
(layers/pairwise.py:33-68), errors for CPU tensors / missing GPU / missing
library (backends/pairwise_tilelang.py:421-436), and bench.py's one-GPU guard."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest
import torch

from oracle import pairwise_torch as orc
from tropnn_amd import PairwiseLinear, pairwise_hip
import importlib

ph = importlib.import_module("tropnn_amd.backends.pairwise_hip")

ROOT = Path(__file__).resolve().parent.parent


def test_constructor_validation():
    with pytest.raises(ValueError, match="tables"):
        PairwiseLinear(8, 5, tables=0)
    with pytest.raises(ValueError, match="comparisons"):
        PairwiseLinear(8, 5, comparisons=0)
    with pytest.raises(ValueError, match="reference"):
        PairwiseLinear(8, 5, backend="torch")
    with pytest.raises(ValueError, match="backend='hip'"):
        PairwiseLinear(8, 5, backend="cuda")
    with pytest.raises(ValueError, match="unsupported surrogate"):
        PairwiseLinear(8, 5, surrogate="relu")
    with pytest.raises(ValueError, match="cpu_lut_dtype"):
        PairwiseLinear(8, 5, cpu_lut_dtype="f64")
    with pytest.raises(ValueError, match="device_lut_dtype"):
        PairwiseLinear(8, 5, device_lut_dtype="bf16")
    with pytest.raises(ValueError, match="in_features"):
        PairwiseLinear(0, 5)


def test_state_dict_layout_matches_reference_module():
    kw = dict(tables=7, comparisons=5, seed=3)
    ref = orc.OraclePairwiseLinear(16, 9, **kw)
    prod = PairwiseLinear(16, 9, **kw)
    rs, ps = ref.state_dict(), prod.state_dict()
    assert list(rs) == list(ps) or set(rs) == set(ps)
    for k in rs:
        assert rs[k].dtype == ps[k].dtype and rs[k].shape == ps[k].shape, k
        assert torch.equal(rs[k], ps[k]), k
    assert prod.output_scale == ref.output_scale
    prod.load_state_dict(rs)


def test_cpu_tensors_are_rejected():
    layer = PairwiseLinear(8, 5, tables=3, comparisons=3)
    if torch.cuda.is_available():
        with pytest.raises(ValueError, match="GPU"):
            layer(torch.randn(4, 8))
    else:
        with pytest.raises((ValueError, RuntimeError)):
            layer(torch.randn(4, 8))


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_no_gpu_raises_runtime_error():
    anchors = torch.zeros(3, 3, 2, dtype=torch.long)
    with pytest.raises(RuntimeError, match="GPU"):
        pairwise_hip(torch.randn(2, 1, 8), anchors, torch.zeros(3, 3), torch.zeros(3, 8, 5))
    assert ph.has_pairwise_hip() is False


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(ph, "_LIB", None)
    monkeypatch.setenv("TROPNN_HIP_LIB", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="not built"):
        ph.load_library()
    bogus = tmp_path / "bogus.so"
    bogus.write_bytes(b"not an ELF file")
    monkeypatch.setenv("TROPNN_HIP_LIB", str(bogus))
    with pytest.raises(RuntimeError, match="cannot load"):
        ph.load_library()


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
    assert proc.stdout == ""
