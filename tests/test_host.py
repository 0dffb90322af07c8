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


def test_route_debug_mode_is_validated():
    layer = PairwiseLinear(8, 5, tables=3, comparisons=2)
    layer.cache_route_debug = "codes"
    with pytest.raises(ValueError, match="cache_route_debug"):
        layer(torch.zeros(2, 8))


def test_lazy_route_debug_materialises_once():
    """The lazy record widens uint8 codes to int64 on first access and calls
    the margin recomputation exactly once."""
    from tropnn_amd.layers.base import RouteDebug

    calls = []

    def recompute():
        calls.append(1)
        return torch.full((2, 1, 3, 2), 0.5)

    codes = torch.tensor([[[0, 3, 255]], [[1, 2, 128]]], dtype=torch.uint8)
    rec = RouteDebug(codes=codes, recompute_margins=recompute)
    assert rec.codes is codes and not calls
    idx = rec.indices
    assert idx.dtype == torch.int64 and idx.tolist() == codes.long().tolist()
    assert rec.indices is idx
    m1, m2 = rec.margins, rec.margins
    assert m1 is m2 and len(calls) == 1
    eager = RouteDebug(indices=idx, margins=m1)
    assert torch.equal(eager.codes, codes) and eager.margins is m1


def test_route_debug_attributes_are_settable():
    """The reference shell assigns _last_indices / _last_margins directly
    (layers/base.py:78-83); the properties accept that."""
    layer = PairwiseLinear(8, 5, tables=3, comparisons=2)
    idx = torch.zeros(2, 1, 3, dtype=torch.long)
    layer._last_indices = idx
    layer._last_margins = torch.ones(2, 1, 3, 2)
    assert layer._last_indices is idx and float(layer._last_margins.sum()) == 12.0
    layer._last_indices = None
    layer._last_margins = None
    assert layer._last_indices is None and layer._last_margins is None and layer._last_codes is None


def test_committed_counter_profiles_match_the_kernel_sources():
    """bench.py takes each kernel's HBM bytes and L2 hit rate from the
    committed rocprofv3 summaries (profiles/traffic*.json) only while the
    kernel sources, comments aside, hash to the digest the profile was made
    from; otherwise its roofline falls back to compulsory bytes. A kernel
    change committed without new counter passes shows up here rather than as
    a silently weaker bench line."""
    root = Path(__file__).resolve().parents[1]
    sys.path.insert(0, str(root))
    import json

    import bench

    digest = bench.source_digest()
    for name in ("traffic.json", "traffic_c1.json", "traffic_c3.json", "traffic_c4.json"):
        rec = json.loads((root / "profiles" / name).read_text())
        assert rec["source_digest"] == digest, f"profiles/{name} was made from other kernel sources"
        assert rec["kernels"], name
        for kernel, k in rec["kernels"].items():
            assert k["fetch_bytes"] > 0 and k["write_bytes"] >= 0, (name, kernel)
    for md in (root / "profiles").glob("c[1-5]_*.md"):
        assert digest in md.read_text(), f"{md.name} names another digest of the kernel sources"
