"""ctypes wrapper for oracle/liblut_cpu.so. TEST INFRASTRUCTURE ONLY.

The library is the C restatement of the reference's Zig CPU forward
(kernels/src/lut.zig:248-318). The wrapper mirrors the reference's Python
side (backends/pairwise_zig.py:35-103, backends/zig_runtime.py:134-164):
float32 inputs, int64 anchors, f32 or f16 weights, caller-owned output,
process-global thread count set before each call.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading
from pathlib import Path

import torch
from torch import Tensor

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liblut_cpu.so"
_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None


def build() -> Path:
    """Compile liblut_cpu.so with the Makefile next to this file."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not _LIB_PATH.exists():
                raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C {_HERE}`")
            lib = ctypes.CDLL(str(_LIB_PATH))
            sz, p = ctypes.c_size_t, ctypes.c_void_p
            for name in ("lut_forward_batch_with_offsets_no_cache", "lut_forward_batch_f16_no_cache"):
                fn = getattr(lib, name)
                fn.argtypes = [sz, sz, sz, sz, sz, p, p, p, p, p]
                fn.restype = None
            lib.tropnn_set_num_threads.argtypes = [sz]
            lib.tropnn_set_num_threads.restype = None
            lib.tropnn_get_num_threads.argtypes = []
            lib.tropnn_get_num_threads.restype = sz
            lib.lut_cpu_worker_count.argtypes = [sz, sz]
            lib.lut_cpu_worker_count.restype = sz
            lib.lut_cpu_test_add4_f32.argtypes = [p, p, p, p, p, sz]
            lib.lut_cpu_test_add4_f16.argtypes = [p, p, p, p, p, sz]
            lib.lut_cpu_test_code.argtypes = [p, p, p, sz, sz]
            lib.lut_cpu_test_code.restype = sz
            lib.lut_cpu_test_half_to_float.argtypes = [ctypes.c_uint16]
            lib.lut_cpu_test_half_to_float.restype = ctypes.c_float
            _LIB = lib
    return _LIB


def default_threads() -> int:
    """TROPNN_ZIG_THREADS, else torch's intra-op thread count
    (backends/zig_runtime.py:134-147)."""
    env = os.environ.get("TROPNN_ZIG_THREADS")
    if env:
        return max(0, int(env))
    return max(1, int(torch.get_num_threads()))


def forward(
    latent: Tensor, anchors: Tensor, thresholds: Tensor, lut: Tensor, *, lut_dtype: str = "f32", threads: int | None = None
) -> Tensor:
    """latent [B,S,I] f32 (CPU) -> output [B,S,O] f32 before output scaling."""
    if latent.device.type != "cpu" or latent.dtype != torch.float32:
        raise TypeError("latent must be a float32 CPU tensor")
    if anchors.dtype != torch.long:
        raise TypeError("anchors must be int64")
    if lut_dtype not in ("f32", "f16"):
        raise ValueError(f"lut_dtype must be 'f32' or 'f16', got {lut_dtype!r}")
    batch, seq, in_dim = latent.shape
    tables, comps, _ = anchors.shape
    if thresholds.shape != (tables, comps) or lut.shape[:2] != (tables, 1 << comps):
        raise ValueError("incompatible thresholds / lut shapes")
    out_dim = lut.shape[-1]
    items = batch * seq
    x = latent.reshape(items, in_dim).contiguous()
    anc = anchors.contiguous()
    thr = thresholds.to(torch.float32).contiguous()
    w = lut.contiguous().to(torch.float16 if lut_dtype == "f16" else torch.float32)
    out = torch.empty(items, out_dim, dtype=torch.float32)
    lib = load()
    lib.tropnn_set_num_threads(default_threads() if threads is None else threads)
    fn = lib.lut_forward_batch_f16_no_cache if lut_dtype == "f16" else lib.lut_forward_batch_with_offsets_no_cache
    fn(items, tables, comps, in_dim, out_dim, w.data_ptr(), anc.data_ptr(), thr.data_ptr(), x.data_ptr(), out.data_ptr())
    return out.view(batch, seq, out_dim)
