"""Backend names and capability probe (backend.py:8, 15-42 of the reference).

The reference's Backend literal is ("auto", "torch", "triton", "tilelang",
"zig"); this package adds "hip", the only backend it implements.
"""
from __future__ import annotations

from typing import Literal

Backend = Literal["auto", "torch", "triton", "tilelang", "zig", "hip"]
REFERENCE_BACKENDS = ("auto", "torch", "triton", "tilelang", "zig")


def has_pairwise_hip() -> bool:
    """True when libtropnn_hip.so loads and a GPU is visible."""
    from .backends.pairwise_hip import has_pairwise_hip as _probe

    return _probe()
