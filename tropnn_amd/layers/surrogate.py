"""Surrogate-gradient names accepted by PairwiseLinear (layers/surrogate.py:9-25).

The HIP kernels evaluate the surrogate on the device; this module only holds
the host-side name check the constructor runs (layers/pairwise.py:42), with
the reference's error for an unknown name.
"""
from __future__ import annotations

SURROGATES = ("fast_sigmoid_odd", "izhikevich")


def check_surrogate(name: str) -> str:
    """Return `name` if the reference knows it, else raise ValueError like
    surrogate_gradient does (layers/surrogate.py:20-25)."""
    if name not in SURROGATES:
        raise ValueError(f"unsupported surrogate {name!r}")
    return name
