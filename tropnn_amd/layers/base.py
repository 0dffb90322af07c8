"""Shell shared by routed layers: input shaping, compute dtype, output scale,
route-debug caching. Same contract as the reference's RoutedLinearBase
(layers/base.py:13-84), with one addition: a subclass whose backend already
applied the output scale inside its kernel sets `fuses_output_scale = True`
and the shell does not scale a second time.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Optional

import torch
import torch.nn as nn
from torch import Tensor

from ..backend import Backend


class RoutedLinearBase(nn.Module, ABC):
    fuses_output_scale = False

    def __init__(self, in_features: int, out_features: int, *, backend: Backend = "hip", output_scale: float = 1.0) -> None:
        super().__init__()
        if in_features < 1:
            raise ValueError(f"in_features must be >= 1, got {in_features}")
        if out_features < 1:
            raise ValueError(f"out_features must be >= 1, got {out_features}")
        self.in_features = in_features
        self.out_features = out_features
        self.backend = backend
        self.output_scale = output_scale
        self._last_indices: Optional[Tensor] = None
        self._last_margins: Optional[Tensor] = None

    def _compute_dtype(self, x: Tensor) -> torch.dtype:
        """f16 / bf16 inputs are computed in f32 (layers/base.py:34-35)."""
        return torch.float32 if x.dtype in {torch.float16, torch.bfloat16} else x.dtype

    @abstractmethod
    def _project_input(self, x: Tensor, compute_dtype: torch.dtype) -> Tensor:
        """Map the input to the latent the router compares."""

    @abstractmethod
    def _route_output(
        self, latent: Tensor, *, input_device: torch.device, compute_dtype: torch.dtype, training: bool
    ) -> tuple[Tensor, Tensor, Tensor]:
        """Return (output, discrete route indices, route margins)."""

    def forward(self, x: Tensor) -> Tensor:
        """[B,I] or [B,S,I] -> [B,S,O] in x's dtype (layers/base.py:64-84)."""
        if x.ndim == 2:
            x = x.unsqueeze(1)
        input_dtype = x.dtype
        compute_dtype = self._compute_dtype(x)
        latent = self._project_input(x, compute_dtype)
        output, indices, margins = self._route_output(
            latent, input_device=x.device, compute_dtype=compute_dtype, training=self.training
        )
        if self.output_scale != 1.0 and not self.fuses_output_scale:
            output = output * self.output_scale
        if getattr(self, "cache_route_debug", True):
            self._last_indices = indices.detach()
            self._last_margins = margins.detach()
        else:
            self._last_indices = None
            self._last_margins = None
        return output.to(dtype=input_dtype)
