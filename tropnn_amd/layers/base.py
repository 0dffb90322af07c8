"""Shell shared by routed layers: input shaping, compute dtype, output scale,
route-debug caching. Same contract as the reference's RoutedLinearBase
(layers/base.py:13-84), with two additions:
  * a subclass whose backend already applied the output scale inside its
    kernel sets `fuses_output_scale = True` and the shell does not scale a
    second time;
  * `cache_route_debug` takes True (the reference's behaviour: int64
    `_last_indices` and f32 `_last_margins` written by every call), False
    (neither is kept) or "lazy": the call writes only uint8 codes [B,S,T]
    (`_last_codes`), `_last_indices` widens them on first access and
    `_last_margins` is recomputed on first access by the subclass's
    `_recompute_margins`, which raises if the inputs it reads have been
    modified in place since the call.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Callable, Optional

import torch
import torch.nn as nn
from torch import Tensor

from ..backend import Backend

ROUTE_DEBUG_MODES = (True, False, "lazy")


class RouteDebug:
    """Route-debug tensors of one call. Eager: int64 indices and f32 margins
    as the call wrote them. Lazy: the call's uint8 codes; indices and margins
    are materialised on first access and then kept."""

    def __init__(
        self,
        *,
        indices: Optional[Tensor] = None,
        margins: Optional[Tensor] = None,
        codes: Optional[Tensor] = None,
        recompute_margins: Optional[Callable[[], Tensor]] = None,
    ) -> None:
        self._indices = indices
        self._margins = margins
        self._codes = codes
        self._recompute_margins = recompute_margins

    @property
    def codes(self) -> Optional[Tensor]:
        if self._codes is None and self._indices is not None and self._indices.numel() > 0:
            self._codes = self._indices.to(torch.uint8)
        return self._codes

    @property
    def indices(self) -> Optional[Tensor]:
        if self._indices is None and self._codes is not None:
            self._indices = self._codes.to(torch.int64)
        return self._indices

    @property
    def margins(self) -> Optional[Tensor]:
        if self._margins is None and self._recompute_margins is not None:
            self._margins = self._recompute_margins()
            self._recompute_margins = None
        return self._margins


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
        self._route_debug: Optional[RouteDebug] = None

    @property
    def _last_indices(self) -> Optional[Tensor]:
        """[B,S,T] int64 route codes of the last call (None if not kept)."""
        return None if self._route_debug is None else self._route_debug.indices

    @_last_indices.setter
    def _last_indices(self, value: Optional[Tensor]) -> None:
        margins = None if self._route_debug is None else self._route_debug._margins
        self._route_debug = None if value is None and margins is None else RouteDebug(indices=value, margins=margins)

    @property
    def _last_margins(self) -> Optional[Tensor]:
        """[B,S,T,C] f32 route margins of the last call (None if not kept)."""
        return None if self._route_debug is None else self._route_debug.margins

    @_last_margins.setter
    def _last_margins(self, value: Optional[Tensor]) -> None:
        indices = None if self._route_debug is None else self._route_debug._indices
        self._route_debug = None if value is None and indices is None else RouteDebug(indices=indices, margins=value)

    @property
    def _last_codes(self) -> Optional[Tensor]:
        """[B,S,T] uint8 route codes of the last call (None if not kept)."""
        return None if self._route_debug is None else self._route_debug.codes

    def _recompute_margins(self, latent: Tensor) -> Callable[[], Tensor]:
        """Return a callable computing the margins of a call on `latent`,
        for cache_route_debug="lazy"; subclasses that support it override."""
        raise NotImplementedError(f"{type(self).__name__} does not support cache_route_debug='lazy'")

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
        mode = getattr(self, "cache_route_debug", True)
        if mode not in ROUTE_DEBUG_MODES:
            raise ValueError(f"cache_route_debug must be True, False or 'lazy', got {mode!r}")
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
        if mode == "lazy":
            # `indices` holds the uint8 codes in this mode
            self._route_debug = RouteDebug(codes=indices.detach(), recompute_margins=self._recompute_margins(latent))
        elif mode:
            self._route_debug = RouteDebug(indices=indices.detach(), margins=margins.detach())
        elif self._route_debug is not None:  # nn.Module.__setattr__ only when it changes
            self._route_debug = None
        return output if output.dtype == input_dtype else output.to(dtype=input_dtype)
