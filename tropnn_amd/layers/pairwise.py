"""PairwiseLinear on the HIP backend.

Constructor arguments, seeded init and state-dict layout follow the
reference module (layers/pairwise.py:15-68) so checkpoints and seeds
interchange with it; `_route_output` dispatches to the HIP kernels
(the reference's dispatch is layers/pairwise.py:202-248).
"""
from __future__ import annotations

import math
from typing import Callable, Literal

import torch
import torch.nn as nn
from torch import Tensor

from ..backend import REFERENCE_BACKENDS, Backend
from ..backends.pairwise_hip import INPUT_GRAD_FORMS, pairwise_hip, pairwise_hip_route
from .base import RoutedLinearBase
from .surrogate import check_surrogate


class PairwiseLinear(RoutedLinearBase):
    """Pairwise-comparator LUT layer with the min-margin STE.

    Per item b and table t: code[b,t] = sum_c [x[a_tc] - x[b_tc] - thr_tc > 0] * 2^c,
    y[b,:] = s * sum_t lut[t, code[b,t], :] with s = 1/sqrt(tables) when
    use_output_scaling. Training carries the fast_sigmoid_odd STE gradient
    through the comparison with the smallest |margin|.

    Extra arguments beyond the reference's:
      device_lut_dtype  "f32" (default) or "f16": the LUT element type the
                        kernels read. "f16" reads an RNE-rounded copy of the
                        f32 parameter, refreshed whenever the parameter's
                        version changes (in-place torch ops and FusedAdam
                        bump it) and cast afresh by every replay of a forward
                        captured in a HIP graph; gradients still go to the
                        f32 LUT.
      input_grad        "auto" (default), "fused" or "scatter": where the
                        backward forms the input gradient of narrow rows
                        (out_features a multiple of 4 up to 64 or of 8 up
                        to 256), in its first launch or in a kernel after it.
                        "auto" decides by the row width, which is right for
                        inputs whose codes spread over the LUT; "fused" pays
                        where the items' codes concentrate on few rows, as in
                        a layer fed by another PairwiseLinear. Results are
                        bit-identical either way.
    Attribute `cache_route_debug` (default True, as the reference's shell
    assumes) keeps `_last_indices` [B,S,T] int64 and `_last_margins`
    [B,S,T,C] f32 of the last call; False skips writing them; "lazy" writes
    only uint8 codes (`_last_codes`, B*T bytes) and materialises the other
    two on first access, the margins by a route-only launch that reads the
    call's latent, anchors and thresholds (an error if any of them has been
    modified in place since, e.g. by an optimizer step).
    """

    fuses_output_scale = True

    def __init__(
        self,
        in_features: int,
        out_features: int,
        *,
        tables: int = 16,
        comparisons: int = 4,
        backend: Backend = "hip",
        seed: int = 0,
        lut_init_std: float = 0.02,
        use_min_margin_ste: bool = True,
        use_output_scaling: bool = True,
        surrogate: str = "fast_sigmoid_odd",
        cpu_lut_dtype: Literal["f32", "f16"] = "f32",
        device_lut_dtype: Literal["f32", "f16"] = "f32",
        input_grad: Literal["auto", "fused", "scatter"] = "auto",
    ) -> None:
        if tables < 1:
            raise ValueError(f"tables must be >= 1, got {tables}")
        if comparisons < 1:
            raise ValueError(f"comparisons must be >= 1, got {comparisons}")
        if backend != "hip":
            if backend in REFERENCE_BACKENDS:
                raise ValueError(
                    f"backend={backend!r} belongs to the reference tropnn package; this package implements backend='hip'"
                )
            raise ValueError(f"PairwiseLinear supports backend='hip', got {backend!r}")
        if cpu_lut_dtype not in {"f32", "f16"}:
            raise ValueError(f"cpu_lut_dtype must be 'f32' or 'f16', got {cpu_lut_dtype!r}")
        if device_lut_dtype not in {"f32", "f16"}:
            raise ValueError(f"device_lut_dtype must be 'f32' or 'f16', got {device_lut_dtype!r}")
        if input_grad not in INPUT_GRAD_FORMS:
            raise ValueError(f"input_grad must be 'auto', 'fused' or 'scatter', got {input_grad!r}")
        check_surrogate(surrogate)

        output_scale = 1.0 / math.sqrt(tables) if use_output_scaling else 1.0
        super().__init__(in_features, out_features, backend=backend, output_scale=output_scale)
        self.tables = tables
        self.comparisons = comparisons
        self.table_size = 1 << comparisons
        self.use_min_margin_ste = use_min_margin_ste
        self.surrogate = surrogate
        self.cpu_lut_dtype = cpu_lut_dtype
        self.device_lut_dtype = device_lut_dtype
        self.input_grad = input_grad
        self.cache_route_debug = True
        self._lut_f16: Tensor | None = None
        self._lut_f16_key: tuple | None = None

        # Seeded init, same draw sequence as layers/pairwise.py:55-68: reseed
        # the global RNG, one scalar randint per anchor endpoint in (table,
        # comparison) order with the second endpoint redrawn while equal to
        # the first, zero thresholds, then randn(T, 2^C, O) * std.
        torch.manual_seed(seed)
        endpoints = torch.zeros(tables * comparisons, 2, dtype=torch.long)
        for k in range(tables * comparisons):
            a = torch.randint(0, in_features, (1,)).item()
            b = torch.randint(0, in_features, (1,)).item()
            while b == a:
                b = torch.randint(0, in_features, (1,)).item()
            endpoints[k, 0] = a
            endpoints[k, 1] = b
        self.register_buffer("anchors", endpoints.view(tables, comparisons, 2))
        self.thresholds = nn.Parameter(torch.zeros(tables, comparisons))
        self.lut = nn.Parameter(torch.randn(tables, self.table_size, out_features) * lut_init_std)
        self.register_buffer("powers", 2 ** torch.arange(comparisons, dtype=torch.long))

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, tables={self.tables}, "
            f"comparisons={self.comparisons}, backend={self.backend!r}, use_min_margin_ste={self.use_min_margin_ste}, "
            f"surrogate={self.surrogate!r}, device_lut_dtype={self.device_lut_dtype!r}"
            + (f", input_grad={self.input_grad!r}" if getattr(self, "input_grad", "auto") != "auto" else "")
        )

    def _project_input(self, x: Tensor, compute_dtype: torch.dtype) -> Tensor:
        return x if x.dtype == compute_dtype else x.to(compute_dtype)

    def _lut_for_reading(self) -> Tensor:
        """The LUT tensor the kernels read: the f32 parameter, or its f16 copy
        re-rounded whenever the parameter changes (like the Zig f16 cache,
        layers/pairwise.py:82-92)."""
        if self.device_lut_dtype == "f32":
            return self.lut
        if self.lut.is_cuda and torch.cuda.is_current_stream_capturing():
            # A captured forward casts on every replay: an optimizer step
            # replayed in the same graph updates the f32 LUT without running
            # any Python, so no version key could tell that the copy is stale.
            # The graph's copy is not cached for eager calls either.
            self._lut_f16 = None
            self._lut_f16_key = None
            with torch.no_grad():
                return self.lut.detach().to(torch.float16)
        key = (self.lut._version, self.lut.data_ptr(), tuple(self.lut.shape), self.lut.device)
        if self._lut_f16 is None or self._lut_f16_key != key:
            with torch.no_grad():
                self._lut_f16 = self.lut.detach().to(torch.float16).contiguous()
            self._lut_f16_key = key
        return self._lut_f16

    def _route_output(
        self, latent: Tensor, *, input_device: torch.device, compute_dtype: torch.dtype, training: bool
    ) -> tuple[Tensor, Tensor, Tensor]:
        del input_device
        if not latent.is_cuda:
            raise ValueError("PairwiseLinear backend='hip' requires GPU input tensors")
        if compute_dtype != torch.float32:
            raise TypeError(f"PairwiseLinear backend='hip' requires float32 compute dtype, got {compute_dtype}")
        # the STE applies in training only, as in the torch path (layers/pairwise.py:245-247)
        ste = training and (latent.requires_grad or self.thresholds.requires_grad)
        return pairwise_hip(
            latent,
            self.anchors,
            self.thresholds,
            self.lut,
            use_min_margin_ste=self.use_min_margin_ste,
            surrogate=self.surrogate,
            output_scale=self.output_scale,
            lut_read=self._lut_for_reading(),
            ste=ste,
            return_route=self._route_mode(),
            input_grad=getattr(self, "input_grad", "auto"),  # modules pickled before the option
        )

    def _compute_indices(self, latent: Tensor) -> tuple[Tensor, Tensor]:
        """Route only, as the reference's method of this name
        (layers/pairwise.py:127-135): latent [B, S, I] f32 on the GPU ->
        (indices int64 [B, S, T], margins f32 [B, S, T, C]), from the route
        kernel (bit-identical to the forward's codes and margins). The margins
        carry no autograd graph; training goes through forward()."""
        if not latent.is_cuda:
            raise ValueError("PairwiseLinear backend='hip' requires GPU input tensors")
        _, indices, margins = pairwise_hip_route(
            latent, self.anchors, self.thresholds.detach(), codes=False, indices=True, margins=True
        )
        return indices, margins

    def _route_mode(self) -> bool | str:
        mode = getattr(self, "cache_route_debug", True)
        return "codes" if mode == "lazy" else bool(mode)

    def _recompute_margins(self, latent: Tensor) -> Callable[[], Tensor]:
        """Margins of the call on `latent`, computed when first asked for by
        the route-only kernel from the same latent, anchors and thresholds;
        their version counters (bumped by every in-place write) must not have
        moved since the call."""
        inputs = (latent.detach(), self.anchors, self.thresholds.detach())
        versions = tuple(t._version for t in inputs)

        def recompute() -> Tensor:
            if tuple(t._version for t in inputs) != versions:
                raise RuntimeError(
                    "cache_route_debug='lazy': the latent, anchors or thresholds of the last call were modified in "
                    "place since (e.g. by an optimizer step), so its margins can no longer be recomputed; read "
                    "_last_margins before that, or set cache_route_debug=True"
                )
            return pairwise_hip_route(*inputs, codes=False, indices=False, margins=True)[2]

        return recompute
