"""Torch restatement of the reference PairwiseLinear `backend="torch"` path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker. The product (`tropnn_amd`) never
imports this module.

It follows the reference op by op so that its float results, autograd graph and
peak memory behave like the reference's torch path:
  * seeded init                 layers/pairwise.py:55-68
  * route (margins, codes)      layers/pairwise.py:127-135
  * chunked gather-sum          layers/pairwise.py:99-125, layers/base.py:37-47
  * min-margin STE              layers/pairwise.py:137-166
  * full STE                    layers/pairwise.py:168-200
  * surrogates + Heaviside STE  layers/surrogate.py:9-42
  * module shell                layers/base.py:64-84, layers/pairwise.py:202-248
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
from torch import Tensor

SURROGATES = ("fast_sigmoid_odd", "izhikevich")


# --------------------------------------------------------------------------
# surrogate gradients (layers/surrogate.py:9-25)
# --------------------------------------------------------------------------
def fast_sigmoid_odd(u: Tensor) -> Tensor:
    """-0.5 * sign(u) / (1 + |u|)^2, evaluated in the reference's op order
    (layers/surrogate.py:16-17): sign, scale, |u|, +1, square, divide."""
    return -0.5 * torch.sign(u) / (1.0 + u.abs()).square()


def izhikevich(u: Tensor) -> Tensor:
    """sign' * 2 * sig(|u|) * (1 - sig(|u|)), sign' = -1 for u > 0 else +1
    (layers/surrogate.py:9-13). No clamp on |u| (the TileLang kernel clamps at
    10, pairwise_tilelang.py:264-265; the torch path is followed here)."""
    sig = torch.sigmoid(u.abs())
    sgn = torch.where(u > 0, -torch.ones_like(u), torch.ones_like(u))
    return sgn * 2.0 * sig * (1.0 - sig)


def surrogate_gradient(u: Tensor, name: str = "fast_sigmoid_odd") -> Tensor:
    """Dispatch by name; unknown names raise ValueError (surrogate.py:20-25)."""
    if name == "fast_sigmoid_odd":
        return fast_sigmoid_odd(u)
    if name == "izhikevich":
        return izhikevich(u)
    raise ValueError(f"unsupported surrogate {name!r}")


class _HeavisideSTE(torch.autograd.Function):
    """Forward [u > 0] in u's dtype; backward g * surrogate(u)
    (layers/surrogate.py:28-38)."""

    @staticmethod
    def forward(ctx, u: Tensor, name: str) -> Tensor:  # type: ignore[override]
        ctx.save_for_backward(u)
        ctx.name = name
        return (u > 0).to(u.dtype)

    @staticmethod
    def backward(ctx, g: Tensor):  # type: ignore[override]
        (u,) = ctx.saved_tensors
        return g * surrogate_gradient(u, ctx.name), None


def heaviside_ste(u: Tensor, name: str = "fast_sigmoid_odd") -> Tensor:
    return _HeavisideSTE.apply(u, name)


# --------------------------------------------------------------------------
# init (layers/pairwise.py:55-68)
# --------------------------------------------------------------------------
def init_params(
    in_features: int, out_features: int, tables: int, comparisons: int, seed: int, lut_init_std: float = 0.02
) -> tuple[Tensor, Tensor, Tensor]:
    """Seeded draw of (anchors int64 [T,C,2], thresholds f32 [T,C], lut f32 [T,2^C,O]).

    Reseeds the *global* torch RNG, then draws one scalar randint per anchor
    endpoint in (table, comparison) order, redrawing the second endpoint while
    it equals the first, then zero thresholds, then randn(T, 2^C, O) * std.
    """
    torch.manual_seed(seed)
    pairs: list[tuple[int, int]] = []
    for _ in range(tables * comparisons):
        first = int(torch.randint(0, in_features, (1,)).item())
        second = int(torch.randint(0, in_features, (1,)).item())
        while second == first:
            second = int(torch.randint(0, in_features, (1,)).item())
        pairs.append((first, second))
    anchors = torch.tensor(pairs, dtype=torch.long).view(tables, comparisons, 2)
    thresholds = torch.zeros(tables, comparisons)
    lut = torch.randn(tables, 1 << comparisons, out_features) * lut_init_std
    return anchors, thresholds, lut


# --------------------------------------------------------------------------
# route (layers/pairwise.py:127-135)
# --------------------------------------------------------------------------
def compute_route(latent: Tensor, anchors: Tensor, thresholds: Tensor) -> tuple[Tensor, Tensor]:
    """latent [B,S,I] -> (indices int64 [B,S,T], margins [B,S,T,C]).

    margin = (x[a] - x[b]) - thr, code = sum_c [margin > 0] * 2^c.
    """
    batch, seq, _ = latent.shape
    tables, comps, _ = anchors.shape
    first = latent[..., anchors[:, :, 0].reshape(-1)].view(batch, seq, tables, comps)
    second = latent[..., anchors[:, :, 1].reshape(-1)].view(batch, seq, tables, comps)
    margins = first - second - thresholds.to(dtype=latent.dtype, device=latent.device)
    weights = (2 ** torch.arange(comps, dtype=torch.long, device=latent.device)).view(1, 1, 1, -1)
    indices = ((margins > 0).to(torch.long) * weights).sum(dim=-1)
    return indices, margins


# --------------------------------------------------------------------------
# chunked gather-sum (layers/base.py:37-47, layers/pairwise.py:99-125)
# --------------------------------------------------------------------------
def route_chunk_size(
    item_count: int, payload_width: int, dtype: torch.dtype, route_count: int, target_bytes: int = 16 * 1024 * 1024
) -> int:
    """Tables per chunk: max(1, min(T, target // (items * width * elem_bytes)))."""
    per_route = item_count * payload_width * torch.finfo(dtype).bits // 8
    return max(1, min(route_count, target_bytes // max(1, per_route)))


def _flat_rows(lut: Tensor, dtype: torch.dtype, device: torch.device) -> Tensor:
    tables, rows, width = lut.shape
    return lut.to(dtype=dtype, device=device).reshape(tables * rows, width)


def lookup_sum(indices: Tensor, lut: Tensor, dtype: torch.dtype) -> Tensor:
    """out[b,s,:] = sum_t lut[t, idx[b,s,t], :], summed chunk by chunk with
    index_select + sum(1) + running add, exactly as the reference."""
    batch, seq, tables = indices.shape
    rows_per_table, width = lut.shape[1], lut.shape[2]
    items = batch * seq
    flat_idx = indices.reshape(items, tables)
    table = _flat_rows(lut, dtype, indices.device)
    chunk = route_chunk_size(items, width, dtype, tables)
    out = torch.zeros(items, width, device=indices.device, dtype=dtype)
    for lo in range(0, tables, chunk):
        hi = min(lo + chunk, tables)
        base = (torch.arange(lo, hi, device=indices.device) * rows_per_table).view(1, -1)
        rows = table.index_select(0, (flat_idx[:, lo:hi] + base).reshape(-1))
        out = out + rows.view(items, hi - lo, width).sum(dim=1)
    return out.view(batch, seq, width)


# --------------------------------------------------------------------------
# STE corrections (value 0, gradient carriers)
# --------------------------------------------------------------------------
def min_margin_select(indices: Tensor, margins: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(r*, u, neighbour): r* = first argmin_c |margin| (NaN counts as
    smallest, torch semantics), u = margin[r*], neighbour = code ^ 2^r*
    (layers/pairwise.py:138-140)."""
    r_star = margins.abs().argmin(dim=-1)
    u = margins.gather(dim=-1, index=r_star.unsqueeze(-1)).squeeze(-1)
    neighbour = indices ^ (2**r_star).long()
    return r_star, u, neighbour


def min_margin_ste(indices: Tensor, margins: Tensor, lut: Tensor, surrogate: str) -> Tensor:
    """corr[b,s,:] = sum_t (H_ste(u) - [u>0]) * (L[t,nb] - L[t,cur])
    (layers/pairwise.py:137-166)."""
    _, u, neighbour = min_margin_select(indices, margins)
    delta = heaviside_ste(u, surrogate) - (u > 0).to(u.dtype)
    batch, seq, tables = indices.shape
    rows_per_table, width = lut.shape[1], lut.shape[2]
    items = batch * seq
    cur_idx = indices.reshape(items, tables)
    nb_idx = neighbour.reshape(items, tables)
    delta = delta.reshape(items, tables, 1).float()
    table = _flat_rows(lut, torch.float32, indices.device)
    chunk = route_chunk_size(items, width, torch.float32, tables)
    corr = torch.zeros(items, width, device=indices.device, dtype=torch.float32)
    for lo in range(0, tables, chunk):
        hi = min(lo + chunk, tables)
        base = (torch.arange(lo, hi, device=indices.device) * rows_per_table).view(1, -1)
        cur = table.index_select(0, (cur_idx[:, lo:hi] + base).reshape(-1)).view(items, hi - lo, width)
        nb = table.index_select(0, (nb_idx[:, lo:hi] + base).reshape(-1)).view(items, hi - lo, width)
        corr = corr + (delta[:, lo:hi] * (nb - cur)).sum(dim=1)
    return corr.view(batch, seq, width)


def full_ste(indices: Tensor, margins: Tensor, lut: Tensor, surrogate: str) -> Tensor:
    """corr[b,s,:] = sum_t sum_c (H_ste(m_c) - [m_c>0]) * (L[t, code^2^c] - L[t,code])
    with an 8 MiB chunk target over width O*(C+1) (layers/pairwise.py:168-200)."""
    batch, seq, tables = indices.shape
    comps = margins.shape[-1]
    rows_per_table, width = lut.shape[1], lut.shape[2]
    items = batch * seq
    powers = 2 ** torch.arange(comps, dtype=torch.long, device=indices.device)
    cur_idx = indices.reshape(items, tables)
    nb_idx = cur_idx.unsqueeze(-1) ^ powers.view(1, 1, -1)
    delta = heaviside_ste(margins, surrogate) - (margins > 0).to(margins.dtype)
    delta = delta.reshape(items, tables, comps, 1).float()
    table = _flat_rows(lut, torch.float32, indices.device)
    chunk = route_chunk_size(items, width * (comps + 1), torch.float32, tables, target_bytes=8 * 1024 * 1024)
    corr = torch.zeros(items, width, device=indices.device, dtype=torch.float32)
    for lo in range(0, tables, chunk):
        hi = min(lo + chunk, tables)
        base = (torch.arange(lo, hi, device=indices.device) * rows_per_table).view(1, -1)
        cur = table.index_select(0, (cur_idx[:, lo:hi] + base).reshape(-1)).view(items, hi - lo, 1, width)
        nb_flat = (nb_idx[:, lo:hi] + base.unsqueeze(-1)).reshape(-1)
        nb = table.index_select(0, nb_flat).view(items, hi - lo, comps, width)
        corr = corr + (delta[:, lo:hi] * (nb - cur)).sum(dim=(1, 2))
    return corr.view(batch, seq, width)


# --------------------------------------------------------------------------
# functional forward of the whole layer
# --------------------------------------------------------------------------
def route_output(
    latent: Tensor,
    anchors: Tensor,
    thresholds: Tensor,
    lut: Tensor,
    *,
    training: bool,
    use_min_margin_ste: bool = True,
    surrogate: str = "fast_sigmoid_odd",
) -> tuple[Tensor, Tensor, Tensor]:
    """(output before scaling, indices, margins) -- the torch branch of
    PairwiseLinear._route_output (layers/pairwise.py:243-248)."""
    indices, margins = compute_route(latent, anchors, thresholds)
    output = lookup_sum(indices, lut, latent.dtype)
    if training and (latent.requires_grad or thresholds.requires_grad):
        ste = min_margin_ste if use_min_margin_ste else full_ste
        output = output + ste(indices, margins, lut, surrogate).to(output.dtype)
    return output, indices, margins


class OraclePairwiseLinear(nn.Module):
    """The reference torch-path module restated: same constructor arguments,
    same state-dict keys (anchors, powers buffers; thresholds, lut
    parameters), same forward shell (layers/base.py:64-84)."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        *,
        tables: int = 16,
        comparisons: int = 4,
        seed: int = 0,
        lut_init_std: float = 0.02,
        use_min_margin_ste: bool = True,
        use_output_scaling: bool = True,
        surrogate: str = "fast_sigmoid_odd",
    ) -> None:
        super().__init__()
        if in_features < 1 or out_features < 1 or tables < 1 or comparisons < 1:
            raise ValueError("in_features, out_features, tables and comparisons must be >= 1")
        surrogate_gradient(torch.zeros((), dtype=torch.float32), surrogate)
        self.in_features = in_features
        self.out_features = out_features
        self.tables = tables
        self.comparisons = comparisons
        self.table_size = 1 << comparisons
        self.use_min_margin_ste = use_min_margin_ste
        self.surrogate = surrogate
        self.output_scale = 1.0 / math.sqrt(tables) if use_output_scaling else 1.0
        anchors, thresholds, lut = init_params(in_features, out_features, tables, comparisons, seed, lut_init_std)
        self.register_buffer("anchors", anchors)
        self.thresholds = nn.Parameter(thresholds)
        self.lut = nn.Parameter(lut)
        self.register_buffer("powers", 2 ** torch.arange(comparisons, dtype=torch.long))
        self._last_indices: Tensor | None = None
        self._last_margins: Tensor | None = None

    def forward(self, x: Tensor) -> Tensor:
        if x.ndim == 2:
            x = x.unsqueeze(1)
        in_dtype = x.dtype
        compute = torch.float32 if x.dtype in (torch.float16, torch.bfloat16) else x.dtype
        latent = x.to(compute)
        out, idx, margins = route_output(
            latent,
            self.anchors,
            self.thresholds,
            self.lut,
            training=self.training,
            use_min_margin_ste=self.use_min_margin_ste,
            surrogate=self.surrogate,
        )
        if self.output_scale != 1.0:
            out = out * self.output_scale
        self._last_indices = idx.detach()
        self._last_margins = margins.detach()
        return out.to(dtype=in_dtype)
