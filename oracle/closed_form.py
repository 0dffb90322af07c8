"""Float64 closed forms of PairwiseLinear's gradients. TEST INFRASTRUCTURE ONLY.

An independent second statement of the backward, beside the autograd of the
torch restatement in pairwise_torch.py: the gradients the reference's
autograd produces (layers/pairwise.py:137-200, layers/surrogate.py:9-42),
written out term by term and summed in float64 on the forward's own f32
codes and margins (so both sides route identically):
  grad_lut[t,r,:]  = s * sum_{b: code[b,t] = r} G[b,:]
  D[b,t,c]         = s * sum_o G[b,o] (L[t, code ^ 2^c, o] - L[t, code, o])
  gu[b,t,c]        = D[b,t,c] * surrogate'(m[b,t,c])
  grad_x[b,i]      = sum_{t,c in S} gu[b,t,c] ([i = a_tc] - [i = b'_tc])
  grad_thr[t,c]    = -sum_b [c in S(b,t)] gu[b,t,c]
with S = {r*} (the first argmin_c |m|, layers/pairwise.py:138-140) for the
min-margin STE and S = every comparison for the full STE (168-200), s the
output scale. Used to tell the HIP path's rounding from the f32 oracle's where
long sums cancel; pinned against the oracle's autograd by
tests/test_oracle_math.py.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import routing_np
from .pairwise_torch import surrogate_gradient


def gradients_f64(x: Tensor, anchors: Tensor, thresholds: Tensor, lut: Tensor, grad_out: Tensor, *,
                  min_margin: bool, surrogate: str, output_scale: float) -> tuple[Tensor, Tensor, Tensor]:
    """x [B,I] f32, anchors [T,C,2] int64, thresholds [T,C] f32, lut [T,R,O]
    (the values the path reads), grad_out [B,O] -> (grad_x [B,I],
    grad_thresholds [T,C], grad_lut [T,R,O]), float64."""
    b, i = x.shape
    t, c = thresholds.shape
    rows, o = lut.shape[1], lut.shape[2]
    m = torch.from_numpy(routing_np.margins_f32(x.detach().cpu().numpy(), anchors.cpu().numpy(),
                                                thresholds.detach().cpu().numpy()))      # [B,T,C] f32
    code = torch.from_numpy(routing_np.codes_from_margins(m.numpy()))                      # [B,T]
    L = lut.detach().cpu().double()
    G = grad_out.detach().cpu().double().reshape(b, o) * output_scale
    anc = anchors.cpu()
    grad_lut = torch.zeros(t, rows, o, dtype=torch.float64)
    for k in range(t):
        grad_lut[k].index_add_(0, code[:, k], G)
    grad_x = torch.zeros(b, i, dtype=torch.float64)
    grad_thr = torch.zeros(t, c, dtype=torch.float64)
    tt = torch.arange(t).view(1, t)
    cur = L[tt, code]                                                                      # [B,T,O]
    if min_margin:
        r = torch.from_numpy(routing_np.min_margin_index(m.numpy()))                        # [B,T]
        picks = [(r, m.gather(-1, r.unsqueeze(-1)).squeeze(-1))]
    else:
        picks = [(torch.full((b, t), cc, dtype=torch.long), m[..., cc]) for cc in range(c)]
    for r, u in picks:
        nb = L[tt, code ^ (1 << r)]
        dot = ((nb - cur) * G.view(b, 1, o)).sum(-1)                                        # [B,T]
        gu = dot * surrogate_gradient(u.double(), surrogate)
        grad_x.scatter_add_(1, anc[tt, r, 0], gu)
        grad_x.scatter_add_(1, anc[tt, r, 1], -gu)
        grad_thr.scatter_add_(1, r.t().contiguous(), -gu.t().contiguous())
    return grad_x, grad_thr, grad_lut
