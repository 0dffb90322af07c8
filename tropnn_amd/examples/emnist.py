"""The pairwise family of the reference's EMNIST classifier on the HIP path.

EmnistPairwiseClassifier mirrors EmnistRoutedClassifier(family="pairwise")
(examples/emnist.py:121-175): a stack of PairwiseLinear layers with no
activation in between, dims [input, hidden x (depth - 1), classes], layer idx
seeded with seed + idx (construction order matters: each init reseeds the
global RNG, layers/pairwise.py:55). The training step is the reference's
_run_epoch body (examples/emnist.py:194-214): zero_grad(set_to_none), logits,
cross_entropy, backward, optimizer step; the reference trains with
AdamW(weight_decay=0) (examples/emnist.py:310), i.e. Adam.

The BASELINE c5 configuration is EmnistPairwiseClassifier(784 -> 128 -> 128
-> 10, depth 3, tables 136, comparisons 6), batch 512, Adam lr 1e-3; there is
no dataset here, so make_c5_batch draws the synthetic EMNIST-like batch
(uniform pixels, ~80 % zeros) from a seeded generator.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from ..layers import PairwiseLinear
from ..losses import unit_gradient


class EmnistPairwiseClassifier(nn.Module):
    def __init__(
        self,
        *,
        input_dim: int = 784,
        hidden_dim: int = 128,
        num_classes: int = 10,
        depth: int = 3,
        comparisons: int = 6,
        pairwise_tables: int = 136,
        seed: int = 0,
        input_grad: str | None = None,
        **layer_kwargs,
    ) -> None:
        """input_grad: PairwiseLinear's input_grad for every layer; None gives
        "auto" to the first layer and "fused" to the layers fed by another
        PairwiseLinear, whose codes concentrate on few LUT rows (in the c5
        step the fused form saves ~4 us on the second layer's backward)."""
        super().__init__()
        dims = [input_dim]
        if depth == 1:
            dims.append(num_classes)
        else:
            dims.extend([hidden_dim] * (depth - 1))
            dims.append(num_classes)
        self.layers = nn.ModuleList(
            [
                PairwiseLinear(
                    d_in,
                    d_out,
                    tables=pairwise_tables,
                    comparisons=comparisons,
                    seed=seed + idx,
                    input_grad=input_grad if input_grad is not None else ("auto" if idx == 0 else "fused"),
                    **layer_kwargs,
                )
                for idx, (d_in, d_out) in enumerate(zip(dims[:-1], dims[1:]))
            ]
        )

    def forward(self, x: Tensor) -> Tensor:
        if x.ndim == 2:
            x = x.unsqueeze(1)
        for layer in self.layers:
            x = layer(x)
        return x.squeeze(1)


def make_c5_batch(batch: int = 512, input_dim: int = 784, num_classes: int = 10, seed: int = 0) -> tuple[Tensor, Tensor]:
    """x = rand * (rand >= 0.8) (about 80 % exact zeros, as EMNIST pixels),
    labels = randint(0, classes), from one CPU generator seeded with `seed`."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.rand(batch, input_dim, generator=gen) * (torch.rand(batch, input_dim, generator=gen) >= 0.8)
    y = torch.randint(0, num_classes, (batch,), generator=gen)
    return x, y


def train_step(model: nn.Module, optimizer: torch.optim.Optimizer, x: Tensor, y: Tensor, loss_fn=F.cross_entropy) -> Tensor:
    """One step of the reference's training loop (examples/emnist.py:218-224);
    returns the loss tensor. loss_fn defaults to the reference's
    F.cross_entropy; tropnn_amd.cross_entropy is its one-launch HIP form. The
    backward starts from the kept unit gradient (loss.backward() computes the
    same): no fill launch for d loss / d loss, and none for scaling
    tropnn_amd.cross_entropy's logits gradient."""
    optimizer.zero_grad(set_to_none=True)
    logits = model(x)
    loss = loss_fn(logits, y)
    loss.backward(unit_gradient(loss))
    optimizer.step()
    return loss
