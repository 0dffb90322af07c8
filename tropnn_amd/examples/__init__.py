"""Callers of the PairwiseLinear path: the pairwise family of the reference's
EMNIST classifier (examples/emnist.py)."""
from .emnist import EmnistPairwiseClassifier, make_c5_batch, train_step

__all__ = ["EmnistPairwiseClassifier", "make_c5_batch", "train_step"]
