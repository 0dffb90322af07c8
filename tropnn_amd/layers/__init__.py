from .base import RoutedLinearBase
from .pairwise import PairwiseLinear

__all__ = ["RoutedLinearBase", "PairwiseLinear"]
