"""MI355X-native PairwiseLinear: `PairwiseLinear(..., backend="hip")` runs the
comparator route, LUT gather-sum and min-margin STE backward as gfx950 HIP
kernels in libtropnn_hip.so (C ABI: include/tropnn_hip.h)."""
from .backends import has_pairwise_hip, pairwise_hip, pairwise_hip_forward, pairwise_hip_route
from .layers import PairwiseLinear, RoutedLinearBase
from .losses import cross_entropy, unit_gradient
from .optim import FusedAdam, FusedAdamW

__all__ = [
    "FusedAdam",
    "FusedAdamW",
    "PairwiseLinear",
    "RoutedLinearBase",
    "cross_entropy",
    "has_pairwise_hip",
    "pairwise_hip",
    "pairwise_hip_forward",
    "pairwise_hip_route",
    "unit_gradient",
]
