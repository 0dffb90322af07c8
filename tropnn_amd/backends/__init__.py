from .pairwise_hip import has_pairwise_hip, pairwise_hip, pairwise_hip_forward, pairwise_hip_route

__all__ = ["has_pairwise_hip", "pairwise_hip", "pairwise_hip_forward", "pairwise_hip_route"]
