"""Pure-PyTorch 3D multi-scale deformable attention (reference src/msda_triton/pytorch/msda_3d.py)."""

from __future__ import annotations

import torch

from ._grid import grid_sample_msda


def msda3d_pytorch(
    value: torch.Tensor,
    value_spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    clamp_grid: bool = True,
    clamp_eps: float = 1e-4,
) -> torch.Tensor:
    """3D MSDA with torch.nn.functional.grid_sample (reference pytorch/msda_3d.py:23-118).

    Args:
        value: (B, K, H, C), K = sum of D_l*H_l*W_l.
        value_spatial_shapes: (L, 3) as (D, H, W).
        sampling_locations: (B, Q, H, L, P, 3) as (x, y, z) in [0, 1].
        attention_weights: (B, Q, H, L, P).
        clamp_grid: clamp the [-1, 1] grid to [-1+eps, 1-eps].
        clamp_eps: the eps above.

    Returns:
        (B, Q, H*C) in value's dtype (accumulated in value's dtype).
    """
    return grid_sample_msda(value, value_spatial_shapes, sampling_locations, attention_weights,
                            clamp_grid, clamp_eps)


__all__ = ["msda3d_pytorch"]


# the attention module, at the reference's import path (pytorch/msda_3d.py)
from msda_triton.modules import MSDA3D  # noqa: E402
