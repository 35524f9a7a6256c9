"""Pure-PyTorch 2D multi-scale deformable attention (reference src/msda_triton/pytorch/msda_2d.py)."""

from __future__ import annotations

import torch

from ._grid import grid_sample_msda


def msda2d_pytorch(
    value: torch.Tensor,
    value_spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    clamp_grid: bool = True,
    clamp_eps: float = 1e-4,
) -> torch.Tensor:
    """2D MSDA with torch.nn.functional.grid_sample (reference pytorch/msda_2d.py:23-114).

    Args:
        value: (B, K, H, C), K = sum of H_l*W_l.
        value_spatial_shapes: (L, 2) as (H, W).
        sampling_locations: (B, Q, H, L, P, 2) as (x, y) in [0, 1].
        attention_weights: (B, Q, H, L, P).
        clamp_grid: clamp the [-1, 1] grid to [-1+eps, 1-eps].
        clamp_eps: the eps above.

    Returns:
        (B, Q, H*C) in value's dtype (accumulated in value's dtype).
    """
    return grid_sample_msda(value, value_spatial_shapes, sampling_locations, attention_weights,
                            clamp_grid, clamp_eps)


__all__ = ["msda2d_pytorch"]


# the attention module, at the reference's import path (pytorch/msda_2d.py)
from msda_triton.modules import MSDA2D  # noqa: E402
