"""2D (bilinear) multi-scale deformable attention on the gfx950 HIP kernels.

Drop-in for the reference's src/msda_triton/triton/msda_2d.py: same names
(``msda2d``, ``msda2d_fwd``, ``MSDA2DFn``), signatures, defaults, tensor contract and
error behaviour. value (B, K, H, C); value_spatial_shapes (L, 2) as (H, W);
sampling_locations (B, Q, H, L, P, 2) as (x, y) in [0, 1]; attention_weights
(B, Q, H, L, P) -> (B, Q, H*C) in value's dtype, accumulated in fp32.
"""

from __future__ import annotations

import torch

from . import _core, ops

_NAME = "MSDA2D"
_DIM = 2


def msda2d_fwd(
    value: torch.Tensor,
    value_spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    clamp_grid: bool = True,
    clamp_eps: float = 1e-4,
) -> torch.Tensor:
    """Forward-only MSDA2D without autograd (reference triton/msda_2d.py:654-718).

    Raises:
        ValueError: inputs not on the GPU, or shape mismatch.
        NotImplementedError: value dtype other than fp32, fp16, bf16.
    """
    if torch.compiler.is_compiling():  # an opaque custom op instead of a graph break
        with torch.no_grad():
            return ops.msda_fwd(value, value_spatial_shapes, sampling_locations, attention_weights,
                                _DIM, clamp_grid, clamp_eps)
    return _core.run_fwd(_NAME, _DIM, value, value_spatial_shapes, sampling_locations,
                         attention_weights, clamp_grid, clamp_eps)


class MSDA2DFn(torch.autograd.Function):
    """Autograd function for MSDA2D (reference triton/msda_2d.py:721-853).

    Saves the contiguous inputs and the device level tables; backward runs one fused HIP
    kernel for all three gradients.
    """

    @staticmethod
    def forward(ctx, value, value_spatial_shapes, sampling_locations, attention_weights,
                clamp_grid=True, clamp_eps=1e-4):
        return _core.fn_forward(ctx, _NAME, _DIM, value, value_spatial_shapes,
                                sampling_locations, attention_weights, clamp_grid, clamp_eps)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_output):
        return _core.fn_backward(ctx, _DIM, grad_output)


def msda2d(
    value: torch.Tensor,
    value_spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    clamp_grid: bool = True,
    clamp_eps: float = 1e-4,
) -> torch.Tensor:
    """MSDA2D with autograd; the primary training entry (reference triton/msda_2d.py:856-907).

    Raises:
        ValueError: If inputs are not GPU tensors.
    """
    if not value.is_cuda:
        raise ValueError(f"{_NAME} HIP kernel requires CUDA tensors. Got CPU tensors instead.")
    if torch.compiler.is_compiling():  # differentiable custom op (msda_triton::msda_fwd)
        return ops.msda_fwd(value, value_spatial_shapes, sampling_locations, attention_weights,
                            _DIM, clamp_grid, clamp_eps)
    return MSDA2DFn.apply(value, value_spatial_shapes, sampling_locations, attention_weights,
                          clamp_grid, clamp_eps)


__all__ = ["msda2d", "msda2d_fwd", "MSDA2DFn"]
