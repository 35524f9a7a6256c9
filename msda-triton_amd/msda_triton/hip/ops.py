"""torch.library custom ops for the HIP path, so msda2d / msda3d trace under torch.compile.

The reference marks its forward entries @torch.compiler.disable (triton/msda_2d.py:586,
:654), which splits a compiled graph at every call. These ops give the compiler an opaque
node with a shape function instead:

  msda_triton::msda_fwd(value, spatial_shapes, loc, attn, dim, clamp_grid, clamp_eps) -> out
  msda_triton::msda_bwd(grad_out, value, spatial_shapes, loc, attn, dim, clamp_grid,
                        clamp_eps) -> (grad_value, grad_loc, grad_attn)

msda_fwd is differentiable through msda_bwd. Both run the same host code and kernels as the
eager entry points (validation, level tables, C ABI), and return fresh tensors in the
input dtypes. The public functions use them only while compiling; eager calls keep the
autograd.Function path of the reference's API.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _core

_NAMES = {2: "MSDA2D", 3: "MSDA3D"}


@torch.library.custom_op("msda_triton::msda_fwd", mutates_args=())
def msda_fwd(value: Tensor, value_spatial_shapes: Tensor, sampling_locations: Tensor,
             attention_weights: Tensor, dim: int, clamp_grid: bool, clamp_eps: float) -> Tensor:
    return _core.run_fwd(_NAMES[dim], dim, value, value_spatial_shapes, sampling_locations,
                         attention_weights, clamp_grid, clamp_eps)


@msda_fwd.register_fake
def _msda_fwd_fake(value, value_spatial_shapes, sampling_locations, attention_weights, dim,
                   clamp_grid, clamp_eps):
    bsz, _, num_heads, ch = value.shape
    return value.new_empty((bsz, sampling_locations.shape[1], num_heads * ch))


@torch.library.custom_op("msda_triton::msda_bwd", mutates_args=())
def msda_bwd(grad_output: Tensor, value: Tensor, value_spatial_shapes: Tensor,
             sampling_locations: Tensor, attention_weights: Tensor, dim: int, clamp_grid: bool,
             clamp_eps: float) -> tuple[Tensor, Tensor, Tensor]:
    levels = _core.prepare_levels(dim, value, value_spatial_shapes)
    cdt = _core.coord_dtype(value, sampling_locations, attention_weights)
    value_c = _core._aligned(value.contiguous())
    loc_c = _core._aligned(sampling_locations.to(dtype=cdt).contiguous())
    attn_c = _core._aligned(attention_weights.to(dtype=cdt).contiguous())
    gv, gl, ga = _core.backward(dim, grad_output, value_c, levels, loc_c, attn_c, clamp_grid,
                                clamp_eps)
    return (gv.to(value.dtype), gl.to(sampling_locations.dtype),
            ga.to(attention_weights.dtype))


@msda_bwd.register_fake
def _msda_bwd_fake(grad_output, value, value_spatial_shapes, sampling_locations,
                   attention_weights, dim, clamp_grid, clamp_eps):
    return (torch.empty_like(value, memory_format=torch.contiguous_format),
            torch.empty_like(sampling_locations, memory_format=torch.contiguous_format),
            torch.empty_like(attention_weights, memory_format=torch.contiguous_format))


def _setup_context(ctx, inputs, output):
    value, shapes, loc, attn, dim, clamp_grid, clamp_eps = inputs
    ctx.save_for_backward(value, shapes, loc, attn)
    ctx.dim, ctx.clamp_grid, ctx.clamp_eps = dim, clamp_grid, clamp_eps


def _backward(ctx, grad_output):
    value, shapes, loc, attn = ctx.saved_tensors
    gv, gl, ga = msda_bwd(grad_output.contiguous(), value, shapes, loc, attn, ctx.dim,
                          ctx.clamp_grid, ctx.clamp_eps)
    return gv, None, gl, ga, None, None, None


msda_fwd.register_autograd(_backward, setup_context=_setup_context)
