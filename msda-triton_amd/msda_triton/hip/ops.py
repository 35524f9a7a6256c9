"""torch.library custom ops for the HIP path, so msda2d / msda3d trace under torch.compile.

The reference marks its forward entries @torch.compiler.disable (triton/msda_2d.py:586,
:654), which splits a compiled graph at every call. These ops give the compiler an opaque
node with a shape function instead:

  msda_triton::msda_fwd(value, spatial_shapes, loc, attn, dim, clamp_grid, clamp_eps) -> out
  msda_triton::msda_bwd(grad_out, value, spatial_shapes, loc, attn, dim, clamp_grid,
                        clamp_eps) -> (grad_value, grad_loc, grad_attn)

  msda_triton::msda_fwd_fused(value, spatial_shapes, reference_points, sampling_offsets,
                              attention_logits, dim, clamp_grid, clamp_eps) -> out
  msda_triton::msda_bwd_fused(grad_out, value, spatial_shapes, reference_points,
                              sampling_offsets, attention_logits, dim, clamp_grid,
                              clamp_eps) -> (grad_value, grad_ref, grad_off, grad_logits)

msda_fwd (msda_fwd_fused) is differentiable through msda_bwd (msda_bwd_fused). They run the
same host code and kernels as the eager entry points (validation, level tables, C ABI),
and return fresh tensors in the input dtypes. The public functions use them only while
compiling; eager calls keep the autograd.Function paths.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _core, fused

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


@torch.library.custom_op("msda_triton::msda_fwd_fused", mutates_args=())
def msda_fwd_fused(value: Tensor, value_spatial_shapes: Tensor, reference_points: Tensor,
                   sampling_offsets: Tensor, attention_logits: Tensor, dim: int, clamp_grid: bool,
                   clamp_eps: float) -> Tensor:
    return fused.fused_forward_only(dim, value, value_spatial_shapes, reference_points,
                                    sampling_offsets, attention_logits, clamp_grid, clamp_eps)


@msda_fwd_fused.register_fake
def _msda_fwd_fused_fake(value, value_spatial_shapes, reference_points, sampling_offsets,
                         attention_logits, dim, clamp_grid, clamp_eps):
    bsz, _, num_heads, ch = value.shape
    return value.new_empty((bsz, sampling_offsets.shape[1], num_heads * ch))


@torch.library.custom_op("msda_triton::msda_bwd_fused", mutates_args=())
def msda_bwd_fused(grad_output: Tensor, value: Tensor, value_spatial_shapes: Tensor,
                   reference_points: Tensor, sampling_offsets: Tensor, attention_logits: Tensor,
                   dim: int, clamp_grid: bool, clamp_eps: float
                   ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    logits, ref = fused.validate_fused_inputs(fused._NAMES[dim], dim, value, value_spatial_shapes,
                                              reference_points, sampling_offsets, attention_logits)
    levels = _core.prepare_levels(dim, value, value_spatial_shapes)
    cdt = _core.coord_dtype(value, sampling_offsets, logits)
    value_c = _core._aligned(value.contiguous())
    ref_c = ref.to(dtype=torch.float32).contiguous()
    off_c = _core._aligned(sampling_offsets.to(dtype=cdt).contiguous())
    logits_c = _core._aligned(logits.to(dtype=cdt).contiguous())
    gv, gr, go, gl = fused.backward(dim, grad_output, value_c, levels, ref_c, off_c, logits_c,
                                    clamp_grid, clamp_eps)
    if reference_points.shape[2] == 1 and gr.shape[2] != 1:
        gr = gr.sum(dim=2, keepdim=True)
    return (gv.to(value.dtype), gr.to(reference_points.dtype), go.to(sampling_offsets.dtype),
            gl.to(attention_logits.dtype).reshape(attention_logits.shape))


@msda_bwd_fused.register_fake
def _msda_bwd_fused_fake(grad_output, value, value_spatial_shapes, reference_points,
                         sampling_offsets, attention_logits, dim, clamp_grid, clamp_eps):
    cf = torch.contiguous_format
    return (torch.empty_like(value, memory_format=cf),
            torch.empty_like(reference_points, memory_format=cf),
            torch.empty_like(sampling_offsets, memory_format=cf),
            torch.empty_like(attention_logits, memory_format=cf))


def _setup_context_fused(ctx, inputs, output):
    value, shapes, ref, off, logits, dim, clamp_grid, clamp_eps = inputs
    ctx.save_for_backward(value, shapes, ref, off, logits)
    ctx.dim, ctx.clamp_grid, ctx.clamp_eps = dim, clamp_grid, clamp_eps


def _backward_fused(ctx, grad_output):
    value, shapes, ref, off, logits = ctx.saved_tensors
    gv, gr, go, gl = msda_bwd_fused(grad_output.contiguous(), value, shapes, ref, off, logits,
                                    ctx.dim, ctx.clamp_grid, ctx.clamp_eps)
    return gv, None, gr, go, gl, None, None, None


msda_fwd_fused.register_autograd(_backward_fused, setup_context=_setup_context_fused)
