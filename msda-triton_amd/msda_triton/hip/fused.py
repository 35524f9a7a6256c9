"""Fused producer ops: msda2d_fused / msda3d_fused.

The attention modules form the sampling locations and weights before calling the sampling
op (reference src/msda_triton/pytorch/msda_2d.py:303-339, msda_3d.py:314-350):

    loc  = reference_points[:, :, None, :, None, :] + sampling_offsets / (W_l, H_l[, D_l])
    attn = softmax(attention_logits over the flattened L*P axis)

These functions take the reference points, offsets and logits instead and form both inside
the HIP forward kernel (msda_fwd_fused in include/msda.h), in fp32, so neither tensor goes
through memory. The backward (msda_bwd_fused) returns gradients for value, reference points,
offsets and logits.

Shapes: value (B, K, H, C); reference_points (B, Q, L, dim), or (B, Q, 1, dim) shared by all
levels; sampling_offsets (B, Q, H, L, P, dim) in pixels of each level; attention_logits
(B, Q, H, L, P) or (B, Q, H, L*P). Offsets and logits share one floating dtype, the value
dtype or float32; reference points are read as float32.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from . import _core

_NAMES = {2: "MSDA2DFused", 3: "MSDA3DFused"}


def validate_fused_inputs(name: str, dim: int, value: torch.Tensor, value_spatial_shapes,
                          reference_points: torch.Tensor, sampling_offsets: torch.Tensor,
                          attention_logits: torch.Tensor):
    """Checks in the order of validate_inputs; returns the logits as (B, Q, H, L, P) and the
    reference points expanded to (B, Q, L, dim)."""
    if not value.is_cuda:
        raise ValueError(f"{name} HIP kernel requires CUDA tensors. Got CPU tensors instead.")
    if value.dtype not in _core._DTYPE_CODE:
        raise NotImplementedError(
            f"{name} HIP kernel only supports fp32, fp16, and bf16. Got {value.dtype}. "
            "The kernel accumulates in fp32 internally."
        )
    if value.dim() != 4:
        raise ValueError(f"value must be (B, K, H, C), got {tuple(value.shape)}")
    if sampling_offsets.dim() != 6:
        raise ValueError(f"sampling_offsets must be {_core._COORD_NAMES[dim]}, "
                         f"got {tuple(sampling_offsets.shape)}")
    bsz, _, num_heads, _ = value.shape
    bsz_s, nq, nh, nl, npt, last = sampling_offsets.shape
    if not (bsz == bsz_s and num_heads == nh and last == dim):
        raise ValueError(
            f"Shape mismatch: value=(B,K,H,C), sampling_offsets="
            f"{_core._COORD_NAMES[dim].replace(' ', '')}. Got value={tuple(value.shape)}, "
            f"sampling_offsets={tuple(sampling_offsets.shape)}")
    if attention_logits.shape == (bsz, nq, nh, nl * npt):
        attention_logits = attention_logits.reshape(bsz, nq, nh, nl, npt)
    if attention_logits.shape != (bsz, nq, nh, nl, npt):
        raise ValueError("attention_logits must be (B,Q,H,L,P) or (B,Q,H,L*P), got "
                         f"{tuple(attention_logits.shape)}")
    if reference_points.dim() != 4 or reference_points.shape[-1] != dim or \
            reference_points.shape[:2] != (bsz, nq) or reference_points.shape[2] not in (1, nl):
        raise ValueError(f"reference_points must be (B,Q,L,{dim}) or (B,Q,1,{dim}), got "
                         f"{tuple(reference_points.shape)}")
    if value_spatial_shapes.shape != (nl, dim):
        raise ValueError(
            f"value_spatial_shapes must be (L,{dim}), got {tuple(value_spatial_shapes.shape)}. "
            f"num_levels={nl}, expected shape=({nl}, {dim})")
    for tname, t in (("reference_points", reference_points), ("sampling_offsets", sampling_offsets),
                     ("attention_logits", attention_logits)):
        if t.device != value.device:
            raise ValueError(f"{tname} is on {t.device} but value is on {value.device}")
        if not t.is_floating_point():
            raise ValueError(f"{tname} must be a floating-point tensor, got {t.dtype}")
    return attention_logits, reference_points.expand(bsz, nq, nl, dim)


def _desc(dim, value, off, cdt, clamp_grid, clamp_eps):
    return _core.make_desc(dim, value, off, cdt, clamp_grid, clamp_eps)


def forward(dim: int, value, levels, ref, off, logits, clamp_grid, clamp_eps):
    """Launch msda_fwd_fused. Returns (out, value_c, ref_c, off_c, logits_c)."""
    lib = _lib.load()
    cdt = _core.coord_dtype(value, off, logits)
    value_c = _core._aligned(value.contiguous())
    ref_c = ref.to(dtype=torch.float32).contiguous()
    off_c = _core._aligned(off.to(dtype=cdt).contiguous())
    logits_c = _core._aligned(logits.to(dtype=cdt).contiguous())
    bsz, _, num_heads, ch = value.shape
    out = torch.empty((bsz, off.shape[1], num_heads * ch), device=value.device, dtype=value.dtype)
    desc = _desc(dim, value_c, off_c, cdt, clamp_grid, clamp_eps)
    ws_bytes = int(lib.msda_fwd_workspace_bytes(ctypes.byref(desc)))
    ws = torch.empty(ws_bytes, device=value.device, dtype=torch.uint8) if ws_bytes else None
    with _core._on_device(value.device):
        rc = lib.msda_fwd_fused(ctypes.byref(desc), value_c.data_ptr(), levels.spatial.data_ptr(),
                                levels.starts.data_ptr(), ref_c.data_ptr(), off_c.data_ptr(),
                                logits_c.data_ptr(), out.data_ptr(),
                                ws.data_ptr() if ws is not None else None, ws_bytes,
                                _core._stream(value.device))
    _lib.check(rc, "msda_fwd_fused")
    return out, value_c, ref_c, off_c, logits_c


def backward(dim: int, grad_output, value_c, levels, ref_c, off_c, logits_c, clamp_grid,
             clamp_eps):
    """Launch msda_bwd_fused. Returns (grad_value, grad_ref (fp32), grad_off, grad_logits)."""
    lib = _lib.load()
    grad_out = _core._aligned(grad_output.to(dtype=value_c.dtype).contiguous())
    grad_value = torch.empty(value_c.shape, device=value_c.device, dtype=value_c.dtype)
    grad_ref = torch.empty(ref_c.shape, device=ref_c.device, dtype=torch.float32)
    grad_off = torch.empty(off_c.shape, device=off_c.device, dtype=off_c.dtype)
    grad_logits = torch.empty(logits_c.shape, device=logits_c.device, dtype=logits_c.dtype)
    desc = _desc(dim, value_c, off_c, off_c.dtype, clamp_grid, clamp_eps)
    if levels.host is not None:
        name, shapes, entry = "msda_bwd_fused", levels.host.data_ptr(), lib.msda_bwd_fused
        ws_bytes = int(lib.msda_bwd_fused_workspace_bytes(ctypes.byref(desc), shapes))
    else:
        # GPU-resident shapes: planned on the device, no host read of the shapes
        name, shapes, entry = "msda_bwd_fused_dev", levels.spatial.data_ptr(), lib.msda_bwd_fused_dev
        ws_bytes = int(lib.msda_bwd_fused_dev_workspace_bytes(ctypes.byref(desc)))
    if ws_bytes == 0 and _lib.last_error():
        _lib.check(_lib.MSDA_ERR_INVALID, name + "_workspace_bytes")
    ws = torch.empty(max(ws_bytes, 1), device=value_c.device, dtype=torch.uint8)
    with _core._on_device(value_c.device):
        rc = entry(ctypes.byref(desc), shapes, value_c.data_ptr(), ref_c.data_ptr(),
                   off_c.data_ptr(), logits_c.data_ptr(), grad_out.data_ptr(),
                   grad_value.data_ptr(), grad_ref.data_ptr(), grad_off.data_ptr(),
                   grad_logits.data_ptr(), ws.data_ptr(), ws_bytes, _core._stream(value_c.device))
    _lib.check(rc, name)
    return grad_value, grad_ref, grad_off, grad_logits


class MSDAFusedFn(torch.autograd.Function):
    """Autograd of the fused op: value, reference points, offsets and logits get gradients."""

    @staticmethod
    def forward(ctx, dim, value, value_spatial_shapes, reference_points, sampling_offsets,
                attention_logits, clamp_grid=True, clamp_eps=1e-4):
        name = _NAMES[dim]
        logits, ref = validate_fused_inputs(name, dim, value, value_spatial_shapes,
                                            reference_points, sampling_offsets, attention_logits)
        levels = _core.prepare_levels(dim, value, value_spatial_shapes)
        out, value_c, ref_c, off_c, logits_c = forward(dim, value, levels, ref, sampling_offsets,
                                                       logits, clamp_grid, clamp_eps)
        ctx.save_for_backward(value_c, ref_c, off_c, logits_c)
        ctx.dim, ctx.levels = dim, levels
        ctx.clamp_grid, ctx.clamp_eps = clamp_grid, clamp_eps
        ctx.meta = (value.dtype, reference_points.dtype, reference_points.shape,
                    sampling_offsets.dtype, attention_logits.dtype, attention_logits.shape)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        value_c, ref_c, off_c, logits_c = ctx.saved_tensors
        gv, gr, go, gl = backward(ctx.dim, grad_output, value_c, ctx.levels, ref_c, off_c,
                                  logits_c, ctx.clamp_grid, ctx.clamp_eps)
        vdt, rdt, rshape, odt, ldt, lshape = ctx.meta
        if rshape[2] == 1 and gr.shape[2] != 1:
            gr = gr.sum(dim=2, keepdim=True)  # reference points shared by all levels
        return (None, gv.to(vdt), None, gr.to(rdt), go.to(odt), gl.to(ldt).reshape(lshape),
                None, None)


def fused_forward_only(dim, value, value_spatial_shapes, reference_points, sampling_offsets,
                       attention_logits, clamp_grid, clamp_eps) -> torch.Tensor:
    name = _NAMES[dim]
    logits, ref = validate_fused_inputs(name, dim, value, value_spatial_shapes, reference_points,
                                        sampling_offsets, attention_logits)
    levels = _core.prepare_levels(dim, value, value_spatial_shapes)
    out, *_ = forward(dim, value, levels, ref, sampling_offsets, logits, clamp_grid, clamp_eps)
    return out


def _fused(dim, value, shapes, ref, off, logits, clamp_grid, clamp_eps):
    if torch.compiler.is_compiling():  # an opaque custom op instead of a graph break
        from . import ops
        return ops.msda_fwd_fused(value, shapes, ref, off, logits, dim, clamp_grid, clamp_eps)
    return MSDAFusedFn.apply(dim, value, shapes, ref, off, logits, clamp_grid, clamp_eps)


def _fused_fwd(dim, value, shapes, ref, off, logits, clamp_grid, clamp_eps):
    with torch.no_grad():
        if torch.compiler.is_compiling():
            from . import ops
            return ops.msda_fwd_fused(value, shapes, ref, off, logits, dim, clamp_grid, clamp_eps)
        return fused_forward_only(dim, value, shapes, ref, off, logits, clamp_grid, clamp_eps)


def msda2d_fused(value, value_spatial_shapes, reference_points, sampling_offsets,
                 attention_logits, clamp_grid: bool = True, clamp_eps: float = 1e-4):
    """2D MSDA with location and weight formation in the kernel (see the module docstring).
    Differentiable with respect to value, reference_points, sampling_offsets and
    attention_logits. Returns (B, Q, H*C) in value's dtype."""
    return _fused(2, value, value_spatial_shapes, reference_points, sampling_offsets,
                  attention_logits, clamp_grid, clamp_eps)


def msda3d_fused(value, value_spatial_shapes, reference_points, sampling_offsets,
                 attention_logits, clamp_grid: bool = True, clamp_eps: float = 1e-4):
    """3D counterpart of msda2d_fused; spatial shapes are (D, H, W) per level."""
    return _fused(3, value, value_spatial_shapes, reference_points, sampling_offsets,
                  attention_logits, clamp_grid, clamp_eps)


def msda2d_fused_fwd(value, value_spatial_shapes, reference_points, sampling_offsets,
                     attention_logits, clamp_grid: bool = True, clamp_eps: float = 1e-4):
    """Forward-only msda2d_fused (no autograd graph), like msda2d_fwd."""
    return _fused_fwd(2, value, value_spatial_shapes, reference_points, sampling_offsets,
                      attention_logits, clamp_grid, clamp_eps)


def msda3d_fused_fwd(value, value_spatial_shapes, reference_points, sampling_offsets,
                     attention_logits, clamp_grid: bool = True, clamp_eps: float = 1e-4):
    """Forward-only msda3d_fused."""
    return _fused_fwd(3, value, value_spatial_shapes, reference_points, sampling_offsets,
                      attention_logits, clamp_grid, clamp_eps)
