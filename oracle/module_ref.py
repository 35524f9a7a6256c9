"""Restatement of the reference attention modules' forward — TEST INFRASTRUCTURE ONLY.

msda_module_ref computes what MSDA2D.forward (src/msda_triton/pytorch/msda_2d.py:230-383) and
MSDA3D.forward (src/msda_triton/pytorch/msda_3d.py:241-394) compute, step by step, from the
modules' parameters passed in as plain tensors, with the sampling step done by
oracle.torch_ref.msda_ref (the reference's msda2d_pytorch / msda3d_pytorch restated):

  value   = query if value is None; identity = query if identity is None   (msda_2d.py:270-271)
  query  += query_pos                                                       (:274)
  (seq-first inputs are permuted to batch-first)                            (:277-279)
  value   = value_proj(value), masked_fill(key_padding_mask, 0), split heads (:294-297)
  offsets = sampling_offsets(query) -> (B, Q, H, L, P, dim)                 (:328-330)
  weights = softmax over L*P of attention_weights(query)                    (:331-337)
  loc     = reference_points[:, :, None, :, None, :] + offsets / (W, H[, D]) (:305-308, :339-342)
  out     = output_proj(msda(value, shapes, loc, weights))                  (:344-379)
  return dropout(out) + identity (dropout is the identity here: p = 0 or eval) (:381-383)

The query and head chunking of the reference (:316-377) does not change the result, so it
is not repeated. Nothing in the msda_triton package imports this file.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import torch_ref


def msda_module_ref(dim, params, query, *, value=None, identity=None, query_pos=None,
                    key_padding_mask=None, reference_points, spatial_shapes, num_heads,
                    num_levels, num_points, batch_first=False, clamp_grid=True, clamp_eps=1e-4):
    """params: dict of value_proj / sampling_offsets / attention_weights / output_proj
    weight and bias tensors (nn.Linear layout: weight (out, in), bias (out,))."""
    value_t = query if value is None else value
    identity_t = query if identity is None else identity
    query_t = query + query_pos if query_pos is not None else query
    if not batch_first:
        query_t = query_t.permute(1, 0, 2)
        value_t = value_t.permute(1, 0, 2)
    bs, nq, _ = query_t.shape
    nv = value_t.shape[1]
    if reference_points.shape[-1] != dim:
        raise ValueError(f"Last dim of reference_points must be {dim}")
    v = F.linear(value_t, params["value_proj.weight"], params["value_proj.bias"])
    if key_padding_mask is not None:
        v = v.masked_fill(key_padding_mask[..., None], 0.0)
    v = v.view(bs, nv, num_heads, -1)
    # (L, dim) shapes ordered (H, W) / (D, H, W); the normaliser is (W, H[, D])
    normalizer = spatial_shapes.flip(-1).to(query_t.dtype)
    off = F.linear(query_t, params["sampling_offsets.weight"], params["sampling_offsets.bias"])
    off = off.view(bs, nq, num_heads, num_levels, num_points, dim)
    aw = F.linear(query_t, params["attention_weights.weight"], params["attention_weights.bias"])
    aw = aw.view(bs, nq, num_heads, num_levels * num_points).softmax(-1)
    aw = aw.view(bs, nq, num_heads, num_levels, num_points)
    loc = reference_points[:, :, None, :, None, :] + off / normalizer[None, None, None, :, None, :]
    out = torch_ref.msda_ref(v, spatial_shapes, loc, aw, clamp_grid, clamp_eps)
    out = F.linear(out, params["output_proj.weight"], params["output_proj.bias"])
    if not batch_first:
        out = out.permute(1, 0, 2)
    return out + identity_t
