"""CPU restatement of the reference's pure-PyTorch oracle — TEST INFRASTRUCTURE ONLY.

``msda_ref`` restates ``msda2d_pytorch`` (src/msda_triton/pytorch/msda_2d.py:58-114) and
``msda3d_pytorch`` (src/msda_triton/pytorch/msda_3d.py:58-118) step by step, in the input
dtype, so its rounding matches the reference oracle's:

1. split value by per-level sizes (msda_2d.py:62-63);
2. grid = 2*loc - 1, optionally clamped to [-1+eps, 1-eps] (msda_2d.py:66-68);
3. per level, F.grid_sample(bilinear, zeros, align_corners=False) of the
   (B*H, C, [D,] H_l, W_l) level against the (B*H, Q, P, [1,] d) grid (msda_2d.py:77-98,
   msda_3d.py:81-102);
4. multiply by the level's attention weights, sum over points, accumulate over levels in
   an accumulator of the input dtype (msda_2d.py:71, 102-110);
5. return (B, Q, H*C) (msda_2d.py:113-114).

``msda_fused_ref`` restates the attention modules' formation of locations and weights
before that call (pytorch/msda_2d.py:303-339, pytorch/msda_3d.py:314-350): the offset
normaliser stacks the level extents in coordinate order (W, H[, D]); locations are
reference_points[:, :, None, :, None, :] + offsets / normaliser; weights are the softmax of
the logits over the flattened L*P axis.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def msda_ref(value: torch.Tensor, value_spatial_shapes: torch.Tensor,
             sampling_locations: torch.Tensor, attention_weights: torch.Tensor,
             clamp_grid: bool = True, clamp_eps: float = 1e-4) -> torch.Tensor:
    bs, _, num_heads, ch = value.shape
    _, nq, _, nl, npt, dim = sampling_locations.shape
    shapes = [tuple(int(s) for s in row) for row in value_spatial_shapes.cpu().tolist()]
    sizes = [int(torch.tensor(s).prod()) for s in shapes]
    value_list = value.split(sizes, dim=1)
    grids = 2 * sampling_locations - 1
    if clamp_grid:
        grids = grids.clamp(min=-1.0 + clamp_eps, max=1.0 - clamp_eps)
    acc = value.new_zeros(bs * num_heads, ch, nq)
    for lvl, shp in enumerate(shapes):
        v_l = value_list[lvl].flatten(2).transpose(1, 2).reshape(bs * num_heads, ch, *shp)
        g_l = grids[:, :, :, lvl].transpose(1, 2).flatten(0, 1)
        if dim == 3:
            g_l = g_l.unsqueeze(-2)
        s_l = F.grid_sample(v_l, g_l, mode="bilinear", padding_mode="zeros",
                            align_corners=False)
        if dim == 3:
            s_l = s_l.squeeze(-1)
        a_l = attention_weights[:, :, :, lvl, :].transpose(1, 2).reshape(bs * num_heads, 1, nq,
                                                                          npt)
        acc = acc + (s_l * a_l).sum(-1)
    return acc.view(bs, num_heads * ch, nq).transpose(1, 2).contiguous()


def msda_ref_grads(value, shapes, loc, attn, grad_out, clamp_grid=True, clamp_eps=1e-4):
    """(out, grad_value, grad_loc, grad_attn) of msda_ref via autograd, on copies of the inputs."""
    v = value.detach().clone().requires_grad_(True)
    lo = loc.detach().clone().requires_grad_(True)
    a = attn.detach().clone().requires_grad_(True)
    out = msda_ref(v, shapes, lo, a, clamp_grid, clamp_eps)
    out.backward(grad_out.to(out.dtype))
    return out.detach(), v.grad, lo.grad, a.grad


def msda_fused_ref(value: torch.Tensor, value_spatial_shapes: torch.Tensor,
                   reference_points: torch.Tensor, sampling_offsets: torch.Tensor,
                   attention_logits: torch.Tensor, clamp_grid: bool = True,
                   clamp_eps: float = 1e-4) -> torch.Tensor:
    """msda_ref of the locations and weights formed from (B, Q, L, d) reference points,
    (B, Q, H, L, P, d) offsets and (B, Q, H, L, P) logits, as the modules form them."""
    bs, nq, nh, nl, npt, dim = sampling_offsets.shape
    shapes = value_spatial_shapes.to(torch.int64)
    # (L, d) in coordinate order: 2D (W, H) = columns (1, 0); 3D (W, H, D) = (2, 1, 0)
    normalizer = torch.stack([shapes[..., dim - 1 - k] for k in range(dim)], -1)
    attn = attention_logits.reshape(bs, nq, nh, nl * npt).softmax(-1).view(bs, nq, nh, nl, npt)
    loc = (reference_points[:, :, None, :, None, :]
           + sampling_offsets / normalizer[None, None, None, :, None, :])
    return msda_ref(value, value_spatial_shapes, loc, attn, clamp_grid, clamp_eps)
