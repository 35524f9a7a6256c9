"""Pure-PyTorch MSDA shared by msda2d_pytorch and msda3d_pytorch.

Same computation, order of operations and dtype behaviour as the reference's pure-PyTorch
functions (src/msda_triton/pytorch/msda_2d.py:58-114, src/msda_triton/pytorch/msda_3d.py:
58-118): grid = 2*loc - 1 with optional clamp, one F.grid_sample per level over the
(B*H, C, [D,] H_l, W_l) view of that level, weighted by attention and summed over points,
accumulated over levels in the input dtype. Runs on any device; this is the portable
(slow) path of the public API, not the HIP kernels.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def grid_sample_msda(value: torch.Tensor, value_spatial_shapes: torch.Tensor,
                     sampling_locations: torch.Tensor, attention_weights: torch.Tensor,
                     clamp_grid: bool, clamp_eps: float) -> torch.Tensor:
    bs, _, num_heads, dims_per_head = value.shape
    _, num_queries, _, _, num_points, dim = sampling_locations.shape
    shapes = [tuple(int(s) for s in row) for row in value_spatial_shapes.cpu().tolist()]
    sections = []
    for shp in shapes:
        n = 1
        for s in shp:
            n *= s
        sections.append(n)
    value_list = value.split(sections, dim=1)

    grids = 2 * sampling_locations - 1
    if clamp_grid:
        grids = grids.clamp(min=-1.0 + clamp_eps, max=1.0 - clamp_eps)

    out = value.new_zeros(bs * num_heads, dims_per_head, num_queries)
    for level, shp in enumerate(shapes):
        # (B, K_l, H, C) -> (B*H, C, [D,] H_l, W_l)
        v_l = value_list[level].flatten(2).transpose(1, 2).reshape(bs * num_heads, dims_per_head,
                                                                   *shp)
        # (B, Q, H, P, d) -> (B*H, Q, P, [1,] d)
        g_l = grids[:, :, :, level].transpose(1, 2).flatten(0, 1)
        if dim == 3:
            g_l = g_l.unsqueeze(-2)
        s_l = F.grid_sample(v_l, g_l, mode="bilinear", padding_mode="zeros", align_corners=False)
        if dim == 3:
            s_l = s_l.squeeze(-1)
        # (B, Q, H, P) -> (B*H, 1, Q, P)
        a_l = attention_weights[:, :, :, level, :].transpose(1, 2).reshape(
            bs * num_heads, 1, num_queries, num_points)
        out = out + (s_l * a_l).sum(-1)
    return out.view(bs, num_heads * dims_per_head, num_queries).transpose(1, 2).contiguous()
