"""Helpers for the parity tests: seeded inputs and error metrics."""

from __future__ import annotations

import numpy as np
import torch


def make_inputs(dim, batch_size=2, num_queries=50, num_heads=8, dim_per_head=32, num_levels=2,
                num_points=4, spatial_shapes=None, dtype=torch.float32, seed=42,
                logits="rand", device="cpu"):
    """Seeded inputs on the CPU (then moved), as the reference tests build them
    (tests/test_msda_2d.py:32-111): value ~ N(0,1), locations ~ U[0,1]^d, weights = softmax
    over L*P of `rand` (or `randn`) logits. Default pyramids: 2D (32,32),(16,16),(8,8),(4,4);
    3D (4,5,5),(2,3,3),(3,4,4),(2,2,2) (test_msda_3d.py:61)."""
    if spatial_shapes is None:
        base = ([(32, 32), (16, 16), (8, 8), (4, 4)] if dim == 2
                else [(4, 5, 5), (2, 3, 3), (3, 4, 4), (2, 2, 2)])
        spatial_shapes = base[:num_levels]
    num_levels = len(spatial_shapes)
    num_keys = sum(int(np.prod(s)) for s in spatial_shapes)
    g = torch.Generator().manual_seed(seed)
    value = torch.randn(batch_size, num_keys, num_heads, dim_per_head, generator=g)
    loc = torch.rand(batch_size, num_queries, num_heads, num_levels, num_points, dim, generator=g)
    raw = (torch.rand if logits == "rand" else torch.randn)(
        batch_size, num_queries, num_heads, num_levels * num_points, generator=g)
    attn = raw.softmax(-1).view(batch_size, num_queries, num_heads, num_levels, num_points)
    shapes = torch.tensor(spatial_shapes, dtype=torch.int64)
    return (value.to(device=device, dtype=dtype), shapes, loc.to(device=device, dtype=dtype),
            attn.to(device=device, dtype=dtype))


def max_rel(a, b) -> float:
    """max|a - b| / max|b| (normwise max-relative error of a against reference b)."""
    a = torch.as_tensor(a).detach().double().cpu()
    b = torch.as_tensor(b).detach().double().cpu()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)


def max_abs(a, b) -> float:
    a = torch.as_tensor(a).detach().double().cpu()
    b = torch.as_tensor(b).detach().double().cpu()
    return (a - b).abs().max().item()


def clamp_active(loc, clamp_eps: float = 1e-4) -> np.ndarray:
    """True per (sample, axis) where the grid clamp of the forward is active: the fp32 grid
    coordinate g = 2*loc - 1 (rounded after each operation, as the kernels and torch's
    fp32 oracle compute it) lies outside [fp32(-1 + eps), fp32(1 - eps)]. There the
    gradient of the location is zero (backward of torch.clamp)."""
    lo = np.asarray(torch.as_tensor(loc).detach().float().cpu().numpy(), dtype=np.float32)
    g = np.float32(2.0) * lo - np.float32(1.0)
    return (g < np.float32(-1.0 + clamp_eps)) | (g > np.float32(1.0 - clamp_eps))
