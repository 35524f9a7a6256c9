"""MSDA2D / MSDA3D attention modules on the HIP op.

Same constructor, parameters, ``init_weights`` patterns and ``forward`` contract as the
reference modules (src/msda_triton/pytorch/msda_2d.py:117-383, msda_3d.py:121-394), which
run the pure-PyTorch function; these run ``msda2d`` / ``msda3d`` (libmsda_hip.so) for the
sampling step, so their tensors must be on the GPU. The projections, masking, chunking, checkpointing, dropout and residual are plain PyTorch,
as in the reference. With ``fused=True`` (the default) the softmax over L*P and the location
formation ``reference + offset / (W, H[, D])`` run inside the HIP kernel (``msda2d_fused`` /
``msda3d_fused``) instead of as separate PyTorch ops; ``fused=False`` keeps the reference's
order of operations.
"""

from __future__ import annotations

import math

import torch
from torch import nn
from torch.utils.checkpoint import checkpoint

from msda_triton.hip.fused import msda2d_fused, msda3d_fused
from msda_triton.hip.msda_2d import msda2d
from msda_triton.hip.msda_3d import msda3d


class _MSDAModule(nn.Module):
    """Shared body of MSDA2D (dim 2) and MSDA3D (dim 3)."""

    dim = 2

    def __init__(self, embed_dims: int, num_heads: int, num_levels: int, num_points: int,
                 dropout: float = 0.1, batch_first: bool = False,
                 query_chunk_size: int | None = None, head_chunk_size: int | None = None,
                 use_checkpoint: bool = False, clamp_grid: bool = True,
                 clamp_eps: float = 1e-4, fused: bool = True, **kwargs) -> None:
        super().__init__()
        if embed_dims % num_heads != 0:
            raise ValueError(
                f"embed_dims must be divisible by num_heads, but got {embed_dims} and {num_heads}")
        self.dropout = nn.Dropout(dropout)
        self.batch_first = batch_first
        self.embed_dims = embed_dims
        self.num_levels = num_levels
        self.num_heads = num_heads
        self.num_points = num_points
        self.query_chunk_size = query_chunk_size
        self.head_chunk_size = head_chunk_size
        self.use_checkpoint = use_checkpoint
        self.clamp_grid = clamp_grid
        self.clamp_eps = clamp_eps
        self.fused = fused
        d = self.dim
        self.sampling_offsets = nn.Linear(embed_dims, num_heads * num_levels * num_points * d)
        self.attention_weights = nn.Linear(embed_dims, num_heads * num_levels * num_points)
        self.value_proj = nn.Linear(embed_dims, embed_dims)
        self.output_proj = nn.Linear(embed_dims, embed_dims)

    # the sampling ops (msda2d / msda3d and their fused variants); a test may substitute
    # other functions
    def _msda(self, value, shapes, loc, attn):
        op = msda2d if self.dim == 2 else msda3d
        return op(value, shapes, loc, attn, self.clamp_grid, self.clamp_eps)

    def _msda_fused(self, value, shapes, ref, off, logits):
        op = msda2d_fused if self.dim == 2 else msda3d_fused
        return op(value, shapes, ref, off, logits, self.clamp_grid, self.clamp_eps)

    def _offset_bias(self, device) -> torch.Tensor:  # (H, L, P, dim)
        raise NotImplementedError

    def init_weights(self) -> None:
        """Zero offset/attention projections with the per-head sampling pattern in the
        offset bias; Xavier-uniform value and output projections with zero bias."""
        nn.init.constant_(self.sampling_offsets.weight, 0.0)
        device = self.sampling_offsets.weight.device
        with torch.no_grad():
            self.sampling_offsets.bias.copy_(self._offset_bias(device).reshape(-1))
        nn.init.constant_(self.attention_weights.weight, 0.0)
        nn.init.constant_(self.attention_weights.bias, 0.0)
        for lin in (self.value_proj, self.output_proj):
            nn.init.xavier_uniform_(lin.weight)
            nn.init.constant_(lin.bias, 0.0)
        self._is_init = True

    def forward(self, query: torch.Tensor, key: torch.Tensor | None = None,
                value: torch.Tensor | None = None, identity: torch.Tensor | None = None,
                query_pos: torch.Tensor | None = None,
                key_padding_mask: torch.Tensor | None = None,
                reference_points: torch.Tensor | None = None,
                spatial_shapes: torch.Tensor | None = None,
                level_start_index: torch.Tensor | None = None, **kwargs) -> torch.Tensor:
        """query (n_q, bs, C) or (bs, n_q, C) with batch_first; value defaults to query and
        identity (the residual) to query; reference_points (bs, n_q, L, dim) in [0, 1];
        spatial_shapes (L, dim) as (H, W) or (D, H, W). key and level_start_index are
        unused. Returns the query-shaped output_proj(attention) + identity, after dropout."""
        d = self.dim
        value = query if value is None else value
        identity = query if identity is None else identity
        q = query if query_pos is None else query + query_pos
        if not self.batch_first:
            q = q.permute(1, 0, 2)
            value = value.permute(1, 0, 2)
        bs, nq, _ = q.shape
        nv = value.shape[1]
        assert spatial_shapes is not None, "spatial_shapes is required"
        assert reference_points is not None, "reference_points is required"
        total = spatial_shapes.prod(-1).sum()
        assert total == nv, f"Spatial shapes product {total} doesn't match value size {nv}"

        v = self.value_proj(value)
        if key_padding_mask is not None:
            v = v.masked_fill(key_padding_mask[..., None], 0.0)
        v = v.view(bs, nv, self.num_heads, -1)
        if reference_points.shape[-1] != d:
            raise ValueError(f"Last dim of reference_points must be {d}, "
                             f"but got {reference_points.shape[-1]} instead.")
        # per-level extents in coordinate order (x, y[, z]) = (W, H[, D]); kept integer so
        # the offsets keep their dtype in the division, as in the reference. The shapes may
        # stay on the host (the op's fastest form); the normalizer goes to the offsets.
        normalizer = None if self.fused else spatial_shapes.flip(-1).to(reference_points.device)

        H, L, P = self.num_heads, self.num_levels, self.num_points
        qc = int(self.query_chunk_size) if self.query_chunk_size else nq
        hc = (int(self.head_chunk_size)
              if self.head_chunk_size and self.head_chunk_size < H else H)
        dph = self.embed_dims // H
        outs = []
        for q0 in range(0, nq, qc):
            q1 = min(q0 + qc, nq)
            qq = q[:, q0:q1]
            off = self.sampling_offsets(qq).view(bs, q1 - q0, H, L, P, d)
            logits = self.attention_weights(qq).view(bs, q1 - q0, H, L, P)
            if self.fused:
                ref = reference_points[:, q0:q1]
                fn = self._msda_fused
            else:
                attn = logits.view(bs, q1 - q0, H, L * P).softmax(-1).view(bs, q1 - q0, H, L, P)
                loc = reference_points[:, q0:q1, None, :, None, :] + off / normalizer[None, None, None, :, None, :]
                fn = self._msda
            out = q.new_zeros(bs, q1 - q0, self.embed_dims)
            for h0 in range(0, H, hc):
                h1 = min(h0 + hc, H)
                if self.fused:
                    args = (v[:, :, h0:h1], spatial_shapes, ref, off[:, :, h0:h1], logits[:, :, h0:h1])
                else:
                    args = (v[:, :, h0:h1], spatial_shapes, loc[:, :, h0:h1], attn[:, :, h0:h1])
                if self.use_checkpoint and self.training:
                    o = checkpoint(fn, *args, use_reentrant=False)
                else:
                    o = fn(*args)
                out[:, :, h0 * dph:h1 * dph] = o
            outs.append(out)
        output = self.output_proj(torch.cat(outs, dim=1))
        if not self.batch_first:
            output = output.permute(1, 0, 2)
        return self.dropout(output) + identity


class MSDA2D(_MSDAModule):
    """2D multi-scale deformable attention module (reference pytorch/msda_2d.py:117-383)."""

    dim = 2

    def _offset_bias(self, device) -> torch.Tensor:
        # head h points along angle 2*pi*h/H, scaled so the larger of |cos|, |sin| is 1;
        # point p of every level at (p + 1) times that step (Deformable DETR's pattern)
        H, L, P = self.num_heads, self.num_levels, self.num_points
        ang = torch.arange(H, dtype=torch.float32, device=device) * (2.0 * math.pi / H)
        dirs = torch.stack([ang.cos(), ang.sin()], -1)
        dirs = dirs / dirs.abs().amax(-1, keepdim=True)
        scale = torch.arange(1, P + 1, dtype=torch.float32, device=device)
        return dirs[:, None, None, :] * scale[None, None, :, None] * torch.ones(1, L, 1, 1, device=device)


class MSDA3D(_MSDAModule):
    """3D multi-scale deformable attention module (reference pytorch/msda_3d.py:121-394)."""

    dim = 3

    def _offset_bias(self, device) -> torch.Tensor:
        # point p of head h at angle 2*pi*(h*P + p)/(H*P), radius 0.02*(p + 1):
        # (x, y, z) = radius * (0.5 cos a, 0.5 sin a, 2 sin 2a), the same on every level
        H, L, P = self.num_heads, self.num_levels, self.num_points
        k = torch.arange(H * P, dtype=torch.float64, device=device).view(H, P)
        ang = 2.0 * math.pi * k / (H * P)
        rad = 0.02 * torch.arange(1, P + 1, dtype=torch.float64, device=device).view(1, P)
        xyz = torch.stack([rad * 0.5 * ang.cos(), rad * 0.5 * ang.sin(), rad * 2.0 * (2 * ang).sin()], -1)
        return xyz[:, None].expand(H, L, P, 3).to(torch.float32)
