"""GPU parity suite shared by tests/test_msda_2d.py and tests/test_msda_3d.py.

It mirrors the reference's own suites (tests/test_msda_2d.py:22-427, tests/test_msda_3d.py)
case by case, and adds oracle parity at the north-star tolerances:
  forward  max|out - ref| / max|ref| <= 1e-5 (fp32), <= 1e-2 (bf16/fp16 vs the fp32 oracle
           on upcast inputs);
  gradients (fp32) normwise max-relative <= 1e-4 against the float64 brute-force oracle
           evaluated with the same fp32 coordinate rounding as the kernel, and against the
           torch oracle with samples within 1e-3 px of a cell edge excluded from
           grad_sampling_locations (there one ulp of coordinate selects another cell).
The HIP op is reached through msda_triton (ctypes -> libmsda_hip.so); the oracle runs on
the CPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import msda_triton
from msda_triton import triton as mt_triton
from oracle import brute, torch_ref
from tests._util import clamp_active, make_inputs, max_abs, max_rel

FWD_TOL_F32 = 1e-5
FWD_TOL_HALF = 1e-2
GRAD_TOL_F32 = 1e-4
EDGE_TOL_PX = 1e-3


@pytest.mark.gpu
class ParitySuite:
    dim = 2

    @pytest.fixture(autouse=True)
    def _setup(self) -> None:
        if not torch.cuda.is_available():
            pytest.skip("no GPU")
        self.device = torch.device("cuda")
        if self.dim == 2:
            self.fwd, self.op, self.fn = msda_triton.msda2d_fwd, msda_triton.msda2d, mt_triton.MSDA2DFn
        else:
            self.fwd, self.op, self.fn = msda_triton.msda3d_fwd, msda_triton.msda3d, mt_triton.MSDA3DFn

    # ------------------------------------------------------------------ helpers
    def inputs(self, **kw):
        return make_inputs(self.dim, **kw)

    def gpu(self, *ts):
        return [t.to(self.device) for t in ts]

    def run_fwd_bwd(self, value, shapes, loc, attn, grad_out, **kw):
        v, lo, a = [t.detach().clone().to(self.device).requires_grad_(True) for t in (value, loc, attn)]
        out = self.op(v, shapes, lo, a, **kw)
        out.backward(grad_out.to(self.device, out.dtype))
        return out.detach().cpu(), v.grad.cpu(), lo.grad.cpu(), a.grad.cpu()

    def check_grads(self, value, shapes, loc, attn, grad_out, gv, gl, ga, clamp_grid=True,
                    clamp_eps=1e-4):
        """fp32 gradients vs the brute-force oracle (fp32 coordinate rounding) and vs the
        torch oracle with edge samples excluded from grad_loc."""
        bv, bl, ba = brute.bwd(value, shapes, loc, attn, grad_out, clamp_grid, clamp_eps,
                               coord_f32=True)
        assert max_rel(gv, bv) <= GRAD_TOL_F32, f"grad_value vs brute {max_rel(gv, bv)}"
        assert max_rel(ga, ba) <= GRAD_TOL_F32, f"grad_attn vs brute {max_rel(ga, ba)}"
        assert max_rel(gl, bl) <= GRAD_TOL_F32, f"grad_loc vs brute {max_rel(gl, bl)}"
        _, tv, tl, ta = torch_ref.msda_ref_grads(value, shapes, loc, attn, grad_out, clamp_grid,
                                                 clamp_eps)
        assert max_rel(gv, tv) <= GRAD_TOL_F32, f"grad_value vs torch {max_rel(gv, tv)}"
        assert max_rel(ga, ta) <= GRAD_TOL_F32, f"grad_attn vs torch {max_rel(ga, ta)}"
        keep = torch.from_numpy(~brute.edge_mask(shapes, loc, EDGE_TOL_PX, clamp_grid, clamp_eps))
        keep = keep.unsqueeze(-1).expand_as(tl)
        assert max_rel(gl[keep], tl[keep]) <= GRAD_TOL_F32, (
            f"grad_loc vs torch {max_rel(gl[keep], tl[keep])} "
            f"({int((~keep).sum()) // self.dim} edge samples excluded)")

    def check_half_grad_loc(self, value, shapes, loc, attn, grad_out, gl, clamp_eps=1e-4):
        """16-bit grad_sampling_locations against the float64 brute-force oracle on the
        upcast inputs with the kernels' fp32 coordinate rounding (same corners on every
        sample), normwise <= 1e-2; exactly zero on axes where the grid clamp was active."""
        vf, lf, af, gf = (t.float() for t in (value, loc, attn, grad_out))
        _, bl, _ = brute.bwd(vf, shapes, lf, af, gf, True, clamp_eps, coord_f32=True)
        gl = gl.float().cpu()
        assert max_rel(gl, bl) <= FWD_TOL_HALF, f"grad_loc vs brute {max_rel(gl, bl)}"
        active = torch.from_numpy(clamp_active(lf, clamp_eps))
        assert torch.all(gl[active] == 0)

    # ------------------------------------------------------- reference-mirrored cases
    def test_forward_pass_basic(self) -> None:
        value, shapes, loc, attn = self.inputs()
        ref = torch_ref.msda_ref(value, shapes, loc, attn, clamp_grid=True, clamp_eps=1e-4)
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn), clamp_grid=True,
                       clamp_eps=1e-4).cpu()
        assert out.shape == ref.shape and out.dtype == torch.float32
        assert max_abs(out, ref) < 1e-4
        assert (out - ref).abs().mean().item() < 1e-5
        assert max_rel(out, ref) <= FWD_TOL_F32
        assert max_rel(out, brute.fwd(value, shapes, loc, attn)) <= FWD_TOL_F32

    @pytest.mark.parametrize("cfg", [(1, 100, 4, 64, 3, 4), (4, 25, 8, 32, 2, 8),
                                     (2, 200, 16, 16, 4, 4)])
    def test_forward_pass_different_configs(self, cfg) -> None:
        bs, nq, nh, dph, nl, npt = cfg
        value, shapes, loc, attn = self.inputs(batch_size=bs, num_queries=nq, num_heads=nh,
                                               dim_per_head=dph, num_levels=nl, num_points=npt)
        ref = torch_ref.msda_ref(value, shapes, loc, attn)
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn)).cpu()
        assert max_abs(out, ref) < 1e-4
        assert max_rel(out, ref) <= FWD_TOL_F32

    def test_backward_pass_basic(self) -> None:
        value, shapes, loc, attn = self.inputs()
        grad_out = torch.randn(value.shape[0], loc.shape[1], value.shape[2] * value.shape[3],
                               generator=torch.Generator().manual_seed(7))
        out, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out, clamp_grid=True,
                                           clamp_eps=1e-4)
        ref, tv, tl, ta = torch_ref.msda_ref_grads(value, shapes, loc, attn, grad_out)
        # the reference suite's own absolute bounds (tests/test_msda_2d.py:207-231)
        assert max_abs(gv, tv) < 1e-5 and (gv - tv).abs().mean() < 1e-7
        assert max_abs(gl, tl) < 0.25 and (gl - tl).abs().mean() < 2e-5
        assert max_abs(ga, ta) < 3e-4 and (ga - ta).abs().mean() < 1e-6
        self.check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga)

    def test_fp64_not_supported(self) -> None:
        value, shapes, loc, attn = self.inputs(batch_size=1, num_queries=10, num_heads=2,
                                               dim_per_head=8, dtype=torch.float64)
        with pytest.raises(NotImplementedError) as exc_info:
            self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn))
        assert "fp32, fp16, and bf16" in str(exc_info.value)
        assert "float64" in str(exc_info.value)

    def test_edge_case_boundary_sampling(self) -> None:
        value, shapes, loc, attn = self.inputs(batch_size=1, num_queries=10)
        loc[0, 0, 0, 0, 0, :] = 0.0
        loc[0, 1, 0, 0, 0, :] = 1.0
        loc[0, 2, 0, 0, 0, :] = torch.tensor([0.0, 1.0] if self.dim == 2 else [0.0, 1.0, 0.5])
        ref = torch_ref.msda_ref(value, shapes, loc, attn)
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn)).cpu()
        assert max_abs(out, ref) < 1e-4
        assert max_rel(out, ref) <= FWD_TOL_F32

    def test_edge_case_out_of_bounds(self) -> None:
        value, shapes, loc, attn = self.inputs(batch_size=1, num_queries=10)
        loc[0, 0, 0, 0, 0, :] = -0.1
        loc[0, 1, 0, 0, 0, :] = 1.1
        ref = torch_ref.msda_ref(value, shapes, loc, attn, clamp_grid=True)
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn), clamp_grid=True).cpu()
        assert max_abs(out, ref) < 1e-4
        assert max_rel(out, ref) <= FWD_TOL_F32
        grad_out = torch.randn(1, 10, value.shape[2] * value.shape[3])
        _, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out, clamp_grid=True)
        # a clamped coordinate passes no gradient (torch.clamp backward)
        assert torch.all(gl[0, 0, 0, 0, 0] == 0) and torch.all(gl[0, 1, 0, 0, 0] == 0)
        self.check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga)

    def test_gradient_flow_end_to_end(self) -> None:
        value, shapes, loc, attn = self.inputs(batch_size=2, num_queries=20, num_heads=4,
                                               dim_per_head=16)
        v1, l1, a1 = [t.clone().requires_grad_(True) for t in (value, loc, attn)]
        loss_ref = (torch_ref.msda_ref(v1, shapes, l1, a1) ** 2).sum()
        loss_ref.backward()
        v2, l2, a2 = [t.clone().to(self.device).requires_grad_(True) for t in (value, loc, attn)]
        loss = (self.op(v2, shapes, l2, a2) ** 2).sum()
        loss.backward()
        assert abs(loss_ref.item() - loss.item()) < 1e-4 * max(1.0, abs(loss_ref.item()))
        keep = torch.from_numpy(~brute.edge_mask(shapes, loc, EDGE_TOL_PX)).unsqueeze(-1)
        keep = keep.expand_as(l1)
        assert max_abs(v2.grad.cpu(), v1.grad) < 1e-3
        assert max_abs(a2.grad.cpu(), a1.grad) < 1e-3
        assert max_abs(l2.grad.cpu()[keep], l1.grad[keep]) < 1e-3

    def test_no_clamp_grid(self) -> None:
        value, shapes, loc, attn = self.inputs()
        # widen the range so zero padding outside the level is exercised
        loc = loc * 1.2 - 0.1
        ref = torch_ref.msda_ref(value, shapes, loc, attn, clamp_grid=False)
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn), clamp_grid=False).cpu()
        assert max_abs(out, ref) < 1e-4
        assert max_rel(out, ref) <= FWD_TOL_F32
        grad_out = torch.randn(out.shape)
        _, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out, clamp_grid=False)
        self.check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga, clamp_grid=False)

    def test_single_level(self) -> None:
        ss = [(32, 32)] if self.dim == 2 else [(4, 5, 5)]
        value, shapes, loc, attn = self.inputs(num_levels=1, spatial_shapes=ss)
        ref = torch_ref.msda_ref(value, shapes, loc, attn)
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn)).cpu()
        assert max_abs(out, ref) < 1e-4
        grad_out = torch.randn(out.shape)
        _, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out)
        self.check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga)

    @pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
    def test_half_precision(self, dtype) -> None:
        value, shapes, loc, attn = self.inputs(batch_size=1, num_queries=50, num_heads=4,
                                               dim_per_head=32, dtype=dtype)
        ref = torch_ref.msda_ref(value.float(), shapes, loc.float(), attn.float())
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn))
        assert out.dtype == dtype and out.shape == ref.shape
        assert max_abs(out.cpu().float(), ref) < (1e-2 if dtype == torch.float16 else 5e-2)
        assert max_rel(out.cpu().float(), ref) <= FWD_TOL_HALF
        grad_out = torch.randn(out.shape)
        _, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out.to(dtype))
        for name, g in (("value", gv), ("loc", gl), ("attn", ga)):
            assert torch.isfinite(g.float()).all(), f"grad_{name} not finite"
        assert gv.dtype == dtype and gl.dtype == dtype and ga.dtype == dtype
        # gradients against the fp32 oracle on the same (rounded) inputs
        _, tv, tl, ta = torch_ref.msda_ref_grads(value.float(), shapes, loc.float(), attn.float(),
                                                 grad_out.to(dtype).float())
        assert max_rel(gv.float(), tv) <= FWD_TOL_HALF
        assert max_rel(ga.float(), ta) <= FWD_TOL_HALF
        self.check_half_grad_loc(value, shapes, loc, attn, grad_out.to(dtype), gl)

    @pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
    def test_half_precision_clamped_points(self, dtype) -> None:
        """16-bit locations on and beyond the level borders (0, 1, -0.1, 1.1 and within the
        clamp band, about a fifth of all coordinates): grad_sampling_locations against the
        float64 oracle, and exactly zero on every clamped axis."""
        value, shapes, loc, attn = self.inputs(batch_size=2, num_queries=40, num_heads=4,
                                               dim_per_head=32)
        g = torch.Generator().manual_seed(9)
        pick = torch.rand(loc.shape, generator=g) < 0.2
        special = torch.tensor([0.0, 1.0, -0.1, 1.1, 2e-5, 1.0 - 2e-5, 3e-3])
        idx = torch.randint(0, len(special), loc.shape, generator=g)
        loc = torch.where(pick, special[idx], loc)
        value, loc, attn = (t.to(dtype) for t in (value, loc, attn))
        grad_out = torch.randn(2, 40, 4 * 32, generator=g).to(dtype)
        out, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out)
        ref = brute.fwd(value.float(), shapes, loc.float(), attn.float(), coord_f32=True)
        assert max_rel(out.float(), ref) <= FWD_TOL_HALF
        assert int(torch.from_numpy(clamp_active(loc.float())).sum()) > 50
        self.check_half_grad_loc(value, shapes, loc, attn, grad_out, gl)
        bv, _, ba = brute.bwd(value.float(), shapes, loc.float(), attn.float(), grad_out.float(),
                              coord_f32=True)
        assert max_rel(gv.float(), bv) <= FWD_TOL_HALF and max_rel(ga.float(), ba) <= FWD_TOL_HALF

    @pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
    def test_half_precision_lattice_points(self, dtype) -> None:
        """16-bit locations on an exact lattice of k / (2 * largest extent) over power-of-two
        levels, so every sample's pixel coordinate is an exact integer, half or quarter
        (corner weights 0 / 1 and ties of floor): the tile kernel re-derives each sample's
        corners from its record's raw 16-bit location, and must pick the fill's corners for
        every one of them. All gradients against the float64 oracle with the kernels' fp32
        coordinate rounding."""
        ss = [(32, 32), (16, 16), (8, 8)] if self.dim == 2 else [(8, 16, 16), (4, 8, 8)]
        value, shapes, loc, attn = self.inputs(batch_size=2, num_queries=60, num_heads=4,
                                               dim_per_head=32, spatial_shapes=ss)
        n = 2 * max(max(s) for s in ss)
        g = torch.Generator().manual_seed(11)
        loc = torch.randint(0, n + 1, loc.shape, generator=g).float() / n
        value, loc, attn = (t.to(dtype) for t in (value, loc, attn))
        assert torch.equal(loc.float() * n, (loc.float() * n).round())  # exact in 16 bits
        grad_out = torch.randn(2, 60, 4 * 32, generator=g).to(dtype)
        out, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out)
        ref = brute.fwd(value.float(), shapes, loc.float(), attn.float(), coord_f32=True)
        assert max_rel(out.float(), ref) <= FWD_TOL_HALF
        self.check_half_grad_loc(value, shapes, loc, attn, grad_out, gl)
        bv, _, ba = brute.bwd(value.float(), shapes, loc.float(), attn.float(), grad_out.float(),
                              coord_f32=True)
        assert max_rel(gv.float(), bv) <= FWD_TOL_HALF and max_rel(ga.float(), ba) <= FWD_TOL_HALF

    @pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
    def test_half_precision_no_clamp_outside_levels(self, dtype) -> None:
        """16-bit inputs without the grid clamp, locations over [-0.3, 1.3]: samples with no
        corner inside their level get exactly zero grad_loc and grad_attn (in the binned
        backward the count pass writes those, the tile kernel all others); every gradient
        against the float64 oracle on the upcast inputs. The allocator's memory is filled
        with NaN first, so a gradient left unwritten cannot pass."""
        value, shapes, loc, attn = self.inputs(batch_size=2, num_queries=60, num_heads=4,
                                               dim_per_head=32)
        loc = loc * 1.6 - 0.3
        value, loc, attn = (t.to(dtype) for t in (value, loc, attn))
        g = torch.Generator().manual_seed(11)
        grad_out = torch.randn(2, 60, 4 * 32, generator=g).to(dtype)
        vf, lf, af, gf = (t.float() for t in (value, loc, attn, grad_out))
        # samples whose pixel coordinate leaves [-1, size) on some axis have no corner inside
        u = torch.from_numpy(brute.coords(shapes, lf, clamp_grid=False, coord_f32=True))
        size = shapes.flip(-1).to(u.dtype).view(1, 1, 1, -1, 1, self.dim)
        outside = ((u < -1) | (u >= size)).any(-1)
        assert int(outside.sum()) > 100
        poison = torch.full((1 << 22,), float("nan"), device=self.device)
        del poison
        out, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out, clamp_grid=False)
        ref = brute.fwd(vf, shapes, lf, af, clamp_grid=False, coord_f32=True)
        assert max_rel(out.float(), ref) <= FWD_TOL_HALF
        bv, bl, ba = brute.bwd(vf, shapes, lf, af, gf, False, 1e-4, coord_f32=True)
        for name, got, want in (("value", gv, bv), ("loc", gl, bl), ("attn", ga, ba)):
            assert torch.isfinite(got.float()).all(), f"grad_{name} not finite"
            assert max_rel(got.float(), want) <= FWD_TOL_HALF, f"grad_{name} {max_rel(got.float(), want)}"
        assert torch.all(ga[outside] == 0) and torch.all(gl[outside] == 0)

    # ------------------------------------------------------------- added cases
    def test_mixed_dtype_fp32_coords(self) -> None:
        """bf16 value with fp32 locations and weights (autocast-style inputs)."""
        value, shapes, loc, attn = self.inputs(batch_size=1, num_queries=64)
        vb = value.to(torch.bfloat16)
        ref = torch_ref.msda_ref(vb.float(), shapes, loc, attn)
        out = self.fwd(vb.to(self.device), shapes, *self.gpu(loc, attn))
        assert out.dtype == torch.bfloat16
        assert max_rel(out.cpu().float(), ref) <= FWD_TOL_HALF
        grad_out = torch.randn(out.shape)
        _, gv, gl, ga = self.run_fwd_bwd(vb, shapes, loc, attn, grad_out.to(torch.bfloat16))
        assert gl.dtype == torch.float32 and ga.dtype == torch.float32
        _, tv, tl, ta = torch_ref.msda_ref_grads(vb.float(), shapes, loc, attn,
                                                 grad_out.to(torch.bfloat16).float())
        assert max_rel(ga, ta) <= FWD_TOL_HALF
        assert max_rel(gv.float(), tv) <= FWD_TOL_HALF
        # fp32 locations and weights: their gradients are computed and stored in fp32
        bv, bl, ba = brute.bwd(vb.float(), shapes, loc, attn, grad_out.to(torch.bfloat16).float(),
                               coord_f32=True)
        assert max_rel(gl, bl) <= GRAD_TOL_F32 and max_rel(ga, ba) <= GRAD_TOL_F32

    def test_gpu_resident_shapes(self) -> None:
        value, shapes, loc, attn = self.inputs(batch_size=1)
        a = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn)).cpu()
        b = self.fwd(*self.gpu(value), shapes.to(self.device, torch.int32),
                     *self.gpu(loc, attn)).cpu()
        assert torch.equal(a, b)

    def test_gpu_resident_shapes_modified_in_place(self) -> None:
        """The level tables cached for a device shapes tensor follow in-place edits."""
        ss = [(32, 32), (16, 16)] if self.dim == 2 else [(4, 5, 5), (2, 3, 3)]
        value, shapes, loc, attn = self.inputs(batch_size=1, spatial_shapes=ss)
        shapes_dev = shapes.to(self.device, torch.int32)
        a = self.fwd(*self.gpu(value), shapes_dev, *self.gpu(loc, attn)).cpu()
        assert max_rel(a, torch_ref.msda_ref(value, shapes, loc, attn)) <= FWD_TOL_F32
        new = torch.tensor([[16, 64], [16, 16]] if self.dim == 2 else [[5, 4, 5], [2, 3, 3]])
        shapes_dev.copy_(new)  # same K, different level geometry
        b = self.fwd(*self.gpu(value), shapes_dev, *self.gpu(loc, attn)).cpu()
        assert max_rel(b, torch_ref.msda_ref(value, new, loc, attn)) <= FWD_TOL_F32
        assert not torch.equal(a, b)

    def test_cpu_shapes_reused_and_modified_in_place(self) -> None:
        """CPU shapes tensors are cached by identity and version counter: a reused tensor
        hits the cache, an in-place change of its first level (same K) is seen, and the
        K check still runs on a cache hit."""
        value, shapes, loc, attn = self.inputs(batch_size=1, num_queries=16)
        v, lo, a = self.gpu(value, loc, attn)
        for _ in range(2):
            out = self.fwd(v, shapes, lo, a).cpu()
            assert max_rel(out, torch_ref.msda_ref(value, shapes, loc, attn)) <= FWD_TOL_F32
        shapes[0] = torch.tensor([16, 64] if self.dim == 2 else [5, 4, 5])
        out = self.fwd(v, shapes, lo, a).cpu()
        assert max_rel(out, torch_ref.msda_ref(value, shapes, loc, attn)) <= FWD_TOL_F32
        with pytest.raises(ValueError, match="does not match sum of spatial shapes"):
            self.fwd(v[:, :-1], shapes, lo, a)

    def test_non_contiguous_inputs(self) -> None:
        value, shapes, loc, attn = self.inputs(batch_size=2, num_queries=30)
        ref = torch_ref.msda_ref(value, shapes, loc, attn)
        vt = value.to(self.device).transpose(0, 1).contiguous().transpose(0, 1)
        lt = loc.to(self.device).transpose(1, 2).contiguous().transpose(1, 2)
        at = attn.to(self.device).transpose(1, 2).contiguous().transpose(1, 2)
        assert not vt.is_contiguous() and not lt.is_contiguous()
        out = self.fwd(vt, shapes, lt, at).cpu()
        assert max_rel(out, ref) <= FWD_TOL_F32

    @pytest.mark.parametrize("heads,ch", [(3, 3), (5, 48), (1, 8), (2, 128)])
    def test_odd_heads_channels(self, heads, ch) -> None:
        """Channel counts that need narrower loads (C=3), idle lanes (C=48 -> 12 of 16 lanes)
        and odd head counts (no shared-line head groups)."""
        value, shapes, loc, attn = self.inputs(batch_size=2, num_queries=33, num_heads=heads,
                                               dim_per_head=ch, num_levels=3, num_points=3)
        ref = torch_ref.msda_ref(value, shapes, loc, attn)
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn)).cpu()
        assert max_rel(out, ref) <= FWD_TOL_F32
        grad_out = torch.randn(out.shape)
        _, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out)
        self.check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga)

    @pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
    @pytest.mark.parametrize("heads,ch", [(3, 3), (2, 48), (5, 16), (2, 128)])
    def test_odd_heads_channels_half(self, heads, ch, dtype) -> None:
        """16-bit values (the binned backward's tile kernel forms grad_loc / grad_attn from its
        staged region rows) with channel counts that change the staged row sizes and owner
        chunks (C=3: 6-byte rows; C=48: 96-byte rows, 6 of 8 lanes; C=128: tiles shrunk to fit
        the owner items), odd head counts and 3 points per level (the generic count and fill
        loops): every gradient against the float64 oracle on the upcast inputs."""
        value, shapes, loc, attn = self.inputs(batch_size=2, num_queries=33, num_heads=heads,
                                               dim_per_head=ch, num_levels=3, num_points=3)
        value, loc, attn = (t.to(dtype) for t in (value, loc, attn))
        vf, lf, af = (t.float() for t in (value, loc, attn))
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn)).cpu()
        assert max_rel(out.float(), brute.fwd(vf, shapes, lf, af, coord_f32=True)) <= FWD_TOL_HALF
        g = torch.Generator().manual_seed(5)
        grad_out = torch.randn(out.shape, generator=g).to(dtype)
        _, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out)
        bv, _, ba = brute.bwd(vf, shapes, lf, af, grad_out.float(), coord_f32=True)
        assert max_rel(gv.float(), bv) <= FWD_TOL_HALF and max_rel(ga.float(), ba) <= FWD_TOL_HALF
        self.check_half_grad_loc(value, shapes, loc, attn, grad_out, gl)

    def test_wide_level_32bit_addressing(self) -> None:
        """A level whose row stride along y (2D) or z (3D) exceeds 2^23 bytes: corner offsets
        take the 32-bit multiply path instead of the 24-bit one, forward and backward."""
        ss = [(2, 16400), (3, 5)] if self.dim == 2 else [(2, 2, 8200), (2, 3, 4)]
        value, shapes, loc, attn = self.inputs(batch_size=1, num_queries=40, num_heads=8,
                                               dim_per_head=32, num_levels=2, num_points=4,
                                               spatial_shapes=ss)
        ref = torch_ref.msda_ref(value, shapes, loc, attn)
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn)).cpu()
        assert max_rel(out, ref) <= FWD_TOL_F32
        # at 16400 cells a float64 pixel coordinate differs from the fp32 one by ~1e-3 px:
        # the brute-force oracle rounds coordinates to fp32 as the kernel does
        assert max_rel(out, brute.fwd(value, shapes, loc, attn, coord_f32=True)) <= FWD_TOL_F32
        grad_out = torch.randn(out.shape, generator=torch.Generator().manual_seed(3))
        _, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out)
        self.check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga)

    @pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
    def test_levels_beyond_binning_atomic_path(self, dtype) -> None:
        """Levels with more than 8192 tiles per head (the backward's LDS binning limit; 2D
        1032 x 1024 cells in 16 x 8 tiles, 3D 72 x 128 x 128 in 4 x 4 x 8) take the atomic
        grad_value path: fp32 sums scattered with global atomics, then rounded once. The
        second, 15-cell level makes most samples collide on a few keys."""
        ss = [(1032, 1024), (3, 5)] if self.dim == 2 else [(72, 128, 128), (3, 5, 1)]
        nb = 2 if self.dim == 2 else 1
        value, shapes, loc, attn = self.inputs(batch_size=nb, num_queries=64, num_heads=1,
                                               dim_per_head=32, num_points=4, spatial_shapes=ss,
                                               dtype=dtype)
        grad_out = torch.randn(nb, 64, 32, generator=torch.Generator().manual_seed(5)).to(dtype)
        out, gv, gl, ga = self.run_fwd_bwd(value, shapes, loc, attn, grad_out)
        assert gv.dtype == dtype and torch.isfinite(gv.float()).all()
        if dtype == torch.float32:
            assert max_rel(out, brute.fwd(value, shapes, loc, attn, coord_f32=True)) <= FWD_TOL_F32
            self.check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga)
        else:
            vf, lf, af, gf = value.float(), loc.float(), attn.float(), grad_out.float()
            assert max_rel(out.float(), brute.fwd(vf, shapes, lf, af, coord_f32=True)) <= FWD_TOL_HALF
            bv, bl, ba = brute.bwd(vf, shapes, lf, af, gf, coord_f32=True)
            assert max_rel(gv.float(), bv) <= FWD_TOL_HALF
            assert max_rel(ga.float(), ba) <= FWD_TOL_HALF
            assert max_rel(gl.float(), bl) <= FWD_TOL_HALF

    def test_empty_inputs(self) -> None:
        value, shapes, loc, attn = self.inputs(batch_size=2, num_queries=0)
        out = self.fwd(*self.gpu(value), shapes, *self.gpu(loc, attn))
        assert out.shape == (2, 0, value.shape[2] * value.shape[3])
        v, lo, a = [t.to(self.device).requires_grad_(True) for t in (value, loc, attn)]
        self.op(v, shapes, lo, a).sum().backward()
        assert torch.all(v.grad == 0)

    def test_autograd_function_import_path(self) -> None:
        value, shapes, loc, attn = self.inputs(batch_size=1, num_queries=8)
        out = self.fn.apply(*self.gpu(value), shapes, *self.gpu(loc, attn), True, 1e-4).cpu()
        assert max_rel(out, torch_ref.msda_ref(value, shapes, loc, attn)) <= FWD_TOL_F32
