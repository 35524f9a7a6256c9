"""GPU parity at BASELINE.json's full workload sizes.

The small-shape suites (tests/_parity.py) never reach the staged forward kernel, which is
chosen only when every workgroup gets at least kFwdStageMinQueries queries; these cases do,
and they cover the configurations bench.py measures:
  C2  2D encoder B=2 Q=K=19947 L=4 P=4 (bf16, fp32)      staged forward
  C3  2D decoder B=8 Q=300                 (bf16)       unstaged forward (few queries)
  C5  3D 4-level B=1 Q=32768 P=8, 10% of points near a face, clamp_eps=1e-4 (bf16)
  C4  3D B=2 L=2 Q=4096 P=4                   (fp32, bf16) unstaged forward, fwd+bwd
plus a 3D fp32 launch that takes the staged forward (C5's pyramid at Q=16384, P=4) and 2D
backward plans near the 8192-bin limit of the LDS binning.
Oracles, on the CPU: oracle/torch_ref (the reference's msda*_pytorch restated) in fp32 on
the same (upcast) inputs, and oracle/msda_brute.c in float64 with the kernels' fp32
coordinate rounding (coord_f32), which selects the same corners as the kernels on every
sample. Tolerances (normwise max|x-ref|/max|ref|):
  forward  <= 1e-5 (fp32), <= 1e-2 (bf16);
  gradients <= 1e-4 (fp32) for grad_value, grad_sampling_locations and
           grad_attention_weights against brute, and against torch with samples within
           1e-3 px of a cell edge excluded from grad_sampling_locations; <= 1e-2 (bf16,
           every input and gradient stored in bf16) for all three against brute on the
           upcast inputs;
  grad_sampling_locations is exactly zero on every axis where the grid clamp was active
           (backward of torch.clamp), the case C5's near-face points stress.
"""

from __future__ import annotations

import pytest
import torch

import bench
import msda_triton
from oracle import brute, torch_ref
from tests._util import clamp_active, max_rel

EDGE_TOL_PX = 1e-3

pytestmark = pytest.mark.gpu


def _case(name, dtype=None):
    cfg = dict(bench.CONFIGS[name])
    if dtype is not None:
        cfg["dtype"] = dtype
    value, shapes, loc, attn = bench.make_inputs(cfg)
    dt = bench.DTYPES[cfg["dtype"]]
    value, loc, attn = (t.to(dt) for t in (value, loc, attn))
    return cfg, value, shapes, loc, attn


def _fwd(cfg):
    return msda_triton.msda2d_fwd if cfg["dim"] == 2 else msda_triton.msda3d_fwd


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.mark.parametrize("name,dtype,tol", [("c2", "bf16", 1e-2), ("c2", "fp32", 1e-5),
                                            ("c3", "bf16", 1e-2), ("c5", "bf16", 1e-2)])
def test_forward_full_size(name, dtype, tol):
    cfg, value, shapes, loc, attn = _case(name, dtype)
    dev = torch.device("cuda")
    print(f"full-size forward {name} {dtype}", flush=True)
    out = _fwd(cfg)(value.to(dev), shapes, loc.to(dev), attn.to(dev), True, 1e-4)
    ref = torch_ref.msda_ref(value.float(), shapes, loc.float(), attn.float(), True, 1e-4)
    assert out.dtype == value.dtype and out.shape == ref.shape
    assert max_rel(out.float().cpu(), ref) <= tol


def test_forward_gpu_shapes_full_size():
    """GPU-resident level shapes take the same staged path without a host copy."""
    cfg, value, shapes, loc, attn = _case("c2")
    dev = torch.device("cuda")
    a = msda_triton.msda2d_fwd(value.to(dev), shapes, loc.to(dev), attn.to(dev))
    b = msda_triton.msda2d_fwd(value.to(dev), shapes.to(dev, torch.int32), loc.to(dev), attn.to(dev))
    assert torch.equal(a, b)


def _grad_out(cfg, dtype):
    g = torch.Generator().manual_seed(7)
    return torch.randn(cfg["B"], cfg["Q"], cfg["H"] * cfg["C"], generator=g).to(dtype)


def _fwd_bwd(cfg, value, shapes, loc, attn, grad_out, shapes_on_device=False):
    dev = torch.device("cuda")
    op = msda_triton.msda2d if cfg["dim"] == 2 else msda_triton.msda3d
    v, lo, a = [t.to(dev).requires_grad_(True) for t in (value, loc, attn)]
    sh = shapes.to(dev, torch.int32) if shapes_on_device else shapes
    out = op(v, sh, lo, a, True, 1e-4)
    out.backward(grad_out.to(dev))
    return out.detach(), v.grad, lo.grad, a.grad


def _check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga, tol):
    """All three gradients against brute (fp32 coordinate rounding) at tol; grad_value and
    grad_attn against torch at tol and grad_loc against torch away from cell edges; exact
    zeros of grad_loc where the clamp was active. Inputs are upcast to fp32 first."""
    vf, lf, af, gf = (t.float() for t in (value, loc, attn, grad_out))
    gv, gl, ga = (t.float().cpu() for t in (gv, gl, ga))
    bv, bl, ba = brute.bwd(vf, shapes, lf, af, gf, True, 1e-4, coord_f32=True)
    for name, x, r in (("grad_value", gv, bv), ("grad_loc", gl, bl), ("grad_attn", ga, ba)):
        err = max_rel(x, r)
        assert err <= tol, f"{name} vs brute: {err:.3e}"
    active = torch.from_numpy(clamp_active(lf, 1e-4))
    assert torch.all(gl[active] == 0), "grad_loc nonzero where the grid clamp was active"
    assert torch.all(torch.from_numpy(bl)[active] == 0)
    _, tv, tl, ta = torch_ref.msda_ref_grads(vf, shapes, lf, af, gf, True, 1e-4)
    assert max_rel(gv, tv) <= tol, f"grad_value vs torch: {max_rel(gv, tv):.3e}"
    assert max_rel(ga, ta) <= tol, f"grad_attn vs torch: {max_rel(ga, ta):.3e}"
    keep = torch.from_numpy(~brute.edge_mask(shapes, lf, EDGE_TOL_PX, True, 1e-4))
    keep = keep.unsqueeze(-1).expand_as(tl)
    assert max_rel(gl[keep], tl[keep]) <= tol, f"grad_loc vs torch: {max_rel(gl[keep], tl[keep]):.3e}"
    return int(active.sum())


@pytest.mark.parametrize("name", ["c2", "c5"])
def test_backward_full_size(name):
    """bf16 C2 and C5 (the bench's workloads): all three gradients, grad_loc included, and
    its exact zeros on clamped axes (C5: 10% of points within 1e-3 of a face)."""
    cfg, value, shapes, loc, attn = _case(name)
    print(f"full-size backward {name}", flush=True)
    grad_out = _grad_out(cfg, value.dtype)
    out, gv, gl, ga = _fwd_bwd(cfg, value, shapes, loc, attn, grad_out)
    assert gv.dtype == gl.dtype == ga.dtype == torch.bfloat16
    clamped = _check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga, 1e-2)
    if cfg["face_frac"] > 0:
        assert clamped > 1000, f"only {clamped} clamped axes: the clamp stress is missing"
    # size-independent identity <grad_value, value> == <grad_out, out> (linearity in value)
    lhs = (gv.double() * value.to(gv.device).double()).sum().item()
    rhs = (grad_out.to(out.device).double() * out.double()).sum().item()
    assert abs(lhs - rhs) <= 1e-2 * max(1.0, abs(rhs))


def test_backward_full_size_c2_fp32():
    """C2 in fp32: forward at 1e-5 and all three gradients at the north-star 1e-4."""
    cfg, value, shapes, loc, attn = _case("c2", "fp32")
    print("full-size backward c2 fp32", flush=True)
    grad_out = _grad_out(cfg, torch.float32)
    out, gv, gl, ga = _fwd_bwd(cfg, value, shapes, loc, attn, grad_out)
    assert max_rel(out.cpu(), brute.fwd(value, shapes, loc, attn, True, 1e-4, coord_f32=True)) <= 1e-5
    _check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga, 1e-4)


@pytest.mark.parametrize("dtype,tol_f,tol_g", [("fp32", 1e-5, 1e-4), ("bf16", 1e-2, 1e-2)])
def test_c4_full_size(dtype, tol_f, tol_g):
    """C4, 3D B=2 L=2 (16,32,32)/(8,16,16) Q=4096 P=4: forward and all three gradients."""
    cfg, value, shapes, loc, attn = _case("c4", dtype)
    print(f"full-size c4 {dtype}", flush=True)
    grad_out = _grad_out(cfg, value.dtype)
    fwd_only = msda_triton.msda3d_fwd(value.cuda(), shapes, loc.cuda(), attn.cuda(), True, 1e-4)
    out, gv, gl, ga = _fwd_bwd(cfg, value, shapes, loc, attn, grad_out)
    assert torch.equal(fwd_only, out)
    ref = torch_ref.msda_ref(value.float(), shapes, loc.float(), attn.float(), True, 1e-4)
    assert max_rel(out.float().cpu(), ref) <= tol_f
    _check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga, tol_g)


def test_staged_forward_3d_fp32():
    """A 3D fp32 launch on the staged forward: B*H = 8 slices need 32 workgroups each for
    256 CUs, so Q = 16384 gives 512 queries per workgroup, the staging threshold. Pyramid of
    C5, P = 4; the backward is checked too."""
    cfg = dict(bench.CONFIGS["c5"], Q=16384, P=4, dtype="fp32", face_frac=0.1)
    value, shapes, loc, attn = bench.make_inputs(cfg)
    print("staged 3D fp32 forward", flush=True)
    grad_out = _grad_out(cfg, torch.float32)
    out, gv, gl, ga = _fwd_bwd(cfg, value, shapes, loc, attn, grad_out)
    assert max_rel(out.cpu(), brute.fwd(value, shapes, loc, attn, True, 1e-4, coord_f32=True)) <= 1e-5
    assert max_rel(out.cpu(), torch_ref.msda_ref(value, shapes, loc, attn, True, 1e-4)) <= 1e-5
    _check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga, 1e-4)


@pytest.mark.parametrize("dtype,heads", [("fp32", 1), ("bf16", 2)])
def test_backward_bins_near_lds_limit(dtype, heads):
    """A 2D pyramid of 75 x 100 + 1 = 7501 tiles (16 x 8 cells) per head, just inside the
    backward's 8192-bin LDS binning (fill kernel with about 100 KB of LDS). bf16 rows of
    two heads share a line, but 2 x 7501 bins exceed the limit, so the plan ungroups them."""
    cfg = dict(dim=2, B=1, H=heads, C=32, shapes=[(800, 1200), (3, 5)], Q=96, P=4,
               dtype=dtype, face_frac=0.0)
    value, shapes, loc, attn = bench.make_inputs(cfg)
    dt = bench.DTYPES[dtype]
    value, loc, attn = (t.to(dt) for t in (value, loc, attn))
    grad_out = _grad_out(cfg, dt)
    out, gv, gl, ga = _fwd_bwd(cfg, value, shapes, loc, attn, grad_out)
    _check_grads(value, shapes, loc, attn, grad_out, gv, gl, ga, 1e-4 if dtype == "fp32" else 1e-2)
