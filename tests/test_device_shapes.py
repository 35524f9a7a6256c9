"""GPU: level shapes resident on the device, forward and backward without a host read.

The reference keeps GPU-resident shapes on the device and never synchronises
(src/msda_triton/triton/msda_2d.py:76-82, backward :799-851). Here the backward of such a
call goes through msda_bwd_dev / msda_bwd_fused_dev: the host sizes the launch from K and
a first kernel derives the tile geometry from the device shapes. Checks:
  * same results as the host-shapes path on the same inputs: the forward and
    grad_sampling_locations / grad_attention_weights bit for bit (same kernels, same
    geometry), grad_value to 1e-6 normwise (fp32; a cell's entries are summed in the order
    LDS atomics ranked them), and all three against the float64 brute-force oracle with
    the kernels' fp32 coordinate rounding at the north-star 1e-4 (fp32) / 1e-2 (bf16);
  * pyramids with thin levels, which need more tiles than the host's estimate from K, fall
    back on the device to the atomic grad_value path, with the same oracle bounds;
  * shapes inconsistent with K give NaN gradients (the error cannot be returned from the
    device), with no fault: every kernel reads the geometry first and exits;
  * the fused producer op's backward with device shapes equals its host-shapes backward;
  * fwd+bwd with device shapes captured in a HIP graph replays correctly on fresh inputs.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import msda_triton
from msda_triton import _lib
from msda_triton.hip import _core
from oracle import brute
from tests._util import make_inputs, max_rel

pytestmark = pytest.mark.gpu

CASES = {
    "2d": dict(dim=2, batch_size=2, num_queries=300, num_heads=8, num_points=4,
               spatial_shapes=[(40, 60), (20, 30), (10, 15), (5, 8)]),
    "3d": dict(dim=3, batch_size=1, num_queries=400, num_heads=4, num_points=4,
               spatial_shapes=[(8, 16, 16), (4, 8, 8), (2, 4, 4)]),
    # thin levels: 1025 tiles along x on the first level, far beyond the estimate from K
    "2d_thin": dict(dim=2, batch_size=1, num_queries=40, num_heads=2, num_points=4,
                    spatial_shapes=[(2, 16400), (3, 5)]),
    "3d_thin": dict(dim=3, batch_size=1, num_queries=40, num_heads=2, num_points=4,
                    spatial_shapes=[(2, 2, 8200), (2, 3, 4)]),
}


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _inputs(case, dtype, seed=42):
    cfg = dict(CASES[case])
    dim = cfg.pop("dim")
    value, shapes, loc, attn = make_inputs(dim, dtype=dtype, seed=seed, **cfg)
    g = torch.Generator().manual_seed(seed + 1)
    grad_out = torch.randn(value.shape[0], loc.shape[1], value.shape[2] * value.shape[3],
                           generator=g).to(dtype)
    return dim, value, shapes, loc, attn, grad_out


def _fwd_bwd(dim, value, shapes, loc, attn, grad_out):
    dev = torch.device("cuda")
    op = msda_triton.msda2d if dim == 2 else msda_triton.msda3d
    v, lo, a = [t.to(dev).requires_grad_(True) for t in (value, loc, attn)]
    out = op(v, shapes, lo, a)
    out.backward(grad_out.to(dev))
    return [t.detach().cpu() for t in (out, v.grad, lo.grad, a.grad)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("case", sorted(CASES))
def test_device_shapes_match_host_shapes_and_oracle(case, dtype):
    print(f"device shapes {case} {dtype}", flush=True)
    dim, value, shapes, loc, attn, grad_out = _inputs(case, dtype)
    host = _fwd_bwd(dim, value, shapes, loc, attn, grad_out)
    dev = _fwd_bwd(dim, value, shapes.to("cuda", torch.int32), loc, attn, grad_out)
    assert torch.equal(host[0], dev[0]), "forward differs"
    thin = case.endswith("thin")
    if not thin:
        # same binned kernels on the same geometry
        assert torch.equal(host[2], dev[2]), "grad_loc differs"
        assert torch.equal(host[3], dev[3]), "grad_attn differs"
    tol_same = 1e-6 if dtype == torch.float32 else 1e-2
    for name, x, y in zip(("grad_value", "grad_loc", "grad_attn"), host[1:], dev[1:]):
        assert max_rel(y, x) <= tol_same, f"{name} host vs device shapes: {max_rel(y, x):.3e}"
    vf, lf, af, gf = (t.float() for t in (value, loc, attn, grad_out))
    bv, bl, ba = brute.bwd(vf, shapes, lf, af, gf, coord_f32=True)
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    for name, x, r in zip(("grad_value", "grad_loc", "grad_attn"), dev[1:], (bv, bl, ba)):
        assert max_rel(x, r) <= tol, f"{name} vs brute: {max_rel(x, r):.3e}"


def test_thin_levels_exceed_the_estimate():
    """The thin-level cases above really take the device-side fallback: with host shapes
    their plan is binned (1026 tiles per head fit the 8192-bin binning), but their tiles
    exceed what msda_bwd_dev_workspace_bytes sized for, which then includes the fp32 sums of
    the atomic path (host-only check)."""
    lib = _lib.load()
    dim, value, shapes, loc, attn, _ = _inputs("2d_thin", torch.float32)
    desc = _core.make_desc(dim, value, loc, torch.float32, True, 1e-4)
    hs = shapes.to(torch.int32).contiguous()
    host_ws = lib.msda_bwd_workspace_bytes(ctypes.byref(desc), ctypes.c_void_p(hs.data_ptr()))
    dev_ws = lib.msda_bwd_dev_workspace_bytes(ctypes.byref(desc))
    assert host_ws > 0 and dev_ws > 0, _lib.last_error()
    sums = value.numel() * 4
    assert dev_ws >= sums  # fp32 sums of the fallback
    # estimate: 1.5 * ceil(K / 128) + 4 * 2^dim * L + 64 tiles per head < 1026
    K = value.shape[1]
    assert (K + 127) // 128 * 3 // 2 + 4 * 4 * 2 + 64 < 1026


@pytest.mark.parametrize("dim", [2, 3])
def test_inconsistent_device_shapes_give_nan_gradients(dim):
    """Device shapes whose sizes do not add up to K: the forward cannot check them (the
    reference's GPU path does not either), and the backward fills every gradient with NaN
    instead of reading or writing outside the level tables. The forward reads value rows
    through the buffer range check, so it stays within value."""
    case = "2d" if dim == 2 else "3d"
    _, value, shapes, loc, attn, grad_out = _inputs(case, torch.float32)
    bad = shapes.clone()
    bad[0, -1] += 1  # one more column (or x-slice) on the first level: sum exceeds K
    dev = torch.device("cuda")
    op = msda_triton.msda2d if dim == 2 else msda_triton.msda3d
    v, lo, a = [t.to(dev).requires_grad_(True) for t in (value, loc, attn)]
    out = op(v, bad.to(dev, torch.int32), lo, a)
    out.backward(grad_out.to(dev))
    torch.cuda.synchronize()
    for name, g in (("grad_value", v.grad), ("grad_loc", lo.grad), ("grad_attn", a.grad)):
        assert torch.isnan(g).all(), f"{name} is not all NaN"


@pytest.mark.parametrize("dim", [2, 3])
def test_fused_device_shapes_match_host_shapes(dim):
    print(f"fused device shapes dim={dim}", flush=True)
    g = torch.Generator().manual_seed(3)
    shapes_l = [(12, 17), (6, 9), (3, 5)] if dim == 2 else [(4, 6, 7), (2, 3, 4)]
    L, B, Q, H, C, P = len(shapes_l), 2, 37, 4, 32, 4
    K = sum(int(torch.tensor(s).prod()) for s in shapes_l)
    dev = torch.device("cuda")
    value = torch.randn(B, K, H, C, generator=g).to(dev)
    ref = torch.rand(B, Q, L, dim, generator=g).to(dev)
    off = (2.0 * torch.randn(B, Q, H, L, P, dim, generator=g)).to(dev)
    logits = torch.randn(B, Q, H, L, P, generator=g).to(dev)
    grad = torch.randn(B, Q, H * C, generator=g).to(dev)
    shapes = torch.tensor(shapes_l)
    op = msda_triton.msda2d_fused if dim == 2 else msda_triton.msda3d_fused
    res = []
    for sh in (shapes, shapes.to(dev, torch.int32)):
        ins = [t.detach().clone().requires_grad_(True) for t in (value, ref, off, logits)]
        out = op(ins[0], sh, *ins[1:])
        out.backward(grad)
        res.append([out.detach()] + [t.grad for t in ins])
    assert torch.equal(res[0][0], res[1][0])
    for name, x, y in zip(("value", "ref", "off", "logits"), res[0][1:], res[1][1:]):
        assert max_rel(y, x) <= 1e-6, f"grad {name}: {max_rel(y, x):.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("case", ["2d", "3d"])
def test_graph_capture_with_device_shapes(case, dtype):
    """Forward + backward with device shapes captured once and replayed on fresh inputs,
    with eager work between replays; each replay matches an eager run."""
    print(f"graph device shapes {case} {dtype}", flush=True)
    dev = torch.device("cuda:0")
    dim, value, shapes, loc, attn, grad_out = _inputs(case, dtype, seed=0)
    v, lo, a, go = (t.to(dev) for t in (value, loc, attn, grad_out))
    shapes_dev = shapes.to(dev, torch.int32)
    levels = _core.prepare_levels(dim, v, shapes_dev)
    assert levels.host is None

    def step():
        out = _core.forward(dim, v, levels, lo, a, True, 1e-4)[0]
        return (out, *_core.backward(dim, go, v, levels, lo, a, True, 1e-4))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    for rep in range(3):
        _, nv, _, nlo, na, ngo = _inputs(case, dtype, seed=rep + 1)
        for dst, src in ((v, nv), (lo, nlo), (a, na), (go, ngo)):
            dst.copy_(src.to(dev))
        graph.replay()
        eager = step()
        torch.cuda.synchronize()
        assert torch.equal(static[0], eager[0]), f"replay {rep}: forward differs"
        for name, x, y in zip(("grad_value", "grad_loc", "grad_attn"), static[1:], eager[1:]):
            assert max_rel(x, y) <= tol, f"replay {rep}: {name} {max_rel(x, y):.3e}"
