"""GPU parity at BASELINE.json's full workload sizes.

The small-shape suites (tests/_parity.py) never reach the staged forward kernel, which is
chosen only when every workgroup gets at least kFwdStageMinQueries queries; these cases do,
and they cover the configurations bench.py measures:
  C2  2D encoder B=2 Q=K=19947 L=4 P=4 (bf16, fp32)      staged forward
  C3  2D decoder B=8 Q=300                 (bf16)       unstaged forward (few queries)
  C5  3D 4-level B=1 Q=32768 P=8, 10% of points near a face, clamp_eps=1e-4 (bf16)
The oracle is oracle/torch_ref (the reference's msda*_pytorch restated) in fp32 on the
same (upcast) inputs, on the CPU. Tolerances: forward max|out-ref|/max|ref| <= 1e-5 (fp32),
<= 1e-2 (bf16); grad_value and grad_attention_weights normwise <= 1e-2 (bf16 storage of
every input and gradient). grad_sampling_locations is left to the fp32 small-shape suites:
in bf16 its derivative jumps at cell edges, where one rounding of a coordinate selects
another cell.
"""

from __future__ import annotations

import pytest
import torch

import bench
import msda_triton
from oracle import torch_ref
from tests._util import max_rel

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


@pytest.mark.parametrize("name", ["c2", "c5"])
def test_backward_full_size(name):
    cfg, value, shapes, loc, attn = _case(name)
    dev = torch.device("cuda")
    print(f"full-size backward {name}", flush=True)
    g = torch.Generator().manual_seed(7)
    grad_out = torch.randn(cfg["B"], cfg["Q"], cfg["H"] * cfg["C"], generator=g).to(value.dtype)
    op = msda_triton.msda2d if cfg["dim"] == 2 else msda_triton.msda3d
    v, lo, a = [t.to(dev).requires_grad_(True) for t in (value, loc, attn)]
    out = op(v, shapes, lo, a, True, 1e-4)
    out.backward(grad_out.to(dev))
    _, tv, tl, ta = torch_ref.msda_ref_grads(value.float(), shapes, loc.float(), attn.float(),
                                             grad_out.float(), True, 1e-4)
    assert max_rel(v.grad.float().cpu(), tv) <= 1e-2
    assert max_rel(a.grad.float().cpu(), ta) <= 1e-2
    # sum over all gradients of grad_value equals sum_q attn * grad_out over valid corners:
    # checked through the oracle above; here the size-independent identity
    # <grad_value, value> == <grad_out, out> (linearity of the op in value)
    lhs = (v.grad.double() * v.detach().double()).sum().item()
    rhs = (grad_out.to(dev).double() * out.detach().double()).sum().item()
    assert abs(lhs - rhs) <= 1e-2 * max(1.0, abs(rhs))
