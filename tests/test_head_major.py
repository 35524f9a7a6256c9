"""GPU tests of the head-major value copy (msda_fwd_workspace_bytes / the backward's plan).

The copy is taken when value rows are shorter than a 128-byte line, there are several
heads, K * 128 bytes exceed an XCD's 4 MB L2 and the gathers outnumber the keys eightfold.
The cases here meet that rule at sizes the oracle finishes in seconds:
  * the forward through the workspace equals the forward without it, bit for bit;
  * forward and backward match the fp32 oracle (oracle/torch_ref) on the same bf16 inputs
    at the bf16 tolerances (forward max-relative <= 1e-2, grad_value / grad_attn normwise
    <= 1e-2), and fp32 inputs of a 16-channel head at the fp32 ones.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import msda_triton
from msda_triton import _lib
from msda_triton.hip import _core
from oracle import torch_ref
from tests._util import make_inputs, max_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _case(dim, dtype, ch=32):
    ss = [(200, 200)] if dim == 2 else [(34, 34, 34)]
    value, shapes, loc, attn = make_inputs(dim, batch_size=1, num_queries=20000 if dim == 2 else 10000,
                                           num_heads=2, dim_per_head=ch, num_levels=1,
                                           num_points=4, spatial_shapes=ss)
    return value.to(dtype), shapes, loc.to(dtype), attn.to(dtype)


def _fwd_direct(dim, value, shapes, loc, attn, use_ws):
    """msda_fwd through the C ABI with or without the optional workspace."""
    lib = _lib.load()
    dev = torch.device("cuda")
    v, lo, a = (t.to(dev).contiguous() for t in (value, loc, attn))
    levels = _core.prepare_levels(dim, v, shapes)
    desc = _core.make_desc(dim, v, lo, lo.dtype, True, 1e-4)
    n = int(lib.msda_fwd_workspace_bytes(ctypes.byref(desc)))
    assert n == v.numel() * v.element_size(), "case does not take the head-major path"
    ws = torch.empty(n, device=dev, dtype=torch.uint8) if use_ws else None
    out = torch.empty(v.shape[0], lo.shape[1], v.shape[2] * v.shape[3], device=dev, dtype=v.dtype)
    rc = lib.msda_fwd(ctypes.byref(desc), v.data_ptr(), levels.spatial.data_ptr(),
                      levels.starts.data_ptr(), lo.data_ptr(), a.data_ptr(), out.data_ptr(),
                      ws.data_ptr() if use_ws else None, n if use_ws else 0,
                      torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "msda_fwd")
    return out.cpu()


@pytest.mark.parametrize("dim", [2, 3])
def test_head_major_forward_bit_identical(dim):
    value, shapes, loc, attn = _case(dim, torch.bfloat16)
    print(f"head-major forward dim={dim}", flush=True)
    a = _fwd_direct(dim, value, shapes, loc, attn, use_ws=True)
    b = _fwd_direct(dim, value, shapes, loc, attn, use_ws=False)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dim,dtype,ch,tol", [(2, torch.bfloat16, 32, 1e-2), (3, torch.bfloat16, 32, 1e-2),
                                              (2, torch.float32, 16, 1e-4)])
def test_head_major_parity(dim, dtype, ch, tol):
    value, shapes, loc, attn = _case(dim, dtype, ch)
    dev = torch.device("cuda")
    print(f"head-major parity dim={dim} {dtype} C={ch}", flush=True)
    op = msda_triton.msda2d if dim == 2 else msda_triton.msda3d
    v, lo, a = [t.to(dev).requires_grad_(True) for t in (value, loc, attn)]
    out = op(v, shapes, lo, a, True, 1e-4)
    grad_out = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(dtype)
    out.backward(grad_out.to(dev))
    ref, tv, tl, ta = torch_ref.msda_ref_grads(value.float(), shapes, loc.float(), attn.float(),
                                               grad_out.float(), True, 1e-4)
    fwd_tol = 1e-2 if dtype != torch.float32 else 1e-5
    assert max_rel(out.detach().float().cpu(), ref) <= fwd_tol
    assert max_rel(v.grad.float().cpu(), tv) <= tol
    assert max_rel(a.grad.float().cpu(), ta) <= tol


def _bwd(dim, value, shapes, loc, attn, grad_out, given_hm):
    """_core.backward on the GPU, with the value's head-major copy supplied by the caller
    (MSDA_FLAG_VALUE_HEAD_MAJOR) or not."""
    dev = torch.device("cuda")
    v, lo, a, g = (t.to(dev).contiguous() for t in (value, loc, attn, grad_out))
    levels = _core.prepare_levels(dim, v, shapes)
    hm = v.permute(0, 2, 1, 3).contiguous() if given_hm else None
    gv, gl, ga = _core.backward(dim, g, v, levels, lo, a, True, 1e-4, value_hm=hm)
    return gv.cpu(), gl.cpu(), ga.cpu()


def _same_grads(x, y, tol):
    """grad_loc and grad_attn come from the same per-sample arithmetic: equal bit for bit;
    grad_value sums the same terms, in an order that LDS atomics (binned path) or global
    atomics (atomic path) do not fix."""
    assert torch.equal(x[1], y[1]) and torch.equal(x[2], y[2])
    assert max_rel(x[0].float(), y[0].float()) <= tol


@pytest.mark.parametrize("dim,dtype,tol", [(2, torch.bfloat16, 1e-2), (3, torch.bfloat16, 1e-2),
                                           (2, torch.float32, 1e-6)])
def test_backward_from_caller_head_major_value(dim, dtype, tol):
    """A caller-supplied head-major value (what the autograd function passes on from the
    forward's workspace) gives the gradients of the backward's own relayout."""
    value, shapes, loc, attn = _case(dim, dtype, 32 if dtype != torch.float32 else 16)
    grad_out = torch.randn(value.shape[0], loc.shape[1], value.shape[2] * value.shape[3],
                           generator=torch.Generator().manual_seed(9)).to(dtype)
    print(f"caller head-major dim={dim} {dtype}", flush=True)
    _same_grads(_bwd(dim, value, shapes, loc, attn, grad_out, True),
                _bwd(dim, value, shapes, loc, attn, grad_out, False), tol)


@pytest.mark.parametrize("dim", [2, 3])
def test_caller_head_major_value_on_small_and_atomic_plans(dim):
    """The flag also holds where the backward would not relayout itself: a small pyramid (the
    plan then keeps one head per group) and levels beyond the LDS binning (atomic path: the
    fp32 sums follow the head-major layout and the rounding pass transposes them back)."""
    if dim == 2:
        cases = [dict(ss=[(32, 32), (16, 16)], q=100, b=1), dict(ss=[(1032, 1024), (3, 5)], q=64, b=2)]
    else:
        cases = [dict(ss=[(8, 8, 8), (4, 4, 4)], q=100, b=1), dict(ss=[(72, 128, 128), (3, 5, 1)], q=64, b=1)]
    for c in cases:
        value, shapes, loc, attn = make_inputs(dim, batch_size=c["b"], num_queries=c["q"], num_heads=2,
                                               dim_per_head=32, num_levels=len(c["ss"]), num_points=4,
                                               spatial_shapes=c["ss"])
        grad_out = torch.randn(c["b"], c["q"], 2 * 32, generator=torch.Generator().manual_seed(3))
        print(f"caller head-major dim={dim} shapes={c['ss']}", flush=True)
        _same_grads(_bwd(dim, value, shapes, loc, attn, grad_out, True),
                    _bwd(dim, value, shapes, loc, attn, grad_out, False), 1e-5)
