"""torch.library custom ops (msda_triton::msda_fwd / msda_bwd) used under torch.compile.

CPU: both ops are registered and their fake (shape) functions follow the tensor contract.
GPU: torch.library.opcheck on both ops; msda2d / msda3d inside torch.compile(fullgraph=True)
(no graph break; aot_eager backend, so no code generation is involved) give the eager
forward and gradients (grad_value to fp32 rounding: its in-tile summation order is not
fixed), and msda*_fwd stays non-differentiable when compiled, as in eager.
"""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import msda_triton
from tests._util import make_inputs, max_rel


def test_ops_registered_with_shape_functions():
    fwd, bwd = torch.ops.msda_triton.msda_fwd, torch.ops.msda_triton.msda_bwd
    with FakeTensorMode():
        v = torch.empty(2, 100, 8, 32, dtype=torch.bfloat16)
        s = torch.empty(2, 3, dtype=torch.int64)
        lo = torch.empty(2, 7, 8, 2, 4, 3)
        a = torch.empty(2, 7, 8, 2, 4)
        out = fwd(v, s, lo, a, 3, True, 1e-4)
        assert out.shape == (2, 7, 256) and out.dtype == torch.bfloat16
        gv, gl, ga = bwd(torch.empty(2, 7, 256, dtype=torch.bfloat16), v, s, lo, a, 3, True, 1e-4)
        assert gv.shape == v.shape and gv.dtype == v.dtype
        assert gl.shape == lo.shape and gl.dtype == lo.dtype and ga.shape == a.shape


def _gpu_inputs(dim, dtype=torch.float32):
    value, shapes, loc, attn = make_inputs(dim, batch_size=2, num_queries=40)
    dev = torch.device("cuda")
    return value.to(dev, dtype), shapes, loc.to(dev, dtype), attn.to(dev, dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("dim", [2, 3])
def test_opcheck(dim):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    v, s, lo, a = _gpu_inputs(dim)
    print(f"opcheck dim={dim}", flush=True)
    v, lo, a = (t.requires_grad_(True) for t in (v, lo, a))
    torch.library.opcheck(torch.ops.msda_triton.msda_fwd.default, (v, s, lo, a, dim, True, 1e-4),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
    g = torch.randn(v.shape[0], lo.shape[1], v.shape[2] * v.shape[3], device=v.device)
    torch.library.opcheck(torch.ops.msda_triton.msda_bwd.default,
                          (g, v.detach(), s, lo.detach(), a.detach(), dim, True, 1e-4),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
@pytest.mark.parametrize("dim", [2, 3])
def test_compiled_matches_eager(dim):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    op = msda_triton.msda2d if dim == 2 else msda_triton.msda3d
    fwd = msda_triton.msda2d_fwd if dim == 2 else msda_triton.msda3d_fwd
    v, s, lo, a = _gpu_inputs(dim)
    print(f"compile dim={dim}", flush=True)

    def step(v, lo, a):
        return (op(v, s, lo, a) * 1.5).sum()

    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    grads = []
    for fn in (step, compiled):
        vv, ll, aa = (t.detach().clone().requires_grad_(True) for t in (v, lo, a))
        loss = fn(vv, ll, aa)
        loss.backward()
        grads.append((loss.detach(), vv.grad, ll.grad, aa.grad))
    (l0, *g0), (l1, *g1) = grads
    assert max_rel(l1, l0) <= 1e-6
    for x, y in zip(g1, g0):
        assert max_rel(x, y) <= 1e-6
    cfwd = torch.compile(lambda v, lo, a: fwd(v, s, lo, a), backend="aot_eager", fullgraph=True)
    out = cfwd(v.requires_grad_(True), lo, a)
    assert out.grad_fn is None
    assert torch.equal(out, fwd(v, s, lo, a))


def _fused_inputs(dim):
    g = torch.Generator().manual_seed(3)
    shapes = torch.tensor([[6, 9], [3, 5]] if dim == 2 else [[3, 4, 5], [2, 2, 3]])
    B, Q, H, C, L, P = 2, 19, 4, 16, 2, 4
    K = int(shapes.prod(-1).sum())
    dev = torch.device("cuda")
    value = torch.randn(B, K, H, C, generator=g).to(dev)
    ref = torch.rand(B, Q, L, dim, generator=g).to(dev)
    off = torch.randn(B, Q, H, L, P, dim, generator=g).to(dev)
    logits = torch.randn(B, Q, H, L, P, generator=g).to(dev)
    return value, shapes, ref, off, logits


def test_fused_ops_registered_with_shape_functions():
    fwd, bwd = torch.ops.msda_triton.msda_fwd_fused, torch.ops.msda_triton.msda_bwd_fused
    with FakeTensorMode():
        v = torch.empty(2, 100, 8, 32, dtype=torch.bfloat16)
        s = torch.empty(2, 2, dtype=torch.int64)
        r = torch.empty(2, 7, 1, 2)
        o = torch.empty(2, 7, 8, 2, 4, 2, dtype=torch.bfloat16)
        lg = torch.empty(2, 7, 8, 8, dtype=torch.bfloat16)
        out = fwd(v, s, r, o, lg, 2, True, 1e-4)
        assert out.shape == (2, 7, 256) and out.dtype == torch.bfloat16
        gv, gr, go, gl = bwd(torch.empty(2, 7, 256, dtype=torch.bfloat16), v, s, r, o, lg, 2, True, 1e-4)
        assert gv.shape == v.shape and gr.shape == r.shape and go.shape == o.shape
        assert gl.shape == lg.shape and gl.dtype == lg.dtype


@pytest.mark.gpu
@pytest.mark.parametrize("dim", [2, 3])
def test_fused_opcheck_and_compile(dim):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"fused opcheck/compile dim={dim}", flush=True)
    value, shapes, ref, off, logits = _fused_inputs(dim)
    args = tuple(t.clone().requires_grad_(True) for t in (value, ref, off, logits))
    torch.library.opcheck(torch.ops.msda_triton.msda_fwd_fused.default,
                          (args[0], shapes, *args[1:], dim, True, 1e-4),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
    op = msda_triton.msda2d_fused if dim == 2 else msda_triton.msda3d_fused

    def step(v, r, o, lg):
        return (op(v, shapes, r, o, lg) * 1.5).sum()

    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    grads = []
    for fn in (step, compiled):
        ins = [t.detach().clone().requires_grad_(True) for t in (value, ref, off, logits)]
        loss = fn(*ins)
        loss.backward()
        grads.append((loss.detach(), *(t.grad for t in ins)))
    for x, y in zip(grads[1], grads[0]):
        err = max_rel(x, y)
        assert err <= 1e-6
