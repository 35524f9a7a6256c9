"""Producer-fused ops msda2d_fused / msda3d_fused (msda_fwd_fused / msda_bwd_fused).

The fused op forms loc = ref + offsets / (W, H[, D]) and attn = softmax over L*P inside the
kernel (reference modules: pytorch/msda_2d.py:303-339, pytorch/msda_3d.py:314-350).

CPU, pinning the oracle (oracle/torch_ref.msda_fused_ref) by what the mathematics fixes:
* samples placed on pixel centres of non-square levels with equal logits give the mean of
  the addressed value rows, read by plain indexing (a swapped normaliser axis or a
  per-level softmax fails this);
* adding a constant to all L*P logits of a (b, q, h) leaves the output unchanged, adding it
  to one level's logits does not (softmax over the flattened axis, not per level);
* a dominant logit selects its sample's value row;
* torch.autograd.gradcheck (finite differences) of the oracle in float64 with respect to
  value, reference points, offsets and logits.
CPU, host side: the workspace size entry point and the CPU-tensor refusal.
GPU: forward against the oracle (fp32 1e-5, bf16 1e-2 normwise); against the unfused HIP op
fed the kernel's own fp32 locations (fma(offset, 1/size, ref), reproduced as one rounding of
the exact float64 value) and torch's softmax weights (1e-6 fp32); gradients against autograd
of the float64 oracle (1e-4 normwise, fp32); and at the C2 / C5 workload sizes (staged
forward) against the unfused HIP op.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import msda_triton
from msda_triton import _lib
from oracle import torch_ref
from tests._util import max_rel


def _pixel_case(dim, seed=0):
    """Integer pixel-centre samples on non-square levels. Returns (value, shapes, ref, off,
    kidx): kidx[b, q, h, l, p] is the row of K each sample lands on exactly."""
    g = torch.Generator().manual_seed(seed)
    shapes_l = [(6, 10), (3, 5)] if dim == 2 else [(3, 4, 6), (2, 3, 5)]
    shapes = torch.tensor(shapes_l)
    B, Q, H, C, P = 2, 5, 3, 4, 2
    L = len(shapes_l)
    sizes = [int(np.prod(s)) for s in shapes_l]
    starts = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    value = torch.randn(B, sum(sizes), H, C, generator=g, dtype=torch.float64)
    ref = torch.empty(B, Q, L, dim, dtype=torch.float64)
    off = torch.empty(B, Q, H, L, P, dim, dtype=torch.float64)
    kidx = torch.empty(B, Q, H, L, P, dtype=torch.int64)
    for b in range(B):
        for q in range(Q):
            for lv, shp in enumerate(shapes_l):
                ext = shp[::-1]  # (W, H[, D]) in coordinate order
                base = [int(torch.randint(0, e, (1,), generator=g)) for e in ext]
                for d in range(dim):
                    ref[b, q, lv, d] = (base[d] + 0.5) / ext[d]
                for h in range(H):
                    for p in range(P):
                        idx = [int(torch.randint(0, e, (1,), generator=g)) for e in ext]
                        k = 0
                        for d in reversed(range(dim)):  # row-major (z, y, x)
                            off[b, q, h, lv, p, d] = idx[d] - base[d]
                            k = k * ext[d] + idx[d]
                        kidx[b, q, h, lv, p] = int(starts[lv]) + k
    return value, shapes, ref, off, kidx


def _rows(value, kidx):
    """value[b, kidx[b, q, h, l, p], h, :] as (B, Q, H, L, P, C)."""
    B, Q, H, L, P = kidx.shape
    bi = torch.arange(B).view(B, 1, 1, 1, 1).expand_as(kidx)
    hi = torch.arange(H).view(1, 1, H, 1, 1).expand_as(kidx)
    return value[bi, kidx, hi]


@pytest.mark.parametrize("dim", [2, 3])
def test_oracle_pixel_centres(dim):
    value, shapes, ref, off, kidx = _pixel_case(dim)
    B, Q, H, L, P = kidx.shape
    logits = torch.zeros(B, Q, H, L, P, dtype=torch.float64)  # equal weights 1 / (L * P)
    out = torch_ref.msda_fused_ref(value, shapes, ref, off, logits)
    expected = _rows(value, kidx).mean(dim=(3, 4)).reshape(B, Q, -1)
    assert torch.allclose(out, expected, atol=1e-12, rtol=0)


@pytest.mark.parametrize("dim", [2, 3])
def test_oracle_softmax_over_all_levels_and_points(dim):
    value, shapes, ref, off, kidx = _pixel_case(dim, seed=1)
    B, Q, H, L, P = kidx.shape
    g = torch.Generator().manual_seed(2)
    logits = torch.randn(B, Q, H, L, P, generator=g, dtype=torch.float64)
    out = torch_ref.msda_fused_ref(value, shapes, ref, off, logits)
    shifted = torch_ref.msda_fused_ref(value, shapes, ref, off, logits + 3.0)
    assert torch.allclose(out, shifted, atol=1e-12, rtol=0)
    one_level = logits.clone()
    one_level[:, :, :, 0] += 3.0
    assert (torch_ref.msda_fused_ref(value, shapes, ref, off, one_level) - out).abs().max() > 1e-3
    # a dominant logit (level 1, point 0) selects its sample's value row
    dom = torch.zeros_like(logits)
    dom[:, :, :, 1, 0] = 200.0
    sel = torch_ref.msda_fused_ref(value, shapes, ref, off, dom)
    assert torch.allclose(sel, _rows(value, kidx)[:, :, :, 1, 0].reshape(B, Q, -1), atol=1e-12, rtol=0)


def test_oracle_gradcheck():
    g = torch.Generator().manual_seed(3)
    shapes = torch.tensor([[5, 7], [3, 4]])
    B, Q, H, L, P, C = 1, 3, 2, 2, 2, 3
    K = int(shapes.prod(-1).sum())
    value = torch.randn(B, K, H, C, generator=g, dtype=torch.float64, requires_grad=True)
    ref = (0.2 + 0.6 * torch.rand(B, Q, L, 2, generator=g, dtype=torch.float64)).requires_grad_(True)
    off = torch.randn(B, Q, H, L, P, 2, generator=g, dtype=torch.float64).requires_grad_(True)
    logits = torch.randn(B, Q, H, L, P, generator=g, dtype=torch.float64).requires_grad_(True)
    assert torch.autograd.gradcheck(
        lambda v, r, o, lg: torch_ref.msda_fused_ref(v, shapes, r, o, lg),
        (value, ref, off, logits), eps=1e-6, atol=1e-6)


def _desc(**kw):
    d = _lib.MsdaDesc()
    base = dict(dim=2, batch=2, num_keys=19947, num_heads=8, channels=32, num_queries=19947,
                num_levels=4, num_points=4, value_dtype=_lib.MSDA_BF16,
                coord_dtype=_lib.MSDA_BF16, clamp_grid=1, flags=0, clamp_eps=1e-4)
    base.update(kw)
    for k, v in base.items():
        setattr(d, k, v)
    return d


def test_fused_workspace_bytes():
    lib = _lib.load()
    vals = (100, 150, 50, 75, 25, 38, 13, 19)
    shapes = ctypes.cast((ctypes.c_int32 * len(vals))(*vals), ctypes.c_void_p)
    d = _desc()
    fused = lib.msda_bwd_fused_workspace_bytes(ctypes.byref(d), shapes)
    d32 = _desc(coord_dtype=_lib.MSDA_F32)
    inner = lib.msda_bwd_workspace_bytes(ctypes.byref(d32), shapes)
    samples = 2 * 19947 * 8 * 4 * 4
    # fp32 locations + weights and their gradients, then the inner backward's workspace
    assert fused >= inner + samples * (2 + 1) * 4 * 2
    assert fused <= inner + samples * (2 + 1) * 4 * 2 + 5 * 256
    assert lib.msda_bwd_fused_workspace_bytes(ctypes.byref(_desc(num_points=0)), shapes) == 0


def test_cpu_tensors_are_refused():
    v = torch.randn(1, 6, 2, 4)
    with pytest.raises(ValueError, match="CUDA"):
        msda_triton.msda2d_fused(v, torch.tensor([[2, 3]]), torch.rand(1, 5, 1, 2),
                                 torch.randn(1, 5, 2, 1, 2, 2), torch.randn(1, 5, 2, 1, 2))


# ---------------------------------------------------------------------------------- GPU
def _inputs(dim, dtype, P=4, ref_levels=None, seed=7, Q=37, B=2, H=4, C=32, shapes=None):
    g = torch.Generator().manual_seed(seed)
    if shapes is None:
        shapes = [(12, 17), (6, 9), (3, 5)] if dim == 2 else [(4, 6, 7), (2, 3, 4)]
    L = len(shapes)
    K = sum(int(np.prod(s)) for s in shapes)
    value = torch.randn(B, K, H, C, generator=g)
    ref = torch.rand(B, Q, ref_levels or L, dim, generator=g)
    off = 2.0 * torch.randn(B, Q, H, L, P, dim, generator=g)  # pixels
    logits = torch.randn(B, Q, H, L, P, generator=g)
    dev = torch.device("cuda")
    return (value.to(dev, dtype), torch.tensor(shapes), ref.to(dev), off.to(dev, dtype),
            logits.to(dev, dtype))


def _op(dim, fwd_only=False):
    if dim == 2:
        return msda_triton.msda2d_fused_fwd if fwd_only else msda_triton.msda2d_fused
    return msda_triton.msda3d_fused_fwd if fwd_only else msda_triton.msda3d_fused


def _unfused(dim, value, shapes, ref, off, logits, autograd=False):
    """The plain HIP op on the locations and weights formed in fp32 by torch on the GPU
    (the autograd op with autograd=True, else the forward-only entry)."""
    B, Q, H, L, P, _ = off.shape
    inv = 1.0 / shapes.flip(-1).to(device=off.device, dtype=torch.float32)  # fp32 reciprocals
    # fma(off, inv, ref): the float64 product of two fp32 values is exact, one rounding after
    loc = (off.double() * inv.double()[None, None, None, :, None, :]
           + ref.double().expand(B, Q, L, dim)[:, :, None, :, None, :]).float()
    attn = logits.float().reshape(B, Q, H, L * P).softmax(-1).view(B, Q, H, L, P)
    if autograd:
        fn = msda_triton.msda2d if dim == 2 else msda_triton.msda3d
    else:
        fn = msda_triton.msda2d_fwd if dim == 2 else msda_triton.msda3d_fwd
    return fn(value, shapes, loc.contiguous(), attn.contiguous())


@pytest.mark.gpu
@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("P,ref_levels", [(4, None), (3, None), (4, 1)])
def test_forward_matches_oracle(dim, dtype, tol, P, ref_levels):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"fused fwd dim={dim} dtype={dtype} P={P} ref_levels={ref_levels}", flush=True)
    value, shapes, ref, off, logits = _inputs(dim, dtype, P=P, ref_levels=ref_levels)
    out = _op(dim, True)(value, shapes, ref, off, logits)
    want = torch_ref.msda_fused_ref(value.cpu().float(), shapes, ref.cpu().float(),
                                    off.cpu().float(), logits.cpu().float())
    assert out.dtype == dtype and out.shape == want.shape
    err = max_rel(out.float().cpu(), want)
    assert err <= tol
    # fp32 locations and weights formed by torch, through the plain op
    err = max_rel(out, _unfused(dim, value, shapes, ref, off, logits))
    assert err <= (1e-6 if dtype == torch.float32 else 1e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("ref_levels", [None, 1])
def test_backward_matches_oracle(dim, ref_levels):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"fused bwd dim={dim} ref_levels={ref_levels}", flush=True)
    _check_backward(dim, *_inputs(dim, torch.float32, ref_levels=ref_levels, Q=23))


@pytest.mark.gpu
@pytest.mark.parametrize("dim", [2, 3])
def test_backward_beyond_binning_matches_unfused(dim):
    """A pyramid with more than 8192 backward tiles per head: the inner backward takes the
    atomic grad_value plan (fp32 sums with global atomics, then one rounding pass). At 1024
    cells per axis one fp32 ulp of a location moves the pixel coordinate by ~6e-5 px, so
    the reference here is the plain autograd op on the same fp32 locations (formed with one
    rounding, as the kernels form them) and torch's softmax; the plain op itself is checked
    on such levels against the brute-force oracle with fp32 coordinates
    (tests/_parity.py::test_levels_beyond_binning_atomic_path)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print(f"fused bwd beyond binning dim={dim}", flush=True)
    shapes = [(1032, 1024), (3, 5)] if dim == 2 else [(72, 128, 128), (3, 5, 1)]
    value, shapes, ref, off, logits = _inputs(dim, torch.float32, Q=23, B=1, H=1, shapes=shapes)
    g = torch.Generator().manual_seed(11)
    grad = torch.randn(1, 23, value.shape[2] * value.shape[3], generator=g).to(value.device)
    a = [t.detach().clone().requires_grad_(True) for t in (value, ref, off, logits)]
    out = _op(dim)(a[0], shapes, *a[1:])
    out.backward(grad)
    b = [t.detach().clone().requires_grad_(True) for t in (value, ref, off, logits)]
    want = _unfused(dim, b[0], shapes, *b[1:], autograd=True)
    want.backward(grad)
    assert max_rel(out.detach(), want.detach()) <= 1e-6
    for name, x, y in zip(("value", "ref", "off", "logits"), a, b):
        assert x.grad is not None and x.grad.shape == y.grad.shape, name
        err = max_rel(x.grad, y.grad)
        assert err <= 1e-4, (name, err)


def _check_backward(dim, value, shapes, ref, off, logits):
    """Fused forward + backward on the GPU against the float64 oracle composition."""
    g = torch.Generator().manual_seed(11)
    grad = torch.randn(value.shape[0], off.shape[1], value.shape[2] * value.shape[3], generator=g)
    ins = [t.detach().clone().requires_grad_(True) for t in (value, ref, off, logits)]
    out = _op(dim)(ins[0], shapes, *ins[1:])
    out.backward(grad.to(out.device))
    cpu = [t.detach().cpu().double().requires_grad_(True) for t in (value, ref, off, logits)]
    want = torch_ref.msda_fused_ref(cpu[0], shapes, *cpu[1:])
    want.backward(grad.double())
    err = max_rel(out.detach().cpu(), want.detach())
    assert err <= 1e-5
    for name, a, b in zip(("value", "ref", "off", "logits"), ins, cpu):
        assert a.grad is not None and a.grad.shape == b.shape, name
        err = max_rel(a.grad.cpu(), b.grad)
        assert err <= 1e-4, name


@pytest.mark.gpu
@pytest.mark.parametrize("name,dtype,tol", [("c2", torch.bfloat16, 1e-2), ("c2", torch.float32, 1e-5),
                                            ("c5", torch.bfloat16, 1e-2)])
def test_full_size_matches_unfused(name, dtype, tol):
    """BASELINE.json's workload sizes (the staged forward and its shared-geometry path)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import bench
    cfg = bench.CONFIGS[name]
    print(f"fused full size {name} {dtype}", flush=True)
    value, shapes, ref, off, logits = _inputs(cfg["dim"], dtype, P=cfg["P"], Q=cfg["Q"], B=cfg["B"],
                                              H=cfg["H"], C=cfg["C"], shapes=cfg["shapes"], seed=5)
    out = _op(cfg["dim"], True)(value, shapes, ref, off, logits)
    want = _unfused(cfg["dim"], value, shapes, ref, off, logits)
    err = max_rel(out, want)
    assert err <= (1e-6 if dtype == torch.float32 else tol)
    # grad through the fused backward: value gradient equals the plain backward's
    if name == "c2" and dtype == torch.float32:
        v1 = value.detach().clone().requires_grad_(True)
        g = torch.randn_like(out)
        _op(2)(v1, shapes, ref, off, logits).backward(g)
        v2 = value.detach().clone().requires_grad_(True)
        B, Q, H, L, P, _ = off.shape
        norm = shapes.flip(-1).to(device=off.device, dtype=torch.float32)
        loc = ref[:, :, None, :, None, :] + off / norm[None, None, None, :, None, :]
        attn = logits.reshape(B, Q, H, L * P).softmax(-1).view(B, Q, H, L, P)
        msda_triton.msda2d(v2, shapes, loc.contiguous(), attn.contiguous()).backward(g)
        err = max_rel(v1.grad, v2.grad)
        assert err <= 1e-5
