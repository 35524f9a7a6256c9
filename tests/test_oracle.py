"""CPU tests that pin the oracle before any kernel is compared against it.

The reference ships no golden vectors or known-answer files for this path (its tests
recompute the PyTorch oracle on the fly, tests/test_msda_2d.py:113-427), so both oracle
functions are pinned here by what the mathematics fixes:

* closed forms of bilinear / trilinear sampling with grid = 2*loc - 1 and
  align_corners=False: a constant field, an affine field (value and exact location
  gradient), pixel-centre sampling that returns value rows, and a permutation gather;
* zero padding and clamp semantics with hand-computed expectations;
* float64 finite differences of the brute-force forward against its analytic backward;
* linearity in value and in attention weights;
* agreement of the two independent restatements (explicit loops in oracle/msda_brute.c,
  F.grid_sample composition in oracle/torch_ref.py) on seeded inputs, and
  torch.autograd.gradcheck of the latter.

Every closed form uses a non-square level and unequal axis slopes, so a swapped x/y (or
z), a dropped chain factor W/H/D, or a sign error in a corner weight fails a test.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import brute, torch_ref
from tests._util import make_inputs, max_rel

SHAPES_2D = [(5, 7), (3, 4)]          # (H, W) per level, deliberately non-square
SHAPES_3D = [(3, 5, 6), (2, 3, 4)]    # (D, H, W)


def _level_sizes(shapes):
    return [int(np.prod(s)) for s in shapes]


def _interior_locs(rng, shape_rev, n):
    """Locations whose pixel coordinate lies in [0.1, size-1.1] on every axis (all corners
    valid). shape_rev is the axis order of loc: (W, H[, D])."""
    out = np.empty((n, len(shape_rev)))
    for k, size in enumerate(shape_rev):
        u = rng.uniform(0.1, size - 1.1, size=n)
        out[:, k] = (u + 0.5) / size           # u = loc*size - 0.5 for align_corners=False
    return out


def _affine_value(shapes, dim, B, H, C, coef):
    """value[b, k, h, c] = coef[h, c] . (x, y[, z]) + coef0[h, c] at key k's pixel position."""
    rows = []
    for shp in shapes:
        if dim == 2:
            hh, ww = shp
            yy, xx = np.meshgrid(np.arange(hh), np.arange(ww), indexing="ij")
            pos = np.stack([xx.ravel(), yy.ravel()], -1)
        else:
            dd, hh, ww = shp
            zz, yy, xx = np.meshgrid(np.arange(dd), np.arange(hh), np.arange(ww), indexing="ij")
            pos = np.stack([xx.ravel(), yy.ravel(), zz.ravel()], -1)
        rows.append(pos)
    pos = np.concatenate(rows, 0).astype(np.float64)          # (K, dim)
    lin = np.einsum("kd,hcd->khc", pos, coef[..., :dim]) + coef[..., dim]
    return np.broadcast_to(lin, (B,) + lin.shape).copy()


@pytest.mark.parametrize("dim", [2, 3])
def test_brute_constant_field(dim):
    shapes = SHAPES_2D if dim == 2 else SHAPES_3D
    rng = np.random.default_rng(1)
    B, Q, H, C, L, P = 2, 9, 3, 4, len(shapes), 3
    K = sum(_level_sizes(shapes))
    value = np.full((B, K, H, C), 2.5)
    loc = np.empty((B, Q, H, L, P, dim))
    for l, shp in enumerate(shapes):
        loc[:, :, :, l] = _interior_locs(rng, shp[::-1], B * Q * H * P).reshape(B, Q, H, P, dim)
    attn = rng.uniform(0, 1, (B, Q, H, L, P))
    out = brute.fwd(value, torch.tensor(shapes), loc, attn)
    expect = 2.5 * attn.sum((-1, -2))                         # (B, Q, H)
    np.testing.assert_allclose(out.reshape(B, Q, H, C), np.repeat(expect[..., None], C, -1),
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dim", [2, 3])
def test_brute_affine_field_value_and_gradient(dim):
    """An affine field is reproduced exactly by bilinear/trilinear interpolation, and
    d out / d loc_axis = attn * slope_axis * size_axis (u = loc*size - 0.5)."""
    shapes = SHAPES_2D if dim == 2 else SHAPES_3D
    rng = np.random.default_rng(2)
    B, Q, H, C, L, P = 1, 7, 2, 3, len(shapes), 2
    coef = rng.uniform(-2, 2, (H, C, dim + 1))
    coef[..., 1] += 3.0                                       # y slope differs from x slope
    value = _affine_value(shapes, dim, B, H, C, coef)
    loc = np.empty((B, Q, H, L, P, dim))
    for l, shp in enumerate(shapes):
        loc[:, :, :, l] = _interior_locs(rng, shp[::-1], B * Q * H * P).reshape(B, Q, H, P, dim)
    attn = rng.uniform(0.1, 1, (B, Q, H, L, P))
    out = brute.fwd(value, torch.tensor(shapes), loc, attn, clamp_grid=False)
    expect = np.zeros((B, Q, H, C))
    for l, shp in enumerate(shapes):
        sizes = shp[::-1]                                     # (W, H[, D]) in loc order
        u = loc[:, :, :, l] * np.array(sizes) - 0.5           # (B, Q, H, P, dim)
        f = np.einsum("bqhpd,hcd->bqhpc", u, coef[..., :dim]) + coef[None, None, :, None, :, dim]
        expect += np.einsum("bqhp,bqhpc->bqhc", attn[:, :, :, l], f)
    np.testing.assert_allclose(out.reshape(B, Q, H, C), expect, rtol=1e-11, atol=1e-11)

    grad_out = rng.standard_normal((B, Q, H * C))
    gv, gl, ga = brute.bwd(value, torch.tensor(shapes), loc, attn, grad_out, clamp_grid=False)
    go = grad_out.reshape(B, Q, H, C)
    for l, shp in enumerate(shapes):
        sizes = np.array(shp[::-1], dtype=np.float64)
        slope = np.einsum("bqhc,hcd->bqhd", go, coef[..., :dim])  # d<go, f>/du
        exp_gl = attn[:, :, :, l][..., None] * slope[:, :, :, None, :] * sizes
        np.testing.assert_allclose(gl[:, :, :, l], exp_gl, rtol=1e-10, atol=1e-10)
        u = loc[:, :, :, l] * sizes - 0.5
        f = np.einsum("bqhpd,hcd->bqhpc", u, coef[..., :dim]) + coef[None, None, :, None, :, dim]
        np.testing.assert_allclose(ga[:, :, :, l], np.einsum("bqhc,bqhpc->bqhp", go, f),
                                   rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("dim", [2, 3])
def test_brute_pixel_centres_and_permutation(dim):
    """L = P = 1 and Q = K with every query at a distinct pixel centre: out is a permutation
    of value rows; the backward scatters grad_out back through the same permutation."""
    shp = (4, 6) if dim == 2 else (2, 3, 5)
    K = int(np.prod(shp))
    rng = np.random.default_rng(3)
    B, H, C = 2, 2, 5
    value = rng.standard_normal((B, K, H, C))
    perm = rng.permutation(K)
    if dim == 2:
        ys, xs = np.unravel_index(perm, shp)
        pix = np.stack([xs, ys], -1)
    else:
        zs, ys, xs = np.unravel_index(perm, shp)
        pix = np.stack([xs, ys, zs], -1)
    loc1 = (pix + 0.5) / np.array(shp[::-1])
    loc = np.broadcast_to(loc1[None, :, None, None, None, :], (B, K, H, 1, 1, dim)).copy()
    attn = np.ones((B, K, H, 1, 1))
    out = brute.fwd(value, torch.tensor([shp]), loc, attn, clamp_grid=False)
    np.testing.assert_allclose(out.reshape(B, K, H, C), value[:, perm], rtol=0, atol=1e-12)
    grad_out = rng.standard_normal((B, K, H * C))
    gv, _, ga = brute.bwd(value, torch.tensor([shp]), loc, attn, grad_out, clamp_grid=False)
    expect = np.zeros_like(value)
    expect[:, perm] = grad_out.reshape(B, K, H, C)
    np.testing.assert_allclose(gv, expect, rtol=0, atol=1e-12)
    np.testing.assert_allclose(ga[..., 0, 0], (grad_out.reshape(B, K, H, C) * value[:, perm]).sum(-1),
                               rtol=1e-12, atol=1e-12)


def test_brute_zero_padding_and_clamp():
    """Hand-computed 1x2 level: value row 0 = 1, row 1 = 3 (W = 2, H = 1)."""
    shapes = torch.tensor([(1, 2)])
    value = np.array([1.0, 3.0]).reshape(1, 2, 1, 1)
    attn = np.ones((1, 1, 1, 1, 1))

    def at(x, y, clamp, eps=1e-4):
        loc = np.array([x, y], dtype=np.float64).reshape(1, 1, 1, 1, 1, 2)
        return brute.fwd(value, shapes, loc, attn, clamp_grid=clamp, clamp_eps=eps)[0, 0, 0]

    # u_x = 2x - 0.5, u_y = y - 0.5; at y = 0.5 the row is hit exactly
    assert at(0.25, 0.5, False) == pytest.approx(1.0)
    assert at(0.75, 0.5, False) == pytest.approx(3.0)
    assert at(0.5, 0.5, False) == pytest.approx(2.0)
    # half a pixel outside on x: only one corner valid, weight 0.5 (zero padding)
    assert at(0.0, 0.5, False) == pytest.approx(0.5)
    assert at(1.0, 0.5, False) == pytest.approx(1.5)
    # y = 0.25: u_y = -0.25, upper corner row valid with weight 0.75
    assert at(0.25, 0.25, False) == pytest.approx(0.75)
    # entirely outside without clamp: zero
    assert at(-0.6, 0.5, False) == 0.0
    assert at(0.25, 1.6, False) == 0.0
    # with clamp, -0.6 is clamped to grid -1+eps: u_x = (eps*2 - 1)/2
    eps = 1e-3
    ux = (eps * 2 - 1) / 2
    assert at(-0.6, 0.5, True, eps) == pytest.approx((1 + ux) * 1.0)
    # clamped coordinate passes no gradient; unclamped one does
    loc = np.array([-0.6, 0.5]).reshape(1, 1, 1, 1, 1, 2)
    _, gl, _ = brute.bwd(value, shapes, loc, attn, np.ones((1, 1, 1)), True, eps)
    assert gl[..., 0].item() == 0.0
    loc = np.array([0.3, 0.5]).reshape(1, 1, 1, 1, 1, 2)
    _, gl, _ = brute.bwd(value, shapes, loc, attn, np.ones((1, 1, 1)), True, eps)
    assert gl[..., 0].item() == pytest.approx(2.0 * 2)  # slope 2 per pixel * W


@pytest.mark.parametrize("dim", [2, 3])
def test_brute_finite_differences(dim):
    value, shapes, loc, attn = make_inputs(dim, batch_size=1, num_queries=5, num_heads=2,
                                           dim_per_head=3, num_levels=2, num_points=2,
                                           dtype=torch.float64)
    value, loc, attn = value.numpy(), loc.numpy(), attn.numpy()
    rng = np.random.default_rng(4)
    grad_out = rng.standard_normal((1, 5, 6))
    gv, gl, ga = brute.bwd(value, shapes, loc, attn, grad_out, clamp_grid=False)

    def f(v, lo, a):
        return float((brute.fwd(v, shapes, lo, a, clamp_grid=False) * grad_out).sum())

    h = 1e-6
    for arr, grad, name in ((value, gv, "value"), (loc, gl, "loc"), (attn, ga, "attn")):
        flat = arr.reshape(-1)
        for i in rng.choice(flat.size, size=min(25, flat.size), replace=False):
            old = flat[i]
            flat[i] = old + h
            fp = f(value, loc, attn)
            flat[i] = old - h
            fm = f(value, loc, attn)
            flat[i] = old
            fd = (fp - fm) / (2 * h)
            assert grad.reshape(-1)[i] == pytest.approx(fd, rel=1e-5, abs=1e-6), (name, i)


@pytest.mark.parametrize("dim", [2, 3])
def test_brute_linearity(dim):
    value, shapes, loc, attn = make_inputs(dim, batch_size=1, num_queries=6, num_heads=2,
                                           dim_per_head=4, dtype=torch.float64)
    v2 = torch.randn(value.shape, dtype=torch.float64)
    a2 = torch.rand(attn.shape, dtype=torch.float64)
    f = lambda v, a: brute.fwd(v, shapes, loc, a)  # noqa: E731
    np.testing.assert_allclose(f(2 * value + 3 * v2, attn), 2 * f(value, attn) + 3 * f(v2, attn),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(f(value, attn - 0.5 * a2), f(value, attn) - 0.5 * f(value, a2),
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("clamp", [True, False])
def test_torch_ref_matches_brute(dim, clamp):
    """The grid_sample restatement agrees with the explicit loops (float64)."""
    value, shapes, loc, attn = make_inputs(dim, batch_size=2, num_queries=40, num_heads=3,
                                           dim_per_head=5, num_levels=3, num_points=3,
                                           dtype=torch.float64)
    loc = loc * 1.3 - 0.15                                   # include out-of-range samples
    loc[0, 0, 0, 0, 0] = 0.0
    loc[0, 1, 0, 0, 0] = 1.0
    out = torch_ref.msda_ref(value, shapes, loc, attn, clamp_grid=clamp, clamp_eps=1e-4)
    ref = brute.fwd(value, shapes, loc, attn, clamp_grid=clamp, clamp_eps=1e-4)
    assert max_rel(out, ref) < 1e-12
    grad_out = torch.randn(out.shape, dtype=torch.float64)
    _, tv, tl, ta = torch_ref.msda_ref_grads(value, shapes, loc, attn, grad_out, clamp, 1e-4)
    bv, bl, ba = brute.bwd(value, shapes, loc, attn, grad_out, clamp, 1e-4)
    assert max_rel(tv, bv) < 1e-12
    assert max_rel(ta, ba) < 1e-12
    keep = ~brute.edge_mask(shapes, loc, 1e-9, clamp, 1e-4)
    keep = np.broadcast_to(keep[..., None], bl.shape)
    assert max_rel(tl.numpy()[keep], bl[keep]) < 1e-10


@pytest.mark.parametrize("dim", [2, 3])
def test_torch_ref_fp32_matches_brute_fp32_coords(dim):
    """In fp32 the torch oracle and the brute oracle with fp32 coordinate rounding select
    the same corners; outputs agree to fp32 accumulation error."""
    value, shapes, loc, attn = make_inputs(dim, batch_size=2, num_queries=64)
    out = torch_ref.msda_ref(value, shapes, loc, attn)
    ref = brute.fwd(value, shapes, loc, attn, coord_f32=True)
    assert max_rel(out, ref) < 2e-6
    u32 = brute.coords(shapes, loc, coord_f32=True)
    u64 = brute.coords(shapes, loc.double(), coord_f32=False)
    assert np.abs(u32 - u64).max() < 1e-4                    # same pixel coordinates


def test_torch_ref_gradcheck():
    for dim in (2, 3):
        value, shapes, loc, attn = make_inputs(dim, batch_size=1, num_queries=3, num_heads=2,
                                               dim_per_head=2, num_levels=2, num_points=2,
                                               dtype=torch.float64)
        value.requires_grad_(True)
        loc.requires_grad_(True)
        attn.requires_grad_(True)
        fn = lambda v, lo, a: torch_ref.msda_ref(v, shapes, lo, a, False)  # noqa: E731
        assert torch.autograd.gradcheck(fn, (value, loc, attn), eps=1e-6, atol=1e-5)


def test_public_pytorch_functions_match_oracle():
    """msda_triton.pytorch (the package's portable functions) equals the oracle."""
    from msda_triton.pytorch import msda2d_pytorch, msda3d_pytorch

    for dim, fn in ((2, msda2d_pytorch), (3, msda3d_pytorch)):
        value, shapes, loc, attn = make_inputs(dim, batch_size=1, num_queries=20)
        assert torch.equal(fn(value, shapes, loc, attn), torch_ref.msda_ref(value, shapes, loc,
                                                                            attn))


def test_planted_mistake_is_caught():
    """A transposed-axis variant of the oracle (x read along H) fails the affine check
    above: the closed form distinguishes it."""
    shapes = SHAPES_2D
    rng = np.random.default_rng(5)
    coef = rng.uniform(-2, 2, (1, 1, 3))
    coef[..., 1] += 3.0
    value = _affine_value(shapes, 2, 1, 1, 1, coef)
    loc = np.empty((1, 4, 1, 2, 1, 2))
    for l, shp in enumerate(shapes):
        loc[:, :, :, l] = _interior_locs(rng, shp[::-1], 4).reshape(1, 4, 1, 1, 2)
    attn = np.ones((1, 4, 1, 2, 1))
    good = brute.fwd(value, torch.tensor(shapes), loc, attn, clamp_grid=False)
    swapped = brute.fwd(value, torch.tensor(shapes), loc[..., ::-1].copy(), attn,
                        clamp_grid=False)
    assert np.abs(good - swapped).max() > 1e-3
