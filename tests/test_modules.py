"""MSDA2D / MSDA3D modules (msda_triton.modules, re-exported from msda_triton.pytorch).

CPU: init_weights patterns against what their geometry fixes (2D: the eight compass
directions scaled to the unit square, times p + 1; 3D: points on circles of radius
0.5 * 0.02 * (p + 1) in (x, y) with z = 2 * radius * sin(2 * angle)), argument checks, and
that the module refuses CPU tensors (no CPU fallback). The module oracle
(oracle/module_ref.msda_module_ref, the reference modules' forward restated) is pinned by
a closed form: identity projections, uniform softmax and integer pixel offsets from
pixel-centre reference points on non-square levels sample exact value rows, so the output
is the identity plus the mean of known rows.
GPU: forward and parameter gradients of MSDA2D / MSDA3D (HIP op, fp32) equal those of the
module oracle evaluated in float64 on the CPU from the same parameters, within 1e-4
normwise; exercised with query and head chunking, padding mask, positional encoding,
sequence-first layout and checkpointing, for the fused (locations and softmax in the
kernel) and unfused paths.
"""

from __future__ import annotations

import math

import pytest
import torch

from msda_triton.pytorch import MSDA2D, MSDA3D
from oracle import module_ref
from tests._util import max_rel


def test_import_paths():
    from msda_triton.pytorch.msda_2d import MSDA2D as A
    from msda_triton.pytorch.msda_3d import MSDA3D as B
    assert A is MSDA2D and B is MSDA3D


def test_init_weights_2d_pattern():
    m = MSDA2D(64, num_heads=8, num_levels=3, num_points=4)
    m.init_weights()
    b = m.sampling_offsets.bias.detach().view(8, 3, 4, 2)
    s = 1.0 / math.sqrt(2.0)
    unit = torch.tensor([[1, 0], [s, s], [0, 1], [-s, s], [-1, 0], [-s, -s], [0, -1], [s, -s]])
    unit = unit / unit.abs().amax(-1, keepdim=True)       # corners of the unit square
    for p in range(4):
        for lvl in range(3):
            assert torch.allclose(b[:, lvl, p], unit * (p + 1), atol=1e-6)
    assert torch.all(m.sampling_offsets.weight == 0) and torch.all(m.attention_weights.weight == 0)
    assert torch.all(m.attention_weights.bias == 0) and torch.all(m.value_proj.bias == 0)
    lim = math.sqrt(6.0 / (64 + 64))                     # Xavier-uniform bound
    assert m.value_proj.weight.abs().max() <= lim and m.output_proj.weight.abs().max() <= lim


def test_init_weights_3d_pattern():
    H, L, P = 4, 2, 3
    m = MSDA3D(32, num_heads=H, num_levels=L, num_points=P)
    m.init_weights()
    b = m.sampling_offsets.bias.detach().double().view(H, L, P, 3)
    assert torch.equal(b[:, 0], b[:, 1])
    for h in range(H):
        for p in range(P):
            r = 0.02 * (p + 1)
            x, y, z = b[h, 0, p]
            assert abs(math.hypot(x, y) - 0.5 * r) < 1e-7
            a = math.atan2(y, x) % (2 * math.pi)
            assert abs(a - 2 * math.pi * (h * P + p) / (H * P)) < 1e-5
            assert abs(z - 2 * r * math.sin(2 * a)) < 1e-7


def test_argument_checks():
    with pytest.raises(ValueError, match="divisible"):
        MSDA2D(30, num_heads=8, num_levels=1, num_points=1)
    m = MSDA2D(16, num_heads=2, num_levels=1, num_points=2, batch_first=True)
    q = torch.randn(1, 5, 16)
    shapes = torch.tensor([[2, 3]])
    with pytest.raises(ValueError, match="Last dim of reference_points must be 2"):
        m(q, value=torch.randn(1, 6, 16), reference_points=torch.rand(1, 5, 1, 3),
          spatial_shapes=shapes)
    with pytest.raises(AssertionError):
        m(q, value=torch.randn(1, 7, 16), reference_points=torch.rand(1, 5, 1, 2),
          spatial_shapes=shapes)


def test_cpu_tensors_are_refused():
    m = MSDA2D(16, num_heads=2, num_levels=1, num_points=2, batch_first=True)
    with pytest.raises(ValueError, match="CUDA"):
        m(torch.randn(1, 5, 16), value=torch.randn(1, 6, 16),
          reference_points=torch.rand(1, 5, 1, 2), spatial_shapes=torch.tensor([[2, 3]]))


def _params(m, dtype=torch.float64):
    return {k: v.detach().cpu().to(dtype) for k, v in m.state_dict().items()}


@pytest.mark.parametrize("dim", [2, 3])
def test_module_oracle_closed_form(dim):
    """Identity value/output projections, zero attention logits (uniform weights over L*P)
    and offsets of whole pixels from pixel-centre reference points: every sample lands on a
    pixel centre and returns that value row exactly, on non-square levels, so the output is
    identity + the mean over (l, p) of known rows. A swapped x/y pixel offset gives
    different rows (the case distinguishes the normaliser's axis order)."""
    E, H, L, P, bs, nq = 8, 2, 2, 3, 2, 5
    C = E // H
    # every extent >= 3: a reference pixel one inside the border plus a shift of at most
    # one pixel stays inside the level
    shapes = torch.tensor([[5, 7], [3, 4]] if dim == 2 else [[3, 4, 5], [3, 3, 4]])
    sizes = shapes.prod(-1).tolist()
    starts = [0, sizes[0]]
    nv = sum(sizes)
    g = torch.Generator().manual_seed(0)
    eye = torch.eye(E, dtype=torch.float64)
    # whole-pixel offsets per (h, l, p, axis): small, so reference + offset stays inside
    shift = torch.randint(-1, 2, (H, L, P, dim), generator=g)
    params = {"value_proj.weight": eye, "value_proj.bias": torch.zeros(E, dtype=torch.float64),
              "output_proj.weight": eye, "output_proj.bias": torch.zeros(E, dtype=torch.float64),
              "attention_weights.weight": torch.zeros(H * L * P, E, dtype=torch.float64),
              "attention_weights.bias": torch.zeros(H * L * P, dtype=torch.float64),
              "sampling_offsets.weight": torch.zeros(H * L * P * dim, E, dtype=torch.float64),
              "sampling_offsets.bias": shift.reshape(-1).to(torch.float64)}
    query = torch.randn(nq, bs, E, generator=g, dtype=torch.float64)   # sequence-first
    value = torch.randn(nv, bs, E, generator=g, dtype=torch.float64)
    # reference pixel (x, y[, z]) per (b, q, l), one pixel inside the level's border
    ext = shapes.flip(-1)  # (W, H[, D]) per level
    pix = torch.stack([torch.randint(1, int(e) - 1, (bs, nq), generator=g) for e in ext.reshape(-1)], -1)
    pix = pix.view(bs, nq, L, dim)
    refp = (pix.to(torch.float64) + 0.5) / ext.to(torch.float64)
    out = module_ref.msda_module_ref(dim, params, query, value=value, reference_points=refp,
                                     spatial_shapes=shapes, num_heads=H, num_levels=L,
                                     num_points=P)

    def expected(sh):
        want = query.clone()
        for b in range(bs):
            for q in range(nq):
                for h in range(H):
                    acc = torch.zeros(C, dtype=torch.float64)
                    for lv in range(L):
                        W_, H_ = int(ext[lv, 0]), int(ext[lv, 1])
                        for p in range(P):
                            x, y = (pix[b, q, lv, :2] + sh[h, lv, p, :2]).tolist()
                            k = starts[lv] + y * W_ + x
                            if dim == 3:
                                z = int(pix[b, q, lv, 2] + sh[h, lv, p, 2])
                                k = starts[lv] + (z * H_ + y) * W_ + x
                            acc += value[k, b, h * C:(h + 1) * C]
                    want[q, b, h * C:(h + 1) * C] += acc / (L * P)
        return want

    assert (out - expected(shift)).abs().max().item() < 1e-10
    swapped = shift.clone()
    swapped[..., [0, 1]] = shift[..., [1, 0]]
    if not torch.equal(swapped, shift):
        assert (out - expected(swapped)).abs().max().item() > 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("fused", [True, False])
def test_module_matches_oracle_module(dim, fused):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.manual_seed(0)
    cls = MSDA2D if dim == 2 else MSDA3D
    shapes = torch.tensor([[12, 10], [6, 5]] if dim == 2 else [[4, 6, 5], [2, 3, 3]])
    nv = int(shapes.prod(-1).sum())
    E, H, L, P, nq, bs = 64, 4, 2, 3, 37, 2
    m = cls(E, num_heads=H, num_levels=L, num_points=P, dropout=0.0, query_chunk_size=16,
            head_chunk_size=3, use_checkpoint=True, fused=fused)
    m.init_weights()
    with torch.no_grad():  # non-trivial offsets and weights
        m.sampling_offsets.weight.normal_(0, 0.05)
        m.attention_weights.weight.normal_(0, 0.2)
    m.train()
    params = {k: v.requires_grad_(True) for k, v in _params(m).items()}
    print(f"module parity dim={dim} fused={fused}", flush=True)
    g = torch.Generator().manual_seed(1)
    query = torch.randn(nq, bs, E, generator=g)          # sequence-first (batch_first=False)
    value = torch.randn(nv, bs, E, generator=g)
    pos = torch.randn(nq, bs, E, generator=g)
    refp = torch.rand(bs, nq, L, dim, generator=g)
    mask = torch.rand(bs, nv, generator=g) < 0.1
    grad = torch.randn(nq, bs, E, generator=g)
    dev = torch.device("cuda")
    m = m.to(dev)
    out = m(query.to(dev), value=value.to(dev), query_pos=pos.to(dev), key_padding_mask=mask.to(dev),
            reference_points=refp.to(dev), spatial_shapes=shapes)
    out.backward(grad.to(dev))
    d = torch.float64
    out_r = module_ref.msda_module_ref(dim, params, query.to(d), value=value.to(d),
                                       query_pos=pos.to(d), key_padding_mask=mask,
                                       reference_points=refp.to(d), spatial_shapes=shapes,
                                       num_heads=H, num_levels=L, num_points=P)
    out_r.backward(grad.to(d))
    assert out.shape == (nq, bs, E)
    assert max_rel(out.detach().cpu(), out_r.detach()) <= 1e-4
    for name, p in m.named_parameters():
        assert p.grad is not None, name
        err = max_rel(p.grad.cpu(), params[name].grad)
        assert err <= 1e-4, (name, err)
