"""GPU: a batch split over several launches.

The C ABI keeps every in-kernel offset within 32 bits by splitting the batch into launches
whose value bytes (and their fp32 view), lanes and records stay below 2^31, offsetting every
pointer to the launch's first batch in 64-bit host arithmetic (msda_api.hip,
batches_per_launch). Here one batch's fp32 view of value is K*H*C*4 = 1.11 GB > 2^30, so
each of the B = 3 batches gets its own launch, forward and backward, and batches 1 and 2
run from offset pointers. (32 heads keep the level at 2114 backward tiles per head, inside
the binning's 8192.) Each batch's output and gradients must equal a separate
single-batch call on that batch's slices (a one-launch path covered by the parity suites):
the forward bit for bit, the gradients to 1e-6 normwise (grad_value sums a cell's entries
in the order LDS atomics ranked them). The whole split call is also held to the float64
brute-force oracle with the kernels' fp32 coordinate rounding: forward <= 1e-5 and all three
gradients <= 1e-4 normwise.
"""

from __future__ import annotations

import pytest
import torch

import msda_triton
from oracle import brute
from tests._util import max_rel

pytestmark = pytest.mark.gpu

SHAPES = [(512, 528), (16, 16)]
B, Q, H, C, P = 3, 64, 32, 32, 4


def test_batch_split_matches_single_batch_calls():
    keys = sum(h * w for h, w in SHAPES)
    assert keys * H * C * 4 > 2**30  # the fp32 view of one batch forces one launch per batch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(11)
    L = len(SHAPES)
    value = torch.randn(B, keys, H, C, device=dev, generator=g)
    loc = torch.rand(B, Q, H, L, P, 2, device=dev, generator=g)
    attn = torch.rand(B, Q, H, L * P, device=dev, generator=g).softmax(-1).view(B, Q, H, L, P)
    grad_out = torch.randn(B, Q, H * C, device=dev, generator=g)
    shapes = torch.tensor(SHAPES, dtype=torch.int64)

    def run(v, lo, a, go):
        v, lo, a = (t.detach().clone().requires_grad_(True) for t in (v, lo, a))
        out = msda_triton.msda2d(v, shapes, lo, a)
        out.backward(go)
        return out.detach(), v.grad, lo.grad, a.grad

    full = run(value, loc, attn, grad_out)
    print("batch split: split call done", flush=True)
    vc, lc, ac, gc = (t.cpu() for t in (value, loc, attn, grad_out))
    assert max_rel(full[0], brute.fwd(vc, shapes, lc, ac, coord_f32=True)) <= 1e-5
    bv, bl, ba = brute.bwd(vc, shapes, lc, ac, gc, coord_f32=True)
    for name, x, r in zip(("grad_value", "grad_loc", "grad_attn"), full[1:], (bv, bl, ba)):
        err = max_rel(x, r)
        assert err <= 1e-4, f"{name} vs brute: {err:.3e}"
    del bv, bl, ba
    for b in range(B):
        one = run(value[b:b + 1], loc[b:b + 1], attn[b:b + 1], grad_out[b:b + 1])
        assert torch.equal(full[0][b:b + 1], one[0]), f"batch {b}: forward differs"
        for name, x, r in zip(("grad_value", "grad_loc", "grad_attn"), full[1:], one[1:]):
            err = max_rel(x[b:b + 1], r)
            assert err <= 1e-6, f"batch {b}: {name} max rel err {err:.3e}"
