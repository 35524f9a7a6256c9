"""GPU: the C ABI on a non-default stream and inside a HIP graph.

Every entry point enqueues its kernels on the caller's stream and clears its buffers with
fill kernels (no hipMemsetAsync node), so a forward + backward can be captured once and
replayed. The graph test replays the captured graph several times on fresh inputs, with the
program's own eager work and synchronisations between the replays, and checks every
replay against an eager run on the same inputs. The 3D case is large enough to take the
head-major copy in bf16 in both the forward (caller workspace) and the backward (inside
its workspace) and runs the unstaged forward kernel; the 2D case takes the staged one.

Tolerances: the forward is deterministic (one lane group per output row, fixed order), so
replay and eager outputs must be identical. grad_value sums a cell's entries in the order
the fill kernel's LDS atomics ranked them, which may differ between runs, so gradients
are compared at 1e-5 (fp32) / 1e-2 (bf16) normwise; a graph that replays a stale buffer
or skips a clear fails these by orders of magnitude.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from msda_triton import _lib
from msda_triton.hip import _core
from tests._util import make_inputs, max_rel

pytestmark = pytest.mark.gpu

CASES = {
    # 2D: 16 (b, h) slices share 256 workgroups, 8192 / 16 = 512 queries each -> staged
    # forward kernel
    "2d_staged": dict(dim=2, batch_size=2, num_queries=8192, num_heads=8, num_points=4,
                      spatial_shapes=[(64, 96), (32, 48), (16, 24)]),
    # 3D: K = 131072 keys x 128 B > 4 MB and gathers >= 8 K -> head-major copies
    "3d_head_major": dict(dim=3, batch_size=1, num_queries=16384, num_heads=2, num_points=8,
                          spatial_shapes=[(32, 64, 64)]),
}


def _device_inputs(case, dtype, seed):
    cfg = dict(CASES[case])
    dim = cfg.pop("dim")
    value, shapes, loc, attn = make_inputs(dim, dtype=torch.float32, seed=seed, **cfg)
    g = torch.Generator().manual_seed(seed + 1000)
    grad_out = torch.randn(value.shape[0], loc.shape[1], value.shape[2] * value.shape[3], generator=g)
    dev = torch.device("cuda:0")
    return dim, shapes, [t.to(dev, dtype) for t in (value, loc, attn, grad_out)]


def _step(dim, levels, v, lo, a, go):
    out = _core.forward(dim, v, levels, lo, a, True, 1e-4)[0]
    gv, gl, ga = _core.backward(dim, go, v, levels, lo, a, True, 1e-4)
    return out, gv, gl, ga


def _check(got, ref, dtype, what):
    out, *grads = got
    rout, *rgrads = ref
    assert torch.equal(out, rout), f"{what}: forward differs"
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    for name, x, r in zip(("grad_value", "grad_loc", "grad_attn"), grads, rgrads):
        err = max_rel(x, r)
        assert err <= tol, f"{what}: {name} max rel err {err:.3e} > {tol}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("case", sorted(CASES))
def test_graph_replay_matches_eager(case, dtype):
    dim, shapes, (v, lo, a, go) = _device_inputs(case, dtype, seed=0)
    levels = _core.prepare_levels(dim, v, shapes)  # level tables uploaded before capture
    if case == "3d_head_major" and dtype == torch.bfloat16:
        desc = _core.make_desc(dim, v, lo, dtype, True, 1e-4)
        assert _lib.load().msda_fwd_workspace_bytes(ctypes.byref(desc)) > 0, "no head-major copy"
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture (library load, workspaces)
        for _ in range(2):
            _step(dim, levels, v, lo, a, go)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = _step(dim, levels, v, lo, a, go)
    for rep in range(3):
        _, _, (nv, nlo, na, ngo) = _device_inputs(case, dtype, seed=rep + 1)
        for dst, src in ((v, nv), (lo, nlo), (a, na), (go, ngo)):
            dst.copy_(src)
        graph.replay()
        eager = _step(dim, levels, v, lo, a, go)  # eager work between the replays
        torch.cuda.synchronize()
        _check(static, eager, dtype, f"{case} replay {rep}")


@pytest.mark.parametrize("case", sorted(CASES))
def test_non_default_stream_matches_default(case):
    dtype = torch.float32
    dim, shapes, (v, lo, a, go) = _device_inputs(case, dtype, seed=3)
    levels = _core.prepare_levels(dim, v, shapes)
    ref = _step(dim, levels, v, lo, a, go)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = _step(dim, levels, v, lo, a, go)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _check(got, ref, dtype, f"{case} side stream")
