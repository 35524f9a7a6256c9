"""GPU: msda_bwd_noalloc, the backward whose workspace is the library's static device scratch.

Called through the C ABI (ctypes), it must equal msda_bwd (the same call with a caller
workspace) on the same inputs: grad_sampling_locations and grad_attention_weights bit for
bit, grad_value within 1e-6 normwise in fp32 (a cell's entries are summed in the order LDS
atomics ranked them) and within one bf16 rounding in bf16. Two calls in a row, the second
with a smaller input, so the second reuses the scratch the first left behind. A problem
whose workspace exceeds the scratch is refused before any launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from msda_triton import _lib
from msda_triton.hip import _core
from tests._util import make_inputs, max_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _call(entry, dim, value, shapes, loc, attn, grad_out):
    """Run msda_bwd (entry == "ws") or msda_bwd_noalloc (entry == "noalloc")."""
    lib = _lib.load()
    desc = _core.make_desc(dim, value, loc, loc.dtype, True, 1e-4)
    hs = shapes.to(torch.int32).contiguous()
    gv, gl, ga = torch.empty_like(value), torch.empty_like(loc), torch.empty_like(attn)
    stream = torch.cuda.current_stream().cuda_stream
    args = [value.data_ptr(), loc.data_ptr(), attn.data_ptr(), grad_out.data_ptr(),
            gv.data_ptr(), gl.data_ptr(), ga.data_ptr()]
    if entry == "ws":
        n = lib.msda_bwd_workspace_bytes(ctypes.byref(desc), ctypes.c_void_p(hs.data_ptr()))
        ws = torch.empty(max(n, 1), dtype=torch.uint8, device=value.device)
        rc = lib.msda_bwd(ctypes.byref(desc), hs.data_ptr(), *args, ws.data_ptr(), n, stream)
    else:
        rc = lib.msda_bwd_noalloc(ctypes.byref(desc), hs.data_ptr(), *args, stream)
    _lib.check(rc, entry)
    torch.cuda.synchronize()
    return gv, gl, ga


def _case(dim, dtype, q, seed):
    dev = torch.device("cuda")
    shapes = ([(100, 150), (50, 75), (25, 38), (13, 19)] if dim == 2
              else [(16, 32, 32), (8, 16, 16)])
    value, shapes, loc, attn = make_inputs(dim, batch_size=2, num_queries=q, num_heads=8,
                                           dim_per_head=32, num_points=4,
                                           spatial_shapes=shapes, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    grad_out = torch.randn(2, q, 8 * 32, generator=g)
    return dim, [t.to(dev, dtype) for t in (value, loc, attn, grad_out)], shapes


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("dim", [2, 3])
def test_noalloc_matches_workspace_entry(dim, dtype):
    # C2's full encoder workload first (about 165 MB of workspace), then a smaller one
    for q, seed in ((19947 if dim == 2 else 4096, 1), (500, 2)):
        print(f"noalloc dim={dim} {dtype} Q={q}", flush=True)
        d, (value, loc, attn, grad_out), shapes = _case(dim, dtype, q, seed)
        want = _call("ws", d, value, shapes, loc, attn, grad_out)
        got = _call("noalloc", d, value, shapes, loc, attn, grad_out)
        assert torch.equal(got[1], want[1]), "grad_loc differs"
        assert torch.equal(got[2], want[2]), "grad_attn differs"
        tol = 1e-6 if dtype == torch.float32 else 1e-2
        err = max_rel(got[0].float(), want[0].float())
        assert err <= tol, f"grad_value {err:.3e}"


def test_noalloc_refuses_problems_beyond_the_scratch():
    """C5 (3D 4-level, Q=32768, P=8) needs more backward workspace than the static scratch:
    refused with MSDA_ERR_WORKSPACE and a message naming both sizes, before any launch."""
    lib = _lib.load()
    d = _lib.MsdaDesc()
    for k, v in dict(dim=3, batch=1, num_keys=149760, num_heads=8, channels=32,
                     num_queries=32768, num_levels=4, num_points=8, value_dtype=_lib.MSDA_BF16,
                     coord_dtype=_lib.MSDA_BF16, clamp_grid=1, flags=0,
                     clamp_eps=1e-4).items():
        setattr(d, k, v)
    hs = torch.tensor([32, 64, 64, 16, 32, 32, 8, 16, 16, 4, 8, 8], dtype=torch.int32)
    need = lib.msda_bwd_workspace_bytes(ctypes.byref(d), ctypes.c_void_p(hs.data_ptr()))
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    fake = 256  # never dereferenced: the call must fail on the host first
    rc = lib.msda_bwd_noalloc(ctypes.byref(d), hs.data_ptr(), fake, fake, fake, fake, fake,
                              fake, fake, None)
    assert rc == _lib.MSDA_ERR_WORKSPACE
    msg = _lib.last_error()
    assert "static scratch" in msg and str(need) in msg
