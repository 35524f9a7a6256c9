"""CPU tests of the C ABI (include/msda.h) and the host layer; no device calls.

* libmsda_hip.so loads and exports every function include/msda.h declares;
* the ctypes mirror of msda_desc has the C layout (checked against gcc's offsetof);
* the host-only entry points (msda_validate, msda_bwd_workspace_bytes) return the
  documented status codes and messages;
* the Python layer raises the reference's exception types with its message substrings
  (reference src/msda_triton/triton/msda_2d.py:541-583, 61-70, 903-904).
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

from msda_triton import _lib

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "msda.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(msda_[a-z_0-9]+)\s*\(",
                                 text, flags=re.M)))


def _desc(**kw):
    d = _lib.MsdaDesc()
    base = dict(dim=2, batch=2, num_keys=19947, num_heads=8, channels=32, num_queries=19947,
                num_levels=4, num_points=4, value_dtype=_lib.MSDA_BF16,
                coord_dtype=_lib.MSDA_BF16, clamp_grid=1, flags=0, clamp_eps=1e-4)
    base.update(kw)
    for k, v in base.items():
        setattr(d, k, v)
    return d


C2_SHAPES = (100, 150, 50, 75, 25, 38, 13, 19)


def _shapes(vals):
    return ctypes.cast((ctypes.c_int32 * len(vals))(*vals), ctypes.c_void_p)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert set(declared) >= {"msda_fwd", "msda_fwd_workspace_bytes", "msda_bwd",
                             "msda_bwd_workspace_bytes", "msda_validate", "msda_last_error",
                             "msda_abi_version"}
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in msda.h but not exported"
    assert set(_lib.EXPORTED_SYMBOLS) <= set(declared)
    assert lib.msda_abi_version() == _lib.ABI_VERSION


def test_desc_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    fields = [f[0] for f in _lib.MsdaDesc._fields_]
    body = "".join(f'printf("{f} %zu\\n", offsetof(msda_desc, {f}));' for f in fields)
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "msda.h"\n'
                   f'int main(void){{printf("size %zu\\n", sizeof(msda_desc));{body}return 0;}}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(REPO / "include"), str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.check_output([str(exe)], text=True).split("\n")
               if line)
    assert int(out["size"]) == ctypes.sizeof(_lib.MsdaDesc)
    for f in fields:
        assert int(out[f]) == getattr(_lib.MsdaDesc, f).offset, f


def test_validate_status_codes():
    lib = _lib.load()
    v = lambda **kw: lib.msda_validate(ctypes.byref(_desc(**kw)))  # noqa: E731
    assert v() == _lib.MSDA_OK and _lib.last_error() == ""
    assert v(dim=4) == _lib.MSDA_ERR_INVALID and "dim must be 2 or 3" in _lib.last_error()
    assert v(value_dtype=7) == _lib.MSDA_ERR_DTYPE
    assert v(value_dtype=_lib.MSDA_BF16, coord_dtype=_lib.MSDA_F16) == _lib.MSDA_ERR_DTYPE
    assert v(value_dtype=_lib.MSDA_BF16, coord_dtype=_lib.MSDA_F32) == _lib.MSDA_OK
    assert v(num_keys=2**31) == _lib.MSDA_ERR_INVALID and "int32" in _lib.last_error()
    assert v(num_levels=65) == _lib.MSDA_ERR_INVALID
    # flags: only the head-major value bit is known, and it is valid for the backward alone
    assert v(flags=2) == _lib.MSDA_ERR_INVALID and "unknown flags" in _lib.last_error()
    assert v(flags=_lib.FLAG_VALUE_HEAD_MAJOR) == _lib.MSDA_OK
    hm = _desc(flags=_lib.FLAG_VALUE_HEAD_MAJOR)
    assert lib.msda_fwd_workspace_bytes(ctypes.byref(hm)) == 0
    assert "backward only" in _lib.last_error()
    assert v(clamp_eps=float("nan")) == _lib.MSDA_ERR_INVALID
    assert v(num_heads=0) == _lib.MSDA_ERR_INVALID
    # one batch's fp32 view of value must stay below 2^31 bytes
    assert v(num_keys=2**24, num_heads=8, channels=32) == _lib.MSDA_ERR_INVALID
    # an empty problem is valid
    assert v(batch=0, num_queries=0) == _lib.MSDA_OK


def test_bwd_workspace_bytes_host_only():
    lib = _lib.load()
    d = _desc()
    n = lib.msda_bwd_workspace_bytes(ctypes.byref(d), _shapes(C2_SHAPES))
    assert n > 0 and n % 256 == 0
    # the plan depends on the shapes, not on pointers: same answer twice
    assert lib.msda_bwd_workspace_bytes(ctypes.byref(d), _shapes(C2_SHAPES)) == n
    bad = list(C2_SHAPES)
    bad[-1] -= 1
    assert lib.msda_bwd_workspace_bytes(ctypes.byref(d), _shapes(bad)) == 0
    assert "does not match sum of spatial shapes" in _lib.last_error()
    # nothing to sample: no workspace and no error
    d0 = _desc(num_queries=0)
    assert lib.msda_bwd_workspace_bytes(ctypes.byref(d0), _shapes(C2_SHAPES)) == 0
    assert _lib.last_error() == ""
    # 3D, the 4-level volumetric configuration
    d3 = _desc(dim=3, batch=1, num_keys=149760, num_queries=32768, num_points=8)
    s3 = (32, 64, 64, 16, 32, 32, 8, 16, 16, 4, 8, 8)
    n3 = lib.msda_bwd_workspace_bytes(ctypes.byref(d3), _shapes(s3))
    assert n3 > 0
    # the backward reads value rows only per tile region, so it never relays value out: a
    # caller-supplied head-major value (the forward's copy) needs the same workspace
    h3 = _desc(dim=3, batch=1, num_keys=149760, num_queries=32768, num_points=8,
               flags=_lib.FLAG_VALUE_HEAD_MAJOR)
    assert lib.msda_fwd_workspace_bytes(ctypes.byref(d3)) == 149760 * 8 * 32 * 2
    assert lib.msda_bwd_workspace_bytes(ctypes.byref(h3), _shapes(s3)) == n3


def test_bwd_levels_beyond_binning_plan_atomic_path():
    """The backward bins samples by tile in LDS, at most 8192 tiles per head: a 2D bf16
    C=32 level of 1024 x 1024 cells (64 x 128 tiles of 16 x 8) is binned; one more tile row
    switches the plan to the atomic grad_value path, whose workspace holds one fp32 sum per
    grad_value element (host-only)."""
    lib = _lib.load()
    ok = _desc(batch=1, num_keys=1024 * 1024, num_queries=64, num_levels=1, num_heads=1)
    binned = lib.msda_bwd_workspace_bytes(ctypes.byref(ok), _shapes((1024, 1024)))
    assert binned > 0, _lib.last_error()
    big = _desc(batch=2, num_keys=1032 * 1024, num_queries=64, num_levels=1, num_heads=2)
    ws = lib.msda_bwd_workspace_bytes(ctypes.byref(big), _shapes((1032, 1024)))
    assert ws >= 2 * 1032 * 1024 * 2 * 32 * 4, _lib.last_error()
    # more than 2^27 samples per (b, h, level) do not fit a record's sample id: same plan,
    # workspace = fp32 sums (plus 256-byte aligned bookkeeping), no records
    q = (1 << 23) + 1
    many = _desc(batch=1, num_keys=32 * 32, num_queries=q, num_levels=1, num_points=16,
                 num_heads=1)
    ws = lib.msda_bwd_workspace_bytes(ctypes.byref(many), _shapes((32, 32)))
    assert 32 * 32 * 32 * 4 <= ws < q * 16 * 4, _lib.last_error()
    fewer = _desc(batch=1, num_keys=32 * 32, num_queries=q - 2, num_levels=1, num_points=16,
                  num_heads=1)  # 2^27 - 16 samples: binned, 12-byte records (bf16)
    assert lib.msda_bwd_workspace_bytes(ctypes.byref(fewer), _shapes((32, 32))) > q * 16 * 4


def test_fwd_workspace_bytes_rule():
    """The head-major value copy is requested only where rows share 128-byte lines across
    heads, the line footprint exceeds an XCD's L2 and gathers dominate (host-only)."""
    lib = _lib.load()
    c2 = _desc()
    assert lib.msda_fwd_workspace_bytes(ctypes.byref(c2)) == 0          # 2.5 MB of lines: fits L2
    c5 = _desc(dim=3, batch=1, num_keys=149760, num_queries=32768, num_points=8)
    assert lib.msda_fwd_workspace_bytes(ctypes.byref(c5)) == 149760 * 8 * 32 * 2
    c5_f32 = _desc(dim=3, batch=1, num_keys=149760, num_queries=32768, num_points=8,
                   value_dtype=_lib.MSDA_F32, coord_dtype=_lib.MSDA_F32)
    assert lib.msda_fwd_workspace_bytes(ctypes.byref(c5_f32)) == 0      # 128-byte rows
    c5_few = _desc(dim=3, batch=1, num_keys=149760, num_queries=300, num_points=8)
    assert lib.msda_fwd_workspace_bytes(ctypes.byref(c5_few)) == 0      # copy would not pay
    c5_h1 = _desc(dim=3, batch=1, num_keys=149760, num_queries=32768, num_points=8, num_heads=1)
    assert lib.msda_fwd_workspace_bytes(ctypes.byref(c5_h1)) == 0       # already head-major
    assert lib.msda_fwd_workspace_bytes(ctypes.byref(_desc(dim=5))) == 0
    assert _lib.last_error() != ""


def test_entry_points_reject_bad_descriptors_before_any_device_work():
    lib = _lib.load()
    d = _desc(dim=5)
    rc = lib.msda_fwd(ctypes.byref(d), None, None, None, None, None, None, None, 0, None)
    assert rc == _lib.MSDA_ERR_INVALID
    rc = lib.msda_bwd(ctypes.byref(d), None, None, None, None, None, None, None, None, None, 0,
                      None)
    assert rc == _lib.MSDA_ERR_INVALID
    d = _desc()
    rc = lib.msda_fwd(ctypes.byref(d), None, None, None, None, None, None, None, 0, None)
    assert rc == _lib.MSDA_ERR_INVALID and "NULL" in _lib.last_error()


def test_check_maps_status_to_reference_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.MSDA_ERR_INVALID, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.MSDA_ERR_DTYPE, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.MSDA_ERR_HIP, "x")
    _lib.check(_lib.MSDA_OK, "x")


@pytest.mark.parametrize("dim", [2, 3])
def test_cpu_tensors_raise_value_error(dim):
    """Reference test_error_on_cpu_tensors (tests/test_msda_2d.py:376-386)."""
    import msda_triton

    from tests._util import make_inputs

    value, shapes, loc, attn = make_inputs(dim, batch_size=1, num_queries=4)
    for fn in ((msda_triton.msda2d, msda_triton.msda2d_fwd) if dim == 2
               else (msda_triton.msda3d, msda_triton.msda3d_fwd)):
        with pytest.raises(ValueError, match="CUDA"):
            fn(value, shapes, loc, attn)


def test_prepare_levels_cpu_shape_checks():
    """CPU-resident shapes: K mismatch and int32 overflow (reference msda_2d.py:53-70)."""
    from msda_triton.hip import _core

    value = torch.zeros(1, 10, 1, 4)
    with pytest.raises(ValueError, match="does not match sum of spatial shapes"):
        _core.prepare_levels(2, value, torch.tensor([[3, 3]]))
    with pytest.raises(ValueError, match="exceeds int32 range"):
        _core.prepare_levels(2, value, torch.tensor([[65536, 65536]]))
    lv = _core.prepare_levels(2, torch.zeros(1, 13, 1, 4), torch.tensor([[3, 3], [2, 2]]))
    assert lv.starts.tolist() == [0, 9]
    assert lv.host.tolist() == [[3, 3], [2, 2]]


def test_cpu_shapes_cache_follows_writes_through_numpy_views():
    """The identity cache of CPU shape tensors compares the tensor's bytes on every hit: a
    write through a numpy view (which does not bump the version counter) is seen, even when
    K is unchanged (H and W swapped)."""
    from msda_triton.hip import _core

    shapes = torch.tensor([[3, 4], [2, 2]])
    value = torch.zeros(1, 16, 1, 4)
    a = _core.prepare_levels(2, value, shapes)
    assert a.host.tolist() == [[3, 4], [2, 2]]
    assert _core.prepare_levels(2, value, shapes) is a  # identity hit
    shapes.numpy()[0] = [4, 3]
    v0 = shapes._version
    b = _core.prepare_levels(2, value, shapes)
    assert shapes._version == v0  # the write did not bump the version
    assert b.host.tolist() == [[4, 3], [2, 2]]


def test_public_api_surface():
    """Same export sites and names as the reference (src/msda_triton/__init__.py:16-27,
    triton/__init__.py:10-22, pytorch/__init__.py:10-20)."""
    import msda_triton
    import msda_triton.pytorch as mp
    import msda_triton.triton as mt

    assert msda_triton.__version__ == "0.1.0"
    for n in ("msda2d", "msda2d_fwd", "msda3d", "msda3d_fwd"):
        assert n in msda_triton.__all__ and callable(getattr(msda_triton, n))
    for n in ("msda2d", "msda2d_fwd", "MSDA2DFn", "msda3d", "msda3d_fwd", "MSDA3DFn"):
        assert hasattr(mt, n)
    for n in ("msda2d_pytorch", "msda3d_pytorch"):
        assert hasattr(mp, n)
    import inspect

    sig = inspect.signature(msda_triton.msda2d)
    assert list(sig.parameters) == ["value", "value_spatial_shapes", "sampling_locations",
                                    "attention_weights", "clamp_grid", "clamp_eps"]
    assert sig.parameters["clamp_grid"].default is True
    assert sig.parameters["clamp_eps"].default == 1e-4


def test_bench_byte_model_matches_baseline_table():
    """bench.py's algorithmic bytes reproduce the per-config figures (MB = 1e6 B)."""
    import bench

    b = bench.algorithmic_bytes
    c2 = dict(bench.CONFIGS["c2"])
    assert round(b(c2)["fwd"] / 1e6, 2) == 71.49
    assert round(b(c2)["fwd_bwd"] / 1e6, 2) == 194.04
    c2f = dict(c2, dtype="fp32")
    assert round(b(c2f)["fwd"] / 1e6, 2) == 142.98
    assert round(b(c2f)["fwd_bwd"] / 1e6, 2) == 388.09
    c5 = dict(bench.CONFIGS["c5"])
    assert round(b(c5)["fwd"] / 1e6, 2) == 160.56
    assert round(b(c5)["fwd_bwd"] / 1e6, 2) == 464.91
    c3 = dict(bench.CONFIGS["c3"])
    assert round(b(c3)["fwd"] / 1e6, 2) == 81.72
    c4 = dict(bench.CONFIGS["c4"], dtype="fp32")
    assert round(b(c4)["fwd"] / 1e6, 2) == 54.53
