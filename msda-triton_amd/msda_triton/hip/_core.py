"""Host layer shared by the 2D and 3D HIP ops: validation, level tables, C-ABI calls.

Mirrors the reference's host side for this path (src/msda_triton/triton/msda_2d.py:17-82,
541-651, 721-853 and src/msda_triton/triton/msda_3d.py:17-77, 684-794, 864-996): the same
checks with the same exception types and messages, the same CPU- versus GPU-resident
spatial-shape handling, and the same autograd contract. The kernels themselves live in
libmsda_hip.so (csrc/msda_kernels.hip) and are reached through include/msda.h.
"""

from __future__ import annotations

import contextlib
import ctypes
import weakref
from collections import OrderedDict

import torch

from .. import _lib

_DTYPE_CODE = {torch.float32: _lib.MSDA_F32, torch.float16: _lib.MSDA_F16,
               torch.bfloat16: _lib.MSDA_BF16}
_COORD_NAMES = {2: "(B, Q, H, L, P, 2)", 3: "(B, Q, H, L, P, 3)"}
_SHAPE_NAMES = {2: "H_l x W_l", 3: "D_l x H_l x W_l"}
_INT32_MAX = 2**31 - 1

# Device copies of CPU-resident level tables, keyed by (dim, shapes, device).
_LEVEL_CACHE: OrderedDict = OrderedDict()
_LEVEL_CACHE_MAX = 64
# Level tables derived from GPU-resident shape tensors, keyed by id(tensor) and valid while
# that tensor is alive and unmodified (same version counter): a loop over one shapes
# tensor pays the device-side conversion once.
_GPU_LEVEL_CACHE: OrderedDict = OrderedDict()
# The same identity cache for CPU-resident shape tensors (entries also hold K and the
# tensor's raw bytes, compared on every hit, since writes through a numpy view of the
# tensor do not bump its version counter): a loop over one shapes tensor skips converting
# it in Python on every call.
_CPU_ID_CACHE: OrderedDict = OrderedDict()


def _raw_bytes(t: torch.Tensor):
    """The raw bytes of a small contiguous CPU tensor, read straight from its memory (None
    for other layouts)."""
    return ctypes.string_at(t.data_ptr(), t.nbytes) if t.is_contiguous() else None


def validate_inputs(name: str, dim: int, value: torch.Tensor, value_spatial_shapes: torch.Tensor,
                    sampling_locations: torch.Tensor, attention_weights: torch.Tensor) -> None:
    """Device, dtype and shape checks; raises on the first violation.

    Same order, types and messages as _validate_inputs_2d (triton/msda_2d.py:541-583) and
    _validate_inputs_3d (triton/msda_3d.py:684-726), plus a same-device check.
    """
    if not value.is_cuda:
        raise ValueError(f"{name} HIP kernel requires CUDA tensors. Got CPU tensors instead.")
    if value.dtype not in _DTYPE_CODE:
        raise NotImplementedError(
            f"{name} HIP kernel only supports fp32, fp16, and bf16. Got {value.dtype}. "
            "The kernel accumulates in fp32 internally."
        )
    if value.dim() != 4:
        raise ValueError(f"value must be (B, K, H, C), got {tuple(value.shape)}")
    if sampling_locations.dim() != 6:
        raise ValueError(
            f"sampling_locations must be {_COORD_NAMES[dim]}, got {tuple(sampling_locations.shape)}"
        )
    bsz, _, num_heads, _ = value.shape
    bsz_s, num_queries, num_heads_s, num_levels, num_points, last = sampling_locations.shape
    if not (bsz == bsz_s and num_heads == num_heads_s and last == dim):
        raise ValueError(
            f"Shape mismatch: value=(B,K,H,C), sampling_locations={_COORD_NAMES[dim].replace(' ', '')}. "
            f"Got value={tuple(value.shape)}, sampling_locations={tuple(sampling_locations.shape)}"
        )
    if attention_weights.shape != (bsz, num_queries, num_heads, num_levels, num_points):
        raise ValueError(
            f"attention_weights must be (B,Q,H,L,P), got {tuple(attention_weights.shape)}"
        )
    if value_spatial_shapes.shape != (num_levels, dim):
        raise ValueError(
            f"value_spatial_shapes must be (L,{dim}), got {tuple(value_spatial_shapes.shape)}. "
            f"num_levels={num_levels}, expected shape=({num_levels}, {dim})"
        )
    for tname, t in (("sampling_locations", sampling_locations),
                     ("attention_weights", attention_weights)):
        if t.device != value.device:
            raise ValueError(f"{tname} is on {t.device} but value is on {value.device}")
        if not t.is_floating_point():
            raise ValueError(f"{tname} must be a floating-point tensor, got {t.dtype}")


class Levels:
    """Level tables of one call: (L, dim) int32 shapes and (L,) int32 starts on the device
    (read by the forward kernel) and, for CPU-resident shapes, a host (L, dim) int32 copy of
    the shapes (planned from by the backward). GPU-resident shapes have no host copy: their
    backward (msda_bwd_dev) derives its plan from the device tables on the device, so no
    call ever waits for the device."""

    __slots__ = ("spatial", "starts", "host")

    def __init__(self, spatial, starts, host):
        self.spatial = spatial
        self.starts = starts
        self.host = host


def prepare_levels(dim: int, value: torch.Tensor, value_spatial_shapes: torch.Tensor) -> Levels:
    """Level tables on value's device, plus the host copy of the shapes.

    CPU-resident shapes are checked against K and the int32 range (as in
    _prepare_spatial_2d, triton/msda_2d.py:53-74) and their device copy is cached.
    GPU-resident shapes are converted on the device without a host sync and without the
    K check (triton/msda_2d.py:76-82), cached for the live, unmodified tensor.
    """
    device = value.device
    if value_spatial_shapes.device.type == "cpu":
        key = id(value_spatial_shapes)
        hit = _CPU_ID_CACHE.get(key)
        raw = _raw_bytes(value_spatial_shapes)
        if hit is not None:
            ref, version, hdim, hdev, total_keys, levels, hraw = hit
            if (ref() is value_spatial_shapes and version == value_spatial_shapes._version
                    and hdim == dim and hdev == device and raw is not None and raw == hraw):
                _check_num_keys(dim, value, total_keys)
                _CPU_ID_CACHE.move_to_end(key)
                return levels
            del _CPU_ID_CACHE[key]
        levels, total_keys = _cpu_levels(dim, value, value_spatial_shapes)
        try:
            ref = weakref.ref(value_spatial_shapes)
        except TypeError:
            return levels
        _CPU_ID_CACHE[key] = (ref, value_spatial_shapes._version, dim, device, total_keys, levels,
                              raw)
        if len(_CPU_ID_CACHE) > _LEVEL_CACHE_MAX:
            _CPU_ID_CACHE.popitem(last=False)
        return levels
    return _gpu_levels(dim, value, value_spatial_shapes)


def _check_num_keys(dim: int, value: torch.Tensor, total_keys: int) -> None:
    if value.size(1) != total_keys:
        raise ValueError(
            f"value dim 1 ({value.size(1)}) does not match sum of spatial shapes "
            f"({total_keys}). Ensure K = Σ({_SHAPE_NAMES[dim]}) across all levels."
        )


def _cpu_levels(dim: int, value: torch.Tensor, value_spatial_shapes: torch.Tensor):
    """(levels, K) for CPU-resident shapes; device tables cached by the shapes' values."""
    device = value.device
    shapes_cpu = value_spatial_shapes.detach().to(dtype=torch.int64)
    rows = tuple(tuple(int(v) for v in r) for r in shapes_cpu.tolist())
    key = (dim, rows, device)
    sizes = [1] * len(rows)
    for i, r in enumerate(rows):
        for v in r:
            sizes[i] *= v
    total_keys = sum(sizes)
    if total_keys > _INT32_MAX:
        raise ValueError(
            f"Total number of keys ({total_keys}) exceeds int32 range. "
            "Reduce spatial dimensions or number of levels."
        )
    _check_num_keys(dim, value, total_keys)
    hit = _LEVEL_CACHE.get(key)
    if hit is not None:
        _LEVEL_CACHE.move_to_end(key)
        return hit, total_keys
    starts = [0] * len(rows)
    for i in range(1, len(rows)):
        starts[i] = starts[i - 1] + sizes[i - 1]
    host = torch.tensor(rows, dtype=torch.int32).reshape(len(rows), dim).contiguous()
    levels = Levels(host.to(device), torch.tensor(starts, dtype=torch.int32).to(device), host)
    _LEVEL_CACHE[key] = levels
    if len(_LEVEL_CACHE) > _LEVEL_CACHE_MAX:
        _LEVEL_CACHE.popitem(last=False)
    return levels, total_keys


def _gpu_levels(dim: int, value: torch.Tensor, value_spatial_shapes: torch.Tensor) -> Levels:
    """Level tables for GPU-resident shapes, cached for the live, unmodified tensor."""
    device = value.device
    key = id(value_spatial_shapes)
    hit = _GPU_LEVEL_CACHE.get(key)
    if hit is not None:
        ref, version, hdim, hdev, levels = hit
        if (ref() is value_spatial_shapes and version == value_spatial_shapes._version
                and hdim == dim and hdev == device):
            _GPU_LEVEL_CACHE.move_to_end(key)
            return levels
        del _GPU_LEVEL_CACHE[key]
    spatial_i32 = value_spatial_shapes.to(device=device, dtype=torch.int32).contiguous()
    sizes = spatial_i32.to(torch.int64).prod(dim=1)
    starts = torch.zeros_like(sizes)
    if sizes.numel() > 1:
        starts[1:] = torch.cumsum(sizes[:-1], dim=0)
    levels = Levels(spatial_i32, starts.to(torch.int32), None)
    try:
        ref = weakref.ref(value_spatial_shapes)
    except TypeError:
        return levels
    _GPU_LEVEL_CACHE[key] = (ref, value_spatial_shapes._version, dim, device, levels)
    if len(_GPU_LEVEL_CACHE) > _LEVEL_CACHE_MAX:
        _GPU_LEVEL_CACHE.popitem(last=False)
    return levels


def coord_dtype(value: torch.Tensor, loc: torch.Tensor, attn: torch.Tensor) -> torch.dtype:
    """dtype the kernels read locations and weights in: the value dtype when all three
    agree, else float32 (both are then upcast, which is exact for fp16/bf16)."""
    if loc.dtype == value.dtype and attn.dtype == value.dtype:
        return value.dtype
    return torch.float32


def make_desc(dim: int, value: torch.Tensor, loc: torch.Tensor, cdt: torch.dtype,
              clamp_grid: bool, clamp_eps: float) -> _lib.MsdaDesc:
    bsz, num_keys, num_heads, ch = value.shape
    _, num_queries, _, num_levels, num_points, _ = loc.shape
    d = _lib.MsdaDesc()
    d.dim = dim
    d.batch = bsz
    d.num_keys = num_keys
    d.num_heads = num_heads
    d.channels = ch
    d.num_queries = num_queries
    d.num_levels = num_levels
    d.num_points = num_points
    d.value_dtype = _DTYPE_CODE[value.dtype]
    d.coord_dtype = _DTYPE_CODE[cdt]
    d.clamp_grid = 1 if clamp_grid else 0
    d.flags = 0
    d.clamp_eps = float(clamp_eps)
    return d


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """t itself if its data is 16-byte aligned (the backward's row loads need it), else an
    aligned copy (only contiguous views with an odd storage offset are affected)."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _on_device(device: torch.device):
    """Context that makes device current, or nothing if it already is."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def _stream(device: torch.device) -> int:
    """The current torch stream of device (a tensor's device: its index is set), as the
    raw hipStream_t handle torch.cuda.current_stream(device).cuda_stream returns, without
    building a Stream object per call."""
    return torch._C._cuda_getCurrentRawStream(device.index)


# Forward descriptors and their workspace sizes, keyed by the problem (shapes, dtypes, clamp):
# a loop over one problem builds the ctypes descriptor and asks for its workspace once.
_FWD_DESC_CACHE: OrderedDict = OrderedDict()


def _fwd_desc(dim: int, value: torch.Tensor, loc: torch.Tensor, cdt: torch.dtype, clamp_grid: bool,
              clamp_eps: float):
    """(msda_desc, forward workspace bytes) for the problem, cached."""
    key = (dim, value.shape, loc.shape, value.dtype, cdt, bool(clamp_grid), float(clamp_eps))
    hit = _FWD_DESC_CACHE.get(key)
    if hit is not None:
        return hit
    desc = make_desc(dim, value, loc, cdt, clamp_grid, clamp_eps)
    ws_bytes = int(_lib.load().msda_fwd_workspace_bytes(ctypes.byref(desc)))
    _FWD_DESC_CACHE[key] = (desc, ws_bytes)
    if len(_FWD_DESC_CACHE) > _LEVEL_CACHE_MAX:
        _FWD_DESC_CACHE.popitem(last=False)
    return desc, ws_bytes


def forward(dim: int, value: torch.Tensor, levels: Levels, loc: torch.Tensor, attn: torch.Tensor,
            clamp_grid: bool, clamp_eps: float):
    """Launch msda_fwd. Returns (out, value_c, loc_c, attn_c, value_hm): the output, the
    contiguous, kernel-dtype inputs it read (saved for backward) and the head-major copy of
    the whole value the kernel gathered from (its workspace), or None when it made none or
    only of one batch chunk."""
    lib = _lib.load()
    cdt = coord_dtype(value, loc, attn)
    value_c = _aligned(value.contiguous())
    loc_c = _aligned(loc.to(dtype=cdt).contiguous())
    attn_c = _aligned(attn.to(dtype=cdt).contiguous())
    bsz, _, num_heads, ch = value.shape
    num_queries = loc.shape[1]
    out = torch.empty((bsz, num_queries, num_heads * ch), device=value.device, dtype=value.dtype)
    # optional workspace: a head-major copy of value for large, line-sharing value slices
    desc, ws_bytes = _fwd_desc(dim, value_c, loc_c, cdt, clamp_grid, clamp_eps)
    ws = torch.empty(ws_bytes, device=value.device, dtype=torch.uint8) if ws_bytes else None
    with _on_device(value.device):
        rc = lib.msda_fwd(ctypes.byref(desc), value_c.data_ptr(), levels.spatial.data_ptr(),
                          levels.starts.data_ptr(), loc_c.data_ptr(), attn_c.data_ptr(),
                          out.data_ptr(), ws.data_ptr() if ws is not None else None, ws_bytes,
                          _stream(value.device))
    _lib.check(rc, "msda_fwd")
    whole = ws is not None and ws_bytes == value_c.numel() * value_c.element_size()
    return out, value_c, loc_c, attn_c, (ws if whole else None)


def backward(dim: int, grad_output: torch.Tensor, value_c: torch.Tensor, levels: Levels,
             loc_c: torch.Tensor, attn_c: torch.Tensor, clamp_grid: bool, clamp_eps: float,
             value_hm: torch.Tensor | None = None):
    """Launch msda_bwd. Returns (grad_value, grad_loc, grad_attn) in the kernel dtypes,
    all freshly allocated and contiguous. value_hm: a head-major (B, H, K, C) copy of value_c,
    such as the forward's workspace, passed instead of value_c (MSDA_FLAG_VALUE_HEAD_MAJOR)."""
    lib = _lib.load()
    grad_out = _aligned(grad_output.to(dtype=value_c.dtype).contiguous())
    value_c = _aligned(value_c)
    grad_value = torch.empty(value_c.shape, device=value_c.device, dtype=value_c.dtype)
    grad_loc = torch.empty(loc_c.shape, device=loc_c.device, dtype=loc_c.dtype)
    grad_attn = torch.empty(attn_c.shape, device=attn_c.device, dtype=attn_c.dtype)
    desc = make_desc(dim, value_c, loc_c, loc_c.dtype, clamp_grid, clamp_eps)
    value_ptr = value_c.data_ptr()
    if value_hm is not None:
        desc.flags = _lib.FLAG_VALUE_HEAD_MAJOR
        value_ptr = value_hm.data_ptr()
    if levels.host is not None:
        # CPU-resident shapes: the host plans every size exactly
        name, shapes = "msda_bwd", levels.host.data_ptr()
        ws_bytes = int(lib.msda_bwd_workspace_bytes(ctypes.byref(desc), shapes))
        entry = lib.msda_bwd
    else:
        # GPU-resident shapes: the plan is derived on the device (no host read, no sync)
        name, shapes = "msda_bwd_dev", levels.spatial.data_ptr()
        ws_bytes = int(lib.msda_bwd_dev_workspace_bytes(ctypes.byref(desc)))
        entry = lib.msda_bwd_dev
    if ws_bytes == 0 and _lib.last_error():
        _lib.check(_lib.MSDA_ERR_INVALID, name + "_workspace_bytes")
    ws = torch.empty(max(ws_bytes, 1), device=value_c.device, dtype=torch.uint8)
    with _on_device(value_c.device):
        rc = entry(ctypes.byref(desc), shapes, value_ptr, loc_c.data_ptr(),
                   attn_c.data_ptr(), grad_out.data_ptr(), grad_value.data_ptr(),
                   grad_loc.data_ptr(), grad_attn.data_ptr(), ws.data_ptr(), ws_bytes,
                   _stream(value_c.device))
    _lib.check(rc, name)
    return grad_value, grad_loc, grad_attn


def fn_forward(ctx, name: str, dim: int, value, value_spatial_shapes, sampling_locations,
               attention_weights, clamp_grid, clamp_eps) -> torch.Tensor:
    """Body of MSDA2DFn.forward / MSDA3DFn.forward (reference triton/msda_2d.py:749-775)."""
    validate_inputs(name, dim, value, value_spatial_shapes, sampling_locations, attention_weights)
    levels = prepare_levels(dim, value, value_spatial_shapes)
    # the forward's head-major copy of value (its workspace) is not kept: the backward reads
    # value rows once per tile region, in either layout
    out, value_c, loc_c, attn_c, _ = forward(dim, value, levels, sampling_locations,
                                             attention_weights, clamp_grid, clamp_eps)
    ctx.save_for_backward(value_c, loc_c, attn_c)
    ctx.levels = levels
    ctx.clamp_grid = clamp_grid
    ctx.clamp_eps = clamp_eps
    ctx.in_dtypes = (value.dtype, sampling_locations.dtype, attention_weights.dtype)
    return out


def fn_backward(ctx, dim: int, grad_output: torch.Tensor):
    """Body of MSDA2DFn.backward / MSDA3DFn.backward (reference triton/msda_2d.py:777-853):
    returns (grad_value, None, grad_loc, grad_attn, None, None) in the input dtypes."""
    value_c, loc_c, attn_c = ctx.saved_tensors
    gv, gl, ga = backward(dim, grad_output, value_c, ctx.levels, loc_c, attn_c,
                          ctx.clamp_grid, ctx.clamp_eps)
    vdt, ldt, adt = ctx.in_dtypes
    return gv.to(vdt), None, gl.to(ldt), ga.to(adt), None, None


def run_fwd(name: str, dim: int, value, value_spatial_shapes, sampling_locations,
            attention_weights, clamp_grid, clamp_eps) -> torch.Tensor:
    """Forward-only entry (msda2d_fwd / msda3d_fwd)."""
    validate_inputs(name, dim, value, value_spatial_shapes, sampling_locations, attention_weights)
    levels = prepare_levels(dim, value, value_spatial_shapes)
    out = forward(dim, value, levels, sampling_locations, attention_weights, clamp_grid,
                  clamp_eps)[0]
    return out
