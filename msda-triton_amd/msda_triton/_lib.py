"""ctypes binding of libmsda_hip.so (the C ABI declared in include/msda.h).

The library is built in-tree by ``msda-triton_amd/build_hip.py`` and loaded from this
package directory. There is no fallback: if the library is missing or fails to load,
every HIP entry point raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libmsda_hip.so")
ABI_VERSION = 5

MSDA_F32, MSDA_F16, MSDA_BF16 = 0, 1, 2
MSDA_OK, MSDA_ERR_INVALID, MSDA_ERR_DTYPE, MSDA_ERR_WORKSPACE, MSDA_ERR_HIP = range(5)

EXPORTED_SYMBOLS = (
    "msda_abi_version",
    "msda_last_error",
    "msda_validate",
    "msda_fwd_workspace_bytes",
    "msda_fwd",
    "msda_bwd_workspace_bytes",
    "msda_bwd",
    "msda_bwd_dev_workspace_bytes",
    "msda_bwd_dev",
    "msda_fwd_fused",
    "msda_bwd_fused_workspace_bytes",
    "msda_bwd_fused",
    "msda_bwd_fused_dev_workspace_bytes",
    "msda_bwd_fused_dev",
    "msda_bwd_noalloc",
)
NOALLOC_SCRATCH_BYTES = 256 << 20  # MSDA_NOALLOC_SCRATCH_BYTES
FLAG_VALUE_HEAD_MAJOR = 1  # MSDA_FLAG_VALUE_HEAD_MAJOR


class MsdaDesc(ctypes.Structure):
    """Mirror of ``msda_desc`` in include/msda.h (64 bytes, natural alignment)."""

    _fields_ = [
        ("dim", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("num_keys", ctypes.c_int64),
        ("num_heads", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("num_queries", ctypes.c_int64),
        ("num_levels", ctypes.c_int32),
        ("num_points", ctypes.c_int32),
        ("value_dtype", ctypes.c_int32),
        ("coord_dtype", ctypes.c_int32),
        ("clamp_grid", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("clamp_eps", ctypes.c_double),
    ]


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library, with argument types declared."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"msda_triton: HIP library {LIB_PATH} is not built. Build it with "
                "`python msda-triton_amd/build_hip.py` (hipcc, gfx950)."
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:
            raise RuntimeError(f"msda_triton: failed to load {LIB_PATH}: {exc}") from exc
        vp, dp = ctypes.c_void_p, ctypes.POINTER(MsdaDesc)
        lib.msda_abi_version.argtypes = []
        lib.msda_abi_version.restype = ctypes.c_int
        lib.msda_last_error.argtypes = []
        lib.msda_last_error.restype = ctypes.c_char_p
        lib.msda_validate.argtypes = [dp]
        lib.msda_validate.restype = ctypes.c_int
        lib.msda_fwd_workspace_bytes.argtypes = [dp]
        lib.msda_fwd_workspace_bytes.restype = ctypes.c_size_t
        lib.msda_fwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
        lib.msda_fwd.restype = ctypes.c_int
        lib.msda_bwd_workspace_bytes.argtypes = [dp, vp]
        lib.msda_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.msda_bwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
        lib.msda_bwd.restype = ctypes.c_int
        lib.msda_bwd_dev_workspace_bytes.argtypes = [dp]
        lib.msda_bwd_dev_workspace_bytes.restype = ctypes.c_size_t
        lib.msda_bwd_dev.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
        lib.msda_bwd_dev.restype = ctypes.c_int
        lib.msda_fwd_fused.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
        lib.msda_fwd_fused.restype = ctypes.c_int
        lib.msda_bwd_fused_workspace_bytes.argtypes = [dp, vp]
        lib.msda_bwd_fused_workspace_bytes.restype = ctypes.c_size_t
        lib.msda_bwd_fused.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                       ctypes.c_size_t, vp]
        lib.msda_bwd_fused.restype = ctypes.c_int
        lib.msda_bwd_fused_dev_workspace_bytes.argtypes = [dp]
        lib.msda_bwd_fused_dev_workspace_bytes.restype = ctypes.c_size_t
        lib.msda_bwd_fused_dev.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                           ctypes.c_size_t, vp]
        lib.msda_bwd_fused_dev.restype = ctypes.c_int
        lib.msda_bwd_noalloc.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        lib.msda_bwd_noalloc.restype = ctypes.c_int
        version = lib.msda_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(
                f"msda_triton: {LIB_PATH} has ABI version {version}, expected {ABI_VERSION}; "
                "rebuild the library"
            )
        _lib = lib
        return lib


def last_error() -> str:
    return load().msda_last_error().decode("utf-8", "replace")


def check(rc: int, what: str) -> None:
    """Raise for a non-OK status returned by the C ABI."""
    if rc == MSDA_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == MSDA_ERR_DTYPE:
        raise NotImplementedError(msg)
    if rc in (MSDA_ERR_INVALID, MSDA_ERR_WORKSPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)
