"""Import-path compatibility for ``msda_triton.triton.msda_3d`` (re-exports the HIP op)."""

from msda_triton.hip.msda_3d import MSDA3DFn, msda3d, msda3d_fwd

__all__ = ["msda3d", "msda3d_fwd", "MSDA3DFn"]
