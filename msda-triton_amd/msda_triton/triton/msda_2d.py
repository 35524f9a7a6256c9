"""Import-path compatibility for ``msda_triton.triton.msda_2d`` (re-exports the HIP op)."""

from msda_triton.hip.msda_2d import MSDA2DFn, msda2d, msda2d_fwd

__all__ = ["msda2d", "msda2d_fwd", "MSDA2DFn"]
