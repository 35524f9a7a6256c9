"""Import-path compatibility with the reference's ``msda_triton.triton`` subpackage
(reference src/msda_triton/triton/__init__.py:10-22). Nothing here uses Triton: every
name re-exports the HIP implementation from ``msda_triton.hip``."""

from msda_triton.hip.msda_2d import MSDA2DFn, msda2d, msda2d_fwd
from msda_triton.hip.msda_3d import MSDA3DFn, msda3d, msda3d_fwd

__all__ = ["msda2d", "msda2d_fwd", "MSDA2DFn", "msda3d", "msda3d_fwd", "MSDA3DFn"]
