"""HIP (gfx950) implementation of the msda_triton ops."""

from .msda_2d import MSDA2DFn, msda2d, msda2d_fwd
from .msda_3d import MSDA3DFn, msda3d, msda3d_fwd
from .fused import MSDAFusedFn, msda2d_fused, msda2d_fused_fwd, msda3d_fused, msda3d_fused_fwd

__all__ = ["msda2d", "msda2d_fwd", "MSDA2DFn", "msda3d", "msda3d_fwd", "MSDA3DFn",
           "msda2d_fused", "msda2d_fused_fwd", "msda3d_fused", "msda3d_fused_fwd", "MSDAFusedFn"]
