"""Pure-PyTorch functions and the attention modules (reference
src/msda_triton/pytorch/__init__.py:10-20). The modules live in msda_triton.modules and run
the HIP op; they are re-exported here, at the reference's import path."""

from msda_triton.pytorch.msda_2d import MSDA2D, msda2d_pytorch
from msda_triton.pytorch.msda_3d import MSDA3D, msda3d_pytorch

__all__ = [
    # 2D
    "msda2d_pytorch",
    "MSDA2D",
    # 3D
    "msda3d_pytorch",
    "MSDA3D",
]
