"""Pure-PyTorch functions (reference src/msda_triton/pytorch/__init__.py:10-20)."""

from msda_triton.pytorch.msda_2d import msda2d_pytorch
from msda_triton.pytorch.msda_3d import msda3d_pytorch

__all__ = ["msda2d_pytorch", "msda3d_pytorch"]
