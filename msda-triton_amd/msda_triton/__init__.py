"""msda_triton — multi-scale deformable attention for AMD MI355X (gfx950).

Drop-in replacement for mach9robotics/msda-triton (reference src/msda_triton/__init__.py:12-27):
the same top-level exports, backed by hand-written HIP kernels in libmsda_hip.so
(C ABI: include/msda.h) instead of Triton. ``msda_triton.pytorch`` keeps the pure-PyTorch
functions and modules; ``msda_triton.triton`` keeps the reference's import path for the
autograd functions. ``msda2d_fused`` / ``msda3d_fused`` are an addition: they take the
modules' reference points, offsets and attention logits and form the sampling locations and
weights inside the kernel.
"""

from __future__ import annotations

__version__ = "0.1.0"

from msda_triton.hip.msda_2d import msda2d, msda2d_fwd
from msda_triton.hip.msda_3d import msda3d, msda3d_fwd
from msda_triton.hip.fused import msda2d_fused, msda2d_fused_fwd, msda3d_fused, msda3d_fused_fwd

__all__ = [
    "__version__",
    # 2D (image)
    "msda2d",
    "msda2d_fwd",
    # 3D (volumetric)
    "msda3d",
    "msda3d_fwd",
    # producer-fused variants (locations and weights formed in the kernel)
    "msda2d_fused",
    "msda2d_fused_fwd",
    "msda3d_fused",
    "msda3d_fused_fwd",
]
