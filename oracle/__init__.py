"""Oracle for the MSDA hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
import this package, and only as the checker (or the timed CPU baseline). The shipped
library ``msda_triton`` never imports, links or calls anything here; its HIP path
raises if its extension is missing instead of falling back to the CPU.

Contents
--------
``torch_ref``  CPU restatement of the reference's pure-PyTorch oracle
               ``msda2d_pytorch`` / ``msda3d_pytorch``
               (src/msda_triton/pytorch/msda_2d.py:58-114, msda_3d.py:58-118):
               ``F.grid_sample`` per level, in the input dtype. Gradients by autograd.
``brute``      ctypes wrapper of ``msda_brute.c``: explicit float64 loops over
               (b, q, h, l, p, corner, channel), forward and analytic backward, that call
               no library sampling routine. It pins ``torch_ref`` independently of
               ``grid_sample``.

How each function is pinned (the tests live in tests/test_oracle.py):
* ``brute`` forward/backward: closed forms (constant field, affine field with its exact
  gradient, pixel-centre sampling returning value rows, permutation gather with
  L = P = 1 and Q = K at all pixel centres), zero padding and clamp semantics with
  hand-computed expectations, float64 finite differences, and linearity in value and
  attention weights.
* ``torch_ref``: agreement with ``brute`` on seeded inputs (2D and 3D, clamp on/off,
  boundary and out-of-range locations), ``torch.autograd.gradcheck`` in float64, and the
  same closed forms.
No golden vectors or known-answer files ship with the reference for this path.
"""
