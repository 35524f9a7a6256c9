"""GPU parity tests for the 3D (trilinear) op; mirrors the reference's tests/test_msda_3d.py."""

from tests._parity import ParitySuite


class TestMSDA3DHip(ParitySuite):
    dim = 3
