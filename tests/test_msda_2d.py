"""GPU parity tests for the 2D (bilinear) op; mirrors the reference's tests/test_msda_2d.py."""

from tests._parity import ParitySuite


class TestMSDA2DHip(ParitySuite):
    dim = 2
