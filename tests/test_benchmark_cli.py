"""Benchmark CLI (benchmarks/, mirroring the reference's benchmarks/ package).

CPU: the scenario tables match the reference's (names, sizes, shapes) and every entry point
refuses to run without a GPU. GPU: the smallest 2D and 3D scenarios run end to end through
run_suite and report both paths.
"""

from __future__ import annotations

import pytest
import torch

from benchmarks import benchmark_msda2d, benchmark_msda3d, run_benchmarks


def test_scenarios_match_reference():
    c2 = {c.name: c for c in benchmark_msda2d.BENCHMARK_CONFIGS}
    c3 = {c.name: c for c in benchmark_msda3d.BENCHMARK_CONFIGS}
    assert list(c2) == ["tiny", "small", "medium", "large", "xl"]
    assert list(c3) == ["small", "medium", "large", "xl"]
    assert c2["medium"].batch_size == 2 and c2["medium"].spatial_shapes[0] == (100, 134)
    assert c2["xl"].num_queries == 32400 and c2["xl"].spatial_shapes[-1] == (32, 32)
    assert c3["small"].num_heads == 4 and c3["small"].num_levels == 2
    assert c3["xl"].spatial_shapes == ((64, 64, 64), (32, 32, 32), (16, 16, 16), (8, 8, 8))
    for c in list(c2.values()) + list(c3.values()):
        assert len(c.spatial_shapes) == c.num_levels and c.embed_dims == c.num_heads * c.dim_per_head


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU path")
def test_cli_needs_gpu():
    assert run_benchmarks.main(["--2d-only"]) == 1
    assert benchmark_msda2d.main(["--config", "tiny"]) == 1
    assert benchmark_msda3d.main(["--config", "small"]) == 1


@pytest.mark.gpu
def test_smallest_scenarios_run():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from benchmarks._common import run_suite
    r2 = run_suite(2, benchmark_msda2d.BENCHMARK_CONFIGS[:1], "fp32")
    r3 = run_suite(3, benchmark_msda3d.BENCHMARK_CONFIGS[:1], "bf16")
    for r in r2 + r3:
        for k in ("pytorch_fwd_ms", "hip_fwd_ms", "pytorch_bwd_ms", "hip_bwd_ms"):
            assert r[k] > 0
    assert len(r2) == 1 and len(r3) == 1
