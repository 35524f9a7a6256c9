"""2D MSDA benchmark: pure PyTorch vs HIP (reference benchmarks/benchmark_msda2d.py).

Usage: python -m benchmarks.benchmark_msda2d [--config tiny|small|medium|large|xl|all]
                                             [--dtype fp32|fp16|bf16]
"""

from __future__ import annotations

import argparse
import sys

import torch

from benchmarks._common import BenchmarkConfig, print_summary_table, run_suite  # noqa: F401

# the reference's 2D scenarios (benchmark_msda2d.py:34-85) with its published times
BENCHMARK_CONFIGS = [
    BenchmarkConfig("tiny", 1, 100, 8, 32, 4, 4, ((64, 64), (32, 32), (16, 16), (8, 8)), (0.16, 0.58)),
    BenchmarkConfig("small", 1, 900, 8, 32, 4, 4, ((80, 80), (40, 40), (20, 20), (10, 10)), (0.22, 0.71)),
    BenchmarkConfig("medium", 2, 900, 8, 32, 4, 4, ((100, 134), (50, 67), (25, 34), (13, 17)), (0.23, 2.23)),
    BenchmarkConfig("large", 1, 8100, 8, 32, 4, 4, ((200, 200), (100, 100), (50, 50), (25, 25)), (0.62, 6.20)),
    BenchmarkConfig("xl", 1, 32400, 8, 32, 4, 4, ((256, 256), (128, 128), (64, 64), (32, 32)), (1.79, 22.28)),
]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Benchmark MSDA2D implementations")
    ap.add_argument("--config", choices=[c.name for c in BENCHMARK_CONFIGS] + ["all"], default="all")
    ap.add_argument("--dtype", choices=["fp32", "fp16", "bf16"], default="fp32")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("ERROR: no GPU available")
        return 1
    print(f"Device: {torch.cuda.get_device_name()}\nHIP: {torch.version.hip}")
    cfgs = BENCHMARK_CONFIGS if args.config == "all" else [c for c in BENCHMARK_CONFIGS if c.name == args.config]
    run_suite(2, cfgs, args.dtype)
    return 0


if __name__ == "__main__":
    sys.exit(main())
