"""3D MSDA benchmark: pure PyTorch vs HIP (reference benchmarks/benchmark_msda3d.py).

Usage: python -m benchmarks.benchmark_msda3d [--config small|medium|large|xl|all]
                                             [--dtype fp32|fp16|bf16]
"""

from __future__ import annotations

import argparse
import sys

import torch

from benchmarks._common import BenchmarkConfig, print_summary_table, run_suite  # noqa: F401

# the reference's 3D scenarios (benchmark_msda3d.py:44-86) with its published times
BENCHMARK_CONFIGS = [
    BenchmarkConfig("small", 1, 256, 4, 32, 2, 4, ((8, 16, 16), (4, 8, 8)), (0.16, 0.62)),
    BenchmarkConfig("medium", 1, 4096, 8, 32, 3, 4, ((16, 32, 32), (8, 16, 16), (4, 8, 8)), (0.22, 3.34)),
    BenchmarkConfig("large", 1, 16384, 8, 32, 4, 4,
                    ((32, 64, 64), (16, 32, 32), (8, 16, 16), (4, 8, 8)), (1.79, 21.87)),
    BenchmarkConfig("xl", 1, 65536, 8, 32, 4, 4,
                    ((64, 64, 64), (32, 32, 32), (16, 16, 16), (8, 8, 8)), (8.92, 89.65)),
]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Benchmark MSDA3D implementations")
    ap.add_argument("--config", choices=[c.name for c in BENCHMARK_CONFIGS] + ["all"], default="all")
    ap.add_argument("--dtype", choices=["fp32", "fp16", "bf16"], default="fp32")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("ERROR: no GPU available")
        return 1
    print(f"Device: {torch.cuda.get_device_name()}\nHIP: {torch.version.hip}")
    cfgs = BENCHMARK_CONFIGS if args.config == "all" else [c for c in BENCHMARK_CONFIGS if c.name == args.config]
    run_suite(3, cfgs, args.dtype)
    return 0


if __name__ == "__main__":
    sys.exit(main())
