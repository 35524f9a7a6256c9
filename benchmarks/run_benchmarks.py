"""Benchmark suite runner (reference benchmarks/run_benchmarks.py).

Usage: python -m benchmarks.run_benchmarks [--2d-only | --3d-only] [--dtype fp32|fp16|bf16]
Runs the 3D then the 2D scenarios (pure PyTorch vs HIP) and prints a summary table for
each, with the reference's published Triton times (RTX 4070 Ti, fp32) beside them.
"""

from __future__ import annotations

import argparse
import sys

import torch

from benchmarks import benchmark_msda2d, benchmark_msda3d
from benchmarks._common import run_suite


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Run the MSDA benchmarks")
    ap.add_argument("--2d-only", dest="only_2d", action="store_true", help="Run only 2D benchmarks")
    ap.add_argument("--3d-only", dest="only_3d", action="store_true", help="Run only 3D benchmarks")
    ap.add_argument("--dtype", choices=["fp32", "fp16", "bf16"], default="fp32")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("ERROR: no GPU available")
        return 1
    print("=" * 80 + "\nMSDA BENCHMARK SUITE (MI355X HIP)\n" + "=" * 80)
    print(f"Device: {torch.cuda.get_device_name()}\nPyTorch: {torch.__version__}\n"
          f"HIP: {torch.version.hip}\nData type: {args.dtype}")
    # --2d-only wins over --3d-only; with neither, 3D runs first, then 2D
    run_3d = not args.only_2d
    run_2d = args.only_2d or not args.only_3d
    if run_3d:
        print("\n" + "=" * 80 + "\n3D MULTI-SCALE DEFORMABLE ATTENTION BENCHMARKS\n" + "=" * 80)
        run_suite(3, benchmark_msda3d.BENCHMARK_CONFIGS, args.dtype)
    if run_2d:
        print("\n" + "=" * 80 + "\n2D MULTI-SCALE DEFORMABLE ATTENTION BENCHMARKS\n" + "=" * 80)
        run_suite(2, benchmark_msda2d.BENCHMARK_CONFIGS, args.dtype)
    print("\n" + "=" * 80 + "\nBENCHMARK COMPLETE\n" + "=" * 80)
    return 0


if __name__ == "__main__":
    sys.exit(main())
