"""Benchmark CLI matching the reference's benchmarks/ package (run_benchmarks.py, benchmark_msda2d.py,
benchmark_msda3d.py): the pure-PyTorch path against the HIP kernels on the same inputs."""
