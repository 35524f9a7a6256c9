"""Shared pieces of the benchmark CLI: configurations, inputs, timing and the summary table.

Methodology of the reference's benchmarks (benchmarks/benchmark_msda2d.py:158-254): inputs
drawn on the device (value ~ N(0,1), locations ~ U[0,1], weights = softmax of U[0,1)
logits over L*P), forward timed with events over 20 calls after 5 warm-up calls, and
forward + backward over 10 iterations after 3, each iteration cloning the inputs and
drawing a fresh grad_output; the extra memory is the peak allocation above the baseline.
"""

from __future__ import annotations

import math
import sys
from collections.abc import Callable
from dataclasses import dataclass
from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parents[1] / "msda-triton_amd"
if str(_PKG) not in sys.path:
    sys.path.insert(0, str(_PKG))

DTYPES = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


@dataclass(frozen=True)
class BenchmarkConfig:
    name: str
    batch_size: int
    num_queries: int
    num_heads: int
    dim_per_head: int
    num_levels: int
    num_points: int
    spatial_shapes: tuple
    # the reference's published Triton times on an RTX 4070 Ti, fp32 (README.md:84-99):
    # (fwd ms, fwd+bwd ms), or None
    published: tuple | None = None

    @property
    def embed_dims(self) -> int:
        return self.num_heads * self.dim_per_head

    @property
    def dim(self) -> int:
        return len(self.spatial_shapes[0])


def make_inputs(cfg: BenchmarkConfig, device, dtype, requires_grad=False) -> dict:
    keys = sum(math.prod(s) for s in cfg.spatial_shapes)
    B, Q, H, L, P = cfg.batch_size, cfg.num_queries, cfg.num_heads, cfg.num_levels, cfg.num_points
    value = torch.randn(B, keys, H, cfg.dim_per_head, device=device, dtype=dtype)
    loc = torch.rand(B, Q, H, L, P, cfg.dim, device=device, dtype=dtype)
    attn = torch.rand(B, Q, H, L * P, device=device, dtype=dtype).softmax(-1).view(B, Q, H, L, P)
    for t in (value, loc, attn):
        t.requires_grad_(requires_grad)
    shapes = torch.tensor(cfg.spatial_shapes, device=device, dtype=torch.int32)
    return {"value": value, "spatial_shapes": shapes, "sampling_locations": loc,
            "attention_weights": attn}


def _timed(step: Callable[[], object], warmup: int, iters: int, device) -> dict:
    for _ in range(warmup):
        step()
    torch.cuda.synchronize(device)
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats(device)
    base = torch.cuda.memory_allocated(device)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        step()
    e1.record()
    torch.cuda.synchronize(device)
    return {"time_ms": e0.elapsed_time(e1) / iters,
            "memory_mb": (torch.cuda.max_memory_allocated(device) - base) / 2**20}


def time_forward(fn: Callable, inp: dict, warmup: int = 5, iters: int = 20) -> dict:
    args = (inp["value"], inp["spatial_shapes"], inp["sampling_locations"], inp["attention_weights"])
    return _timed(lambda: fn(*args), warmup, iters, inp["value"].device)


def time_forward_backward(fn: Callable, inp: dict, warmup: int = 3, iters: int = 10) -> dict:
    def step():
        v = inp["value"].detach().clone().requires_grad_(True)
        lo = inp["sampling_locations"].detach().clone().requires_grad_(True)
        a = inp["attention_weights"].detach().clone().requires_grad_(True)
        out = fn(v, inp["spatial_shapes"], lo, a)
        out.backward(torch.randn_like(out))
        return v.grad, lo.grad, a.grad
    return _timed(step, warmup, iters, inp["value"].device)


def run_benchmark(cfg: BenchmarkConfig, device, dtype, torch_fwd: Callable, hip_fwd: Callable,
                  hip_op: Callable) -> dict:
    print(f"\n{'=' * 70}\nConfig: {cfg.name}\n  Queries: {cfg.num_queries}, Heads: {cfg.num_heads}, "
          f"Levels: {cfg.num_levels}\n  Spatial shapes: {list(cfg.spatial_shapes)}\n  Dtype: {dtype}\n{'=' * 70}")
    res = {"config": cfg.name, "published": cfg.published}
    inp = make_inputs(cfg, device, dtype)
    inp_g = make_inputs(cfg, device, dtype, requires_grad=True)
    print("\nForward pass:")
    for key, fn, label in (("pytorch_fwd", torch_fwd, "PyTorch"), ("hip_fwd", hip_fwd, "HIP")):
        r = time_forward(fn, inp)
        res[key + "_ms"], res[key + "_mb"] = r["time_ms"], r["memory_mb"]
        print(f"  {label + ':':<9}{r['time_ms']:.3f} ms, {r['memory_mb']:.1f} MB")
    res["fwd_speedup"] = res["pytorch_fwd_ms"] / max(res["hip_fwd_ms"], 1e-6)
    print(f"  Speedup: {res['fwd_speedup']:.2f}x")
    print("\nForward + Backward pass:")
    for key, fn, label in (("pytorch_bwd", torch_fwd, "PyTorch"), ("hip_bwd", hip_op, "HIP")):
        r = time_forward_backward(fn, inp_g)
        res[key + "_ms"], res[key + "_mb"] = r["time_ms"], r["memory_mb"]
        print(f"  {label + ':':<9}{r['time_ms']:.3f} ms, {r['memory_mb']:.1f} MB")
    res["bwd_speedup"] = res["pytorch_bwd_ms"] / max(res["hip_bwd_ms"], 1e-6)
    print(f"  Speedup: {res['bwd_speedup']:.2f}x")
    return res


def print_summary_table(dim: int, results: list[dict]) -> None:
    print("\n" + "=" * 104)
    print(f"SUMMARY: {dim}D MSDA Benchmarks (PyTorch vs HIP; last columns: the reference's "
          f"published Triton times, RTX 4070 Ti fp32)")
    print("=" * 104)
    print(f"{'Config':<10} | {'Forward (ms)':<23} | {'Fwd+Bwd (ms)':<23} | {'Speedup':<11} | "
          f"{'Published Triton (ms)':<22}")
    print(f"{'':10} | {'PyTorch':>10} {'HIP':>10}  | {'PyTorch':>10} {'HIP':>10}  | "
          f"{'Fwd':>5} {'Bwd':>5} | {'fwd':>10} {'fwd+bwd':>10}")
    print("-" * 104)
    for r in results:
        pub = r.get("published")
        pubs = f"{pub[0]:>10.2f} {pub[1]:>10.2f}" if pub else f"{'-':>10} {'-':>10}"
        print(f"{r['config']:<10} | {r['pytorch_fwd_ms']:>10.2f} {r['hip_fwd_ms']:>10.2f}  | "
              f"{r['pytorch_bwd_ms']:>10.2f} {r['hip_bwd_ms']:>10.2f}  | "
              f"{r['fwd_speedup']:>4.1f}x {r['bwd_speedup']:>4.1f}x | {pubs}")
    print("=" * 104)


def run_suite(dim: int, configs: list, dtype_name: str) -> list[dict]:
    """Benchmark every config; a failing config is reported and skipped, as in the reference."""
    import msda_triton
    from msda_triton.pytorch import msda2d_pytorch, msda3d_pytorch

    torch_fwd = msda2d_pytorch if dim == 2 else msda3d_pytorch
    hip_fwd = msda_triton.msda2d_fwd if dim == 2 else msda_triton.msda3d_fwd
    hip_op = msda_triton.msda2d if dim == 2 else msda_triton.msda3d
    device = torch.device("cuda")
    out = []
    for cfg in configs:
        try:
            out.append(run_benchmark(cfg, device, DTYPES[dtype_name], torch_fwd, hip_fwd, hip_op))
        except Exception as exc:  # noqa: BLE001 - report and continue, like the reference
            print(f"ERROR running {cfg.name}: {exc}")
    if out:
        print_summary_table(dim, [dict(r, published=r["published"] if dtype_name == "fp32" else None)
                                  for r in out])
    return out
