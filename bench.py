"""Benchmark of the MSDA hot path on one MI355X.

Metric: "MSDA fwd & fwd+bwd ms + achieved HBM GB/s, 2D encoder & 3D 4-level,
bf16". One step = one msda2d forward + backward (autograd API, preallocated grad_output) of
the 2D Deformable-DETR encoder workload (bf16):
B=2, H=8, C=32, L=4 levels (100x150, 50x75, 25x38, 13x19; K=19947), Q=19947, P=4.
The 3D 4-level workload (configs[4], bf16, 10% of points within 1e-3 of a volume face) is
timed in the same run and reported under "also".

value = algorithmic bytes of fwd+bwd per step / step time, in GB/s, with inputs resident in
HBM. Algorithmic bytes, s = element size: V = B*K*H*C*s, G = B*Q*H*L*P*2^d*C*s,
S = B*Q*H*L*P*d*s, A = B*Q*H*L*P*s, O = B*Q*H*C*s, V' = min(V, G);
fwd = V' + S + A + O, bwd = 2V' + 2S + 2A + O.

Beside the warm (back-to-back) times, each workload is also timed MALL-flushed (a 512 MiB
buffer written between iterations, outside the timed events; median of per-iteration times)
and, for fwd+bwd, the reference benchmark's way (inputs cloned and grad_output drawn with
randn_like inside the timed region, benchmarks/benchmark_msda2d.py:210-218).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
       python bench.py --mode copy   (plain copy kernel of known size, for PMC calibration)
       python bench.py --mode gather (random 64-byte row gather of known size, for PMC
                                      calibration of gathers)
       python bench.py --mode fwd|bwd --config c2|c5 (one entry only, for rocprofv3)
       python bench.py --mode fused --config c2|c5 (producer-fused op against the modules'
                                                    order of operations)
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "msda-triton_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import torch  # noqa: E402

METRIC = "MSDA fwd & fwd+bwd ms + achieved HBM GB/s, 2D encoder & 3D 4-level, bf16"
HBM_PEAK_GBPS = 8000.0
# kernels behind the roofline objects (the C2 bf16 launch: 2D, bf16 value and coordinates,
# 8 channels per lane, 4 points per coordinate block, quad-shared geometry)
FWD_KERNEL = "msda::msda_fwd_staged_kernel<2, msda::BF16, msda::BF16, 8, 4, true, false>"
BWD_KERNELS = ("msda_bwd entry (16-bit values): bwd_count_kernel, bwd_colscan_kernel, "
               "bwd_plan_kernel, bwd_fill_kernel, bwd_tile_kernel, bwd_fold_kernel")

CONFIGS = {
    "c1": dict(dim=2, B=1, H=8, C=32, shapes=[(32, 32), (16, 16)], Q=100, P=4, dtype="fp32",
               face_frac=0.0),
    "c2": dict(dim=2, B=2, H=8, C=32, shapes=[(100, 150), (50, 75), (25, 38), (13, 19)],
               Q=19947, P=4, dtype="bf16", face_frac=0.0),
    "c3": dict(dim=2, B=8, H=8, C=32, shapes=[(100, 150), (50, 75), (25, 38), (13, 19)],
               Q=300, P=4, dtype="bf16", face_frac=0.0),
    "c4": dict(dim=3, B=2, H=8, C=32, shapes=[(16, 32, 32), (8, 16, 16)], Q=4096, P=4,
               dtype="bf16", face_frac=0.0),
    "c5": dict(dim=3, B=1, H=8, C=32, shapes=[(32, 64, 64), (16, 32, 32), (8, 16, 16), (4, 8, 8)],
               Q=32768, P=8, dtype="bf16", face_frac=0.1),
}
DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def num_keys(cfg) -> int:
    k = 0
    for s in cfg["shapes"]:
        n = 1
        for v in s:
            n *= v
        k += n
    return k


def algorithmic_bytes(cfg, q=None) -> dict:
    """Compulsory HBM bytes of fwd, bwd and fwd+bwd (zero-init and workspace excluded)."""
    s = torch.tensor([], dtype=DTYPES[cfg["dtype"]]).element_size()
    d, B, H, C, P = cfg["dim"], cfg["B"], cfg["H"], cfg["C"], cfg["P"]
    L, Q, K = len(cfg["shapes"]), (cfg["Q"] if q is None else q), num_keys(cfg)
    n = B * Q * H * L * P
    V, G = B * K * H * C * s, n * (2 ** d) * C * s
    S, A, O = n * d * s, n * s, B * Q * H * C * s
    Vp = min(V, G)
    fwd = Vp + S + A + O
    bwd = 2 * Vp + 2 * S + 2 * A + O
    return {"fwd": fwd, "bwd": bwd, "fwd_bwd": fwd + bwd, "gathered": G}


def make_inputs(cfg, q=None, seed=42):
    """Seeded CPU inputs: value ~ N(0,1), locations ~ U[0,1]^d, weights = softmax over L*P of
    N(0,1) logits; with face_frac > 0, that fraction of points gets one random coordinate
    moved within 1e-3 of a volume face (exercises clamp_grid with clamp_eps=1e-4)."""
    g = torch.Generator().manual_seed(seed)
    d, B, H, C, P = cfg["dim"], cfg["B"], cfg["H"], cfg["C"], cfg["P"]
    L, Q, K = len(cfg["shapes"]), (cfg["Q"] if q is None else q), num_keys(cfg)
    value = torch.randn(B, K, H, C, generator=g)
    loc = torch.rand(B, Q, H, L, P, d, generator=g)
    logits = torch.randn(B, Q, H, L * P, generator=g)
    if cfg["face_frac"] > 0:
        n = B * Q * H * L * P
        pick = torch.rand(n, generator=g) < cfg["face_frac"]
        axis = torch.randint(0, d, (n,), generator=g)
        side = torch.rand(n, generator=g) < 0.5
        off = torch.rand(n, generator=g) * 1e-3
        flat = loc.view(n, d)
        rows = torch.nonzero(pick).squeeze(1)
        newv = torch.where(side[rows], 1.0 - off[rows], off[rows])
        flat[rows, axis[rows]] = newv
    attn = logits.softmax(-1).view(B, Q, H, L, P)
    shapes = torch.tensor(cfg["shapes"], dtype=torch.int64)
    return value, shapes, loc, attn


class GpuCase:
    """Device-resident inputs of one workload plus direct entry-point timers."""

    def __init__(self, cfg, device):
        from msda_triton.hip import _core

        self.core = _core
        self.cfg = cfg
        self.dim = cfg["dim"]
        dt = DTYPES[cfg["dtype"]]
        value, shapes, loc, attn = make_inputs(cfg)
        self.shapes = shapes
        self.value = value.to(device, dt)
        self.loc = loc.to(device, dt)
        self.attn = attn.to(device, dt)
        self.levels = _core.prepare_levels(self.dim, self.value, shapes)
        g = torch.Generator().manual_seed(7)
        B, Q, HC = cfg["B"], cfg["Q"], cfg["H"] * cfg["C"]
        self.grad_out = torch.randn(B, Q, HC, generator=g).to(device, dt)
        self.op = None

    def fwd(self):
        return self.core.forward(self.dim, self.value, self.levels, self.loc, self.attn,
                                 True, 1e-4)[0]

    def bwd(self):
        return self.core.backward(self.dim, self.grad_out, self.value, self.levels, self.loc,
                                  self.attn, True, 1e-4)

    def step(self, shapes=None):
        import msda_triton

        op = msda_triton.msda2d if self.dim == 2 else msda_triton.msda3d
        v = self.value.detach().requires_grad_(True)
        lo = self.loc.detach().requires_grad_(True)
        a = self.attn.detach().requires_grad_(True)
        out = op(v, self.shapes if shapes is None else shapes, lo, a, True, 1e-4)
        out.backward(self.grad_out)
        return out

    def step_cloning(self):
        """fwd+bwd the way the reference benchmark times it (benchmark_msda2d.py:210-218):
        inputs cloned and grad_output drawn with randn_like inside the timed region."""
        import msda_triton

        op = msda_triton.msda2d if self.dim == 2 else msda_triton.msda3d
        v = self.value.clone().detach().requires_grad_(True)
        lo = self.loc.clone().detach().requires_grad_(True)
        a = self.attn.clone().detach().requires_grad_(True)
        out = op(v, self.shapes, lo, a, True, 1e-4)
        out.backward(torch.randn_like(out))
        return v.grad, lo.grad, a.grad


def time_events(fn, iters, warmup):
    """Average ms per call of fn, from HIP events on the current stream (the launch stream)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


FLUSH_BYTES = 512 << 20  # larger than MI355X's 256 MB MALL


def time_flushed(fn, iters, warmup, flush):
    """Median ms per call of fn with the caches flushed before each call: `flush` (a buffer
    larger than the MALL) is rewritten between calls, outside each call's event pair."""
    for _ in range(warmup):
        fn()
    evs = []
    for i in range(iters):
        flush.fill_(i & 0xFF)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        evs.append((e0, e1))
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in evs)


def measure_case(cfg, device, steps, warmup, flush=None):
    case = GpuCase(cfg, device)
    byt = algorithmic_bytes(cfg)
    fwd_ms = time_events(case.fwd, max(steps, 20), warmup)
    bwd_ms = time_events(case.bwd, max(steps, 20), warmup)
    # timed region: exactly `steps` autograd steps between synchronisations
    for _ in range(warmup):
        case.step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        case.step()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    step_ms = max(e0.elapsed_time(e1) / steps, wall_ms)
    gbps = lambda b, ms: b / (ms * 1e-3) / 1e9  # noqa: E731
    res = {
        "config": cfg,
        "bytes": byt,
        "fwd_ms": fwd_ms,
        "bwd_ms": bwd_ms,
        "step_ms": step_ms,
        "fwd_gbps": gbps(byt["fwd"], fwd_ms),
        "bwd_gbps": gbps(byt["bwd"], bwd_ms),
        "step_gbps": gbps(byt["fwd_bwd"], step_ms),
    }
    if flush is not None:
        n = max(steps, 20)
        res["fwd_ms_flushed"] = time_flushed(case.fwd, n, warmup, flush)
        res["step_ms_flushed"] = time_flushed(case.step, n, warmup, flush)
        res["step_ms_cloning"] = time_events(case.step_cloning, max(steps, 10), warmup)
    return res


def measure_fused(cfg, device, steps, warmup):
    """The producer-fused op (msda2d_fused / msda3d_fused: locations and softmax weights
    formed in the kernel) against the attention modules' order of operations (softmax over
    L*P, reference + offset / normaliser, then the plain op), forward and fwd+bwd."""
    import msda_triton
    from msda_triton.hip import _core, fused

    g = torch.Generator().manual_seed(5)
    d, B, H, C, P = cfg["dim"], cfg["B"], cfg["H"], cfg["C"], cfg["P"]
    L, Q, K = len(cfg["shapes"]), cfg["Q"], num_keys(cfg)
    dt = DTYPES[cfg["dtype"]]
    shapes = torch.tensor(cfg["shapes"], dtype=torch.int64)
    value = torch.randn(B, K, H, C, generator=g).to(device, dt)
    ref = torch.rand(B, Q, L, d, generator=g).to(device)
    off = (2.0 * torch.randn(B, Q, H, L, P, d, generator=g)).to(device, dt)  # pixels
    logits = torch.randn(B, Q, H, L, P, generator=g).to(device, dt)
    grad_out = torch.randn(B, Q, H * C, generator=g).to(device, dt)
    norm = shapes.flip(-1).to(device)
    levels = _core.prepare_levels(d, value, shapes)
    op_f = msda_triton.msda2d_fused if d == 2 else msda_triton.msda3d_fused
    op_p = msda_triton.msda2d if d == 2 else msda_triton.msda3d

    def form(o, lg, r):
        attn = lg.view(B, Q, H, L * P).softmax(-1).view(B, Q, H, L, P)
        return r[:, :, None, :, None, :] + o / norm[None, None, None, :, None, :], attn

    def fwd_fused():
        return fused.forward(d, value, levels, ref, off, logits, True, 1e-4)[0]

    def fwd_unfused():
        loc, attn = form(off, logits, ref)
        return _core.forward(d, value, levels, loc.to(dt), attn, True, 1e-4)[0]

    def leaves():
        return (value.detach().requires_grad_(True), ref.detach().requires_grad_(True),
                off.detach().requires_grad_(True), logits.detach().requires_grad_(True))

    def step_fused():
        v, r, o, lg = leaves()
        op_f(v, shapes, r, o, lg).backward(grad_out)

    def step_unfused():
        v, r, o, lg = leaves()
        loc, attn = form(o, lg, r)
        op_p(v, shapes, loc.to(dt), attn).backward(grad_out)

    n = max(steps, 20)
    return {"fwd_ms": round(time_events(fwd_fused, n, warmup), 5),
            "unfused_fwd_ms": round(time_events(fwd_unfused, n, warmup), 5),
            "fwd_bwd_ms": round(time_events(step_fused, n, warmup), 5),
            "unfused_fwd_bwd_ms": round(time_events(step_unfused, n, warmup), 5),
            "note": "fused: msda*_fused (reference points, pixel offsets and logits in; "
                    "locations and softmax formed in the kernel); unfused: the modules' torch "
                    "softmax and location formation, then msda*; fwd_bwd with gradients for "
                    "value, reference points, offsets and logits"}


def cpu_model() -> str:
    """The host CPU's model name (from /proc/cpuinfo), else the platform's description."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(cfg, q_sample=None, reps=3):
    """The oracle (torch grid_sample restatement, fp32 on upcast inputs) timed on the host
    CPU: fwd + backward of out.sum(), on the first q_sample queries of the workload."""
    from oracle import torch_ref

    torch.set_num_threads(min(torch.get_num_threads(), len(os.sched_getaffinity(0))))
    q_sample = cfg["Q"] if q_sample is None else min(q_sample, cfg["Q"])
    value, shapes, loc, attn = make_inputs(cfg, q=q_sample)
    dt = DTYPES[cfg["dtype"]]
    value, loc, attn = (t.to(dt).float() for t in (value, loc, attn))

    def run():
        v = value.clone().requires_grad_(True)
        lo = loc.clone().requires_grad_(True)
        a = attn.clone().requires_grad_(True)
        torch_ref.msda_ref(v, shapes, lo, a, True, 1e-4).sum().backward()

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    byt = algorithmic_bytes(cfg, q=q_sample)["fwd_bwd"]
    return {
        "value": round(byt / t / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"oracle/torch_ref.msda_ref fwd+bwd(out.sum()) in fp32 on bf16-rounded inputs, "
                   f"first {q_sample} of {cfg['Q']} queries, median of {reps}; "
                   f"{t * 1e3:.1f} ms per sample, {t * 1e3 * cfg['Q'] / q_sample:.0f} ms "
                   f"per full step by linear scaling; CPU {cpu_model()}"),
    }


def load_traffic(key: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary profiles/traffic.json:
    (FETCH_SIZE scaled by the streaming-copy factor + WRITE_SIZE, the same with the
    random-row gather factor), or (None, None)."""
    f = REPO / "profiles" / "traffic.json"
    try:
        e = json.loads(f.read_text()).get(key)
    except (OSError, ValueError):
        return None, None
    if isinstance(e, dict):
        return e.get("copy_calibrated"), e.get("gather_calibrated")
    return e, None


def load_ceiling(key: str):
    """The forward's counter-backed ceiling from profiles/fwd_ceiling.json: its L2 request
    counts (rocprofv3 TCC counters) served at the gather probes' L2 and MALL row rates, as
    {"ms", "frac"} of the HBM roofline, or None."""
    try:
        e = json.loads((REPO / "profiles" / "fwd_ceiling.json").read_text()).get(key)
    except (OSError, ValueError):
        return None
    if not isinstance(e, dict):
        return None
    return {"bound": "L2 line requests: hits at the L2 gather rate, misses at the MALL rate",
            "l2_requests": e["l2_requests"], "l2_misses": e["l2_misses"],
            "ms": e["ceiling_ms"], "frac": e["ceiling_frac"], "source": "profiles/fwd_ceiling.md"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--mode", choices=["full", "fwd", "bwd", "step", "copy", "gather", "fused"],
                    default="full")
    ap.add_argument("--config", choices=sorted(CONFIGS), default="c2")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-queries", type=int, default=None)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(MSDA shards by (batch, head) with no exchange between shards). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)

    if args.mode == "copy":
        n = 1 << 28  # 256 MiB read + 256 MiB written per copy
        src = torch.ones(n, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        ms = time_events(lambda: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"mode": "copy", "bytes_read": n, "bytes_written": n, "ms": ms}))
        return
    if args.mode == "gather":
        # 16 M random 64-byte rows (bf16, 32 channels) out of a 4 GiB table, far beyond the
        # MALL: each row is fetched from HBM once; int32 indices, output written once
        rows, n = (4 << 30) // 64, 1 << 24
        table = torch.empty(rows, 32, dtype=torch.bfloat16, device=device).fill_(1.0)
        idx = torch.randperm(rows, device=device)[:n].to(torch.int32)
        out = torch.empty(n, 32, dtype=torch.bfloat16, device=device)
        ms = time_events(lambda: torch.index_select(table, 0, idx, out=out), args.steps, args.warmup)
        print(json.dumps({"mode": "gather", "bytes_read": n * 64 + n * 4, "bytes_written": n * 64,
                          "rows": n, "ms": ms}))
        return
    if args.mode == "fused":
        r = measure_fused(CONFIGS[args.config], device, args.steps, args.warmup)
        print(json.dumps({"mode": "fused", "config": args.config, **r}))
        return
    if args.mode in ("fwd", "bwd", "step"):
        case = GpuCase(CONFIGS[args.config], device)
        fn = {"fwd": case.fwd, "bwd": case.bwd, "step": case.step}[args.mode]
        ms = time_events(fn, args.steps, args.warmup)
        print(json.dumps({"mode": args.mode, "config": args.config, "ms": ms}))
        return

    main_cfg, also_cfg = CONFIGS["c2"], CONFIGS["c5"]
    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=device)
    r = measure_case(main_cfg, device, args.steps, args.warmup, flush)
    r5 = measure_case(also_cfg, device, args.steps, args.warmup, flush)
    # C2 with the level shapes resident on the GPU (the backward plans on the device)
    c2 = GpuCase(main_cfg, device)
    shapes_dev = c2.shapes.to(device, torch.int32)
    c2_gpu_shapes_ms = time_events(lambda: c2.step(shapes_dev), max(args.steps, 20), args.warmup)
    del flush
    # the other BASELINE.json configurations: C2 in fp32, C4 (3D 2-level) in fp32 and bf16,
    # and C3 (decoder cross-attention, forward only: host and launch latency bound)
    extra = {}
    for key, name, dt in (("c2_fp32", "c2", "fp32"), ("c4_fp32", "c4", "fp32"), ("c4_bf16", "c4", "bf16")):
        extra[key] = measure_case(dict(CONFIGS[name], dtype=dt), device, args.steps, args.warmup)
    c3 = GpuCase(CONFIGS["c3"], device)
    import msda_triton
    c3_args = (c3.value, c3.shapes, c3.loc, c3.attn)
    c3_fwd_ms = time_events(lambda: msda_triton.msda2d_fwd(*c3_args), max(args.steps, 20), args.warmup)
    fused_c2 = measure_fused(main_cfg, device, args.steps, args.warmup)
    fused_c5 = measure_fused(also_cfg, device, args.steps, args.warmup)

    # roofline: the forward kernel, which is one launch per msda2d_fwd call (the kernel the
    # bf16 forward target is stated on); the backward entry (sample-gradient, record fill,
    # scans, tile and fold kernels on the same stream) is reported beside it as a group
    def roof(kname, kbytes, kms, key):
        achieved = kbytes / (kms * 1e-3) / 1e9
        traffic, traffic_g = load_traffic(key)
        return {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": traffic, "traffic_gather_calibrated": traffic_g, "kernel": kname,
                "algorithmic_bytes_per_launch": kbytes, "avg_launch_ms": round(kms, 5)}

    roofline = roof(FWD_KERNEL, r["bytes"]["fwd"], r["fwd_ms"], "msda_fwd:c2_bf16")
    # what bounds this design below the HBM roofline: its L2 line requests
    roofline["ceiling"] = load_ceiling("msda_fwd:c2_bf16")
    roofline_bwd = roof(BWD_KERNELS, r["bytes"]["bwd"], r["bwd_ms"], "msda_bwd:c2_bf16")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(main_cfg, q_sample=args.cpu_queries)

    def summary(x):
        out = {"fwd_ms": round(x["fwd_ms"], 5), "fwd_bwd_ms": round(x["step_ms"], 5),
               "bwd_ms": round(x["bwd_ms"], 5), "bwd_gbps": round(x["bwd_gbps"], 2),
               "fwd_gbps": round(x["fwd_gbps"], 2),
               "fwd_roofline_frac": round(x["fwd_gbps"] / HBM_PEAK_GBPS, 4),
               "fwd_bwd_gbps": round(x["step_gbps"], 2),
               "bytes_fwd": x["bytes"]["fwd"], "bytes_fwd_bwd": x["bytes"]["fwd_bwd"]}
        for k in ("fwd_ms_flushed", "step_ms_flushed", "step_ms_cloning"):
            if k in x:
                out[k.replace("step_", "fwd_bwd_")] = round(x[k], 5)
        return out

    line = {
        "metric": METRIC,
        "value": round(r["step_gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["step_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "2D Deformable-DETR encoder self-attention fwd+bwd "
                               "(BASELINE.json configs[1])",
                   "B": 2, "H": 8, "C": 32, "levels": main_cfg["shapes"], "K": num_keys(main_cfg),
                   "Q": main_cfg["Q"], "P": 4, "clamp_grid": True, "clamp_eps": 1e-4},
        "c2_bf16": dict(summary(r), fwd_bwd_ms_gpu_shapes=round(c2_gpu_shapes_ms, 5)),
        "also": {"c5_bf16_3d_4level": dict(summary(r5), fwd_ceiling=load_ceiling("msda_fwd:c5_bf16")),
                 **{k: summary(v) for k, v in extra.items()},
                 "c3_bf16_decoder": {"fwd_ms": round(c3_fwd_ms, 5),
                                     "note": "msda2d_fwd through the Python API (host time included)"},
                 "c2_bf16_fused_producer": fused_c2,
                 "c5_bf16_fused_producer": fused_c5},
        "roofline": roofline,
        "roofline_bwd": roofline_bwd,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
