"""Microbenchmark probes behind the kernels' design (gather line-request ceiling, atomic
and LDS-atomic throughput) on one MI355X. Measurement only; see benchmarks/probes.hip.

    python benchmarks/probes.py build     # compile libmsda_probes.so (hipcc, gfx950)
    python benchmarks/probes.py           # build if needed, run every probe, print markdown

Times are HIP events around one launch (after one warm-up launch); rates divide the work
of that launch by its time. The gather table sizes put it in one XCD's 4 MB L2 (2 MB),
in the 256 MB MALL (64 MB) or in HBM (4 GB).
"""

from __future__ import annotations

import ctypes
import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "probes.hip"
LIB = HERE / "_build" / "libmsda_probes.so"
ARCH = os.environ.get("MSDA_OFFLOAD_ARCH", "gfx950")


def build() -> Path:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    LIB.parent.mkdir(exist_ok=True)
    cmd = [hipcc, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-munsafe-fp-atomics", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           str(SRC), "-o", str(LIB)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {SRC.name}:\n{res.stderr}")
    return LIB


def _load():
    if not LIB.exists():
        build()
    lib = ctypes.CDLL(str(LIB))
    vp, u32, u64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64
    lib.probe_gather.argtypes = [vp, u64, ctypes.c_int, u32, u32, vp, vp]
    lib.probe_atomic.argtypes = [vp, u64, ctypes.c_int, u32, u32, vp]
    lib.probe_lds.argtypes = [ctypes.c_int, u32, u32, vp, vp]
    for f in (lib.probe_gather, lib.probe_atomic, lib.probe_lds):
        f.restype = ctypes.c_int
    return lib


def run() -> dict:
    import torch

    lib = _load()
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    cus = props.multi_processor_count
    clk_ghz = 2.4  # MI355X peak engine clock
    stream = torch.cuda.current_stream().cuda_stream

    def timed(launch):
        launch()  # warm-up
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        rc = launch()
        e1.record()
        torch.cuda.synchronize()
        assert rc == 0, f"launch failed ({rc})"
        return e0.elapsed_time(e1) * 1e-3  # s

    out = {"device": props.name, "cus": cus, "gather": [], "atomic": [], "lds": []}
    blocks = cus * 8
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    for size, where in ((2 << 20, "L2"), (64 << 20, "MALL"), (4 << 30, "HBM")):
        table = torch.ones(size // 4, dtype=torch.int32, device=dev)
        for row in (64, 128):
            iters = 256 if where != "HBM" else 64
            t = timed(lambda: lib.probe_gather(table.data_ptr(), size, row, blocks, iters,
                                               sink.data_ptr(), stream))
            nrows = blocks * 256 // (row // 16) * iters * 8
            out["gather"].append({"table": where, "table_bytes": size, "row_bytes": row,
                                  "rows": nrows, "s": t, "G_rows_per_s": nrows / t / 1e9,
                                  "TB_per_s": nrows * row / t / 1e12})
        del table
    table = torch.zeros((256 << 20) // 4, dtype=torch.float32, device=dev)
    for bf16 in (0, 1):
        iters = 64
        t = timed(lambda: lib.probe_atomic(table.data_ptr(), table.numel() * 4, bf16, blocks, iters,
                                           stream))
        elems = blocks * 256 * iters * (2 if bf16 else 1)
        out["atomic"].append({"kind": "packed bf16" if bf16 else "fp32", "element_adds": elems,
                              "s": t, "T_elem_adds_per_s": elems / t / 1e12})
    del table
    lsink = torch.empty(cus * 4, dtype=torch.int32, device=dev)
    for mode, name in ((0, "ds_add_u32"), (1, "ds_add_f32"), (2, "ds_write_b32")):
        iters, lblocks = 4096, cus * 4
        t = timed(lambda: lib.probe_lds(mode, lblocks, iters, lsink.data_ptr(), stream))
        ops = lblocks * 256 * iters
        out["lds"].append({"op": name, "lane_ops": ops, "s": t,
                           "lane_ops_per_clk_per_cu": ops / t / (clk_ghz * 1e9) / cus})
    return out


def markdown(r: dict) -> str:
    lines = [f"Device: {r['device']}, {r['cus']} CUs; clock for per-clock rates: 2.4 GHz.", "",
             "| gather table | row bytes | G rows/s | TB/s of rows |", "|---|---:|---:|---:|"]
    for g in r["gather"]:
        lines.append(f"| {g['table']} ({g['table_bytes'] >> 20} MiB) | {g['row_bytes']} | "
                     f"{g['G_rows_per_s']:.1f} | {g['TB_per_s']:.2f} |")
    lines += ["", "| global atomics on random 128-byte rows | T element adds/s |", "|---|---:|"]
    for a in r["atomic"]:
        lines.append(f"| {a['kind']} | {a['T_elem_adds_per_s']:.3f} |")
    lines += ["", "| LDS op, random word of 64 KB | lane ops / clk / CU |", "|---|---:|"]
    for x in r["lds"]:
        lines.append(f"| {x['op']} | {x['lane_ops_per_clk_per_cu']:.2f} |")
    return "\n".join(lines)


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "build":
        print(build())
    else:
        res = run()
        print(markdown(res))
        print(json.dumps(res))
