#!/usr/bin/env python3
"""Benchmark of the decode-step hot path on one MI355X.

Workload (default): the affine 4-bit group-64 quantised GEMV
  y bf16 [8, 6144] = x bf16 [8, 2048] . W[6144, 2048]^T
streamed over ROTATE distinct weight copies (> 512 MB in total, so the 256 MB
Infinity Cache cannot serve them). One step = one GEMV launch on the next copy.
Prints one JSON line (see the driver contract in the repository README).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "rust-ts-tokio-inference-engine_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

METRIC = "decode tokens/sec @ ragged batch 64 (1 GPU); qGEMV HBM GB/s % of peak"
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def qgemv_bytes(m, n, k, group=64, bits=4):
    """Algorithmic HBM bytes of one launch: packed W + bf16 scales/biases + x + y."""
    return n * k * bits // 8 + 2 * 2 * n * (k // group) + 2 * m * k + 2 * m * n


def cpu_baseline_qgemv(x_bits, packed, s_bits, b_bits, m, n, k, budget_s=10.0):
    import oracle
    from hip_bridge import quant

    x = quant.bf16_value(x_bits)
    s = quant.bf16_value(s_bits)
    b = quant.bf16_value(b_bits)
    threads = oracle.lib().orc_max_threads()
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.qmm(x, packed, s, b, 64, 4, threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    per = el / reps
    return {"value": qgemv_bytes(m, n, k) / per / 1e9, "unit": "GB/s", "cores": int(threads), "kind": "port",
            "sample": f"{reps} full qGEMV calls x[{m},{k}].W[{n},{k}]^T (FP64 oracle, OpenMP) in {el:.1f} s"}


def bench_qgemv(args):
    import hip_bridge as hb
    from hip_bridge import DeviceBuffer, Event, Stream, quant

    m, n, k = 8, 6144, 2048
    x, packed, s, b = quant.qgemv_workload(m, n, k)
    per_copy = packed.nbytes + s.nbytes + b.nbytes
    rotate = max(48, int(np.ceil(520e6 / per_copy)))
    log(f"qgemv {m}x{n}x{k}: {rotate} weight copies, {rotate * per_copy / 1e6:.0f} MB rotated")
    stream = Stream()
    dx = DeviceBuffer.from_array(x)
    dy = DeviceBuffer(m * n * 2)
    copies = [hb.TiledWeight(packed, s, b, stream) for _ in range(rotate)]
    hb.synchronize(stream.handle)

    def launch(i):
        hb.qmm_tiled(dx, copies[i % rotate], dy, m, stream=stream)

    # parity gate on the benchmarked buffers before timing
    launch(0)
    hb.synchronize(stream.handle)
    import oracle
    y = quant.bf16_value(dy.download(np.uint16, (m, n)))
    ref = oracle.qmm(quant.bf16_value(x), packed, quant.bf16_value(s), quant.bf16_value(b), 64, 4)
    err = float(np.max(np.abs(y - ref)) / np.sqrt(np.mean(ref * ref)))
    if err > 2e-2:
        raise SystemExit(f"parity gate failed: max err / rms = {err}")
    log(f"parity gate ok (max err / rms = {err:.2e})")

    # One HIP graph replays the rotation of launches: host launch overhead
    # (~5 us per Python call) would otherwise exceed the kernel time.
    graph = hb.CapturedGraph(stream)
    for i in range(rotate):
        launch(i)
    graph.end()
    replays = max(1, args.steps // rotate)
    steps = replays * rotate
    for _ in range(max(1, args.warmup // rotate)):
        graph.launch()
    hb.synchronize(stream.handle)
    start, end = Event(), Event()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(replays):
        graph.launch()
    end.record(stream)
    hb.synchronize(stream.handle)
    wall = time.perf_counter() - t0
    ms = start.elapsed_ms(end)
    per_launch_s = ms / 1e3 / steps
    args.steps = steps
    nbytes = qgemv_bytes(m, n, k)
    gbs = nbytes / per_launch_s / 1e9
    log(f"{args.steps} launches: {ms:.3f} ms on-stream ({per_launch_s * 1e6:.2f} us/launch), wall {wall:.3f} s")
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": per_launch_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 x int4 (fp32 accumulate)",
        "data": "synthetic (seeded x ~ N(0,1), W ~ N(0,0.02) quantised 4-bit g64)",
        "config": {"workload": "qgemv x[8,2048] . W[6144,2048]^T, affine 4-bit g64, bf16 out",
                   "rotated_weight_copies": rotate, "rotated_bytes": rotate * per_copy},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": nbytes, "kernel": "qmm4_tiled"},
    }
    if not args.no_cpu:
        log("timing the CPU baseline (oracle restatement)")
        result["cpu_baseline"] = cpu_baseline_qgemv(x, packed, s, b, m, n, k, args.cpu_budget)
    return result


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="qgemv", choices=["qgemv"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (see DESIGN.md, sharding).",
              file=sys.stderr)
        sys.exit(2)
    import hip_bridge

    lib = hip_bridge.load()
    if lib.hb_device_count() < 1:
        raise SystemExit("no HIP device visible")
    log(f"device 0: {lib.hb_device_name(0).decode()}")
    result = bench_qgemv(args)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
