#!/usr/bin/env python3
"""Benchmark of the continuous-batching decode step on one MI355X.

Default workload (decode): the random-init 4-bit 48-layer hybrid decoder
(36 Gated-DeltaNet + 12 gated GQA layers, hidden 2048, vocab 151936, 512
experts top-10 + shared expert, single-layer MTP head) serving greedy
continuous-batching decode at batch 64 with MTP k = 3 (verify width 4).
Each row holds a synthetic prompt context of U[256, 8192] tokens (seeded KV,
recurrent state and conv history standing in for the prefill) and decodes up
to 256 new tokens. One step = one packed target forward of every live row's
block [pending, drafts...], device selection + acceptance, and the MTP
refresh and drafting calls. value = emitted tokens per second.

The roofline object covers the dominant kernel, the grouped 4-bit MoE
gate/up GEMM: algorithmic bytes per launch (the routed experts it touched,
counted on the device, plus the shared expert and the activations) over its
average duration, timed with HIP events on the engine's stream.

--workload qgemv: the affine 4-bit g64 GEMV y[8,6144] = x[8,2048].W^T streamed
over > 512 MB of distinct weight copies (also reported inside the decode line).
Prints one JSON line.
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


GU_PROBE, DOWN_PROBE = 0, 1
# HIP events bracket the grouped GEMMs of every 8th MoE block of the timed
# steps: each event record stalls the stream for a few microseconds, so
# sampling keeps the probes from slowing the steps they measure.
PROBE_STRIDE = 8
GU_KERNEL = "stream_gemm_kernel<16, 16, 4, true, 0, true, false>"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "moe_gate_up_b64_traffic.json")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the two --pmc runs (FETCH_SIZE, then
    WRITE_SIZE, each scaled by its reading for a 256 MiB copy) recorded in
    profiles/; None when no record for this kernel exists."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    return rec.get("bytes_per_launch") if rec.get("kernel") == kernel else None


def moe_bytes(cfg, stats, kind):
    """Algorithmic HBM bytes per grouped-GEMM launch: the weights of the routed
    experts the launch touched plus the shared expert (4-bit codes + bf16
    scale/bias pairs), the activations read and the outputs written."""
    H, I, top = cfg.hidden, cfg.intermediate, cfg.top
    n = stats["launches"]
    experts = stats["active"] / n + 1.0
    tokens = stats["tokens"] / n
    rows_out = tokens * (top + 1)
    if kind == GU_PROBE:
        w = 2 * I * H // 2 + 2 * I * (H // 64) * 4
        act = tokens * H * 2 + rows_out * I * 2
    else:
        w = H * I // 2 + H * (I // 64) * 4
        act = rows_out * I * 2 + rows_out * H * 2
    return experts * w + act


def cpu_baseline_decode(eng, contexts, budget_s):
    """One period of the layer program (3 DeltaNet layers + 1 attention layer)
    plus the lm_head, for all rows at one token each, on the host cores with
    the oracle's restatement; tokens/s = rows / (periods * period time + head)."""
    import oracle
    from oracle.model import DecodeStepCPU, HybridModel

    cfg = eng.config
    rows = len(contexts)
    model = HybridModel(cfg.dims(), eng.export)
    step = DecodeStepCPU(model, range(cfg.interval), contexts, seed=3)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((rows, cfg.hidden)).astype(np.float32)
    for layer in range(cfg.interval):  # materialise the weights outside the timed region
        for slot in range(13):
            try:
                model.w(16 + 16 * layer + slot)
            except Exception:
                pass
    model.w(2)
    model.w(1)
    threads = int(oracle.lib().orc_max_threads())
    t0 = time.perf_counter()
    for layer in range(cfg.interval):
        x = step.layer(layer, x)
    t_period = time.perf_counter() - t0
    t1 = time.perf_counter()
    model.head(x)
    t_head = time.perf_counter() - t1
    per_step = t_period * (cfg.layers // cfg.interval) + t_head
    return {"value": rows / per_step, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"one greedy decode token for {rows} rows: layers 0-{cfg.interval - 1} (3 DeltaNet + 1 attention,"
                       f" contexts as the GPU rows) {t_period:.2f} s x {cfg.layers // cfg.interval} periods + lm_head "
                       f"{t_head:.2f} s; FP64 oracle restatement with OpenMP, not MLX")}


def calibration_copy(nbytes=256 << 20):
    """One device-to-device copy of a known size: the reference dispatch for
    scaling the FETCH_SIZE / WRITE_SIZE counters of a --pmc run."""
    import hip_bridge as hb
    from hip_bridge import DeviceBuffer

    a, b = DeviceBuffer(nbytes), DeviceBuffer(nbytes)
    a.zero()
    hb.synchronize()
    hb.call("hb_memcpy_d2d", b, a, nbytes, None)
    hb.synchronize()
    log(f"calibration copy: {nbytes} bytes device to device")


def bench_decode(args):
    import hip_bridge as hb
    from hip_bridge import Event
    from hip_bridge.engine import DecodeLoop, Engine, hybrid_config

    if args.calibrate:
        calibration_copy()

    rows, width, budget = 64, 4, 256
    cfg = hybrid_config()
    rng = np.random.default_rng(20261201)
    contexts = rng.integers(256, 8193, rows).astype(np.int32)
    max_context = (8192 + budget + width + 15) // 16 * 16
    t0 = time.perf_counter()
    eng = Engine(cfg, rows, max_context, 8, rows * width, seed=20261201, mtp=True)
    log(f"engine: {eng.weight_bytes / 1e9:.2f} GB weights, {eng.state_bytes / 1e9:.2f} GB state pools "
        f"({time.perf_counter() - t0:.1f} s)")
    eng.synthetic_context(contexts, seed=20261202)
    pending = rng.integers(0, cfg.vocab, rows).astype(np.uint32)
    loop = DecodeLoop(eng, width=width, gate_margin=1.25)
    for r in range(rows):
        loop.admit(r, int(contexts[r]), int(pending[r]), budget)
    for i in range(args.warmup):
        loop.step()
    stats0 = loop.stats()
    eng.profile(PROBE_STRIDE)
    stream = hb._p(eng.stream)
    start, end = Event(), Event()
    t0 = time.perf_counter()
    start.record(stream)
    emitted = 0
    for i in range(args.steps):
        emitted += loop.step()
    end.record(stream)
    hb.synchronize(stream)
    wall = time.perf_counter() - t0
    on_stream_ms = start.elapsed_ms(end)
    gu, dn = eng.profile_read(GU_PROBE), eng.profile_read(DOWN_PROBE)
    stats = {k: v - stats0.get(k, 0) for k, v in loop.stats().items()}
    eng.profile(0)
    tps = emitted / wall
    gu_us = gu["ms"] / gu["launches"] * 1e3
    gu_bytes = moe_bytes(cfg, gu, GU_PROBE)
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9
    dn_us = dn["ms"] / dn["launches"] * 1e3
    dn_gbs = moe_bytes(cfg, dn, DOWN_PROBE) / (dn_us * 1e-6) / 1e9
    log(f"{args.steps} steps: {emitted} tokens in {wall:.3f} s ({on_stream_ms:.1f} ms on-stream): {tps:.1f} tokens/s; "
        f"accepted {stats['accepted']}/{stats['proposed']} drafts, {stats['target_tokens']} target tokens, "
        f"{stats['mtp_calls']} MTP calls")
    log(f"grouped gate/up: {gu['launches']} launches, {gu_us:.1f} us avg, {gu['active'] / gu['launches']:.1f} experts, "
        f"{gu_bytes / 1e6:.1f} MB -> {gu_gbs:.0f} GB/s; down: {dn_us:.1f} us avg -> {dn_gbs:.0f} GB/s")
    result = {
        "metric": METRIC,
        "value": round(tps, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 activations x int4 weights (fp32 accumulate, fp32 recurrent state)",
        "data": "synthetic: random-init seeded weights and seeded prompt contexts (KV, state, conv history)",
        "config": {"workload": "greedy continuous-batching decode, 48-layer hybrid (36 DeltaNet + 12 gated GQA), "
                               "512 experts top-10 + shared, 4-bit g64, MTP k=3",
                   "rows": rows, "verify_width": width, "contexts": "U[256, 8192]", "new_tokens": budget,
                   "accepted_drafts": stats["accepted"], "proposed_drafts": stats["proposed"],
                   "target_tokens": stats["target_tokens"], "mtp_calls": stats["mtp_calls"],
                   "weight_bytes": eng.weight_bytes, "state_bytes": eng.state_bytes},
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(GU_KERNEL),
                     "kernel": GU_KERNEL + " (grouped MoE gate/up + SwiGLU)",
                     "algorithmic_bytes_per_launch": round(gu_bytes), "avg_launch_us": round(gu_us, 2),
                     "launches": gu["launches"], "avg_experts_touched": round(gu["active"] / gu["launches"], 1),
                     "down_kernel": {"avg_launch_us": round(dn_us, 2), "achieved": round(dn_gbs, 1)}},
    }
    if not args.no_cpu:
        log("timing the CPU baseline (oracle restatement)")
        result["cpu_baseline"] = cpu_baseline_decode(eng, contexts, args.cpu_budget)
    loop.close()
    eng.close()
    return result


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode", choices=["decode", "qgemv"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--calibrate", action="store_true",
                    help="run a 256 MiB device copy first (reference dispatch for --pmc byte counters)")
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
    if args.workload == "qgemv":
        args.steps = 2000 if args.steps is None else args.steps
        args.warmup = 200 if args.warmup is None else args.warmup
        result = bench_qgemv(args)
    else:
        args.steps = 48 if args.steps is None else args.steps
        args.warmup = 4 if args.warmup is None else args.warmup
        result = bench_decode(args)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
