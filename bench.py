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
average duration, timed with HIP events on the engine's stream. The line also
carries:
- kernels: the same figures for the grouped down GEMM, paged attention with
  its split combine, and the DeltaNet recurrence (bytes from the step's row
  contexts and token count);
- forced_width: the same engine and contexts with the draft gate at 0, so
  every row proposes all 3 drafts and each step verifies 256 target tokens;
- qgemv: the metric's second half, config 1 (y[8,6144] = x[8,2048].W^T,
  4-bit g64) behind its parity gate: single launches and launches replayed
  in one HIP graph over > 512 MB of distinct weight copies, in GB/s and as a
  fraction of HBM peak, beside its read floor: a plain streaming-read kernel
  over the same bytes with the same graph replay and rotation;
- device_rates: the device's streaming read and copy rates over 1 GiB
  (hand-written kernels), the ceilings the HBM-bound kernels are read against;
- prefill: the chunked DeltaNet prefill (32 prompts of U[64, 2048] tokens
  in 64-token chunks) beside the token-serial kernel on the same inputs,
  behind a state parity gate, with algorithmic TFLOP/s and HBM GB/s;
- cpu_baseline: the oracle's FP64 restatement on the host cores.

--workload qgemv: config 1 alone, its graph figure as the value.
--workload prefill: the prefill leg alone.
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


def measure_qgemv(steps, warmup, log_prefix="qgemv", floor=True):
    """Config 1 on the device: parity gate, then the mean time of single
    launches (HIP events around each, every launch on another weight copy so
    it reads from HBM) and of launches replayed back to back in one HIP graph
    over > 512 MB of distinct copies (beyond the 256 MB Infinity Cache)."""
    import hip_bridge as hb
    from hip_bridge import DeviceBuffer, Event, Stream, quant

    m, n, k = 8, 6144, 2048
    x, packed, s, b = quant.qgemv_workload(m, n, k)
    per_copy = packed.nbytes + s.nbytes + b.nbytes
    rotate = max(48, int(np.ceil(520e6 / per_copy)))
    log(f"{log_prefix} {m}x{n}x{k}: {rotate} weight copies, {rotate * per_copy / 1e6:.0f} MB rotated")
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
        raise SystemExit(f"qgemv parity gate failed: max err / rms = {err}")
    log(f"{log_prefix} parity gate ok (max err / rms = {err:.2e})")
    nbytes = qgemv_bytes(m, n, k)

    # single launches, each bracketed by its own events
    singles = max(rotate, 96)
    evs = [(Event(), Event()) for _ in range(singles)]
    for i in range(singles):
        evs[i][0].record(stream)
        launch(i + 1)
        evs[i][1].record(stream)
    hb.synchronize(stream.handle)
    single_us = float(np.mean([a.elapsed_ms(bb) for a, bb in evs])) * 1e3

    # One HIP graph replays the rotation of launches: host launch overhead
    # (~5 us per Python call) would otherwise exceed the kernel time.
    graph = hb.CapturedGraph(stream)
    for i in range(rotate):
        launch(i)
    graph.end()
    replays = max(1, steps // rotate)
    for _ in range(max(1, warmup // rotate)):
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
    launches = replays * rotate
    graph_us = ms * 1e3 / launches
    log(f"{log_prefix}: single launch {single_us:.2f} us ({nbytes / single_us / 1e3:.0f} GB/s); graph of {rotate}: "
        f"{graph_us:.2f} us/launch ({nbytes / graph_us / 1e3:.0f} GB/s), {launches} launches in {wall:.3f} s")
    del graph, copies
    floor = read_floor(nbytes, rotate, replays, stream, log_prefix) if floor else None
    return dict(x=x, packed=packed, s=s, b=b, m=m, n=n, k=k, nbytes=nbytes, rotate=rotate,
                rotated_bytes=rotate * per_copy, launches=launches, err=err, single_us=single_us, graph_us=graph_us,
                floor=floor)


def read_floor(nbytes, rotate, replays, stream, log_prefix="qgemv"):
    """The same bytes read by a plain streaming-read kernel (hb_stream_read), with
    the qGEMV's graph replay and rotation: `rotate` distinct buffers of the
    qGEMV's algorithmic bytes, one launch each, replayed `replays` times. The
    fastest of a few launch shapes is the platform's floor for one launch of
    that size."""
    import hip_bridge as hb
    from hip_bridge import DeviceBuffer, Event, load

    size = (nbytes + 15) // 16 * 16
    bufs = [DeviceBuffer(size) for _ in range(rotate)]
    for b in bufs:
        b.zero(stream)
    shapes = []
    for blocks in (256, 512, 1024, 2048):
        for nt in (0, 1):
            sink = DeviceBuffer(int(load().hb_stream_read_sink_bytes(blocks)))
            graph = hb.CapturedGraph(stream)
            for i in range(rotate):
                hb.call("hb_stream_read", bufs[i], size, sink, blocks, nt, stream)
            graph.end()
            graph.launch()
            hb.synchronize(stream.handle)
            start, end = Event(), Event()
            start.record(stream)
            for _ in range(replays):
                graph.launch()
            end.record(stream)
            hb.synchronize(stream.handle)
            us = start.elapsed_ms(end) * 1e3 / (replays * rotate)
            shapes.append({"blocks": blocks, "nontemporal": bool(nt), "graph_launch_us": round(us, 3),
                           "gbs": round(size / us / 1e3, 1)})
            del graph
    best = min(shapes, key=lambda r: r["graph_launch_us"])
    log(f"{log_prefix} read floor: {size} bytes per launch, fastest {best['graph_launch_us']:.2f} us "
        f"({best['gbs']:.0f} GB/s) at {best['blocks']} blocks, nontemporal={best['nontemporal']}")
    return {"kernel": "stream_read_kernel (hb_stream_read)", "bytes_per_launch": size, "rotated_buffers": rotate,
            "graph_launches_per_shape": replays * rotate, "best": best, "shapes": shapes}


def device_rates(nbytes=1 << 30, reps=10):
    """Streaming read and copy rates of the device over `nbytes` (hand-written
    kernels, hb_stream_read / hb_stream_copy and their chunked forms), the
    ceilings the HBM-bound kernels are read against: a copy moves 2 x nbytes
    (read + write)."""
    import hip_bridge as hb
    from hip_bridge import DeviceBuffer, Event, Stream, load

    stream = Stream()
    a, b = DeviceBuffer(nbytes), DeviceBuffer(nbytes)
    a.zero(stream)
    b.zero(stream)
    out = {"bytes": nbytes}
    # grid-stride over 1024-8192 workgroups, then contiguous chunks of 128 KiB
    # and 1 MiB per workgroup (the chunked forms: one block of state per
    # workgroup); each kind keeps its best
    shapes = [("grid", blocks) for blocks in (1024, 2048, 4096, 8192)] + [("chunk", c) for c in (1 << 17, 1 << 20)]
    for kind in ("read", "copy"):
        best = None
        for form, arg in shapes:
            blocks = arg if form == "grid" else nbytes // arg
            sink = DeviceBuffer(int(load().hb_stream_read_sink_bytes(blocks)))

            def one():
                if form == "grid" and kind == "read":
                    hb.call("hb_stream_read", a, nbytes, sink, blocks, 1, stream)
                elif form == "grid":
                    hb.call("hb_stream_copy", b, a, nbytes, blocks, stream)
                elif kind == "read":
                    hb.call("hb_stream_read_chunked", a, nbytes, arg, sink, 1, stream)
                else:
                    hb.call("hb_stream_copy_chunked", b, a, nbytes, arg, stream)
            one()
            hb.synchronize(stream.handle)
            start, end = Event(), Event()
            start.record(stream)
            for _ in range(reps):
                one()
            end.record(stream)
            hb.synchronize(stream.handle)
            ms = start.elapsed_ms(end) / reps
            moved = nbytes * (1 if kind == "read" else 2)
            gbs = moved / (ms * 1e-3) / 1e9
            if best is None or gbs > best["gbs"]:
                best = {"form": "grid-stride" if form == "grid" else f"chunks of {arg >> 10} KiB",
                        "blocks": blocks, "ms": round(ms, 4), "gbs": round(gbs, 1),
                        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        out[kind] = best
        log(f"device {kind} rate over {nbytes >> 20} MiB: {best['gbs']:.0f} GB/s "
            f"({100 * best['frac_of_hbm_peak']:.1f} % of peak), {best['form']}, {best['blocks']} blocks")
    return out


def qgemv_summary(q):
    gbs = q["nbytes"] / q["graph_us"] / 1e3
    return {"workload": "x[8,2048] . W[6144,2048]^T, affine 4-bit g64, bf16 out", "kernel": "qmm4_tiled",
            "algorithmic_bytes_per_launch": q["nbytes"], "rotated_weight_copies": q["rotate"],
            "rotated_bytes": q["rotated_bytes"], "parity_max_err_over_rms": q["err"],
            "single_launch_us": round(q["single_us"], 3),
            "single_launch_gbs": round(q["nbytes"] / q["single_us"] / 1e3, 1),
            "graph_launch_us": round(q["graph_us"], 3), "graph_launches": q["launches"],
            "achieved": round(gbs, 1), "unit": "GB/s", "peak": HBM_PEAK_GBS, "frac": round(gbs / HBM_PEAK_GBS, 4),
            "read_floor": q["floor"],
            "frac_of_read_floor": round(q["floor"]["best"]["graph_launch_us"] / q["graph_us"], 4) if q["floor"] else None}


def bench_qgemv(args):
    q = measure_qgemv(args.steps, args.warmup, floor=not args.no_probes)
    args.steps = q["launches"]
    gbs = q["nbytes"] / q["graph_us"] / 1e3
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": q["graph_us"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 x int4 (fp32 accumulate)",
        "data": "synthetic (seeded x ~ N(0,1), W ~ N(0,0.02) quantised 4-bit g64)",
        "config": {"workload": "qgemv x[8,2048] . W[6144,2048]^T, affine 4-bit g64, bf16 out",
                   "rotated_weight_copies": q["rotate"], "rotated_bytes": q["rotated_bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": q["nbytes"], "kernel": "qmm4_tiled"},
        "qgemv": qgemv_summary(q) if q else None,
    }
    if not args.no_cpu:
        log("timing the CPU baseline (oracle restatement)")
        result["cpu_baseline"] = cpu_baseline_qgemv(q["x"], q["packed"], q["s"], q["b"], q["m"], q["n"], q["k"],
                                                    args.cpu_budget)
    return result


GU_PROBE, DOWN_PROBE, ATTN_PROBE, GDN_PROBE = 0, 1, 2, 3
# HIP events bracket the grouped GEMMs of every 8th MoE block of the timed
# steps: each event record stalls the stream for a few microseconds, so
# sampling keeps the probes from slowing the steps they measure.
PROBE_STRIDE = 8
GU_KERNEL = "moe_gemm_kernel<16, true>"
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
    the oracle's restatement, repeated until budget_s has passed; tokens/s =
    rows / (periods * mean period time + mean head time)."""
    import oracle
    from oracle.model import DecodeStepCPU, HybridModel

    cfg = eng.config
    rows = len(contexts)
    model = HybridModel(cfg.dims(), eng.export, fp32=True)
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
    t_period = t_head = 0.0
    reps = 0
    start = time.perf_counter()
    while reps == 0 or time.perf_counter() - start < budget_s:
        t0 = time.perf_counter()
        for layer in range(cfg.interval):
            x = step.layer(layer, x)
        t1 = time.perf_counter()
        model.head(x)
        t_period += t1 - t0
        t_head += time.perf_counter() - t1
        reps += 1
    t_period /= reps
    t_head /= reps
    per_step = t_period * (cfg.layers // cfg.interval) + t_head
    return {"value": rows / per_step, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"one greedy decode token for {rows} rows: layers 0-{cfg.interval - 1} (3 DeltaNet + 1 attention,"
                       f" contexts as the GPU rows) {t_period:.2f} s x {cfg.layers // cfg.interval} periods + lm_head "
                       f"{t_head:.2f} s, means of {reps} repetitions in {time.perf_counter() - start:.1f} s; the "
                       f"oracle's restatement with every 4-bit product in FP32 (weights dequantised once per "
                       f"row and group, OpenMP over output rows and experts), norms, attention and the DeltaNet state "
                       f"in FP64; not MLX")}


MFMA_BF16_PEAK_TFLOPS = 2500.0
FP32_MATRIX_PEAK_TFLOPS = 157.3


def prefill_flops(chunk_tokens, d=128):
    """Algorithmic flops of one head's chunks (c tokens each) in the chunked
    form at key = value dim d: K S^T, Q S^T and K^T U (2 c d^2 each), the
    state decay (d^2), the strict-lower K K^T and lower Q K^T (about c^2 d
    together), and the triangular solve for U and P U (about c^2 d)."""
    c = np.asarray(chunk_tokens, np.float64)
    return float(np.sum(6 * c * d * d + 2 * c * c * d + d * d))


def prefill_bytes(row_tokens, hk=16, hv=32, d=128):
    """Algorithmic HBM bytes of one launch: every (row, head) state read once
    and written once (fp32); per token q_hat and k_hat (f32, key heads), v and
    the output o (f32, value heads), decay and beta, and the gated norm's z
    read and y written (bf16)."""
    T = float(np.sum(row_tokens))
    state = 2 * len(row_tokens) * hv * d * d * 4
    per_token = 2 * hk * d * 4 + 2 * hv * d * 4 + 2 * hv * 4 + 2 * hv * d * 2
    return state + T * per_token


def measure_prefill(reps=5):
    """DeltaNet prefill at 32 prompts of U[64, 2048] tokens (16 key heads, 32
    value heads, 128 dims, conv 4): gdn_prep on seeded device inputs, then the
    chunked MFMA kernel and the token-serial kernel, each timed with HIP events
    around single launches that read every row's state from one slot and write
    it to another (no drift between repetitions). A parity gate checks the
    chunked states against the token-serial ones first (1e-3 of the RMS)."""
    import hip_bridge as hb
    from hip_bridge import DeviceBuffer, Event, Stream

    hk, hv, d, conv = 16, 32, 128, 4
    C = 2 * hk * d + hv * d
    rng = np.random.default_rng(20261203)
    rows = 32
    row_tokens = rng.integers(64, 2049, rows)
    T = int(row_tokens.sum())
    maxt = int(row_tokens.max())
    cu = np.concatenate([[0], np.cumsum(row_tokens)]).astype(np.int32)
    stream = Stream()
    st = stream.handle
    dev = dict(conv_w=DeviceBuffer.from_array((rng.standard_normal((C, conv)) * 0.5).astype(np.float32)),
               alog=DeviceBuffer.from_array(rng.uniform(0, 1, hv).astype(np.float32)),
               dt=DeviceBuffer.from_array(np.zeros(hv, np.float32)),
               norm=DeviceBuffer.from_array((1 + 0.1 * rng.standard_normal(d)).astype(np.float32)),
               win=DeviceBuffer(rows * (conv - 1 + maxt) * C * 2), cu=DeviceBuffer.from_array(cu),
               hoff=DeviceBuffer.from_array(np.zeros(rows, np.int32)), qkv=DeviceBuffer(T * C * 2),
               ab=DeviceBuffer(T * 2 * hv * 2), z=DeviceBuffer(T * hv * d * 2),
               q=DeviceBuffer(T * hk * d * 4), k=DeviceBuffer(T * hk * d * 4), v=DeviceBuffer(T * hv * d * 4),
               g=DeviceBuffer(T * hv * 4), b=DeviceBuffer(T * hv * 4), o=DeviceBuffer(T * hv * d * 4),
               y=DeviceBuffer(T * hv * d * 2), state=DeviceBuffer(2 * rows * hv * d * d * 4),
               src=DeviceBuffer.from_array(np.arange(rows, dtype=np.int32)),
               dst=DeviceBuffer.from_array(np.arange(rows, 2 * rows, dtype=np.int32)))
    dev["win"].zero(st)
    hb.call("hb_random_normal", 31, rows * hv * d * d, 0.01, 0.0, 0, dev["state"], st)
    hb.call("hb_random_normal", 32, T * C, 1.0, 0.0, 4, dev["qkv"], st)
    hb.call("hb_random_normal", 33, T * 2 * hv, 1.0, 0.0, 4, dev["ab"], st)
    hb.call("hb_random_normal", 34, T * hv * d, 1.0, 0.0, 4, dev["z"], st)
    hb.call("hb_gdn_prep", dev["qkv"], C, dev["ab"], hb._p(dev["ab"].ptr + 2 * hv), 2 * hv, dev["conv_w"],
            dev["alog"], dev["dt"], dev["win"], dev["hoff"], None, None, dev["cu"], rows, hk, hv, d, d, conv, maxt,
            dev["q"], dev["k"], dev["v"], dev["g"], dev["b"], st)

    def launch(kind):
        if kind == "chunked":
            hb.call("hb_gdn_chunked", dev["q"], dev["k"], dev["v"], dev["g"], dev["b"], dev["cu"], rows, hk, hv, d, d,
                    dev["state"], dev["src"], dev["dst"], dev["o"], dev["z"], hv * d, dev["norm"], dev["y"], st)
        else:
            hb.call("hb_gdn_recurrence", dev["q"], dev["k"], dev["v"], dev["g"], dev["b"], dev["cu"], rows, hk, hv,
                    d, d, dev["state"], dev["src"], dev["dst"], None, None, None, None, 0, 0, dev["o"], dev["z"],
                    hv * d, dev["norm"], dev["y"], st)

    finals = {}
    for kind in ("serial", "chunked"):
        launch(kind)
        hb.synchronize(st)
        finals[kind] = dev["state"].download(np.float32, (rows, hv * d * d), rows * hv * d * d * 4)
    ref = finals["serial"].astype(np.float64)
    err = float(np.max(np.abs(finals["chunked"] - ref)) / np.sqrt(np.mean(ref * ref)))
    if err > 1e-3:
        raise SystemExit(f"prefill parity gate failed: chunked vs token-serial state max err / rms = {err}")
    times = {}
    for kind in ("chunked", "serial"):
        launch(kind)
        evs = [(Event(), Event()) for _ in range(reps)]
        for a, bb in evs:
            a.record(stream)
            launch(kind)
            bb.record(stream)
        hb.synchronize(st)
        times[kind] = float(np.mean([a.elapsed_ms(bb) for a, bb in evs]))
    chunks = []
    for n in row_tokens:
        chunks += [64] * (int(n) // 64) + ([int(n) % 64] if n % 64 else [])
    flops = prefill_flops(chunks) * hv
    nbytes = prefill_bytes(row_tokens)
    ms = times["chunked"]
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"prefill {rows} prompts, {T} tokens ({len(chunks)} chunks per head): chunked {ms:.3f} ms "
        f"({T / ms * 1e3 / 1e6:.2f} M tokens/s, {tflops:.1f} TFLOP/s algorithmic, {gbs:.0f} GB/s), token-serial "
        f"{times['serial']:.3f} ms; parity max err / rms {err:.2e}")
    return {"workload": "Gated DeltaNet prefill: 32 prompts of U[64, 2048] tokens in 64-token chunks, 16 key / 32 "
                        "value heads x 128, fp32 state",
            "kernel": "gdn_chunk_kernel", "tokens": T, "chunks_per_head": len(chunks),
            "chunked_ms": round(ms, 4), "tokens_per_s": round(T / ms * 1e3, 1),
            "token_serial_ms": round(times["serial"], 4),
            "speedup_vs_token_serial": round(times["serial"] / ms, 2),
            "parity_max_err_over_rms": err,
            "algorithmic_flops": flops, "achieved_tflops": round(tflops, 2),
            "frac_of_fp32_matrix_peak": round(tflops / FP32_MATRIX_PEAK_TFLOPS, 4),
            "mfma_issued_tflops": round(3 * tflops, 2),
            "frac_of_bf16_mfma_peak": round(3 * tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "algorithmic_bytes": nbytes, "achieved_gbs": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


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


def kernel_figures(eng, cfg):
    """Per-launch time and algorithmic bytes of the four probed kernels over
    the sampled launches of the timed steps."""
    out = {}
    names = {GU_PROBE: "moe_gate_up", DOWN_PROBE: "moe_down", ATTN_PROBE: "paged_attention",
             GDN_PROBE: "gdn_decode"}
    for kind, name in names.items():
        st = eng.profile_read(kind)
        if not st["launches"]:
            continue
        us = st["ms"] / st["launches"] * 1e3
        nbytes = moe_bytes(cfg, st, kind) if kind in (GU_PROBE, DOWN_PROBE) else st["bytes"] / st["launches"]
        gbs = nbytes / (us * 1e-6) / 1e9
        fig = {"launches": st["launches"], "avg_launch_us": round(us, 2),
               "algorithmic_bytes_per_launch": round(nbytes), "achieved": round(gbs, 1), "unit": "GB/s",
               "frac": round(gbs / HBM_PEAK_GBS, 4), "tokens_per_launch": round(st["tokens"] / st["launches"], 1)}
        if kind == GU_PROBE:
            fig["avg_experts_touched"] = round(st["active"] / st["launches"], 1)
        out[name] = fig
    return out


def run_loop(eng, contexts, pending, width, gate, warmup, steps, budget):
    """Admit every row on a fresh copy of the synthetic context, warm up, then
    time `steps` decode steps (HIP events on the engine's stream and the wall
    clock). Returns (emitted, wall s, on-stream ms, stats delta, kernel figures)."""
    import hip_bridge as hb
    from hip_bridge import Event
    from hip_bridge.engine import DecodeLoop

    eng.synthetic_context(contexts, seed=20261202)
    loop = DecodeLoop(eng, width=width, gate_margin=gate)
    for r in range(len(contexts)):
        loop.admit(r, int(contexts[r]), int(pending[r]), budget)
    for _ in range(warmup):
        loop.step()
    stats0 = loop.stats()
    eng.profile(PROBE_STRIDE)
    stream = hb._p(eng.stream)
    start, end = Event(), Event()
    t0 = time.perf_counter()
    start.record(stream)
    emitted = 0
    for _ in range(steps):
        emitted += loop.step()
    end.record(stream)
    hb.synchronize(stream)
    wall = time.perf_counter() - t0
    figures = kernel_figures(eng, eng.config)
    eng.profile(0)
    stats = {k: v - stats0.get(k, 0) for k, v in loop.stats().items()}
    loop.close()
    return emitted, wall, start.elapsed_ms(end), stats, figures


def bench_decode(args):
    from hip_bridge.engine import Engine, hybrid_config

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
    pending = rng.integers(0, cfg.vocab, rows).astype(np.uint32)

    # headline: the reference's margin gate (1.25) on MTP drafts
    emitted, wall, on_stream_ms, stats, kern = run_loop(eng, contexts, pending, width, 1.25, args.warmup, args.steps,
                                                        budget)
    tps = emitted / wall
    gu = kern["moe_gate_up"]
    log(f"{args.steps} steps: {emitted} tokens in {wall:.3f} s ({on_stream_ms:.1f} ms on-stream): {tps:.1f} tokens/s; "
        f"accepted {stats['accepted']}/{stats['proposed']} drafts, {stats['target_tokens']} target tokens, "
        f"{stats['mtp_calls']} MTP calls")
    for name, f in kern.items():
        log(f"  {name}: {f['launches']} sampled launches, {f['avg_launch_us']} us avg, "
            f"{f['algorithmic_bytes_per_launch'] / 1e6:.1f} MB -> {f['achieved']:.0f} GB/s ({100 * f['frac']:.1f} %)")

    # forced width: every row proposes all 3 drafts, so each step verifies 4 tokens per row
    f_steps = max(4, args.steps // 2)
    f_emitted, f_wall, f_ms, f_stats, f_kern = run_loop(eng, contexts, pending, width, 0.0, 2, f_steps, budget)
    log(f"forced width: {f_steps} steps, {f_stats['target_tokens'] / f_steps:.0f} target tokens per step, "
        f"{f_emitted / f_wall:.1f} tokens/s, {f_wall * 1e3 / f_steps:.2f} ms/step")
    eng.close()

    q = None if args.decode_only else measure_qgemv(2000, 200, floor=not args.no_probes)
    prefill = None if args.decode_only else measure_prefill()
    rates = None if args.no_probes or args.decode_only else device_rates()

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
                               "512 experts top-10 + shared, 4-bit g64, MTP k=3 (verify width 4, draft margin gate "
                               "1.25)",
                   "rows": rows, "verify_width": width, "contexts": "U[256, 8192]", "new_tokens": budget,
                   "accepted_drafts": stats["accepted"], "proposed_drafts": stats["proposed"],
                   "target_tokens": stats["target_tokens"],
                   "target_tokens_per_step": round(stats["target_tokens"] / args.steps, 1),
                   "mtp_calls": stats["mtp_calls"],
                   "weight_bytes": eng.weight_bytes, "state_bytes": eng.state_bytes},
        "roofline": {"bound": "hbm", "achieved": gu["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gu["frac"], "traffic": measured_traffic(GU_KERNEL),
                     "kernel": GU_KERNEL + " (grouped MoE gate/up + SwiGLU)",
                     "algorithmic_bytes_per_launch": gu["algorithmic_bytes_per_launch"],
                     "avg_launch_us": gu["avg_launch_us"], "launches": gu["launches"],
                     "avg_experts_touched": gu["avg_experts_touched"]},
        "kernels": kern,
        "forced_width": {"gate": 0.0, "steps": f_steps, "tokens_per_s": round(f_emitted / f_wall, 2),
                         "ms_per_step": round(f_wall * 1e3 / f_steps, 3),
                         "target_tokens_per_step": round(f_stats["target_tokens"] / f_steps, 1),
                         "accepted_drafts": f_stats["accepted"], "proposed_drafts": f_stats["proposed"],
                         "kernels": f_kern},
        "qgemv": qgemv_summary(q) if q else None,
        "prefill": prefill,
        "device_rates": rates,
    }
    if not args.no_cpu:
        log("timing the CPU baseline (oracle restatement)")
        eng = Engine(cfg, 1, 64, 8, 8, seed=20261201, mtp=False)  # same seeded weights, small state pools
        result["cpu_baseline"] = cpu_baseline_decode(eng, contexts, args.cpu_budget)
        eng.close()
    return result


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode", choices=["decode", "qgemv", "prefill"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-probes", action="store_true",
                    help="skip the memory-rate probes (the qGEMV read floor and the device read/copy rates)")
    ap.add_argument("--calibrate", action="store_true",
                    help="run a 256 MiB device copy first (reference dispatch for --pmc byte counters)")
    ap.add_argument("--decode-only", action="store_true",
                    help="run the two decode legs only (no qGEMV, prefill or probe legs), e.g. under a profiler")
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
    if args.workload == "prefill":
        if args.calibrate:
            calibration_copy()
        args.steps = 5 if args.steps is None else args.steps
        args.warmup = 1 if args.warmup is None else args.warmup
        pf = measure_prefill(args.steps)
        result = {"metric": "DeltaNet prefill tokens/sec (chunked, 1 GPU)", "value": pf["tokens_per_s"],
                  "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                  "ms_per_step": pf["chunked_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                  "dtype": "f32 (3xbf16 MFMA products)", "data": "synthetic: seeded device inputs",
                  "config": {"workload": pf["workload"]}, "prefill": pf}
    elif args.workload == "qgemv":
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
