#!/usr/bin/env python3
"""Decode-path benchmark on one MI355X (gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--m 1] [--mode 2] [--no-detail] [--no-cpu]

Workload (the headline): TQ2_0 (ternary, BitNet b1.58) decode steps at BitNet-2B FFN shapes.  One step runs the chain
x[m][2560] -> W1[6912 x 2560] -> W2[2560 x 6912]: each GEMV quantizes its f32 input to q8_K inside the same launch
(tq2_0_gemv_f32), so a step is two dependent dispatches.  The reference-shaped path (quant_q8_K then tq2_0_gemv, four
dispatches) is timed beside it and must agree bit for bit (both plan alike at these shapes).  Weights are synthetic ternary ({-1, 0, +1} with
p 0.3/0.4/0.3, f16 d ~ U(0.01, 0.05)), the input N(0, 1), all resident in HBM before the timed region.  Each step reads a different copy of both matrices (>= 1 GiB of copies), so no call is
served from the 256 MB Infinity Cache ("cold").  The K timed steps run as HIP-graph replays, so the host launch rate
does not bound them.

Every timing is a stretch of calls captured into one HIP graph, between two device clock marks (komp_clock) after an
untimed lead call, replayed once after the warm-up.

Printed: one JSON line of a few KB.  value = algorithmic bytes of the K steps (per GEMV: weights + f32 activations in +
f32 outputs) / their wall time (GB/s); roofline = the fused tq2_0_gemv launches' algorithmic bytes / their average
in-graph span (first wave's entry to last wave's stored outputs, from the library's wave stamps over a graph of the same
steps; events_us beside it is the events around the timed replays / the launches, gaps between dispatches included,
and dispatch_us each dispatch timed alone with hipExtLaunchKernel events); cpu_baseline = the C oracle (the
reference's arithmetic restated) on a bounded sample of the same steps on this host; configs = every configuration of
the workload list in the modes (dp4a, bytes) and knob sets it names, one compact row each (us/call, GB/s, % of peak,
streaming-read floor / GEMV).

Written to --detail-out (default gpurun_out/bench_detail.json): the same line plus detail = per-shape GEMV us/call and
GB/s for the Q4_0 / TQ2_0 shape list and Llama-3-8B shapes of Q8_0, IQ4_NL and Q4_K (cold, library-chosen knobs; and
hot: one weight copy, resident in the 256 MB MALL where it fits); configs in full; multi_matrix = projections stored apart (BitNet-2B gate/up, Llama-3-8B Q/K/V) in one gemv_multi launch
against one launch per matrix; batched_gemm = 4, 16 and 64 decode tokens at once on Llama-3-8B (Q4_0, and 14336 x
4096 in Q8_0, IQ4_NL and Q4_K) and BitNet-2B (TQ2_0) projections, the matrix-core GEMM against GEMV launches of 3
columns; ingest = ggml block bytes split into the planes on the device; quantizers = quant_q8_0 / quant_q8_K alone.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "GEMV µs/call + achieved HBM GB/s (% of peak), Q4_0 & TQ2_0 decode shapes"
PEAK_GBS = 8000.0  # MI355X HBM3E, published
MODE_NAMES = {0: "bytes", 1: "dp4a-emulated", 2: "dp4a"}
COLD_BYTES = 1 << 30  # weight copies rotated per workload (4x the 256 MB Infinity Cache)
# HBM bytes per launch of the headline's fused tq2_0 kernel (mean of the two shapes, m=1, dp4a, library-chosen knobs),
# from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE, each scaled by its reading for a 256 MiB copy:
# profiles/tq2_0_gemv_bitnet2b_decode_chain.md.  Reported only for that configuration.
TRAFFIC_FUSED_BITNET_M1 = 4829049


# (values per weight block, weight bytes per block, values per activation block) of each weight format
BLOCKS = {"q4_0": (32, 18, 32), "tq2_0": (256, 66, 256), "q8_0": (32, 34, 32), "iq4_nl": (32, 18, 32),
          "q4_k": (256, 144, 256)}


def gemv_bytes(fmt, n, k, m):
    """Algorithmic HBM bytes of one GEMV call: weights (quant + scale planes), q8 activations, f32 outputs."""
    blk, nbytes, ablk = BLOCKS[fmt]
    return n * k * nbytes // blk + m * (k + 4 * k // ablk) + 4 * m * n


def quant_bytes(fmt, k, m):
    """Algorithmic bytes of one quantizer call: f32 read, int8 + f32 scale written (no bsums)."""
    ablk = BLOCKS[fmt][2]
    return 4 * m * k + m * k + 4 * m * (k // ablk)


# ---------------------------------------------------------------------------------------------------------------------
# synthetic weights, generated on the device


def tq2_0_weights(n, k, gen, torch):
    """Split planes of ternary TQ2_0 weights: crumb c = trit + 1 from {0, 1, 2} with p 0.3/0.4/0.3; f16 d ~ U(.01,.05).
    Byte h*32 + i of a block holds value h*128 + j*32 + i at bits 2j."""
    nb = k // 256
    u = torch.rand((n, nb, 2, 4, 32), generator=gen, device="cuda")
    c = (u > 0.3).to(torch.uint8) + (u > 0.7).to(torch.uint8)
    qs = c[:, :, :, 0] | (c[:, :, :, 1] << 2) | (c[:, :, :, 2] << 4) | (c[:, :, :, 3] << 6)
    wq = qs.reshape(n, nb * 64).contiguous()
    d = torch.rand((n, nb), generator=gen, device="cuda") * 0.04 + 0.01
    ws = d.half().view(torch.int16).contiguous()
    return wq, ws


def q4_0_weights(n, k, gen, torch):
    """Split planes of Q4_0 weights: W ~ N(0, 0.02) quantized by ggml's q4_0 rule (d = max / -8 with max the signed
    value of largest |w|, q = min(15, trunc(w / d + 8.5)))."""
    nb = k // 32
    w = torch.randn((n, nb, 32), generator=gen, device="cuda") * 0.02
    idx = w.abs().argmax(dim=2, keepdim=True)
    mx = torch.gather(w, 2, idx)
    d = mx / -8.0
    idv = torch.where(d != 0, 1.0 / torch.where(d != 0, d, torch.ones_like(d)), torch.zeros_like(d))
    q = torch.clamp(torch.trunc(w * idv + 8.5), 0, 15).to(torch.uint8)
    wq = (q[:, :, :16] | (q[:, :, 16:] << 4)).reshape(n, nb * 16).contiguous()
    ws = d[:, :, 0].half().view(torch.int16).contiguous()
    return wq, ws


def q8_0_weights(n, k, gen, torch):
    """Split planes of Q8_0 weights: W ~ N(0, 0.02), d = max |w| / 127 per block, q = round(w / d)."""
    nb = k // 32
    w = torch.randn((n, nb, 32), generator=gen, device="cuda") * 0.02
    d = w.abs().amax(dim=2, keepdim=True) / 127.0
    q = torch.round(w / torch.where(d > 0, d, torch.ones_like(d))).clamp(-127, 127).to(torch.int8)
    return q.view(torch.uint8).reshape(n, nb * 32).contiguous(), d[:, :, 0].half().view(torch.int16).contiguous()


IQ4_NL_VALUES = (-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113)


def iq4_nl_weights(n, k, gen, torch):
    """Split planes of IQ4_NL weights: W ~ N(0, 0.02), d = max |w| / 127 per block, each value the nearest entry of
    the IQ4_NL table to w / d (index i of value i in the low nibble of byte i, value i + 16 in the high nibble)."""
    nb = k // 32
    w = torch.randn((n, nb, 32), generator=gen, device="cuda") * 0.02
    d = w.abs().amax(dim=2, keepdim=True) / 127.0
    t = torch.tensor(IQ4_NL_VALUES, dtype=torch.float32, device="cuda")
    q = torch.bucketize(w / torch.where(d > 0, d, torch.ones_like(d)), (t[1:] + t[:-1]) / 2).to(torch.uint8)
    wq = (q[:, :, :16] | (q[:, :, 16:] << 4)).reshape(n, nb * 16).contiguous()
    return wq, d[:, :, 0].half().view(torch.int16).contiguous()


def q4_k_weights(n, k, gen, torch):
    """Split planes of Q4_K weights: uniform nibbles and 6-bit scale / min bytes, d and dmin ~ U(0.0002, 0.001)
    (the scale plane holds each block's d, dmin and 12 scale bytes: int16 [n][8 * blocks])."""
    nb = k // 256
    wq = torch.randint(0, 256, (n, nb * 128), dtype=torch.uint8, device="cuda", generator=gen)
    meta = torch.randint(0, 256, (n, nb, 16), dtype=torch.uint8, device="cuda", generator=gen)
    dd = (torch.rand((n, nb, 2), generator=gen, device="cuda") * 0.0008 + 0.0002).half()
    meta[:, :, :4] = dd.view(torch.uint8).reshape(n, nb, 4)
    return wq, meta.view(torch.int16).reshape(n, nb * 8).contiguous()


WEIGHTS = {"q4_0": q4_0_weights, "tq2_0": tq2_0_weights, "q8_0": q8_0_weights, "iq4_nl": iq4_nl_weights,
           "q4_k": q4_k_weights}


def weight_copies(fmt, n, k, gen, torch, total=COLD_BYTES):
    make = WEIGHTS[fmt]
    wq, ws = make(n, k, gen, torch)
    per = wq.numel() + 2 * ws.numel()
    copies = max(2, math.ceil(total / per))
    return [(wq.clone(), ws.clone()) for _ in range(copies)]


# ---------------------------------------------------------------------------------------------------------------------


def run_graph(torch, fn, count, replays):
    """Capture fn(0..count-1) in one HIP graph; return (graph, replay function)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(min(count, 2)):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(count):
            fn(i)
    return g


def timed_steps(torch, step, ncopies, steps, warmup):
    """Run `warmup` untimed calls (graph replays), then exactly `steps` calls back to back inside one graph, between
    two device clock marks after an untimed lead call (timed_one_graph); returns (ms of the calls, host wall ms of the
    replay).  The per-call time of a decode loop captured once: no graph start falls inside the interval."""
    from comp_amd import _abi

    # three warm replays: a shape's first stretch measured after a single one ran 3-5% slow (the first plan of a knob
    # sweep read 12.29 us against 11.95 for the same plan measured later)
    ms, wall, _ = timed_one_graph(torch, _abi, step, ncopies, steps, warmup, warm_replays=3)
    return ms, wall


def timed_one_graph(torch, abi, step, ncopies, steps, warmup, warm_replays=1):
    """The headline's timing: `warmup` untimed steps (graph replays), then ONE graph holding a lead step, a clock mark,
    exactly `steps` steps and a second clock mark, replayed once.  The marks are the library's one-lane komp_clock
    kernel writing the device's real-time counter, since the runtime records no events inside a graph; the graph's
    own start latency on the GPU (about 11 us a replay) falls on the lead step, outside the interval, which holds the
    K steps back to back (and the first mark's own end, a fraction of a microsecond).  -> (ms of the K steps, host wall
    ms of the replay, events ms around the whole replay: lead step and start latency included)."""
    marks = torch.zeros(2, dtype=torch.int64, device="cuda")
    khz = abi.clock_khz()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(min(ncopies, 2)):
            step(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(0)
        abi.clock_into(marks[0:1])
        for i in range(steps):
            step(1 + i)
        abi.clock_into(marks[1:2])
    if warmup > 0:
        per_graph = ncopies * max(1, math.ceil(64 / ncopies))
        g_warm = run_graph(torch, step, min(per_graph, warmup), 1)
        for _ in range(max(warm_replays, math.ceil(warmup / per_graph))):
            g_warm.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    t = marks.cpu().tolist()
    ms = (t[1] - t[0]) / khz
    if not ms > 0.0:
        raise RuntimeError(f"clock marks {t} at {khz} kHz give no interval")
    return ms, wall, e0.elapsed_time(e1)


def read_floor_us(torch, host, nbytes):
    """Graph-replay us per call of the library's streaming-read probe (komp_stream_read: the bytes read once with
    streaming 16-byte buffer loads, nothing computed) over cold copies of nbytes, the same harness as the GEMVs: the
    time of moving that many bytes alone, which a GEMV over them can at best reach."""
    nb = -(-nbytes // 16) * 16
    ncopy = max(2, math.ceil((COLD_BYTES // 2) / nb))
    bufs = [torch.zeros(nb, dtype=torch.uint8, device="cuda") for _ in range(ncopy)]
    out = torch.empty(host.stream_read_words(nb), dtype=torch.int32, device="cuda")

    def call(i):
        host.stream_read_into(bufs[i % ncopy], nb, out)

    per_graph = ncopy * math.ceil(64 / ncopy)
    reps = 4 * per_graph
    ms, _ = timed_steps(torch, call, ncopy, reps, per_graph)
    del bufs
    torch.cuda.empty_cache()
    return ms * 1e3 / reps


def dispatch_times(abi, torch, step, count):
    """Run `count` eager steps with per-dispatch timing; -> {kind: (total_ms, dispatches)}."""
    torch.cuda.synchronize()
    abi.timing_begin(count * 8 + 16)
    for i in range(count):
        step(i)
    torch.cuda.synchronize()
    return abi.timing_end()


PHASES = ("entry", "staged", "dots", "stored")


def stamped_spans(torch, abi, step, ncopies, replays=4):
    """In-graph kernel spans from the library's wave stamps (komp_stamps_begin / komp_stamps_end): one graph of
    ncopies steps is captured with stamping on (the TQ2_0 dp4a one-pass launches then run their stamped
    instantiation, which reads the real-time counter in every wave on entry, once the staged activations are
    published, after its last weight chunk's dot and once its outputs are stored), replayed `replays` times after one
    warm replay, and the last replay's records read back.  -> (per-shape summary, us per step of the stamped replays)
    with, per (N, K): launches, span_us (mean of last stored - first entry), and each phase's median and 95th
    percentile over the waves (ns from the launch's first entry), averaged over the launches."""
    import numpy as np

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(min(ncopies, 2)):
            step(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    buf = torch.zeros(8 << 20, dtype=torch.int32, device="cuda")  # 32 MiB of records
    g = torch.cuda.CUDAGraph()
    abi.stamps_begin(buf)
    try:
        with torch.cuda.graph(g):
            for i in range(ncopies):
                step(i)
    finally:
        used, khz = abi.stamps_end()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us_step = e0.elapsed_time(e1) * 1e3 / (replays * ncopies)
    recs = abi.parse_stamps(buf[:used].cpu().numpy().view(np.uint32), khz)
    del g, buf
    shapes = {}
    for r in recs:
        shapes.setdefault((r["n"], r["k"]), []).append(r)
    out = {}
    for (n, k), rs in shapes.items():
        row = {"launches": len(rs), "waves": rs[0]["waves"],
               "span_us": round(float(np.mean([r["span_ns"] for r in rs])) / 1e3, 3)}  # fmt: skip
        for ph in PHASES:
            row[ph + "_ns_median_p95"] = [round(float(np.mean([np.median(r[ph]) for r in rs]))),
                                          round(float(np.mean([np.percentile(r[ph], 95) for r in rs])))]  # fmt: skip
        out[f"{n}x{k}"] = row
    return out, us_step


def step_bytes_fused(fmt, n, k, m):
    """Algorithmic bytes of one quantize-and-GEMV: weights, f32 activations in, f32 outputs."""
    blk, nbytes, _ = BLOCKS[fmt]
    return n * k * nbytes // blk + 4 * m * k + 4 * m * n


def headline(torch, host, abi, args):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)
    m = args.m
    shapes = ((6912, 2560), (2560, 6912))  # W1 then W2; W2 reads W1's output
    copies = [weight_copies("tq2_0", n, k, gen, torch, COLD_BYTES // len(shapes)) for n, k in shapes]
    ncopies = min(len(c) for c in copies)
    x = torch.randn((m, shapes[0][1]), generator=gen, device="cuda")
    y1 = torch.empty((m, shapes[0][0]), dtype=torch.float32, device="cuda")
    y2 = torch.empty((m, shapes[1][0]), dtype=torch.float32, device="cuda")
    # block_n None = the library's own plan for each launch (reported in the config)
    knobs = [(None, 0, 0) if args.block_n is None else (args.block_n, args.nb, args.num_warps) for _ in shapes]
    plan_keys = ("block_n", "nb", "waves", "lanes_per_row", "passes")
    plans = [[host.auto_plan("tq2_0", m, n, k, fused=True, mode=args.mode)[key] for key in plan_keys]
             if args.block_n is None else list(knobs[j]) for j, (n, k) in enumerate(shapes)]  # fmt: skip
    same_plans = args.block_n is not None or all(
        host.auto_plan("tq2_0", m, n, k, True, args.mode) == host.auto_plan("tq2_0", m, n, k, False, args.mode)
        for n, k in shapes)
    (n1, k1), (n2, k2) = shapes

    def step(i):  # fused: 2 dispatches
        w1, s1 = copies[0][i % ncopies]
        w2, s2 = copies[1][i % ncopies]
        host.gemv_f32_into("tq2_0", w1, s1, x, y1, n1, k1, *knobs[0][:2], args.mode, knobs[0][2])
        host.gemv_f32_into("tq2_0", w2, s2, y1, y2, n2, k2, *knobs[1][:2], args.mode, knobs[1][2])

    q1 = (torch.empty((m, k1), dtype=torch.int8, device="cuda"), torch.empty((m, k1 // 256), device="cuda"))
    q2 = (torch.empty((m, k2), dtype=torch.int8, device="cuda"), torch.empty((m, k2 // 256), device="cuda"))
    u1, u2 = torch.empty_like(y1), torch.empty_like(y2)

    def step_two_launch(i):  # the reference's shape: quantizer then GEMV, 4 dispatches
        w1, s1 = copies[0][i % ncopies]
        w2, s2 = copies[1][i % ncopies]
        host.quantize_into("tq2_0", x, *q1)
        host.gemv_into("tq2_0", w1, s1, *q1, u1, n1, k1, *knobs[0][:2], args.mode, knobs[0][2])
        host.quantize_into("tq2_0", u1, *q2)
        host.gemv_into("tq2_0", w2, s2, *q2, u2, n2, k2, *knobs[1][:2], args.mode, knobs[1][2])

    ms, wall_ms, replay_ms = timed_one_graph(torch, abi, step, ncopies, args.steps, args.warmup)
    last = args.steps % ncopies  # the timed graph's last step
    # the graph must reproduce the eager result of the same (last) step bit for bit, and the fused and two-launch
    # paths must agree bit for bit
    got = (y1.clone(), y2.clone())
    step(last)
    step_two_launch(last)
    torch.cuda.synchronize()
    if not (torch.equal(y1, got[0]) and torch.equal(y2, got[1])):
        raise RuntimeError("graph replay and eager outputs differ")
    if same_plans and not (torch.equal(y1, u1) and torch.equal(y2, u2)):
        raise RuntimeError("fused and two-launch outputs differ")
    rel = max(float((a - b).abs().max() / b.abs().max()) for a, b in ((y1, u1), (y2, u2)))
    if rel > 1e-6:
        raise RuntimeError(f"fused and two-launch outputs differ by {rel:.2e} (relative)")
    ms2, _, _ = timed_one_graph(torch, abi, step_two_launch, ncopies, args.steps, args.warmup)

    step_bytes = sum(step_bytes_fused("tq2_0", n, k, m) for n, k in shapes)
    ms_per_step = ms / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    disp = dispatch_times(abi, torch, step, min(args.steps, 4 * ncopies))
    g_ms, g_n = disp["tq2_0_gemv"]
    launch_b = step_bytes / len(shapes)
    g_us = g_ms * 1e3 / g_n
    # The kernel's average duration: its in-graph span (first wave's entry to last wave's stored outputs, from the
    # wave stamps of a graph of the same steps), averaged over both shapes' launches.  Beside it: the events around
    # the timed replays / the launches in them (gaps between dispatches included), and each dispatch timed alone
    # with hipExtLaunchKernel events (an eager launch leaves the GPU idle in between).
    spans, us_step_stamped = stamped_spans(torch, abi, step, ncopies)
    events_us = ms_per_step * 1e3 / len(shapes)
    if len(spans) == len(shapes):
        launch_us, timing = sum(v["span_us"] for v in spans.values()) / len(spans), "wave stamps (in-graph span)"
    else:  # no stamped instantiation for this mode / plan: the events' share of the step
        launch_us, timing = events_us, "events over the timed replays / launches"
    achieved = launch_b / (launch_us * 1e-6) / 1e9
    default_cfg = m == 1 and args.mode == 2 and args.block_n is None
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBS, 4), "traffic": TRAFFIC_FUSED_BITNET_M1 if default_cfg else None,
                "traffic_source": "profiles/tq2_0_gemv_bitnet2b_decode_chain.md (rocprofv3 --pmc FETCH_SIZE + "
                                  "WRITE_SIZE, scaled by a copy kernel's readings; not measured in this run)",
                "kernel": "tq2_0_gemv (fused quantize)", "launch_us": round(launch_us, 3), "launch_timing": timing,
                "stamps": spans,
                "events_us": round(events_us, 3), "stamped_us_per_step": round(us_step_stamped, 3),
                "dispatch_us": round(g_us, 3), "bytes_per_launch": int(launch_b),
                "read_floor_us": round(read_floor_us(torch, host, int(launch_b)), 3)}  # fmt: skip
    config = {"workload": "tq2_0 decode chain at BitNet-2B FFN shapes: x[m][2560] -> W1[6912x2560] -> W2[2560x6912], "
                          "activations quantized to q8_K inside each launch",  # fmt: skip
              "shapes_nk": [list(s) for s in shapes], "m": m, "mode": MODE_NAMES[args.mode],
              "plan_rows_nb_waves_lanes_passes": plans, "cold_copies": ncopies, "seed": args.seed,
              "step_bytes": step_bytes,
              "step_timing": "device clock marks (komp_clock) around the K steps inside one graph, after a lead step",
              "replay_events_ms": round(replay_ms, 4), "wall_ms_host": round(wall_ms, 3),
              "us_per_step_graph": round(ms_per_step * 1e3, 3),
              "gemv_us_per_call_dispatch": round(g_us, 3),
              "two_launch_us_per_step_graph": round(ms2 / args.steps * 1e3, 3)}  # fmt: skip
    return value, ms_per_step, roofline, config, step_bytes


def cpu_baseline(args, step_bytes_m, seconds=10.0):
    """The C restatement of the reference path (oracle/oracle.c: ggml's q8_K quantizer, int32 block dots, f32 scale
    and accumulate in block order) on whole steps of the same chain, each GEMV's rows split evenly over
    args.cpu_threads host threads (the C calls run outside the GIL); the chain's order is kept, as in a decode."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    from oracle import coracle as C
    from oracle import oracle as O

    threads = max(1, args.cpu_threads or min(16, len(os.sched_getaffinity(0))))
    rng = np.random.default_rng(args.seed)
    m = args.m
    mats = []
    for n, k in ((6912, 2560), (2560, 6912)):
        nb = k // 256
        crumbs = rng.choice(3, size=(n, k), p=[0.3, 0.4, 0.3]).astype(np.uint8)
        d = rng.uniform(0.01, 0.05, size=(n, nb)).astype(np.float32).astype(np.float16).view(np.uint16)
        wq, ws = O.split("tq2_0", O.pack_tq2_0(crumbs, d), n, k)
        mats.append((n, k, wq, ws))
    x0 = rng.normal(size=(m, 2560)).astype(np.float32)
    C.lib()
    pool = ThreadPoolExecutor(threads)

    def gemv(n, k, wq, ws, xq, xd):
        cuts = [n * t // threads for t in range(threads + 1)]
        parts = pool.map(lambda t: C.gemv_f32("tq2_0", wq[cuts[t]:cuts[t + 1]], ws[cuts[t]:cuts[t + 1]], xq, xd,
                                              cuts[t + 1] - cuts[t], k), range(threads))  # fmt: skip
        return np.concatenate(list(parts), axis=1)

    # the row-split chain equals the one-thread chain bit for bit (rows are independent)
    x1 = x2 = x0
    for n, k, wq, ws in mats:
        q1, d1, _ = C.quant_q8_K(x1)
        q2, d2, _ = C.quant_q8_K(x2)
        x1, x2 = C.gemv_f32("tq2_0", wq, ws, q1, d1, n, k), gemv(n, k, wq, ws, q2, d2)
    assert np.array_equal(x1, x2), "row-split CPU chain differs from the one-thread chain"
    steps = 0
    t0 = time.perf_counter()
    while True:
        x = x0
        for n, k, wq, ws in mats:
            xq, xd, _ = C.quant_q8_K(x)
            x = gemv(n, k, wq, ws, xq, xd)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    pool.shutdown()
    value = step_bytes_m * steps / el / 1e9
    return {"value": round(value, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{steps} whole steps of the same chain (m={m}, both matrices) through the C oracle "
                      f"(oracle/oracle.c: quant_q8_K, int32 block dots, f32 block-order accumulation), gcc -O2, "
                      f"each GEMV's rows split over {threads} threads, {el:.1f} s; host has "
                      f"{len(os.sched_getaffinity(0))} cores"}  # fmt: skip


DETAIL_SHAPES = (  # (fmt, n, k, m)
    ("q4_0", 4096, 4096, 1), ("q4_0", 6144, 4096, 1), ("q4_0", 14336, 4096, 1), ("q4_0", 28672, 4096, 1),
    ("q4_0", 4096, 14336, 1),
    ("q4_0", 4096, 14336, 3), ("q4_0", 128256, 4096, 1), ("q4_0", 28672, 8192, 1), ("tq2_0", 6912, 2560, 1),
    ("tq2_0", 2560, 6912, 1), ("tq2_0", 6912, 2560, 3), ("tq2_0", 32768, 8192, 1), ("q4_0", 4097, 4192, 1),
    ("tq2_0", 6913, 2816, 1), ("q8_0", 4096, 4096, 1), ("q8_0", 14336, 4096, 1), ("q8_0", 4096, 14336, 1),
    ("q8_0", 128256, 4096, 1), ("iq4_nl", 4096, 4096, 1), ("iq4_nl", 14336, 4096, 1), ("iq4_nl", 4096, 14336, 1),
    ("iq4_nl", 28672, 8192, 1), ("q4_k", 4096, 4096, 1), ("q4_k", 14336, 4096, 1), ("q4_k", 4096, 14336, 1),
    ("q4_k", 128256, 4096, 1), ("q4_k", 14336, 4096, 3),
)  # fmt: skip


def detail(torch, host, abi, args):
    """Per-shape GEMV us/call (graph replay) and dispatch duration, cold, library-chosen knobs, dp4a."""
    rows = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 1)
    for fmt, n, k, m in DETAIL_SHAPES:
        copies = weight_copies(fmt, n, k, gen, torch, COLD_BYTES // 2)
        x = torch.randn((m, k), generator=gen, device="cuda")
        xq, xd = host.quantize(fmt, x)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        nc = len(copies)

        def call(i, copies=copies, xq=xq, xd=xd, y=y, fmt=fmt, n=n, k=k):  # the GEMV alone, q8 activations in
            wq, ws = copies[i % nc]
            host.gemv_into(fmt, wq, ws, xq, xd, y, n, k, None, 0, 2, 0)

        per_graph = nc * math.ceil(64 / nc)
        reps = 4 * per_graph
        ms, _ = timed_steps(torch, call, nc, reps, per_graph)
        disp = dispatch_times(abi, torch, call, min(reps, 256))
        kind = f"{fmt}_gemv"
        d_us = disp[kind][0] * 1e3 / disp[kind][1]
        b = gemv_bytes(fmt, n, k, m)
        us = ms * 1e3 / reps

        def call_hot(i, w=copies[0], xq=xq, xd=xd, y=y, fmt=fmt, n=n, k=k):  # one copy: resident in the 256 MB MALL
            host.gemv_into(fmt, w[0], w[1], xq, xd, y, n, k, None, 0, 2, 0)

        ms_hot, _ = timed_steps(torch, call_hot, 1, reps, per_graph)
        us_hot = ms_hot * 1e3 / reps
        del copies, call, call_hot
        torch.cuda.empty_cache()
        floor = read_floor_us(torch, host, b)
        if host.uses_gemm(fmt, m, n, k):  # block_n=None routes this many columns to the matrix-core GEMM
            path, gp = "gemm", host.gemm_plan(fmt, m, n, k)
            plan = [gp[key] for key in ("rows", "cols", "waves")]
        elif host.uses_mfma(fmt, m, n, k):  # ... or (three TQ2_0 columns) the matrix-core GEMV: [rows, waves]
            path, plan = "mfma_gemv", list(host.mfma_plan(fmt, m, n, k))
        else:
            path, ap = "gemv", host.auto_plan(fmt, m, n, k)
            plan = [ap[key] for key in ("block_n", "nb", "waves", "lanes_per_row", "passes")]
        rows.append({"fmt": fmt, "n": n, "k": k, "m": m, "path": path, "plan": plan,
                     "bytes": b, "us_per_call": round(us, 3), "gbs": round(b / us / 1e3, 1),
                     "pct_peak": round(b / us / 1e3 / PEAK_GBS * 100, 1), "dispatch_us": round(d_us, 3),
                     "gbs_dispatch": round(b / d_us / 1e3, 1), "read_floor_us": round(floor, 3),
                     "of_read_floor": round(floor / us, 3), "copies": nc, "us_per_call_hot": round(us_hot, 3),
                     "gbs_hot": round(b / us_hot / 1e3, 1)})  # fmt: skip
    return rows


QUANT_SHAPES = (("q4_0", 4096), ("q4_0", 14336), ("tq2_0", 2560), ("tq2_0", 6912))  # (weight format, K)


def quant_detail(torch, host, args):
    """The activation quantizers alone (quant_q8_0 for Q4_0's activations, quant_q8_K for TQ2_0's, without bsums),
    graph replays over 8 rotated inputs, 1 and 3 columns: us per call and GB/s of the f32 read plus the q8 planes
    written (quant_bytes)."""
    rows = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 5)
    for fmt, k in QUANT_SHAPES:
        ablk = BLOCKS[fmt][2]
        for m in (1, 3):
            xs = [torch.randn((m, k), generator=gen, device="cuda") for _ in range(8)]
            xq = torch.empty((m, k), dtype=torch.int8, device="cuda")
            xd = torch.empty((m, k // ablk), dtype=torch.float32, device="cuda")

            def call(i, xs=xs, xq=xq, xd=xd, fmt=fmt):
                host.quantize_into(fmt, xs[i % 8], xq, xd)

            reps = 256
            ms, _ = timed_steps(torch, call, 8, reps, 64)
            us = ms * 1e3 / reps
            b = quant_bytes(fmt, k, m)
            rows.append({"quantizer": "quant_q8_0" if ablk == 32 else "quant_q8_K", "k": k, "m": m, "bytes": b,
                         "us_per_call": round(us, 3), "gbs": round(b / us / 1e3, 1)})  # fmt: skip
    return rows


# The workload list's configurations with the modes and knobs each names: (config, fmt, N, K, column counts, modes,
# knob sets (block_n, nb, num_warps), None = the library's plan, activation outlier fraction).  Knob sets apply at the
# first column count only (config 3's tune space is the spec's, at one column).
CONFIG_ROWS = (
    (1, "q4_0", 4096, 4096, (1,), (2, 0), (None, (64, 4, 4)), 0.0),
    (2, "tq2_0", 6912, 2560, (1, 2, 3), (2, 0), (None, (64, 1, 4)), 0.0),
    (2, "tq2_0", 2560, 6912, (1, 2, 3), (2, 0), (None, (64, 1, 4)), 0.0),
    (3, "q4_0", 6144, 4096, (1, 2, 3), (2, 0), (None,), 0.01),
    (3, "q4_0", 4096, 4096, (1, 2, 3), (2, 0), (None, (32, 4, 4), (32, 8, 4), (64, 4, 4), (64, 8, 4)), 0.01),
    (3, "q4_0", 28672, 4096, (1, 2, 3), (2, 0), (None,), 0.01),
    (3, "q4_0", 4096, 14336, (1, 2, 3), (2, 0), (None,), 0.01),
    (4, "q4_0", 128256, 4096, (1,), (2,), (None,), 0.0),
    (4, "q4_0", 28672, 8192, (1,), (2,), (None,), 0.0),
    (4, "tq2_0", 32768, 8192, (1,), (2,), (None,), 0.0),
    (5, "q4_0", 4097, 4192, (1, 3), (2, 0), (None,), 0.0),
    (5, "q4_0", 6913, 4192, (1, 3), (2, 0), (None,), 0.0),
    (5, "q4_0", 127, 4192, (1, 3), (2, 0), (None,), 0.0),
    (5, "tq2_0", 4097, 2816, (1, 3), (2, 0), (None,), 0.0),
    (5, "tq2_0", 6913, 2816, (1, 3), (2, 0), (None,), 0.0),
    (5, "tq2_0", 127, 2816, (1, 3), (2, 0), (None,), 0.0),
)  # fmt: skip


def config_detail(torch, host, args):
    """Every configuration of the workload list in each mode and knob set it names: quantizer output (q8 planes) in,
    the GEMV alone as graph replays over cold weight copies; us/call, GB/s, % of peak and the streaming-read floor of
    the shape's bytes.  Mode 0 is the bytes mode (bytes unpacked to int first), 2 dp4a (v_dot4c_i32_i8)."""
    rows = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 5)
    for cfg, fmt, n, k, ms, modes, knob_sets, outliers in CONFIG_ROWS:
        copies = weight_copies(fmt, n, k, gen, torch, COLD_BYTES // 2)
        nc = len(copies)
        floor = read_floor_us(torch, host, gemv_bytes(fmt, n, k, 1))
        for m in ms:
            x = torch.randn((m, k), generator=gen, device="cuda")
            if outliers:
                x = torch.where(torch.rand((m, k), generator=gen, device="cuda") < outliers, x * 20.0, x)
            xq, xd = host.quantize(fmt, x)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            for mode in modes:
                for knobs in knob_sets if m == ms[0] else (None,):
                    bn, nb, nw = knobs if knobs else (None, 0, 0)

                    def call(i, copies=copies, xq=xq, xd=xd, y=y, fmt=fmt, n=n, k=k, kn=(bn, nb, nw), mode=mode):
                        wq, ws = copies[i % nc]
                        host.gemv_into(fmt, wq, ws, xq, xd, y, n, k, kn[0], kn[1], mode, kn[2])

                    per_graph = nc * math.ceil(64 / nc)
                    reps = 2 * per_graph
                    ms_t, _ = timed_steps(torch, call, nc, reps, per_graph)
                    b = gemv_bytes(fmt, n, k, m)
                    us = ms_t * 1e3 / reps
                    gemm = knobs is None and host.uses_gemm(fmt, m, n, k, mode=mode)
                    mfma = knobs is None and host.uses_mfma(fmt, m, n, k, mode=mode)
                    rows.append({"config": cfg, "fmt": fmt, "n": n, "k": k, "m": m,
                                 "mode": MODE_NAMES[mode],
                                 "knobs": list(knobs) if knobs else "library plan",
                                 "path": "gemm" if gemm else ("mfma_gemv" if mfma else "gemv"), "outliers": outliers,
                                 "bytes": b,
                                 "us_per_call": round(us, 3), "gbs": round(b / us / 1e3, 1),
                                 "pct_peak": round(b / us / 1e3 / PEAK_GBS * 100, 1), "read_floor_us": round(floor, 3),
                                 "of_read_floor": round(floor / us, 3), "copies": nc})  # fmt: skip
        del copies
        torch.cuda.empty_cache()
    return rows


def config_summary(rows):
    """The configs rows in compact form for the result line: {"<config> <fmt> <N>x<K>": {"m<M> <mode> <knobs>":
    [us/call, GB/s, % of 8 TB/s, read floor / GEMV]}}, knobs "lib" for the library's plan, else block_n/nb/waves."""
    out = {}
    for r in rows:
        key = f"{r['config']} {r['fmt']} {r['n']}x{r['k']}"
        knobs = "lib" if r["knobs"] == "library plan" else "/".join(str(v) for v in r["knobs"])
        out.setdefault(key, {})[f"m{r['m']} {r['mode']} {knobs}"] = [
            round(r["us_per_call"], 2), round(r["gbs"]), round(r["pct_peak"], 1), round(r["of_read_floor"], 2)]
    return out


MULTI_CASES = (  # (name, fmt, [rows per matrix], K): projections stored as separate tensors that share one input
    ("bitnet2b_ffn_gate_up", "tq2_0", (6912, 6912), 2560),
    ("llama3_8b_q_k_v", "q4_0", (4096, 1024, 1024), 4096),
)


def multi_detail(torch, host, args):
    """Several matrices sharing one f32 input (quantized inside each launch): one gemv_multi launch vs one gemv_f32
    launch per matrix, both as graph replays over cold weight copies, m=1, dp4a, library plans."""
    rows = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 2)
    for name, fmt, ns, k in MULTI_CASES:
        make = WEIGHTS[fmt]
        per = sum(gemv_bytes(fmt, n, k, 0) for n in ns)
        ncopy = max(2, math.ceil((COLD_BYTES // 2) / per))
        base = [make(n, k, gen, torch) for n in ns]
        copies = [[(wq.clone(), ws.clone(), n) for (wq, ws), n in zip(base, ns)] for _ in range(ncopy)]
        x = torch.randn((1, k), generator=gen, device="cuda")
        ys = [torch.empty((1, n), dtype=torch.float32, device="cuda") for n in ns]
        ys1 = [torch.empty_like(y) for y in ys]

        def multi(i, copies=copies, x=x, ys=ys, fmt=fmt, k=k):
            host.gemv_multi_into(fmt, copies[i % len(copies)], ys, k, x=x)

        def singles(i, copies=copies, x=x, ys1=ys1, fmt=fmt, k=k):
            for (wq, ws, n), y in zip(copies[i % len(copies)], ys1):
                host.gemv_f32_into(fmt, wq, ws, x, y, n, k)

        per_graph = ncopy * math.ceil(64 / ncopy)
        reps = 4 * per_graph
        ms_m, _ = timed_steps(torch, multi, ncopy, reps, per_graph)
        ms_s, _ = timed_steps(torch, singles, ncopy, reps, per_graph)
        multi(0)
        singles(0)
        torch.cuda.synchronize()
        rel = max(float((a - b).abs().max() / b.abs().max()) for a, b in zip(ys, ys1))
        if rel > 1e-6:
            raise RuntimeError(f"{name}: multi-matrix and single launches differ by {rel:.2e} (relative)")
        b = sum(n * k * BLOCKS[fmt][1] // BLOCKS[fmt][0] for n in ns) + 4 * k + 4 * sum(ns)
        us_m, us_s = ms_m * 1e3 / reps, ms_s * 1e3 / reps
        rows.append({"case": name, "fmt": fmt, "rows": list(ns), "k": k, "bytes": b, "us_multi": round(us_m, 3),
                     "us_singles": round(us_s, 3), "launches_singles": len(ns), "speedup": round(us_s / us_m, 3),
                     "gbs_multi": round(b / us_m / 1e3, 1), "copies": ncopy})  # fmt: skip
        del copies, base
        torch.cuda.empty_cache()
    return rows


BATCH_CASES = (  # (name, fmt, N, K): decode projections, several tokens at once
    ("llama3_8b_attn_o", "q4_0", 4096, 4096),
    ("llama3_8b_ffn_gate", "q4_0", 14336, 4096),
    ("llama3_8b_ffn_down", "q4_0", 4096, 14336),
    ("bitnet2b_ffn_gate", "tq2_0", 6912, 2560),
    ("bitnet2b_ffn_down", "tq2_0", 2560, 6912),
    ("llama3_8b_ffn_gate", "q8_0", 14336, 4096),
    ("llama3_8b_ffn_gate", "iq4_nl", 14336, 4096),
    ("llama3_8b_ffn_gate", "q4_k", 14336, 4096),
)
BATCH_M = (4, 16, 64)


def batched_detail(torch, host, args):
    """Several activation columns (batched decode tokens) per weight matrix, q8 activations in: the matrix-core GEMM
    (what gemv with block_n=None runs from 4 columns) vs the GEMV in launches of 3 columns (its own knobs for that
    column count), both as graph replays over cold weight copies.  Bytes: weights + q8 activations + f32 outputs."""
    rows = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 3)
    for name, fmt, n, k in BATCH_CASES:
        copies = weight_copies(fmt, n, k, gen, torch, COLD_BYTES // 2)
        nc = len(copies)
        for m in BATCH_M:
            x = torch.randn((m, k), generator=gen, device="cuda")
            xq, xd = host.quantize(fmt, x)
            y_g = torch.empty((m, n), dtype=torch.float32, device="cuda")
            y_c = torch.empty_like(y_g)
            bn, nb, nw = host.auto_config(fmt, m, n, k)

            def gemm(i, copies=copies, xq=xq, xd=xd, y=y_g, fmt=fmt, n=n, k=k):
                wq, ws = copies[i % nc]
                host.gemm_into(fmt, wq, ws, xq, xd, y, n, k)

            def chunks(i, copies=copies, xq=xq, xd=xd, y=y_c, fmt=fmt, n=n, k=k, knobs=(bn, nb, nw)):
                wq, ws = copies[i % nc]
                host.gemv_into(fmt, wq, ws, xq, xd, y, n, k, knobs[0], knobs[1], 2, knobs[2])

            per_graph = nc * math.ceil(64 / nc)
            reps = 2 * per_graph
            ms_g, _ = timed_steps(torch, gemm, nc, reps, per_graph)
            ms_c, _ = timed_steps(torch, chunks, nc, reps, per_graph)
            gemm(0)
            chunks(0)
            torch.cuda.synchronize()
            rel = float((y_g - y_c).abs().max() / y_c.abs().max())
            if rel > 1e-5:
                raise RuntimeError(f"{name} m={m}: GEMM and GEMV outputs differ by {rel:.2e} (relative)")
            b = gemv_bytes(fmt, n, k, m)
            us_g, us_c = ms_g * 1e3 / reps, ms_c * 1e3 / reps
            plan = host.gemm_plan(fmt, m, n, k)
            rows.append({"case": name, "fmt": fmt, "n": n, "k": k, "m": m, "bytes": b,
                         "gemm_plan_rows_cols_waves": [plan["rows"], plan["cols"], plan["waves"]],
                         "us_gemm": round(us_g, 3), "us_gemv_chunks": round(us_c, 3),
                         "launches_chunks": math.ceil(m / 3), "speedup": round(us_c / us_g, 3),
                         "gbs_gemm": round(b / us_g / 1e3, 1), "pct_peak_gemm": round(b / us_g / 1e3 / PEAK_GBS * 100, 1),
                         "copies": nc})  # fmt: skip
        del copies
        torch.cuda.empty_cache()
    return rows


INGEST_CASES = (  # (name, fmt, N, K): one weight matrix's ggml block bytes, split on the device
    ("llama3_8b_ffn_gate", "q4_0", 14336, 4096),
    ("llama3_8b_lm_head", "q4_0", 128256, 4096),
    ("llama3_8b_ffn_gate", "q8_0", 14336, 4096),
    ("llama3_8b_ffn_gate", "q4_k", 14336, 4096),
    ("bitnet2b_ffn_gate", "tq2_0", 6912, 2560),
)


def ingest_detail(torch, host, args):
    """ggml block bytes -> split planes on the device (split_into), graph replays over copies of the block bytes;
    bytes = block bytes read + plane bytes written."""
    rows = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 4)
    for name, fmt, n, k in INGEST_CASES:
        f = host.FORMATS[fmt]
        nb = k // f["block"]
        size = n * nb * f["nbytes"]
        ncopy = max(2, math.ceil((COLD_BYTES // 2) / size))
        blocks = [torch.randint(0, 256, (size,), dtype=torch.uint8, device="cuda", generator=gen) for _ in range(ncopy)]
        wq = torch.empty((n, nb * f["qbytes"]), dtype=torch.uint8, device="cuda")
        ws = torch.empty((n, nb * f["sbytes"] // 2), dtype=torch.int16, device="cuda")

        def call(i, blocks=blocks, wq=wq, ws=ws, fmt=fmt, n=n, k=k):
            host.split_into(fmt, blocks[i % len(blocks)], wq, ws, n, k)

        per_graph = ncopy * math.ceil(16 / ncopy)
        reps = 2 * per_graph
        ms, _ = timed_steps(torch, call, ncopy, reps, per_graph)
        b = size + n * nb * (f["qbytes"] + f["sbytes"])
        us = ms * 1e3 / reps
        rows.append({"case": name, "fmt": fmt, "n": n, "k": k, "bytes": b, "us": round(us, 3),
                     "gbs": round(b / us / 1e3, 1), "pct_peak": round(b / us / 1e3 / PEAK_GBS * 100, 1),
                     "copies": ncopy})  # fmt: skip
        del blocks, wq, ws
        torch.cuda.empty_cache()
    return rows


def batched_calls(torch, host, args):
    """The batched_gemm cases' GEMMs, args.batched_calls eager calls each over cold weight copies, untimed: the
    dispatches a hardware-counter run reads (graph replays of hundreds of calls per case are too many for one)."""
    rows = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 3)
    for name, fmt, n, k in BATCH_CASES:
        copies = weight_copies(fmt, n, k, gen, torch, COLD_BYTES // 2)
        for m in BATCH_M:
            x = torch.randn((m, k), generator=gen, device="cuda")
            xq, xd = host.quantize(fmt, x)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            for i in range(args.batched_calls):
                wq, ws = copies[i % len(copies)]
                host.gemm_into(fmt, wq, ws, xq, xd, y, n, k)
            torch.cuda.synchronize()
            rows.append({"case": name, "fmt": fmt, "n": n, "k": k, "m": m, "calls": args.batched_calls,
                         "bytes": gemv_bytes(fmt, n, k, m)})
        del copies
        torch.cuda.empty_cache()
    return rows


COUNTER_CASES = (  # (fmt, N, K, columns, launch, mode): the kernels the hardware-counter tables cover
    ("tq2_0", 6912, 2560, 1, "fused", 2), ("tq2_0", 2560, 6912, 1, "fused", 2),
    ("tq2_0", 6912, 2560, 3, "fused", 2), ("tq2_0", 2560, 6912, 3, "fused", 2),
    ("tq2_0", 6912, 2560, 2, "gemv", 2), ("tq2_0", 6912, 2560, 3, "gemv", 2),
    ("tq2_0", 2560, 6912, 2, "gemv", 2), ("tq2_0", 2560, 6912, 3, "gemv", 2),
    ("tq2_0", 32768, 8192, 1, "gemv", 2), ("tq2_0", 32768, 8192, 3, "gemv", 2),
    ("q4_0", 4096, 14336, 1, "gemv", 2), ("q4_0", 4096, 14336, 3, "gemv", 2),
    ("q4_0", 128256, 4096, 1, "gemv", 2), ("q4_0", 14336, 4096, 64, "gemm", 2),
    ("q4_k", 14336, 4096, 1, "gemv", 2), ("q8_0", 14336, 4096, 1, "gemv", 2),
    # bytes mode (every value unpacked to an integer, no dot instruction) beside dp4a
    ("tq2_0", 6912, 2560, 1, "fused", 0), ("tq2_0", 32768, 8192, 1, "gemv", 0), ("q4_0", 4096, 14336, 1, "gemv", 0),
)  # fmt: skip


def counter_calls(torch, host, args):
    """COUNTER_CASES, args.counter_calls eager launches each over cold weight copies, untimed (library plans, the
    case's mode; fused = f32 activations quantized inside the launch, gemv / gemm = q8 activations in): the dispatches
    one rocprofv3 --pmc pass reads."""
    rows = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed + 6)
    for fmt, n, k, m, launch, mode in COUNTER_CASES:
        copies = weight_copies(fmt, n, k, gen, torch, COLD_BYTES // 2)
        x = torch.randn((m, k), generator=gen, device="cuda")
        xq, xd = host.quantize(fmt, x)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        for i in range(args.counter_calls):
            wq, ws = copies[i % len(copies)]
            if launch == "fused":
                host.gemv_f32_into(fmt, wq, ws, x, y, n, k, None, 0, mode, 0)
            elif launch == "gemm":
                host.gemm_into(fmt, wq, ws, xq, xd, y, n, k)
            else:
                host.gemv_into(fmt, wq, ws, xq, xd, y, n, k, None, 0, mode, 0)
        torch.cuda.synchronize()
        rows.append({"fmt": fmt, "n": n, "k": k, "m": m, "launch": launch, "mode": MODE_NAMES[mode],
                     "calls": args.counter_calls,
                     "bytes": step_bytes_fused(fmt, n, k, m) if launch == "fused" else gemv_bytes(fmt, n, k, m)})
        del copies
        torch.cuda.empty_cache()
    return rows


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--m", type=int, default=1, help="activation columns (1..3 in the workload list)")
    ap.add_argument("--mode", type=int, default=2, choices=(0, 1, 2))
    ap.add_argument("--block-n", type=int, default=None)
    ap.add_argument("--nb", type=int, default=4)
    ap.add_argument("--num-warps", type=int, default=4)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-detail", action="store_true")
    ap.add_argument("--detail-out", default=os.path.join("gpurun_out", "bench_detail.json"), metavar="PATH",
                    help="where the full per-shape tables (detail, configs, multi_matrix, batched_gemm, ingest, "
                         "quantizers) go "
                         "(empty: not written); the result line carries a compact row per workload configuration")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="host threads for cpu_baseline (default: the usable cores, at most 16)")
    ap.add_argument("--batched-only", action="store_true",
                    help="only run the batched_gemm block (for profiling the GEMM by itself)")
    ap.add_argument("--batched-calls", type=int, default=0, metavar="N",
                    help="with --batched-only: run each case's GEMM N times eagerly instead of timing it (a few "
                         "dispatches, for hardware-counter runs)")
    ap.add_argument("--counter-calls", type=int, default=0, metavar="N",
                    help="only launch the COUNTER_CASES kernels N times each, untimed (for rocprofv3 --pmc passes)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only copy a MIB-MiB device buffer 10 times (the known-size kernel that scales the PMC "
                         "FETCH_SIZE / WRITE_SIZE readings)")  # fmt: skip
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU: the decode path is single-device, and --gpus {args.gpus} is not supported "
              f"(value is the one GPU's throughput)", file=sys.stderr)  # fmt: skip
        return 2
    if args.steps < 1:
        print("--steps must be >= 1", file=sys.stderr)
        return 2

    import torch

    from comp_amd import _abi, host

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    _abi.lib()
    if args.calibrate_copy:
        nbytes = args.calibrate_copy << 20
        src = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": nbytes, "copies": 10}), flush=True)
        return 0

    if args.counter_calls > 0:
        print(json.dumps({"counter_calls": counter_calls(torch, host, args)}), flush=True)
        return 0

    if args.batched_only:
        rows = batched_calls(torch, host, args) if args.batched_calls > 0 else batched_detail(torch, host, args)
        print(json.dumps({"batched_gemm": rows}), flush=True)
        return 0

    value, ms_per_step, roofline, config, step_bytes = headline(torch, host, _abi, args)
    out = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8", "data": "synthetic", "config": config, "roofline": roofline,
           "pct_peak": round(value / PEAK_GBS * 100, 2)}  # fmt: skip
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args, step_bytes, args.cpu_seconds)
    if not args.no_detail:
        full = {"detail": detail(torch, host, _abi, args), "configs": config_detail(torch, host, args),
                "multi_matrix": multi_detail(torch, host, args), "batched_gemm": batched_detail(torch, host, args),
                "ingest": ingest_detail(torch, host, args), "quantizers": quant_detail(torch, host, args)}  # fmt: skip
        out["configs"] = config_summary(full["configs"])
        if args.detail_out:
            os.makedirs(os.path.dirname(os.path.abspath(args.detail_out)), exist_ok=True)
            with open(args.detail_out, "w") as f:
                json.dump({**out, **full, "configs_summary": out["configs"]}, f, indent=1)
            out["detail_file"] = args.detail_out
    # the result line stays a few KB (the per-shape tables go to the detail file)
    print(json.dumps(out, separators=(",", ":")), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
