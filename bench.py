#!/usr/bin/env python3
"""Benchmark: batch-1 decode through a stack of 48 routed-expert MoE layers on one
MI355X, tokens/s, plus the HBM roofline of the dominant kernel and the CPU baseline beside it.

    python bench.py [--steps K] [--warmup W] [--layers 48] [--cpu-seconds 10] [--no-cpu]

A step is one token through all layers: router GEMV (x . Wr, fp16 weights), top-k 8 of 128 (renormalised),
gate/up + SwiGLU and down + weighted combine read straight from GGUF Q4_0 blocks, residual add; the whole step
replays as one HIP graph. Weights are Gaussian N(0, 0.02^2) quantized to Q4_0 on the device (seed 0); each step
takes a fresh N(0, 1) fp16 activation row, all resident in HBM before timing. One JSON line on stdout.
"""
import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK = 8.0e12  # MI355X published HBM3E bandwidth, bytes/s
MFMA_PEAK = 2.5e15  # MI355X dense f16 / bf16 matrix peak, flop/s
# HBM bytes a launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (scaled by a 256 MiB copy) at the cfg2 shape,
# per kernel; see profiles/decode_cfg2_traffic.md for the commands. Reported as roofline.traffic for that kernel.
MEASURED_TRAFFIC = {"k_gate_up_xr": 14350080, "k_down_xr": 7321600, "k_router_gemv": 622080}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-config-seconds", type=float, default=4.0,
                    help="seconds of CPU baseline at each of the other configurations")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-grouped", action="store_true", help="skip the cfg3 prefill / cfg4 batched lines")
    ap.add_argument("--extra-only", action="store_true",
                    help="only the Q4_1 / Q8_0 / Q5_K / Q6_K lines (decode chain and grouped path), the trunk's "
                         "qmv_rows lines and the cache-biased route / GGUF loader lines, one JSON line")
    ap.add_argument("--grouped-only", action="store_true",
                    help="run only the grouped-path lines (cfg3 prefill, cfg4, cfg5) and print them: a short run to "
                         "profile the grouped GEMMs with rocprofv3 counters, not a benchmark line")
    ap.add_argument("--timeline", action="store_true",
                    help="only the cfg2 decode stack's per-workgroup phase timeline (the kernels' stamping forms, "
                         "replayed as one HIP graph a step), one JSON object: a measurement, not a benchmark line")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB (the scale for rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE counters)")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gpu_leg(args):
    import torch

    from larder_amd import _lib, layer as lay, workloads

    cfg = workloads.CONFIGS[2]
    g = torch.Generator(device="cuda").manual_seed(0)
    t0 = time.time()
    layers = [workloads.make_layer(cfg, g) for _ in range(args.layers)]
    torch.cuda.synchronize()
    log(f"built {args.layers} layers ({sum(L.wg.numel() * 3 for L in layers) / 1e9:.1f} GB Q4_0) in "
        f"{time.time() - t0:.1f}s")
    n = args.steps + args.warmup
    xs = torch.randn((n, 1, cfg["H"]), generator=g, device="cuda").half()
    st = lay.DecodeStack(layers, 1)
    st.capture()
    for i in range(args.warmup):
        st.x_in.copy_(xs[i])
        st.graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.warmup, n):
        st.x_in.copy_(xs[i])
        st.graph.replay()
    e1.record()
    torch.cuda.synchronize()
    secs = e0.elapsed_time(e1) / 1e3
    step_ms = secs / args.steps * 1e3

    # each decode kernel timed kernel-exactly: the stack runs eagerly for min(K, 64) more steps with the library's
    # launch hook armed, so every router / gate-up / down launch is bracketed by start / stop events that the HIP
    # runtime records at the kernel's own begin and end (the timestamps rocprofv3 reads), on the stream it runs on
    k, I, H, E = cfg["k"], cfg["I"], cfg["H"], cfg["E"]
    per_layer = [("k_router_gemv", E * H * 2 + H * 2 + E * 4 + H // 64 * 144),
                 ("k_gate_up_xr", k * 2 * I * (H // 32 * 18) + E * 4 + H // 64 * 144 + k * (I // 64 * 144)),
                 ("k_down_xr", k * H * (I // 32 * 18) + k * (I // 64 * 144) + 3 * H * 2)]
    prof_steps = min(args.steps, 64)
    M = prof_steps * args.layers * len(per_layer)
    _lib.call("lmoe_profile_arm", M)
    for i in range(prof_steps):
        st.x_in.copy_(xs[args.warmup + i])
        st.step()
    ms = (ctypes.c_float * M)()
    cnt = ctypes.c_int()
    _lib.call("lmoe_profile_read", ms, M, ctypes.byref(cnt))
    if cnt.value != M:
        raise RuntimeError(f"expected {M} timed launches, recorded {cnt.value}")
    timing = {}
    for j, (name, byts) in enumerate(per_layer):
        us = sum(ms[j::len(per_layer)]) / (M // len(per_layer)) * 1e3
        timing[name] = dict(us=round(us, 3), bytes=byts, gbps=round(byts / (us * 1e-6) / 1e9, 1),
                            launches=M // len(per_layer))
    dom = max(timing, key=lambda n: timing[n]["us"])
    token_bytes = args.layers * (workloads.decode_bytes(cfg, k) + 2 * H * 2)
    return dict(secs=secs, step_ms=step_ms, timing=timing, dom=dom, token_bytes=token_bytes, cfg=cfg, layers=layers)


def timeline_leg(args):
    """The cfg2 48-layer decode stack captured with the decode kernels' stamping forms (larder_amd.timeline), replayed
    back to back as in the headline line; after each batch of 16 replays the last replay's stamps are read. Per kernel
    and phase: the first, median and last workgroup's stamp in µs from the layer's first router workgroup start
    (medians over layers and batches), and the layer period (one router start to the next)."""
    import numpy as np
    import torch

    from larder_amd import layer as lay, timeline, workloads

    cfg = workloads.CONFIGS[2]
    g = torch.Generator(device="cuda").manual_seed(0)
    layers = [workloads.make_layer(cfg, g) for _ in range(args.layers)]
    xs = torch.randn((64, 1, cfg["H"]), generator=g, device="cuda").half()
    st = lay.DecodeStack(layers, 1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        st.step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with timeline.Timeline(args.layers * 4096) as tl:
        with torch.cuda.graph(graph):
            st.step()
    if len(tl.launches) != 3 * args.layers:
        raise RuntimeError(f"{len(tl.launches)} stamped launches, expected {3 * args.layers}")
    khz = timeline.clock_khz()
    for i in range(64):
        st.x_in.copy_(xs[i % 64])
        graph.replay()
    torch.cuda.synchronize()
    per = {name: {p: [] for p in timeline.PHASES} for name in timeline.KERNELS.values()}
    periods = []
    for b in range(16):
        for i in range(16):
            st.x_in.copy_(xs[(16 * b + i) % 64])
            graph.replay()
        torch.cuda.synchronize()
        stamps = tl.buf.cpu().numpy()
        res = timeline.layer_phases(stamps, tl.launches, khz)
        for name in per:
            for p in per[name]:
                per[name][p] += res[name][p]
        starts = [stamps[r0:r0 + n, 0].min() for name, r0, n in tl.launches if name == "router"]
        periods += list(np.diff(starts) * 1e3 / khz)
    out = timeline.summary(per)
    out["layer_period_us"] = round(float(np.median(periods)), 2)
    out["clock_khz"] = khz
    out["note"] = (f"cfg2, {args.layers} layers, one HIP graph a step; 16 batches of 16 back-to-back replays, the "
                   "last replay of each read; µs from the layer's first router workgroup start; each workgroup "
                   "stamps from its first thread (wavefront 0)")
    return out


def entry_leg(g):
    """The drop-in entry at cfg2's decode shape, as the reference's caller drives it for one token
    (gguf_experts.experts, gguf_experts.py:803-819): experts(x (1, 1, 1, H), bufs, rhs (1, 1, k), "Q4_0/Q4_0/Q4_0")
    with the token's k slots given, each call on the next layer of the decode line's stack (no expert is read from
    the caches). Reported: the kernels' durations a call (launch-exact, as the decode line's), the call replayed in
    a HIP graph (one call a layer), and eager calls (host launch bound); the HBM fraction over the k experts' bytes."""
    import torch

    from larder_amd import _lib, gguf_experts as ge

    log("[bench] entry decode: start")
    cfg, layers = g["cfg"], g["layers"]
    H, I, E, k = cfg["H"], cfg["I"], cfg["E"], cfg["k"]
    nl = len(layers)
    bufs = [tuple((b,) for b in (L.wg, L.wu, L.wd)) for L in layers]
    gen = torch.Generator(device="cuda").manual_seed(11)
    n = 4 * nl
    xs = torch.randn((n, 1, 1, 1, H), generator=gen, device="cuda").half()
    rhs = torch.stack([torch.randperm(E, generator=gen, device="cuda")[:k] for _ in range(n)]).to(torch.int32)
    rhs = rhs.reshape(n, 1, 1, k)
    types = "Q4_0/Q4_0/Q4_0"

    def call(i):
        return ge.experts(xs[i], bufs[i % nl], rhs[i], types)

    for i in range(2 * nl):
        call(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n):
        call(i)
    e1.record()
    torch.cuda.synchronize()
    us_eager = e0.elapsed_time(e1) / n * 1e3
    # kernel-exact: gate/up + SwiGLU with x prepared in the launch, down (two launches a call)
    names = ("k_gate_up_xr<raw x>", "k_down_slots")
    calls = 2 * nl
    M = calls * len(names)
    _lib.call("lmoe_profile_arm", M)
    for i in range(calls):
        call(i)
    ms = (ctypes.c_float * M)()
    cnt = ctypes.c_int()
    _lib.call("lmoe_profile_read", ms, M, ctypes.byref(cnt))
    if cnt.value != M:
        raise RuntimeError(f"entry: expected {M} timed launches, recorded {cnt.value}")
    kern = {nm: round(sum(ms[j::len(names)]) / calls * 1e3, 3) for j, nm in enumerate(names)}
    # one call a layer in a HIP graph
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(nl):
            call(i)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(nl):
            call(i)
    for _ in range(8):
        graph.replay()
    torch.cuda.synchronize()
    reps = 16
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us_graph = e0.elapsed_time(e1) / (reps * nl) * 1e3
    byts = k * (2 * I * (H // 32 * 18) + H * (I // 32 * 18)) + H * 2 + k * H * 2
    layer_us = g["timing"]["k_gate_up_xr"]["us"] + g["timing"]["k_down_xr"]["us"]
    ksum = sum(kern.values())
    log(f"[bench] entry decode: kernels {ksum:.2f} us a call, graph {us_graph:.2f}, eager {us_eager:.2f}")
    return {"us_kernels": round(ksum, 2), "kernels_us": kern, "hbm_frac_kernels": round(byts / (ksum * 1e-6) / HBM_PEAK, 4),
            "us_graph": round(us_graph, 2), "hbm_frac_graph": round(byts / (us_graph * 1e-6) / HBM_PEAK, 4),
            "us_eager": round(us_eager, 2), "bytes": byts,
            "layer_decode_gate_up_down_us": round(layer_us, 2),
            "kernels_vs_layer_decode": round(ksum / layer_us, 3),
            "note": "experts() at cfg2's shape, one token's 8 slots given; the layer line's gate/up + down kernels "
                    "(the fused top-k and the weighted combine included) beside it"}


def grouped_leg():
    """The other configurations (BASELINE.json configs[0] and [2..4]), reported beside the decode line:
    cfg3 = one 8192-token bf16 prefill chunk through one cfg-2 layer with skewed router logits (MFMA roofline over
    the routed experts' 2 R 3 H I flops); cfg4 = 512 steps of 64 tokens with a fresh Zipf-prior draw each step
    (HBM roofline over the unique experts touched); cfg1 = batch-1 decode through 16 layers with a 5,632-wide shared
    expert; cfg5 = the 512-expert Q4_K layer at T = 1 (decode chain) and T = 2048 (grouped path)."""
    import ctypes

    import torch

    from larder_amd import _lib, grouped, workloads

    out = {}
    g = torch.Generator(device="cuda").manual_seed(3)
    cfg = workloads.CONFIGS[3]
    T = cfg["T"]
    L = workloads.make_layer(cfg, g, with_router=False)
    lg = workloads.skewed_logits(T, cfg["E"], g)
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").bfloat16()
    B = grouped.PrefillBuffers(L, T)
    y = torch.empty((T, cfg["H"]), dtype=torch.bfloat16, device="cuda")
    flops = workloads.expert_flops(cfg, T * cfg["k"])
    R = T * cfg["k"]
    gu, dn = 2 * R * 2 * cfg["H"] * cfg["I"], 2 * R * cfg["H"] * cfg["I"]
    # per-kernel names in launch order (7 launches a pass: top-k and x to f16 in the K order in one launch, 3 grouping,
    # gate/up, down, combine; 8 with LMOE_FUSED_TOPK=0: the first two apart)
    names = (["k_to_f16", "k_router_topk"] if os.environ.get("LMOE_FUSED_TOPK", "1") == "0" else ["k_topk_and_f16"]) + \
        ["k_group_count", "k_group_scan", "k_group_scatter", "k_grouped<gate_up>", "k_grouped<down>", "k_combine_sorted"]

    def cfg3_pass(label):
        log(f"[bench] cfg3 prefill on {label}: start")
        # untimed until the clocks settle: the first ~30 ms of back-to-back chunks run ~12% slower than steady state
        for _ in range(60):
            grouped.prefill(L, x, B, y, logits=lg)
        torch.cuda.synchronize()
        n = 20
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            grouped.prefill(L, x, B, y, logits=lg)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / n * 1e3
        # per kernel, kernel-exact, over 5 more passes
        M = 5 * len(names)
        _lib.call("lmoe_profile_arm", M)
        for _ in range(5):
            grouped.prefill(L, x, B, y, logits=lg)
        ms = (ctypes.c_float * M)()
        cnt = ctypes.c_int()
        _lib.call("lmoe_profile_read", ms, M, ctypes.byref(cnt))
        kern = {nm: round(sum(ms[j:cnt.value:len(names)]) / 5 * 1e3, 2) for j, nm in enumerate(names)}
        log(f"[bench] cfg3 prefill on {label}: {us:.1f} us a chunk")
        return {"us_per_chunk": round(us, 1), "tokens_per_s": round(T / (us * 1e-6), 1),
                "mfma_frac": round(flops / (us * 1e-6) / MFMA_PEAK, 4), "kernels_us": kern,
                "gate_up_mfma_frac": round(gu / (kern["k_grouped<gate_up>"] * 1e-6) / MFMA_PEAK, 4),
                "down_mfma_frac": round(dn / (kern["k_grouped<down>"] * 1e-6) / MFMA_PEAK, 4)}

    out["cfg3_prefill"] = dict(cfg3_pass("the GGUF layout"), flops=flops,
                               rows_per_expert_max=int(B.G.counts.max().item()),
                               experts_empty=int((B.G.counts == 0).sum().item()),
                               weights="GGUF Q4_0 blocks as stored (the layout the reference's dense path reads)")
    # the same layer holding stream-layout copies of its experts (MoELayer.keep_stream: the Q4 bytes twice in HBM),
    # as a resident prefill layer may: a variant, not the figure of record
    stream_bytes = L.keep_stream()
    out["cfg3_prefill"]["resident_stream_copies"] = dict(
        cfg3_pass("stream copies"), extra_hbm_bytes=stream_bytes,
        note="the grouped GEMMs read a second, reordered copy of the Q4_0 experts (MoELayer.keep_stream); same bits")
    L.drop_stream()
    del B, x, y, lg
    # cfg4: 64 sequences x 1 token a step, 512 steps, a fresh draw of logits and x each step
    cfg4 = workloads.CONFIGS[4]
    T4, steps = cfg4["T"], 512
    lgs = torch.stack([workloads.zipf_logits(T4, cfg4["E"], g) for _ in range(steps)])
    xs = torch.randn((steps, T4, cfg4["H"]), generator=g, device="cuda").half()
    # each step's x and logits packed in one row of bytes, staged into the graph's static inputs by one copy a step
    # (as a serving loop stages its batch), so the step pays one copy instead of two
    xb, lb = T4 * cfg4["H"] * 2, T4 * cfg4["E"] * 4
    packed = torch.cat([xs.view(torch.uint8).reshape(steps, xb), lgs.view(torch.uint8).reshape(steps, lb)], 1)
    stage = packed[0].clone()
    x4 = stage[:xb].view(torch.float16).view(T4, cfg4["H"])
    lg4 = stage[xb:].view(torch.float32).view(T4, cfg4["E"])
    B4 = grouped.PrefillBuffers(L, T4)
    y4 = torch.empty((T4, cfg4["H"]), dtype=torch.float16, device="cuda")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def cfg4_pass(label):
        log(f"[bench] cfg4 batched decode on {label}: start")
        # one step as a HIP graph over static input buffers (a serving loop would capture it the same way)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            grouped.prefill(L, x4, B4, y4, logits=lg4)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            grouped.prefill(L, x4, B4, y4, logits=lg4)
        for i in range(200):
            stage.copy_(packed[i % steps])
            graph.replay()
        uniq = rmax = 0
        torch.cuda.synchronize()
        e0.record()
        for i in range(steps):
            stage.copy_(packed[i])
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us4 = e0.elapsed_time(e1) / steps * 1e3
        for i in range(0, steps, 64):  # unique experts a step (for the HBM roofline), sampled
            stage.copy_(packed[i])
            graph.replay()
            uniq += int((B4.G.counts > 0).sum().item())
            rmax += int(B4.G.counts.max().item())
        uniq /= len(range(0, steps, 64))
        rmax /= len(range(0, steps, 64))
        byts = uniq * (2 * cfg4["I"] * workloads.row_bytes("Q4_0", cfg4["H"]) +
                       cfg4["H"] * workloads.row_bytes("Q4_0", cfg4["I"])) + T4 * cfg4["H"] * 2 * 2
        log(f"[bench] cfg4 batched decode on {label}: {us4:.1f} us a step")
        return {"us_per_step": round(us4, 1), "tokens_per_s": round(T4 / (us4 * 1e-6), 1),
                "unique_experts_per_step": round(uniq, 1), "rows_per_expert_max": round(rmax, 1),
                "hbm_frac": round(byts / (us4 * 1e-6) / HBM_PEAK, 4)}

    out["cfg4_batched"] = dict(cfg4_pass("the GGUF layout"),
                               note="one HIP graph a step; one copy a step of the packed x and logits into the graph's "
                                    "inputs, inside the timed loop; the grouped GEMMs read the GGUF blocks as stored")
    stream_bytes = L.keep_stream()
    out["cfg4_batched"]["resident_stream_copies"] = dict(
        cfg4_pass("stream copies"), extra_hbm_bytes=stream_bytes,
        note="the grouped GEMMs read a second, reordered copy of the Q4_0 experts (MoELayer.keep_stream); same bits")
    L.drop_stream()
    del B4, xs, lgs, packed
    # cfg1: E 60, top-4 without renorm, I 1408, a 5,632-wide shared expert with a sigmoid gate, Q4_0; batch-1 decode
    # through 16 such layers (each step touches 16 x 39.2 MB, over twice the 256 MB MALL), one HIP graph a step.
    from larder_amd import layer as lay
    log("[bench] cfg1 decode stack: start")
    cfg1 = workloads.CONFIGS[1]
    L1s = [workloads.make_layer(cfg1, g) for _ in range(16)]  # 627 MB a step: over twice the 256 MB MALL
    st1 = lay.DecodeStack(L1s, 1)
    st1.capture()
    n1 = 128
    x1 = torch.randn((n1 + 16, 1, cfg1["H"]), generator=g, device="cuda").half()
    for i in range(100):
        st1.x_in.copy_(x1[i % 16])
        st1.graph.replay()
    torch.cuda.synchronize()
    e0.record()
    for i in range(16, 16 + n1):
        st1.x_in.copy_(x1[i])
        st1.graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us1 = e0.elapsed_time(e1) / n1 * 1e3 / len(L1s)
    b1 = workloads.decode_bytes(cfg1, cfg1["k"]) + 2 * cfg1["H"] * 2
    out["cfg1_decode_T1"] = {"us_per_layer": round(us1, 2), "bytes_per_layer": b1,
                             "hbm_frac": round(b1 / (us1 * 1e-6) / HBM_PEAK, 4),
                             "note": "16-layer stack; the 5,632-wide shared expert folded into the decode kernels as four slices of the routed width (3 launches a layer)"}
    del st1, L1s, x1
    # cfg5: H 4096, 512 experts top-10, I 512, shared expert, Q4_K. T = 1 through the decode chain (one layer as a
    # HIP graph, a fresh x each step so the touched experts change), T = 2048 through the grouped path.
    log("[bench] cfg5 decode: start")
    cfg5 = workloads.CONFIGS[5]
    L5 = workloads.make_layer(cfg5, g)
    st5 = lay.DecodeStack([L5], 1)
    st5.capture()
    n5 = 256
    x5 = torch.randn((n5 + 16, 1, cfg5["H"]), generator=g, device="cuda").half()
    for i in range(400):
        st5.x_in.copy_(x5[i % 16])
        st5.graph.replay()
    torch.cuda.synchronize()
    e0.record()
    for i in range(16, 16 + n5):
        st5.x_in.copy_(x5[i])
        st5.graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us5 = e0.elapsed_time(e1) / n5 * 1e3
    b5 = workloads.decode_bytes(cfg5, cfg5["k"]) + 2 * cfg5["H"] * 2
    # the same layer shape as an 8-layer stack (seven more layers of fresh weights, 14.5 GB in all), timed per
    # layer as cfg1 is: a one-layer graph also pays its own launch and the input copy on every token
    del st5
    L5s = [L5] + [workloads.make_layer(cfg5, g) for _ in range(7)]
    st5s = lay.DecodeStack(L5s, 1)
    st5s.capture()
    for i in range(100):
        st5s.x_in.copy_(x5[i % 16])
        st5s.graph.replay()
    torch.cuda.synchronize()
    e0.record()
    for i in range(16, 16 + n5 // 2):
        st5s.x_in.copy_(x5[i])
        st5s.graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us5s = e0.elapsed_time(e1) / (n5 // 2) * 1e3 / len(L5s)
    del st5s, L5s[1:]
    out["cfg5_decode_T1"] = {"us_per_token": round(us5, 2), "tokens_per_s": round(1 / (us5 * 1e-6), 1),
                             "bytes": b5, "hbm_frac": round(b5 / (us5 * 1e-6) / HBM_PEAK, 4),
                             "note": "one layer as its own HIP graph a token, with the input copy",
                             "stacked_us_per_layer": round(us5s, 2),
                             "stacked_hbm_frac": round(b5 / (us5s * 1e-6) / HBM_PEAK, 4),
                             "stacked_note": "8 layers of this shape in one graph a token (as cfg1), per layer"}
    T5 = 2048
    x5p = torch.randn((T5, cfg5["H"]), generator=g, device="cuda").bfloat16()
    B5 = grouped.PrefillBuffers(L5, T5)
    y5 = torch.empty((T5, cfg5["H"]), dtype=torch.bfloat16, device="cuda")
    f5 = workloads.expert_flops(cfg5, T5 * cfg5["k"]) + 2 * T5 * 3 * cfg5["H"] * cfg5["Is"]

    def cfg5_pass(label):
        log(f"[bench] cfg5 prefill on {label}: start")
        for _ in range(40):
            grouped.prefill(L5, x5p, B5, y5)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(10):
            grouped.prefill(L5, x5p, B5, y5)
        e1.record()
        torch.cuda.synchronize()
        us5p = e0.elapsed_time(e1) / 10 * 1e3
        u5 = int((B5.G.counts[:cfg5["E"]] > 0).sum().item())  # routed experts (the folded shared one apart)
        by5 = workloads.decode_bytes(cfg5, u5) + T5 * cfg5["H"] * 2 * 2
        log(f"[bench] cfg5 prefill on {label}: {us5p:.1f} us")
        return {"us": round(us5p, 1), "tokens_per_s": round(T5 / (us5p * 1e-6), 1),
                "mfma_frac": round(f5 / (us5p * 1e-6) / MFMA_PEAK, 4),
                "hbm_frac": round(by5 / (us5p * 1e-6) / HBM_PEAK, 4), "experts_touched": u5}

    out["cfg5_prefill_T2048"] = dict(
        cfg5_pass("the GGUF layout"),
        note="routing from x: router logits by the router GEMM and the certified refine (ids bit-exact to the decode "
             "router's fixed order) inside the timing; the shared expert folded into the routed GEMMs as expert E "
             "(slot k of every token); the grouped GEMMs read the GGUF blocks as stored")
    stream_bytes = L5.keep_stream()
    out["cfg5_prefill_T2048"]["resident_stream_copies"] = dict(
        cfg5_pass("stream copies"), extra_hbm_bytes=stream_bytes,
        note="the grouped GEMMs read a second, reordered copy of the Q4_K experts (MoELayer.keep_stream); same bits")
    L5.drop_stream()
    return out


def types_leg():
    """The block types beyond Q4_0 / Q4_K on a cfg2-shaped layer (H 2048, E 128, I 768, top-8), each type for all
    three projections, plus the 35B's Q4_K / Q4_K / Q6_K mix: the decode chain for one token (the general gate/up
    and down kernels, kernel-exact durations against the HBM roofline over the 8 experts' bytes) and the grouped
    path for 2048 tokens (dequant of the experts to f16, then the f16-weight grouped GEMMs; MFMA roofline over the
    routed GEMM flops)."""
    import ctypes

    import torch

    from larder_amd import _lib, gguf_experts as ge, workloads

    H, E, I, k = 2048, 128, 768, 8
    g = torch.Generator(device="cuda").manual_seed(5)
    out = {}

    def kernels(fn, n_launch, reps):
        M = n_launch * reps
        _lib.call("lmoe_profile_arm", M)
        for _ in range(reps):
            fn()
        ms = (ctypes.c_float * M)()
        cnt = ctypes.c_int()
        _lib.call("lmoe_profile_read", ms, M, ctypes.byref(cnt))
        return [sum(ms[j:cnt.value:n_launch]) / reps * 1e3 for j in range(n_launch)]

    for types in (("Q4_1",) * 3, ("Q8_0",) * 3, ("Q5_K",) * 3, ("Q6_K",) * 3, ("Q4_K", "Q4_K", "Q6_K")):
        w = tuple(workloads.random_blocks(t, E, r, c, g) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
        x = torch.randn((1, H), generator=g, device="cuda").half()
        picks = torch.randperm(E, generator=g, device="cuda")[:k].to(torch.int32)
        dec = lambda: ge.gemv(x, w, picks, k, types, torch.float16)  # noqa: E731
        for _ in range(8):
            dec()
        torch.cuda.synchronize()
        gu, dn = kernels(dec, 2, 32)
        wbytes = k * (2 * I * _lib.row_bytes(types[0], H) + H * _lib.row_bytes(types[2], I))
        byts = wbytes + H * 2 + k * I * 4 * 2 + k * H * 2
        T = 2048
        xt = torch.randn((T * k, H), generator=g, device="cuda").half()
        rows = torch.randint(0, E, (T * k,), generator=g, device="cuda", dtype=torch.int32)
        den = lambda: ge.dense(xt, w, rows, types, torch.float16)  # noqa: E731
        for _ in range(2):
            den()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            den()
        e1.record()
        torch.cuda.synchronize()
        us_dense = e0.elapsed_time(e1) / 5 * 1e3
        flops = 2 * T * k * 3 * H * I
        # the layer path with the f16 K-order weights held resident (MoELayer.keep_prefill_f16): no dequant a call
        from larder_amd import grouped, layer as lay
        L = lay.MoELayer(*w, types, k, True)
        L.keep_prefill_f16()
        lg = torch.randn((T, E), generator=g, device="cuda")
        xl = xt[:T]
        B = grouped.PrefillBuffers(L, T)
        yl = torch.empty((T, H), dtype=torch.float16, device="cuda")
        for _ in range(2):
            grouped.prefill(L, xl, B, yl, logits=lg)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(5):
            grouped.prefill(L, xl, B, yl, logits=lg)
        e1.record()
        torch.cuda.synchronize()
        us_layer = e0.elapsed_time(e1) / 5 * 1e3
        del L, B
        # batch-1 decode through a stack of 8 such layers (own experts and router each) as one HIP graph a token,
        # the route layer.decode takes for these types (decode_general: fp32 h, the general or Q6_K down)
        shapes = ((I, H), (I, H), (H, I))
        Ls = [lay.MoELayer(*(workloads.random_blocks(t, E, r, c, g) for (r, c), t in zip(shapes, types)), types, k,
                           True, wr=workloads.router_weight(E, H, g)) for _ in range(8)]
        st = lay.DecodeStack(Ls, 1)
        st.capture()
        xs = torch.randn((80, 1, H), generator=g, device="cuda").half()
        for i in range(40):
            st.x_in.copy_(xs[i % 16])
            st.graph.replay()
        torch.cuda.synchronize()
        e0.record()
        for i in range(16, 80):
            st.x_in.copy_(xs[i])
            st.graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us_stack = e0.elapsed_time(e1) / 64 * 1e3 / len(Ls)
        del st, Ls
        out["/".join(types)] = {
            "decode_stack_us_per_layer": round(us_stack, 2),
            "decode_stack_hbm_frac": round(wbytes / (us_stack * 1e-6) / HBM_PEAK, 4),
            "decode_gate_up_us": round(gu, 2), "decode_down_us": round(dn, 2), "decode_bytes": byts,
            "decode_hbm_frac": round(byts / ((gu + dn) * 1e-6) / HBM_PEAK, 4),
            "dense_2048x8_us": round(us_dense, 1), "dense_mfma_frac": round(flops / (us_dense * 1e-6) / MFMA_PEAK, 4),
            "prefill_2048_resident_f16_us": round(us_layer, 1),
            "prefill_mfma_frac": round(flops / (us_layer * 1e-6) / MFMA_PEAK, 4)}
        del w, xt, rows
    return out


def trunk_leg():
    """The trunk's 4-bit affine matmul (lmoe_qmv_rows) at the 35B's dense shapes the reference's test uses (K -> N,
    group 64), T = 1 and T = 5 rows: kernel-exact durations against the HBM roofline over the weight, scale and
    bias bytes plus x and out."""
    import ctypes

    import torch

    from larder_amd import _lib, trunk

    g = torch.Generator(device="cuda").manual_seed(7)
    out = {}
    for K, N in ((2048, 8192), (2048, 4096), (4096, 2048), (2048, 512)):
        G = 64
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 8), generator=g, device="cuda", dtype=torch.int32)
        sc = (torch.rand((N, K // G), generator=g, device="cuda") * 0.01).bfloat16()
        bi = (torch.rand((N, K // G), generator=g, device="cuda") * -0.05).bfloat16()
        for T in (1, 5):
            x = torch.randn((T, K), generator=g, device="cuda").bfloat16()
            for _ in range(5):
                trunk.qmv_rows(x, w, sc, bi, G)
            torch.cuda.synchronize()
            reps = 50
            _lib.call("lmoe_profile_arm", reps)
            for _ in range(reps):
                trunk.qmv_rows(x, w, sc, bi, G)
            ms = (ctypes.c_float * reps)()
            cnt = ctypes.c_int()
            _lib.call("lmoe_profile_read", ms, reps, ctypes.byref(cnt))
            us = sum(ms[:cnt.value]) / cnt.value * 1e3
            byts = N * K // 2 + 2 * N * (K // G) * 2 + T * K * 2 + T * N * 2
            out[f"{K}->{N} T{T}"] = {"us": round(us, 2), "bytes": byts,
                                     "hbm_frac": round(byts / (us * 1e-6) / HBM_PEAK, 4)}
        del w, sc, bi
    return out


def route_loader_leg():
    """The cache-biased route (lmoe_route_bias: route_cuda.route / bias_probs) at the reference's shapes, kernel-exact;
    and the GGUF pack / loader on a synthetic ~1 GB two-layer Q4_0 GGUF file in a temporary directory: pack
    (GGUF -> experts.bin, each chunk written, synced and read back) and load_layer (experts.bin -> HBM through pinned
    staging) throughput."""
    import ctypes
    import struct
    import tempfile
    import time
    from pathlib import Path

    import numpy as np
    import torch

    from larder_amd import _lib, gguf_pack, route, workloads

    out = {}
    g = torch.Generator(device="cuda").manual_seed(9)
    for E, k, T, dt in ((512, 10, 1, torch.bfloat16), (512, 10, 5, torch.bfloat16), (256, 8, 5, torch.float32)):
        gates = torch.softmax(torch.randn((T, E), generator=g, device="cuda"), -1).to(dt)
        slot = torch.full((E,), -1, dtype=torch.int32, device="cuda")
        slot[:E // 3] = torch.arange(E // 3, dtype=torch.int32, device="cuda")
        f = lambda: route.route(gates, None, slot, 0.5, 0.2, k, lim=E // 4)  # noqa: E731
        for _ in range(5):
            f()
        torch.cuda.synchronize()
        reps = 50
        _lib.call("lmoe_profile_arm", reps)
        for _ in range(reps):
            f()
        ms = (ctypes.c_float * reps)()
        cnt = ctypes.c_int()
        _lib.call("lmoe_profile_read", ms, reps, ctypes.byref(cnt))
        out[f"route_bias E{E} k{k} T{T} {str(dt).split('.')[-1]}"] = {"us": round(sum(ms[:cnt.value]) / cnt.value * 1e3, 2)}
    H, I, E = 2048, 768, 128
    rb_gu, rb_d = workloads.row_bytes("Q4_0", H), workloads.row_bytes("Q4_0", I)
    with tempfile.TemporaryDirectory() as d:
        d = Path(d)
        tensors = []
        for L in range(2):
            for p, (rows, rb, ne0) in (("gate", (I, rb_gu, H)), ("up", (I, rb_gu, H)), ("down", (H, rb_d, I))):
                blocks = np.random.default_rng(L).integers(0, 256, (E, rows, rb // 18, 18), dtype=np.uint8)
                blocks[..., 0:2] = np.frombuffer(np.float16(0.001).tobytes(), np.uint8)
                tensors.append((f"blk.{L}.ffn_{p}_exps.weight", [ne0, rows, E], 2, blocks.tobytes()))
        hdr = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 0)
        off, data = 0, []
        for name, ne, tid, raw in tensors:
            nb = name.encode()
            hdr += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", x) for x in ne)
            hdr += struct.pack("<IQ", tid, off)
            pad = (-len(raw)) % 32
            data.append(raw + b"\0" * pad)
            off += len(raw) + pad
        src = d / "m.gguf"
        with open(src, "wb") as fh:
            fh.write(hdr + b"\0" * ((-len(hdr)) % 32))
            for blob in data:
                fh.write(blob)
        del data, tensors
        nbytes = src.stat().st_size
        t0 = time.perf_counter()
        gguf_pack.pack([src], d / "experts.bin", log=None)
        t_pack = time.perf_counter() - t0
        packed = gguf_pack.load_packed(d)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        bufs = [gguf_pack.load_layer(packed, L)[0] for L in range(2)]
        torch.cuda.synchronize()
        t_load = time.perf_counter() - t0
        packed["fd"].close()
        loaded = sum(b.numel() for bb in bufs for b in bb)
        out["loader"] = {"gguf_bytes": nbytes, "pack_s": round(t_pack, 3), "pack_gbps": round(nbytes / t_pack / 1e9, 2),
                         "load_s": round(t_load, 3), "load_gbps": round(loaded / t_load / 1e9, 2),
                         "note": "synthetic 2-layer Q4_0 GGUF (H 2048, I 768, E 128) in a temporary directory; pack "
                                 "syncs and reads back every chunk; load = experts.bin -> HBM through pinned staging"}
        del bufs
    return out


def cpu_leg(args, g):
    """The C++ restatement of the reference CPU kernel (cpu_kern gather_qmm) over the same experts, converted to
    its affine 4-bit layout, run layer after layer for about --cpu-seconds; tokens/s = 1 / (48 x mean layer time).
    Threads follow the reference's rule (MOE_CPU_THREADS, else the physical cores of a socket), and every other
    configuration gets a bounded sample of its own (cpu_configs)."""
    import numpy as np

    from oracle import cpu_baseline as cb

    cores = cb.threads()
    cb.lib().ckp_set_threads(cores)
    cfg = g["cfg"]
    nl = min(8, len(g["layers"]))
    sample = []
    for L in g["layers"][:nl]:
        G = cb.Affine(L.wg.cpu().numpy(), "Q4_0", cfg["H"])
        U = cb.Affine(L.wu.cpu().numpy(), "Q4_0", cfg["H"])
        D = cb.Affine(L.wd.cpu().numpy(), "Q4_0", cfg["I"])
        sample.append((G, U, D, L.wr.cpu().numpy()))
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, cfg["H"])).astype(np.float32)
    cb.moe_layer(x, sample[0][3], cfg["k"], True, *sample[0][:3], residual=x)
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < args.cpu_seconds or done < nl:
        G, U, D, wr = sample[done % nl]
        x = cb.moe_layer(x, wr, cfg["k"], True, G, U, D, residual=x)
        if done % nl == nl - 1:
            x = rng.standard_normal((1, cfg["H"])).astype(np.float32)   # a fresh token every pass over the sample
        done += 1
    secs = time.perf_counter() - t0
    per_layer = secs / done
    hw = cb.host()
    from larder_amd import workloads
    return dict(value=1.0 / (per_layer * args.layers), unit="tokens/s", cores=cores, kind="port",
                sample=f"{done} layer passes (batch 1, cfg-2 layer shape) over {nl} of the stack's layers in "
                       f"{secs:.1f} s, {hw['isa']}, {hw['model']}; tokens/s = 1 / ({len(g['layers'])} x mean "
                       f"layer time)",
                gb_s=round(workloads.decode_bytes(cfg, cfg["k"]) / per_layer / 1e9, 2),
                host=hw, configs=cpu_configs(cb, args.cpu_config_seconds))


def cpu_configs(cb, secs):
    """The CPU baseline at the other configurations, each a bounded sample of about ``secs`` seconds on the same
    restated kernel: synthetic experts in the affine layout at the configuration's shapes (the kernel's time does
    not depend on the values), routing by the layer's own router on random weights. gb_s is the GGUF algorithmic
    bytes over the time, the GPU lines' measure (the affine layout the kernel reads is 0.75 B a weight, Q4_0 0.5625,
    Q4_K 0.5625)."""
    import numpy as np

    from larder_amd import workloads
    rng = np.random.default_rng(2)

    def timed(fn):
        fn()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < secs or n < 2:
            fn()
            n += 1
        return (time.perf_counter() - t0) / n, n

    def layer(cfg):
        E, H, I, Is = cfg["E"], cfg["H"], cfg["I"], cfg["Is"]
        ex = (cb.synthetic(E, I, H, 1), cb.synthetic(E, I, H, 2), cb.synthetic(E, H, I, 3))
        wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float16)
        sh = (cb.synthetic(1, Is, H, 4), cb.synthetic(1, Is, H, 5), cb.synthetic(1, H, Is, 6)) if Is else None
        wsg = (rng.standard_normal(H) * 0.02).astype(np.float32)

        def run(x):
            y = cb.moe_layer(x, wr, cfg["k"], cfg["norm"], *ex)
            if sh is not None:   # the shared expert through the same kernel, gated by sigmoid(x . wsg)
                z = np.zeros(x.shape[0], np.uint32)
                gg, uu = cb.gather_qmm(x, sh[0], z), cb.gather_qmm(x, sh[1], z)
                hh = gg / (1.0 + np.exp(-gg)) * uu
                y = y + cb.gather_qmm(hh.astype(np.float32), sh[2], z) / (1.0 + np.exp(-(x @ wsg)))[:, None]
            return y
        return run

    out = {}
    runs = {}  # one layer a shape: cfg3 and cfg4 share cfg2's, cfg5's two lines share one
    for name, cid, T, unit in (("cfg1_decode_T1", 1, 1, "layer"), ("cfg3_prefill", 3, 256, "chunk"),
                               ("cfg4_batched", 4, 64, "step"), ("cfg5_decode_T1", 5, 1, "token"),
                               ("cfg5_prefill_T2048", 5, 128, "chunk")):
        cfg = workloads.CONFIGS[cid]
        key = tuple(cfg[f] for f in ("H", "E", "k", "I", "Is", "norm"))
        if key not in runs:
            runs.clear()
            runs[key] = layer(cfg)
        run = runs[key]
        x = rng.standard_normal((T, cfg["H"])).astype(np.float32)
        per, n = timed(lambda: run(x))
        line = {"tokens_per_s": round(T / per, 2), "passes": n, "tokens_a_pass": T}
        if T == 1:
            line["us_per_" + unit] = round(per * 1e6, 1)
            line["gb_s"] = round(workloads.decode_bytes(cfg, cfg["k"]) / per / 1e9, 2)
        else:
            rows = T * cfg["k"]
            line["tflops"] = round((workloads.expert_flops(cfg, rows) + 2 * T * 3 * cfg["H"] * cfg["Is"]) / per / 1e12,
                                   3)
            full = cfg.get("T", 2048 if cid == 5 else T)
            if full != T:
                line["sample"] = f"{T} of the {full}-token {unit}; tokens/s scales with rows"
            if cid == 4:
                line["us_per_step"] = round(per * 1e6, 1)
        out[name] = line
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for {args.gpus})", file=sys.stderr)
        sys.exit(2)
    os.environ.setdefault("HSA_ENABLE_IPC_MODE_LEGACY", "0")
    if args.copy_probe_mib:
        import torch
        src = torch.empty(args.copy_probe_mib << 18, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.timeline:
        log("[bench] cfg2 decode timeline: start")
        print(json.dumps({"timeline": timeline_leg(args)}), flush=True)
        return
    if args.grouped_only:
        log("[bench] grouped lines only: start")
        print(json.dumps({"secondary": grouped_leg()}), flush=True)
        return
    if args.extra_only:
        log("[bench] block types, trunk, route and loader only: start")
        print(json.dumps({"types": types_leg(), "trunk": trunk_leg(), "route_loader": route_loader_leg()}), flush=True)
        return
    log("[bench] cfg2 decode stack: start")
    g = gpu_leg(args)
    log(f"[bench] cfg2 decode stack: {g['step_ms']:.4f} ms a token")
    secondary = {"entry_decode": entry_leg(g)}
    if not args.no_cpu:
        log("[bench] CPU baseline: start")
    cpu = None if args.no_cpu else cpu_leg(args, g)
    if not args.no_grouped:
        secondary.update(grouped_leg())
        log("[bench] block types: start")
        secondary["types"] = types_leg()
        log("[bench] trunk: start")
        secondary["trunk"] = trunk_leg()
        log("[bench] route and loader: start")
        secondary["route_loader"] = route_loader_leg()
    value = args.steps / g["secs"]
    dom = g["timing"][g["dom"]]
    achieved = dom["bytes"] / (dom["us"] * 1e-6)
    out = {
        "metric": "MoE-layer tokens/s (decode, batch 1, 48-layer stack)",
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: Gaussian weights quantized to GGUF Q4_0 on the device (seed 0), fresh N(0,1) fp16 "
                "activations each step",
        "config": {"workload": "cfg2: batch-1 decode through a stack of MoE layers", "layers": args.layers,
                   "hidden": g["cfg"]["H"], "experts": g["cfg"]["E"], "top_k": g["cfg"]["k"],
                   "intermediate": g["cfg"]["I"], "weights": "Q4_0", "renorm": True, "parallelism": "none"},
        "step_hbm_gbps": round(g["token_bytes"] / (g["step_ms"] * 1e-3) / 1e9, 1),
        "step_hbm_frac": round(g["token_bytes"] / (g["step_ms"] * 1e-3) / HBM_PEAK, 4),
        "roofline": {"kernel": g["dom"], "bound": "hbm", "achieved": round(achieved / 1e9, 1),
                     "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                     "traffic": MEASURED_TRAFFIC.get(g["dom"]),
                     "traffic_source": "profiles/decode_cfg2_traffic.md (rocprofv3 FETCH_SIZE + WRITE_SIZE)",
                     "bytes_per_launch": dom["bytes"], "us_per_launch": dom["us"]},
        "kernels": g["timing"],
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
