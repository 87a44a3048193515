#!/usr/bin/env python3
"""Benchmark of the routed-MoE layer on one MI355X.

Workload: BASELINE config 1 by default (K3-shape single-token decode:
hidden 7168, 896 resident MXFP4 experts, top-16, FFN 2048, SwiGLU, scale
2.5), seeded synthetic inputs, everything resident in HBM before timing.
A step is one call of k3_moe_forward_bf16 (router -> top-k -> experts ->
combine + residual).

Prints one JSON line. `value` is layer tokens/s (wall clock over exactly
--steps steps, synchronised on both sides). `roofline` is for the dominant
kernel (decode gate/up for T = 1, timed live with HIP events recorded
around its stage); `cpu_baseline` is the C oracle of the same layer timed
on this host's cores on a bounded token sample. For one token, `graph`
adds the same steps replayed from a HIP graph (a serving loop's form; no
host launch cost between kernels) -- reported beside `value`, not as it.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0
MXFP4_PEAK_TFLOPS = 10066.0  # dense MXFP4 MFMA (vendor figure)
FP8_PEAK_TFLOPS = 5033.0
BF16_PEAK_TFLOPS = 2516.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Hip:
    """Just enough of the HIP runtime for events (libamdhip64)."""

    def __init__(self):
        self.h = ctypes.CDLL("libamdhip64.so")
        self.h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                               ctypes.c_void_p]
        self.h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.h.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def event(self):
        e = ctypes.c_void_p()
        assert self.h.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def elapsed_ms(self, a, b):
        f = ctypes.c_float()
        assert self.h.hipEventElapsedTime(ctypes.byref(f), a, b) == 0
        return f.value


def graph_ms_per_step(torch, call, R, steps):
    """The same steps replayed from a HIP graph: R consecutive calls (one per
    input rotation) captured once on a side stream, replayed ceil(steps / R)
    times, wall clock per step. call(i, stream_handle) enqueues step i."""
    s = torch.cuda.Stream()  # default priority
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        call(0, s.cuda_stream)
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            for i in range(R):
                call(i, s.cuda_stream)
    torch.cuda.synchronize()
    reps = max(1, -(-steps // R))
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / (reps * R) * 1e3
    del g
    return ms


def algorithmic_bytes(cfg, T, unique):
    """Bytes the layer must move: each selected expert once, the router,
    the bias, hidden/residual/output rows and the routes."""
    per_expert = 3 * (cfg.ffn * cfg.hidden // 2 + cfg.ffn * cfg.hidden // 32)
    return (unique * per_expert + cfg.experts * cfg.hidden * 2 + 4 * cfg.experts +
            3 * T * cfg.hidden * 2 + T * cfg.top_k * 8)


def gate_up_bytes(cfg, T, unique):
    """Bytes of the gate/up stage: gate and up tensors of each selected
    expert, the hidden rows, the routes and the bf16 activations written."""
    per = 2 * (cfg.ffn * cfg.hidden // 2 + cfg.ffn * cfg.hidden // 32)
    return unique * per + T * cfg.hidden * 2 + T * cfg.top_k * (4 + 2 * cfg.ffn)


def recorded_traffic(workload, T, precision):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE, each scaled by what
    the same counter reads for a plain copy of known size), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "pmc_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(f"{workload}/T{T}/p{precision}")
    except (OSError, ValueError):
        return None
    return rec["bytes"] if rec else None


def cpu_threads():
    """Every core this process may run on (sched_getaffinity)."""
    return len(os.sched_getaffinity(0))


def cpu_baseline(cfg, inputs_cpu, store, budget_s, threads, full_tokens):
    """The C oracle of the same layer (router, top-k, every route's MXFP4
    gate/up/down and activation, combine, residual) on this host's cores,
    OpenMP over (route, 64-row block) work items, token by token through a
    bounded sample of the workload's own tokens. Returns tok/s; for a
    batch larger than the sample the figure is extrapolated (the port does
    the same work per token at any batch size: it reuses no weights)."""
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests"))
    import _oracle as O  # CPU checker / baseline only
    logits = O.router_logits(inputs_cpu.router_weight, inputs_cpu.hidden)
    ids, _ = O.router_topk(logits, inputs_cpu.router_bias, cfg.top_k, cfg.scale)
    T = inputs_cpu.hidden.shape[0]
    experts = {}
    t0 = time.perf_counter()
    for e in np.unique(ids):
        experts[int(e)] = [t.cpu().numpy() for t in store.device_expert(int(e))]
    copy_s = time.perf_counter() - t0
    O.layer(cfg, inputs_cpu, experts, tokens=[0], threads=threads)  # warm-up
    t0 = time.perf_counter()
    n = 0
    while n < T:
        O.layer(cfg, inputs_cpu, experts, tokens=[n], threads=threads)
        n += 1
        if n % 64 == 0:
            log(f"bench: CPU baseline {n}/{T} tokens, {time.perf_counter() - t0:.0f} s")
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    rate = n / dt
    extrap = full_tokens > n
    return {"value": rate, "unit": "tok/s", "cores": threads, "kind": "port",
            "extrapolated": extrap,
            "sample": f"{n} token(s) of {cfg.name} through the C oracle (router, top-k, "
                      f"{cfg.top_k} MXFP4 experts, activation, combine, residual), OpenMP over "
                      f"(route, 64-row block) on {threads} cores; {dt:.1f} s"
                      + (f"; the full {full_tokens}-token batch extrapolates to "
                         f"{full_tokens / rate:.0f} s" if extrap else "")
                      + f" (+{copy_s:.1f} s copying {len(experts)} experts to the host, untimed)"}


def run_native(args):
    """The K3-native layer (router, Q8-128 latent projection, experts on the
    latent, RMSNorm, up projection, SiTU shared expert, adds) at T tokens."""
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from moonshine_amd import native as N
    from moonshine_amd._lib import lib
    from moonshine_amd.synth import f32_to_bf16_bits

    cfg = N.K3_NATIVE_LAYER
    T = args.tokens or cfg.tokens
    R = args.rotate or (16 if T == 1 else 1)
    log(f"bench: {cfg.name} T={T} building weights and resident expert store ...")
    layer = N.NativeLayer(cfg, device="cuda")
    rng = np.random.default_rng(cfg.seed + 1)
    xs = torch.from_numpy(f32_to_bf16_bits(rng.normal(0, 1, (R, T, cfg.hidden)).astype(
        np.float32)).view(np.int16)).cuda()
    rs = torch.from_numpy(f32_to_bf16_bits(rng.normal(0, 1, (R, T, cfg.hidden)).astype(
        np.float32)).view(np.int16)).cuda()
    out = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
    ids = torch.zeros((T, cfg.top_k), dtype=torch.int32, device="cuda")
    wts = torch.zeros((T, cfg.top_k), dtype=torch.float32, device="cuda")
    ws = layer.workspace(T)
    stream = torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()  # default priority, like every stream here
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    argvs = [[P(out), P(xs[i]), P(rs[i]), ctypes.byref(layer.weights), ctypes.byref(layer.shape),
              T, args.precision, P(ids), P(wts), P(ws), ws.numel()] for i in range(R)]

    def call(i, st, streams):
        shared = ctypes.c_void_p(side.cuda_stream) if streams == 2 else None
        if not lib().k3_moe_native_forward_bf16(*argvs[i % R], ctypes.c_void_p(st), shared):
            raise RuntimeError("k3_moe_native_forward_bf16 failed")

    def step(i):
        call(i, stream, args.streams)

    unique_per_batch = []
    for i in range(max(args.warmup, R)):
        step(i)
        if i < R:
            torch.cuda.synchronize()
            unique_per_batch.append(int(np.unique(ids.cpu().numpy()).size))
    torch.cuda.synchronize()
    log(f"bench: timing {args.steps} steps ...")
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    unique = float(np.mean([unique_per_batch[i % R] for i in range(args.steps)]))
    per_expert = 3 * (cfg.ffn * cfg.latent // 2 + cfg.ffn * cfg.latent // 32)
    nbytes = (unique * per_expert + layer.static_bytes() + cfg.experts * cfg.hidden * 2 +
              4 * cfg.experts + 2 * cfg.latent + 3 * T * cfg.hidden * 2 + T * cfg.top_k * 8)
    gbps = nbytes / (ms * 1e-3) / 1e9
    result = {
        "metric": "K3-native MoE layer tok/s (HBM GB/s)",
        "value": T / (ms * 1e-3), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4 experts, q8-128 static projections, bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded; resident in HBM)",
        "config": {"workload": cfg.name, "tokens": T, "hidden": cfg.hidden,
                   "latent": cfg.latent, "experts": cfg.experts, "top_k": cfg.top_k,
                   "ffn": cfg.ffn, "shared": cfg.shared, "activation": "situ",
                   "scale": cfg.scale, "static": "q8_128", "streams": args.streams,
                   "precision": ["exact", "mx8", "mx8-1term"][args.precision],
                   "unique_experts": unique, "distinct_batches": R},
        "roofline": {"kernel": "whole layer", "bound": "hbm", "achieved": gbps,
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": gbps / HBM_PEAK_GBPS,
                     "traffic": None, "algorithmic_bytes": nbytes, "avg_ms": ms},
    }
    if not args.no_graph:
        log("bench: the same steps replayed from a HIP graph ...")
        gms = graph_ms_per_step(torch, lambda i, st: call(i, st, args.streams), R, args.steps)
        result["graph"] = {"streams": args.streams, "ms_per_step": gms,
                           "value": T / (gms * 1e-3), "hbm_gbps": nbytes / (gms * 1e-3) / 1e9}
    if not args.no_cpu_baseline and T == 1:
        log("bench: CPU baseline (composed C oracle) ...")
        sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests"))
        import _oracle as O  # CPU baseline only
        statics = {n: w.host() for n, w in layer.statics().items()}
        x0 = xs[0].cpu().numpy().view(np.uint16)
        r0 = rs[0].cpu().numpy().view(np.uint16)
        logits = O.router_logits(layer.router_weight_bits, x0)
        sel, _ = O.router_topk(logits, layer.router_bias, cfg.top_k, cfg.scale)
        experts = {int(e): layer.store.host_expert(int(e)) for e in np.unique(sel)}
        threads = cpu_threads()
        n, t0 = 0, time.perf_counter()
        while n == 0 or time.perf_counter() - t0 < args.cpu_budget:
            O.native_layer(cfg, layer.router_weight_bits, layer.router_bias, layer.norm_bits,
                           statics, x0, r0, experts)
            n += 1
        dt = time.perf_counter() - t0
        result["cpu_baseline"] = {
            "value": n / dt, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} run(s) of one {cfg.name} token through the composed C oracle "
                      f"(OpenMP in the projections and experts); {dt:.1f} s"}
    print(json.dumps(result), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, help="BASELINE.json config index")
    ap.add_argument("--tokens", type=int, default=0, help="override token count")
    ap.add_argument("--precision", type=int, default=0, help="0 exact, 1 mx8")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--rotate", type=int, default=0,
                    help="distinct token batches cycled through the steps (default: 16 for "
                         "T = 1, so consecutive steps route to different experts and no step "
                         "finds its weights in the 256 MB last-level cache; 1 for T > 1)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true",
                    help="with the default config 1: skip the batched/prefill lines (configs "
                         "2-4 on the MFMA path, `prefill` in the JSON line)")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--prefill-cpu-budget", type=float, default=6.0)
    ap.add_argument("--native", action="store_true",
                    help="the K3-native layer (Q8-128 static projections around the routed "
                         "experts, shared expert) instead of a BASELINE config")
    ap.add_argument("--streams", type=int, default=1, choices=(1, 2),
                    help="--native: 2 runs the latent projection and the shared expert's gate/up "
                         "on a second stream (host-bound when not in a graph)")
    ap.add_argument("--misalign", action="store_true",
                    help="start the odd experts' tensors 8 bytes past a 16-byte boundary, as "
                         "about a quarter of a real checkpoint's tensors do")
    ap.add_argument("--cpu-full", action="store_true",
                    help="run the CPU baseline over every token of the batch (no time budget, "
                         "no extrapolation; config 3 takes ~3 minutes)")
    ap.add_argument("--no-graph", action="store_true",
                    help="skip the extra HIP-graph replay figure (`graph` in the JSON line)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB, --steps times (the known-size "
                         "kernel that scales FETCH_SIZE/WRITE_SIZE counter readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X; "
              "the layer would shard by tensor-parallel F slices (each GPU holding F / N "
              "rows of every expert)", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": args.steps}), flush=True)
        return

    if args.native:
        run_native(args)
        return

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from moonshine_amd.synth import CONFIGS

    cfg = CONFIGS[args.config]
    T = args.tokens or cfg.tokens
    result = run_layer(args, cfg, T, args.precision, args.steps, args.warmup,
                       args.rotate or (16 if T == 1 else 1), not args.no_cpu_baseline)
    if not args.no_prefill and args.config == 1 and not args.tokens:
        # the metric's other halves: batched decode, 512 and 8K prefill on
        # the grouped scaled-MFMA path (two-term MXFP8 activations)
        result["prefill"] = {}
        for ci in (2, 3, 4):
            pc = CONFIGS[ci]
            # the CPU baseline runs config 2's whole 64-token batch (~20 s);
            # the larger batches are sampled and labelled extrapolated
            budget = max(args.prefill_cpu_budget, 40.0) if ci == 2 else args.prefill_cpu_budget
            r = run_layer(args, pc, pc.tokens, 1, args.prefill_steps, min(args.warmup, 3), 1,
                          not args.no_cpu_baseline, cpu_budget=budget)
            keep = ("value", "unit", "ms_per_step", "config", "layer", "roofline",
                    "cpu_baseline")
            result["prefill"][pc.name] = {k: r[k] for k in keep if k in r}
            result["prefill"][pc.name]["steps"] = args.prefill_steps
    print(json.dumps(result), flush=True)


def run_layer(args, cfg, T, precision, steps, warmup, R, with_cpu, cpu_budget=None):
    """k3_moe_forward_bf16 on one configuration: a fresh resident expert
    store, R distinct token batches cycled through the steps, `steps`
    timed calls (wall clock, synchronised on both sides), then the same
    steps again with HIP events at the stage boundaries."""
    import torch
    from moonshine_amd import layer as L
    from moonshine_amd._lib import STAGES, K3MoeProfile, lib
    from moonshine_amd.synth import make_inputs

    log(f"bench: {cfg.name} T={T} building resident expert store ...")
    torch.cuda.empty_cache()
    inputs = make_inputs(cfg, tokens=T * R)
    store = None
    if getattr(args, "misalign", False):  # odd experts' tensors at 8 mod 16
        store = L.ExpertStore(cfg.experts, cfg.hidden, cfg.ffn, seed=cfg.seed, device="cuda",
                              misalign=8, misalign_odd=True)
    moe = L.build_layer(cfg, inputs, device="cuda", store=store)
    xs = L.bf16_tensor(inputs.hidden).view(R, T, cfg.hidden)
    rs = L.bf16_tensor(inputs.residual).view(R, T, cfg.hidden)
    out = torch.empty((T, cfg.hidden), dtype=xs.dtype, device=xs.device)
    ids = torch.zeros((T, cfg.top_k), dtype=torch.int32, device="cuda")
    wts = torch.zeros((T, cfg.top_k), dtype=torch.float32, device="cuda")
    ws = moe.workspace(T)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    hip = Hip()
    profiles = [K3MoeProfile() for _ in range(steps)]
    for p in profiles:
        for i in range(len(STAGES)):
            p.stage_events[i] = hip.event().value
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    argvs = [[P(out), P(xs[i]), P(rs[i]), P(moe.router_weight), P(moe.router_bias),
              P(moe.store.table), ctypes.byref(moe.shape), T, precision, P(ids), P(wts),
              P(ws), ws.numel()] for i in range(R)]
    unique_per_batch = []

    def step(i, profile):
        if not lib().k3_moe_forward_profiled_bf16(*argvs[i % R], profile,
                                                  ctypes.c_void_p(stream)):
            raise RuntimeError("k3_moe_forward_profiled_bf16 failed")

    log(f"bench: warmup {warmup} ({R} distinct token batches) ...")
    for i in range(max(warmup, R)):
        step(i, None)
        if i < R:
            torch.cuda.synchronize()
            unique_per_batch.append(int(np.unique(ids.cpu().numpy()).size))
    torch.cuda.synchronize()
    log(f"bench: timing {steps} steps ...")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i, None)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / steps * 1e3
    # second pass: the same steps with HIP events at the stage boundaries
    # (each event record adds a few microseconds, so this pass only
    # apportions time; `value` comes from the event-free pass above)
    log(f"bench: {steps} profiled steps ...")
    for i in range(steps):
        step(i, ctypes.byref(profiles[i]))
    torch.cuda.synchronize()

    graph = None
    if not args.no_graph and T == 1:
        log("bench: the same steps replayed from a HIP graph ...")

        def gcall(i, st):
            if not lib().k3_moe_forward_profiled_bf16(*argvs[i % R], None, ctypes.c_void_p(st)):
                raise RuntimeError("k3_moe_forward_profiled_bf16 failed")
        gms = graph_ms_per_step(torch, gcall, R, steps)
        graph = {"ms_per_step": gms, "value": T / (gms * 1e-3)}

    stage_ms = {s: 0.0 for s in STAGES[:-1]}
    gpu_ms = 0.0
    for p in profiles:
        ev = list(p.stage_events)
        for i, s in enumerate(STAGES[:-1]):
            stage_ms[s] += hip.elapsed_ms(ev[i], ev[i + 1]) / steps
        gpu_ms += hip.elapsed_ms(ev[0], ev[-1]) / steps

    # steps cycle through the R batches: the mean over them is each step's work
    unique = float(np.mean([unique_per_batch[i % R] for i in range(steps)]))
    total_bytes = algorithmic_bytes(cfg, T, unique)
    flops = T * cfg.top_k * 2 * 3 * cfg.ffn * cfg.hidden
    kms = stage_ms["gate_up"]
    layer_gbps = total_bytes / (ms_per_step * 1e-3) / 1e9
    traffic = recorded_traffic(cfg.name, T, precision)
    if T == 1:
        # The stage events bracket the gate/up launch, but every event record
        # adds time to the stream's timeline. The event-free pass above runs
        # the same five kernels back to back (no gaps in a trace), so its
        # step time is the sum of their durations; the events' cost per
        # kernel stage is then (sum of the five kernel stages - that step
        # time) / 5, measured live, and the kernel-only time is the gate/up
        # stage minus it. (The plan stage launches nothing at T = 1; its
        # two back-to-back events are reported as event_gap_ms.)
        kstages = ("router", "topk", "gate_up", "down", "combine")
        overhead = max(0.0, (sum(stage_ms[k] for k in kstages) - ms_per_step) / len(kstages))
        kbytes = gate_up_bytes(cfg, T, unique)
        kernel_ms = kms - overhead
        achieved = kbytes / (kernel_ms * 1e-3) / 1e9
        roofline = {"kernel": "gateup_kernel", "bound": "hbm", "achieved": achieved,
                    "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBPS,
                    "traffic": traffic, "algorithmic_bytes": kbytes, "avg_ms": kernel_ms,
                    "stage_ms_events": kms, "event_overhead_ms": overhead,
                    "event_gap_ms": stage_ms["plan"],
                    "frac_event_stage": kbytes / (kms * 1e-3) / 1e9 / HBM_PEAK_GBPS}
    else:
        # grouped gate/up on scaled MFMA (every tile-class launch of the
        # stage). The bound is whichever ideal time of the stage is longer:
        # its bytes at the HBM peak, or the instruction stream actually
        # issued (terms x the useful flops) at the fp8 MFMA rate. Batched
        # decode and 512-token prefill are HBM-bound (few rows per expert);
        # 8K prefill is MFMA-bound.
        kflops = T * cfg.top_k * 2 * 2 * cfg.ffn * cfg.hidden
        kbytes = gate_up_bytes(cfg, T, unique)
        terms = 2 if precision == 1 else 1
        t_hbm = kbytes / (HBM_PEAK_GBPS * 1e9)
        t_mfma = kflops * terms / (FP8_PEAK_TFLOPS * 1e12)
        tflops = kflops / (kms * 1e-3) / 1e12
        gbps = kbytes / (kms * 1e-3) / 1e9
        common = {"kernel": "gateup_mfma*_kernel (every tile-class launch)",
                  "traffic": traffic, "algorithmic_flops": kflops, "algorithmic_bytes": kbytes,
                  "avg_ms": kms, "mfma_terms": terms,
                  "ideal_ms": {"hbm": t_hbm * 1e3, "mfma_fp8_rate": t_mfma * 1e3},
                  "tflops": tflops, "mxfp4_frac": tflops / MXFP4_PEAK_TFLOPS,
                  "fp8_instr_frac": tflops * terms / FP8_PEAK_TFLOPS,
                  "hbm_gbps": gbps, "hbm_frac": gbps / HBM_PEAK_GBPS}
        if precision == 0 or t_mfma > t_hbm:
            roofline = {"bound": "mfma", "achieved": tflops, "peak": MXFP4_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": tflops / MXFP4_PEAK_TFLOPS, **common}
        else:
            roofline = {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS,
                        "unit": "GB/s", "frac": gbps / HBM_PEAK_GBPS, **common}
    result = {
        "metric": "routed-MoE layer tok/s; decode HBM GB/s; 8K-prefill MXFP4 TFLOP/s",
        "value": T / (ms_per_step * 1e-3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4 weights, bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded; experts from a counter-based generator, resident in HBM)",
        "config": {"workload": cfg.name, "tokens": T, "hidden": cfg.hidden,
                   "experts": cfg.experts, "top_k": cfg.top_k, "ffn": cfg.ffn,
                   "activation": "swiglu" if cfg.activation == 1 else "situ",
                   "scale": cfg.scale, "precision": ["exact", "mx8", "mx8-1term"][precision],
                   "unique_experts": unique, "distinct_batches": R},
        "layer": {"bytes": total_bytes, "hbm_gbps": layer_gbps,
                  "hbm_frac": layer_gbps / HBM_PEAK_GBPS,
                  "tflops": flops / (ms_per_step * 1e-3) / 1e12,
                  "mxfp4_frac": flops / (ms_per_step * 1e-3) / 1e12 / MXFP4_PEAK_TFLOPS,
                  "gpu_ms_events": gpu_ms, "stage_ms": stage_ms},
        "roofline": roofline,
    }
    if graph:
        result["graph"] = graph
    if with_cpu:
        log(f"bench: CPU baseline (C oracle) for {cfg.name} ...")
        # a bounded sample of the same workload: its first tokens (for T = 1
        # the rotated decode tokens), each run through the oracle layer
        full = getattr(args, "cpu_full", False) and T > 1
        cpu_inputs = make_inputs(cfg, tokens=T if full else (min(64, max(T * R, 1)) if T > 1 else R))
        result["cpu_baseline"] = cpu_baseline(
            cfg, cpu_inputs, moe.store, float("inf") if full else (cpu_budget or args.cpu_budget),
            cpu_threads(), T)
    del moe, xs, rs, out, ws
    return result


if __name__ == "__main__":
    main()
