#!/usr/bin/env python3
"""Benchmark of the decode-time fused MoE layer on one MI355X.

Workload: one Mixtral-8x7B-shape MoE layer at batch
1 -- h=4096, I=14336, E=8, top-2 with renormalised weights, fp16 expert
weights, fp32 gating and accumulation, x ~ N(0,1) fp32.  A "step" is one call
of the fused layer (warp_route.functional.fused_moe) on inputs already
resident in HBM.  Layers rotate over --layers independent random layers
(default 4, 11.3 GB) so that the 256 MB Infinity Cache holds no reuse between
calls.

Prints one JSON line: value = microseconds per layer (lower is better),
roofline = selected-expert weight bytes / the FFN kernel's average duration
(HIP events around k_fused_ffn alone, through the C-ABI's split entry points)
against 8 TB/s HBM3E, with the whole layer's rate beside it,
cpu_baseline = the reference's pure-torch MoE (fp32, host cores) timed on a
bounded sample of the same layer.

  python bench.py [--steps K] [--warmup W] [--layers L] [--config mixtral]
  python bench.py --weights fp8    # the same layers in bf16 or fp8 E4M3 (not the headline)
  python bench.py --copy-probe     # plain device copy, for counter calibration
  python bench.py --op naive       # the naive multi-kernel path, with fused beside it
  python bench.py --read-probe     # read-only streaming ceiling over the same bytes
  python bench.py --throughput     # batched vs a loop of single-token calls (Mixtral, DBRX)
  python bench.py --timeline 20    # per-phase timeline of the single-token kernel; needs
                                   # WR_HIPCC_FLAGS=-DWR_TIMELINE=1 python warp-route_amd/build.py

The headline line also carries roofline.read_ceiling: the best rate of a
plain read-only streaming kernel (libwr_probe.so) over exactly the selected
experts' bytes of the same rotated layers, measured in the same run, so the
kernel's rate can be read against what the chip streams, not only against
the 8 TB/s peak.

Two further workloads of BASELINE.json configs[4] print their own JSON line
(not the headline): --batch B[,B...] times batched_fused_moe on clustered
Mixtral batches; --stack N [--graph] times one decode step through N
independent Mixtral layers chained with residual adds (end-to-end MoE time
per token), launched op by op and, with --graph, from one captured HIP graph.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "warp-route_amd")]

HBM_PEAK_GBPS = 8000.0
METRIC = ("µs per MoE layer at batch=1 (Mixtral shape); "
          "achieved HBM GB/s as % of peak")


WLABEL = {"fp16": "f16", "bf16": "bf16", "fp8": "fp8 e4m3 (per-row fp32 scales)",
          "mxfp4": "mxfp4 (e2m1, e8m0 scale per 32)", "fp32": "f32"}


def weight_dtype(name: str):
    """torch dtype of a --weights choice."""
    import torch
    return {"fp16": torch.float16, "bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn,
            "mxfp4": torch.float4_e2m1fn_x2, "fp32": torch.float32}[name]


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def cpu_baseline(x, gw, buf, cfg, seconds: float):
    """The reference's pure-torch MoE (tests/test_python.py:15-37, plus
    renormalisation) in fp32 on the host, on the same layer: router, softmax,
    top-k and the selected experts' FFN.  Only the selected experts are
    materialised as fp32 host tensors (upcast from the same fp16 weights;
    bf16 and fp8 blocks are decoded, fp8 with its scales)."""
    import torch
    from oracle import moe_oracle as O

    n = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    xc, gwc = x.float().cpu(), gw.float().cpu()
    logits = gwc @ xc
    sel = torch.topk(torch.softmax(logits, 0), k).indices.tolist()
    fmt = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16",
           torch.float8_e4m3fn: "fp8", torch.float4_e2m1fn_x2: "mxfp4"}[buf.dtype]
    stride = O.weight_layout(E, h, I, fmt)["expert_stride"]
    raw = buf.view(torch.uint8)
    gp, up, dp = [None] * E, [None] * E, [None] * E
    for e in sel:
        blk = raw[e * stride:(e + 1) * stride].cpu().numpy()
        gp[e], up[e], dp[e] = (torch.from_numpy(m).float()
                               for m in O.expert_matrices(blk, 0, E, h, I, fmt))
    for _ in range(2):
        O.torch_moe_reference_cpu(xc, gwc, gp, up, dp, k, cfg.renormalize)
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 1000):
        t0 = time.perf_counter()
        O.torch_moe_reference_cpu(xc, gwc, gp, up, dp, k, cfg.renormalize)
        times.append(time.perf_counter() - t0)
    med_us = statistics.median(times) * 1e6
    fp32_bytes = k * 3 * h * I * 4
    return {
        "value": round(med_us, 1),
        "unit": "us/layer",
        "cores": n,
        "kind": "port",
        "sample": (f"{len(times)} calls of one {cfg.name} layer (batch 1, fp32 torch on the host, "
                   f"median), after 2 warm-ups; {fp32_bytes / med_us / 1e3:.1f} GB/s on the "
                   f"{fp32_bytes / 1e6:.0f} MB of fp32 selected weights; CPU: {cpu_model()}"),
    }


def ffn_kernel_us(layers, cfg, steps: int, warmup: int) -> float:
    """Average duration of the expert-FFN kernel alone (k_fused_ffn): each
    call goes through the C-ABI's two halves of wr_fused_moe, with HIP events
    recorded on the current stream between wr_fused_moe_route and
    wr_fused_moe_ffn and after the latter, so each pair brackets exactly the
    FFN launch."""
    import torch
    from warp_route import capi
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    lib = capi.lib()
    nws = lib.wr_workspace_bytes(capi.WR_KIND_FUSED, E, h, I, k, 1)
    wtag = {torch.float32: capi.WR_F32, torch.float16: capi.WR_F16, torch.bfloat16: capi.WR_BF16,
            torch.float8_e4m3fn: capi.WR_FP8_E4M3, torch.float4_e2m1fn_x2: capi.WR_MXFP4}
    keep, calls = [], []
    for x, gw, buf in layers:
        out = torch.empty_like(x)
        ws = torch.empty(nws, dtype=torch.uint8, device=x.device)
        a = capi.WrMoeArgs()
        a.gate_w, a.weight_buf = gw.data_ptr(), buf.data_ptr()
        a.weight_bytes = buf.numel() * buf.element_size()
        a.weight_dtype = wtag[buf.dtype]
        a.act_dtype = capi.WR_F16 if x.dtype == torch.float16 else capi.WR_F32
        a.num_experts, a.hidden_dim, a.intermediate_dim, a.top_k = E, h, I, k
        a.renormalize, a.batch_size = int(cfg.renormalize), 1
        a.x, a.out = x.data_ptr(), out.data_ptr()
        a.workspace, a.workspace_bytes = ws.data_ptr(), nws
        keep.append((out, ws))
        calls.append(a)
    stream = torch.cuda.current_stream().cuda_stream

    def call(name, a):
        st = capi.call(name, a, stream)
        if st != capi.WR_OK:
            raise RuntimeError(f"{name}: {capi.status_str(st)}")

    for i in range(warmup):
        call("wr_fused_moe", calls[i % len(calls)])
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    torch.cuda.synchronize()
    for i, (e0, e1) in enumerate(evs):
        a = calls[i % len(calls)]
        call("wr_fused_moe_route", a)
        e0.record()
        call("wr_fused_moe_ffn", a)
        e1.record()
    torch.cuda.synchronize()
    return statistics.fmean(e0.elapsed_time(e1) for e0, e1 in evs) * 1e3


TL_EVENTS = 8


def timeline_summary(step, n_calls: int) -> dict:
    """Per-phase timeline of the single-token kernel from its per-workgroup
    records (include/wr_timeline.h; the library must be built with
    WR_HIPCC_FLAGS=-DWR_TIMELINE=1).  Each of n_calls calls (layers rotating
    as in the timed region, each after the previous call's stream drained)
    gives one record set; every figure is in microseconds from the first
    workgroup's start, as the median over the calls of that call's statistic."""
    import ctypes
    import numpy as np
    import torch
    from warp_route import capi
    lib = capi.lib()
    khz = lib.wr_timeline_clock_khz()
    buf = (ctypes.c_uint64 * (65536 * TL_EVENTS))()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows = []
    for i in range(n_calls):
        step(i)
        n = lib.wr_timeline_read(buf, 65536, stream)
        if n == -1:
            raise RuntimeError("the library was built without WR_TIMELINE: rebuild with "
                               "WR_HIPCC_FLAGS=-DWR_TIMELINE=1 python warp-route_amd/build.py")
        if n < 0 or khz <= 0:
            raise RuntimeError(f"wr_timeline_read: {n}, clock {khz} kHz")
        rec = np.frombuffer(buf, dtype=np.uint64, count=n * TL_EVENTS).reshape(n, TL_EVENTS)
        t = rec[:, :5].astype(np.int64)
        t = (t - t[:, 0].min()) / (khz / 1e3)  # microseconds
        gu = rec[:, 6] == 0
        dn = ~gu

        def q(v, p):
            return float(np.percentile(v, p)) if len(v) else float("nan")
        rows.append({
            "gateup_blocks": int(gu.sum()), "down_blocks": int(dn.sum()),
            "gu_start_p50": q(t[gu, 0], 50), "gu_start_max": q(t[gu, 0], 100),
            "gu_selection_p50": q(t[gu, 1] - t[gu, 0], 50),
            "gu_life_p50": q(t[gu, 3] - t[gu, 0], 50),
            # x staged in LDS: the copy and the first weight round landed
            "gu_first_round_p50": q((rec[gu, 2].astype(np.int64) - rec[gu, 0].astype(np.int64))
                                    [rec[gu, 2] > 0] / (khz / 1e3), 50),
            "gu_computed_p50": q((rec[gu, 7].astype(np.int64) - rec[gu, 0].astype(np.int64))
                                 [rec[gu, 7] > 0] / (khz / 1e3), 50),
            "gu_end_p50": q(t[gu, 3], 50),
            "gu_last_arrival": q(t[gu, 3], 100),
            "dn_start_min": q(t[dn, 0], 0), "dn_start_p50": q(t[dn, 0], 50),
            "dn_start_max": q(t[dn, 0], 100),
            "dn_selection_p50": q(t[dn, 1] - t[dn, 0], 50),
            "dn_release_min": q(t[dn, 3], 0), "dn_release_p50": q(t[dn, 3], 50),
            "dn_release_max": q(t[dn, 3], 100),
            "dn_after_release_p50": q(t[dn, 4] - t[dn, 3], 50),
            "dn_after_release_max": q(t[dn, 4] - t[dn, 3], 100),
            "kernel_end": float(max(t[gu, 3].max() if gu.any() else 0.0,
                                    t[dn, 4].max() if dn.any() else 0.0)),
        })
        # Down workgroups by start: per fifth of them in start order, the
        # median start and end relative to the call's median release.
        if dn.sum() >= 5:
            rel = np.median(t[dn, 3])
            order = np.argsort(t[dn, 0])
            for f in range(5):
                sel = order[f * len(order) // 5:(f + 1) * len(order) // 5]
                rows[-1][f"dn_fifth{f}_start_rel_release"] = q(t[dn, 0][sel] - rel, 50)
                rows[-1][f"dn_fifth{f}_end_after_release"] = q(t[dn, 4][sel] - rel, 50)
    import warnings
    with warnings.catch_warnings():  # a phase this kernel variant does not mark is all NaN
        warnings.simplefilter("ignore", RuntimeWarning)
        out = {k: round(float(np.nanmedian([r[k] for r in rows])), 2) for k in rows[0]}
    out = {k: v for k, v in out.items() if v == v}  # phases this kernel variant does not mark
    out["calls"] = n_calls
    out["clock_khz"] = int(khz)
    return out


def _timed(step, steps: int, warmup: int) -> float:
    """Microseconds per call of step(i), K back-to-back calls between two
    events on the current stream, after W untimed calls."""
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        step(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / steps


def batched_bench(args) -> int:
    """Batched decode: Mixtral layers, B tokens whose router logits
    are biased toward one expert pair (synthetic.clustered_batch, alpha = 4),
    through batched_fused_moe.  Bytes = the distinct selected experts' weights
    per call, averaged over the rotated layers."""
    import torch
    from warp_route import functional as F
    from warp_route.synthetic import CONFIGS, clustered_batch, expert_weight_bytes, make_config_layer
    cfg = CONFIGS["mixtral"].with_weights(weight_dtype(args.weights))
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    dev = torch.device("cuda:0")
    layers = [make_config_layer(cfg, seed=s, device=dev, gen_device=dev)
              for s in range(args.layers)]
    for B in [int(v) for v in args.batch.split(",")]:
        xs = [clustered_batch(gw, B, pair=(1, 2), alpha=4.0, seed=s, device=dev)
              for s, (_, gw, _) in enumerate(layers)]
        ids = torch.empty(B, k, dtype=torch.int32, device=dev)
        distinct = []
        for i, (_, gw, buf) in enumerate(layers):
            F.batched_fused_moe(xs[i], gw, buf, E, h, I, k, cfg.renormalize, ids)
            distinct.append(len(set(ids.cpu().numpy().ravel().tolist())))
        L = len(layers)
        us = _timed(lambda i: F.batched_fused_moe(xs[i % L], layers[i % L][1], layers[i % L][2],
                                                  E, h, I, k, cfg.renormalize),
                    args.steps, args.warmup)
        nbytes = sum(distinct) / L * expert_weight_bytes(h, I, cfg.weight_dtype)
        gbps = nbytes / us / 1e3
        print(json.dumps({
            "metric": "µs per batched MoE layer call (Mixtral shape, clustered routing)",
            "value": round(us, 2), "unit": "us/call", "higher_is_better": False,
            "tokens_per_s": round(B / us * 1e6, 1), "us_per_token": round(us / B, 3),
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "dtype": f"{WLABEL[args.weights]} weights, f32 accumulate",
            "data": "synthetic (seeded random-init layers; clustered tokens, alpha 4)",
            "config": {"workload": "mixtral MoE layer, batched decode", "batch": B,
                       "distinct_experts_per_layer": distinct, "layers_rotated": L},
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                         "bytes": f"distinct selected experts' {args.weights} weights"},
        }), flush=True)
    return 0


def throughput_bench(args) -> int:
    """Batched against a loop of single-token calls, as the reference's
    benchmarks/bench_throughput.py:60-118 times them: Mixtral (top-2) and
    DBRX with top-2 (the reference's throughput configs), B in 1..64 (or
    --batch), uniformly random tokens (no clustering), the layers rotated.
    The loop makes B fused_moe calls, one per token of the batch (the
    reference repeats token 0 B times; distinct tokens route like a real
    batch).  One JSON line per model."""
    import torch
    from warp_route import functional as F
    from warp_route.synthetic import CONFIGS, make_config_layer
    sizes = [int(v) for v in args.batch.split(",")] if args.batch else [1, 2, 4, 8, 16, 32, 64]
    dev = torch.device("cuda:0")
    for name in ("mixtral", "dbrx"):
        cfg = dataclasses.replace(CONFIGS[name], top_k=2).with_weights(weight_dtype(args.weights))
        E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
        log(f"[bench] throughput: {args.layers} {name} {args.weights} layers, top-{k}")
        layers = [make_config_layer(cfg, seed=s, batch=max(sizes), device=dev, gen_device=dev)
                  for s in range(args.layers)]
        L = len(layers)
        rows = []
        for B in sizes:
            xs = [x[:B].contiguous() for x, _, _ in layers]
            batched = _timed(lambda i: F.batched_fused_moe(xs[i % L], layers[i % L][1],
                                                           layers[i % L][2], E, h, I, k,
                                                           cfg.renormalize),
                             args.steps, args.warmup)

            def loop(i):
                x, gw, buf = xs[i % L], layers[i % L][1], layers[i % L][2]
                for b in range(B):
                    F.fused_moe(x[b], gw, buf, E, h, I, k, cfg.renormalize)

            iters = max(10, args.steps // B)
            looped = _timed(loop, iters, max(2, args.warmup // B))
            rows.append({"batch": B, "batched_us": round(batched, 2), "loop_us": round(looped, 2),
                         "batched_tok_per_s": round(B / batched * 1e6, 1),
                         "loop_tok_per_s": round(B / looped * 1e6, 1),
                         "us_per_tok_batched": round(batched / B, 3),
                         "us_per_tok_loop": round(looped / B, 3),
                         "speedup": round(looped / batched, 3)})
        print(json.dumps({
            "metric": "batched vs single-token loop, µs per call (benchmarks/bench_throughput.py)",
            "unit": "us/call", "higher_is_better": False, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "dtype": f"{WLABEL[args.weights]} weights, f32 accumulate",
            "data": "synthetic (seeded random-init layers, x ~ N(0, 1), unclustered)",
            "config": {"workload": f"{name} MoE layer, top-{k}", "experts": E, "hidden": h,
                       "intermediate": I, "layers_rotated": L},
            "rows": rows,
        }), flush=True)
        del layers
        torch.cuda.empty_cache()
    return 0


def stack_bench(args) -> int:
    """End-to-end MoE time per token through N independent Mixtral layers
    (configs[4]: 32 layers, 90 GB of fp16 experts), chained with residual adds
    (warp_route.stack.MoEStack): one decode step, launched op by op and, with
    --graph, replayed from one captured HIP graph."""
    import torch
    from warp_route.stack import MoEStack
    from warp_route.synthetic import CONFIGS, make_config_layer
    cfg = CONFIGS["mixtral"]
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    dev = torch.device("cuda:0")
    N = args.stack
    log(f"[bench] generating {N} mixtral layers on the GPU")
    layers, x0 = [], None
    for s in range(N):
        x, gw, buf = make_config_layer(cfg, seed=s, device=dev, gen_device=dev)
        layers.append((gw, buf))
        x0 = x if x0 is None else x0
        if (s + 1) % 8 == 0:
            log(f"[bench]   {s + 1} layers")
    torch.cuda.synchronize()
    weight_gb = sum(buf.numel() * buf.element_size() for _, buf in layers) / 1e9
    stack = MoEStack(layers, E, h, I, k, cfg.renormalize, residual=True)
    steps = max(1, args.steps // N)
    warm = max(1, args.warmup // N)
    us_eager = _timed(lambda i: stack(x0), steps, warm)
    us_graph = None
    if args.graph:
        graphed = stack.capture(x0)
        us_graph = _timed(lambda i: graphed(x0), steps, warm)
    us = us_graph if us_graph is not None else us_eager
    nbytes = N * cfg.selected_bytes
    gbps = nbytes / us / 1e3
    print(json.dumps({
        "metric": f"ms per token through a {N}-layer MoE stack (Mixtral shape, batch 1)",
        "value": round(us / 1e3, 4), "unit": "ms/token", "higher_is_better": False,
        "us_per_layer": round(us / N, 2), "n_gpus": 1, "tokens": steps,
        "eager_ms_per_token": round(us_eager / 1e3, 4),
        "graph_ms_per_token": None if us_graph is None else round(us_graph / 1e3, 4),
        "dtype": "f16 weights, f32 accumulate",
        "data": "synthetic (seeded random-init layers drawn on the GPU)",
        "config": {"workload": f"{N} independent mixtral MoE layers, residual chain",
                   "weights_GB": round(weight_gb, 1), "graph": bool(args.graph)},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4)},
    }), flush=True)
    return 0


def bench_config(args):
    """The layer shape of this run: --config with --weights, and with
    --tp-shard G one GPU's share of a G-way split over I (the same packed
    layout with I' = I / G; the router is replicated, so every shard routes
    as the whole layer does).  Exits with status 2 if G does not divide I
    into whole rows of the format."""
    from warp_route.synthetic import CONFIGS
    cfg = CONFIGS[args.config].with_weights(weight_dtype(args.weights))
    G = args.tp_shard
    if G > 1:
        if cfg.intermediate_dim % G or (args.weights == "mxfp4"
                                        and (cfg.intermediate_dim // G) % 32):
            print(f"--tp-shard {G} does not divide I = {cfg.intermediate_dim} "
                  f"into whole rows for {args.weights}", file=sys.stderr)
            raise SystemExit(2)
        cfg = dataclasses.replace(cfg, intermediate_dim=cfg.intermediate_dim // G,
                                  name=f"{cfg.name}_tp{G}")
    return cfg


def probe_lib():
    """ctypes handle of libwr_probe.so (include/wr_probe.h)."""
    import ctypes
    path = os.path.join(ROOT, "warp-route_amd", "warp_route", "libwr_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (python warp-route_amd/build.py)")
    lib = ctypes.CDLL(path)
    lib.wr_probe_read.argtypes = [ctypes.POINTER(ctypes.c_void_p),
                                  ctypes.POINTER(ctypes.c_int64), ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.wr_probe_read.restype = ctypes.c_int
    lib.wr_probe_gateup.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int,
                                    ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p, ctypes.c_void_p]
    lib.wr_probe_gateup.restype = ctypes.c_int
    lib.wr_probe_down.argtypes = lib.wr_probe_gateup.argtypes
    lib.wr_probe_down.restype = ctypes.c_int
    return lib


# (blocks per CU, loads in flight per lane) tried by read_ceiling: the best
# shapes of a wider sweep (1-8 blocks of 4 waves per CU, 1-8 loads in
# flight) on the Mixtral and DeepSeek selected experts.  24-32 KB in flight
# per CU streams fastest; 64 KB or more per CU is 10-20% slower.
PROBE_SHAPES = [(6, 1), (8, 1), (3, 2), (4, 2), (2, 4), (1, 8)]
# --probe-sweep: the wider sweep those came from
PROBE_SWEEP = [(1, 1), (1, 2), (1, 4), (1, 8), (2, 1), (2, 2), (2, 4), (2, 8), (3, 2), (3, 4),
               (4, 1), (4, 2), (4, 4), (6, 1), (8, 1)]


def read_ceiling(range_sets, steps: int, warmup: int = 5, shapes=None) -> dict:
    """Best rate of the read-only streaming probe over range_sets (one list
    of (ptr, bytes) per rotated layer, read in one launch per call, rotating),
    over `shapes` (default PROBE_SHAPES): the achievable HBM read bandwidth
    for these bytes."""
    import ctypes
    import torch
    lib = probe_lib()
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    calls = []
    for rs in range_sets:
        ptrs = (ctypes.c_void_p * len(rs))(*[p for p, _ in rs])
        nb = (ctypes.c_int64 * len(rs))(*[n for _, n in rs])
        calls.append((ptrs, nb, len(rs), sum(n for _, n in rs)))
    results = []
    for bpc, unroll in (shapes or PROBE_SHAPES):
        def step(i):
            ptrs, nb, n, _ = calls[i % len(calls)]
            if lib.wr_probe_read(ptrs, nb, n, bpc, unroll, ctypes.c_void_p(sink.data_ptr()),
                                 ctypes.c_void_p(stream)) != 0:
                raise RuntimeError("wr_probe_read failed")
        us = _timed(step, steps, warmup)
        nbytes = sum(c[3] for c in calls) / len(calls)
        results.append({"blocks_per_cu": bpc, "loads_in_flight": unroll,
                        "us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1)})
    best = max(results, key=lambda r: r["GBps"])
    return {"GBps": best["GBps"], "us": best["us"], "shape": [best["blocks_per_cu"],
                                                              best["loads_in_flight"]],
            "bytes_per_call": int(sum(c[3] for c in calls) / len(calls)), "sweep": results}


def selected_ranges(layers, cfg):
    """Per layer, the (device pointer, bytes) of each selected expert's
    weights (its three matrices and, for fp8 / MXFP4, their scales: the
    algorithmic bytes), rounded down to 16 bytes."""
    from warp_route import functional as F
    from warp_route.synthetic import expert_weight_bytes
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    stride = F.weight_layout(E, h, I, cfg.weight_dtype)["expert_stride"]
    nb = expert_weight_bytes(h, I, cfg.weight_dtype) // 16 * 16
    out = []
    for x, gw, buf in layers:
        ids, _ = F.gate_topk(x, gw, E, h, k, cfg.renormalize)
        out.append([(buf.data_ptr() + int(e) * stride, nb) for e in ids.tolist()])
    return out


def read_probe_bench(args) -> int:
    """The read-only streaming ceiling: the probe over the selected experts'
    bytes of the rotated layers (what one MoE call must read), and over one
    contiguous 1 GiB buffer."""
    import torch
    from warp_route.synthetic import make_config_layer
    cfg = bench_config(args)
    dev = torch.device("cuda:0")
    layers = [make_config_layer(cfg, seed=s, device=dev, gen_device=dev)
              for s in range(args.layers)]
    shapes = PROBE_SWEEP if args.probe_sweep else None
    sel = read_ceiling(selected_ranges(layers, cfg), args.steps, shapes=shapes)
    flat = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    big = read_ceiling([[(flat.data_ptr(), flat.numel())]], max(20, args.steps // 10),
                       shapes=shapes)
    print(json.dumps({
        "metric": "read-only HBM streaming ceiling (GB/s)", "value": sel["GBps"],
        "unit": "GB/s", "higher_is_better": True, "n_gpus": 1, "steps": args.steps,
        "config": {"workload": f"{cfg.name} selected experts ({args.weights}), "
                               f"{args.layers} layers rotated",
                   "bytes_per_call": sel["bytes_per_call"]},
        "selected_experts": sel, "contiguous_1GiB": big,
        "peak_GBps": HBM_PEAK_GBPS, "frac_of_peak": round(sel["GBps"] / HBM_PEAK_GBPS, 4),
    }), flush=True)
    return 0


def gateup_probe_bench(args) -> int:
    """The gate/up phase's read order against the streaming ceiling: over the
    gate and up matrices of the selected experts of the rotated layers (16-bit
    weights), the read-only probe in the single-token kernel's slot order
    (one workgroup per 8-row slot, as that kernel launches them, and the same
    slots looped over by 4 workgroups per CU), in a workgroup-level grid
    stride over 4-row groups, and the grid-stride streaming ceiling
    (wr_probe_read) over the same bytes."""
    import ctypes
    import torch
    from warp_route import functional as F
    from warp_route.synthetic import make_config_layer
    cfg = bench_config(args)
    if cfg.weight_dtype not in (torch.float16, torch.bfloat16):
        raise SystemExit("--gateup-probe takes 16-bit weights")
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    row_bytes = 2 * h
    dev = torch.device("cuda:0")
    layers = [make_config_layer(cfg, seed=s, device=dev, gen_device=dev)
              for s in range(args.layers)]
    stride = F.weight_layout(E, h, I, cfg.weight_dtype)["expert_stride"]
    bases = []
    for x, gw, buf in layers:
        ids, _ = F.gate_topk(x, gw, E, h, k, cfg.renormalize)
        bases.append([buf.data_ptr() + int(e) * stride for e in ids.tolist()])
    nbytes = k * 2 * I * row_bytes
    lib = probe_lib()
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    arrs = [(ctypes.c_void_p * k)(*b) for b in bases]
    rows = []
    for name, pattern, blocks in [("kernel slots, one workgroup per slot", 0, k * I // 8),
                                  ("kernel slots, 4 workgroups per CU looping", 0, 4 * cus),
                                  ("4-row groups, workgroup grid stride", 1, 4 * cus),
                                  ("4-row groups, workgroup grid stride", 1, 3 * cus)]:
        def step(i, pattern=pattern, blocks=blocks):
            if lib.wr_probe_gateup(arrs[i % len(arrs)], k, row_bytes, I, pattern, blocks,
                                   ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(stream)) != 0:
                raise RuntimeError("wr_probe_gateup failed")
        us = _timed(step, args.steps, 10)
        rows.append({"order": name, "workgroups": blocks, "us": round(us, 2),
                     "GBps": round(nbytes / us / 1e3, 1)})
    ceil = read_ceiling([[(b, 2 * I * row_bytes) for b in bs] for bs in bases], args.steps)
    # The down matrices (h rows of I weights each, after gate and up), in the
    # kernel's down order (4-row groups, one workgroup per group as launched)
    # and row-contiguous, against the ceiling over the same bytes.
    dn_row = 2 * I
    dn_bases = [[b + 2 * I * row_bytes for b in bs] for bs in bases]
    dn_arrs = [(ctypes.c_void_p * k)(*b) for b in dn_bases]
    dn_bytes = k * h * dn_row
    dn_rows = []
    for name, pattern, blocks in [("kernel down order, one workgroup per 4 rows", 0, h // 4),
                                  ("row-contiguous, one workgroup per 4 rows", 1, h // 4)]:
        def dstep(i, pattern=pattern, blocks=blocks):
            if lib.wr_probe_down(dn_arrs[i % len(dn_arrs)], k, dn_row, h, pattern, blocks,
                                 ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(stream)) != 0:
                raise RuntimeError("wr_probe_down failed")
        us = _timed(dstep, args.steps, 10)
        dn_rows.append({"order": name, "workgroups": blocks, "us": round(us, 2),
                        "GBps": round(dn_bytes / us / 1e3, 1)})
    dn_ceil = read_ceiling([[(b, h * dn_row) for b in bs] for bs in dn_bases], args.steps)
    print(json.dumps({
        "metric": "read-only rate of gate/up read orders (GB/s)", "unit": "GB/s",
        "config": {"workload": f"{cfg.name} gate and up matrices of the selected experts "
                               f"({args.weights}), {args.layers} layers rotated",
                   "bytes_per_call": nbytes, "steps": args.steps},
        "orders": rows,
        "grid_stride_ceiling": {k2: ceil[k2] for k2 in ("GBps", "us", "shape")},
        "down": {"bytes_per_call": dn_bytes, "orders": dn_rows,
                 "grid_stride_ceiling": {k2: dn_ceil[k2] for k2 in ("GBps", "us", "shape")}},
    }), flush=True)
    return 0


def naive_bench(args) -> int:
    """The naive multi-kernel path (warp_route.functional.naive_moe: router,
    host softmax / top-K after one stream synchronisation, then per selected
    expert gate, up, SwiGLU, down and weighted-accumulate launches) on the
    headline layers, with the fused op timed on the same layers beside it:
    the comparison of benchmarks/bench_latency.cu:83-122 in the reference."""
    import torch
    from warp_route import functional as F
    from warp_route.synthetic import make_config_layer
    cfg = bench_config(args)
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    dev = torch.device("cuda:0")
    layers = [make_config_layer(cfg, seed=s, device=dev, gen_device=dev)
              for s in range(args.layers)]
    L = len(layers)
    steps = max(10, args.steps // 4)  # each naive call synchronises the stream once

    def naive(i):
        x, gw, buf = layers[i % L]
        return F.naive_moe(x, gw, buf, E, h, I, k, cfg.renormalize)

    def fused(i):
        x, gw, buf = layers[i % L]
        return F.fused_moe(x, gw, buf, E, h, I, k, cfg.renormalize)

    us_naive = _timed(naive, steps, args.warmup)
    us_fused = _timed(fused, args.steps, args.warmup)
    nbytes = cfg.selected_bytes
    print(json.dumps({
        "metric": f"µs per MoE layer at batch=1 ({cfg.name} shape), naive multi-kernel path",
        "value": round(us_naive, 2), "unit": "us/layer", "higher_is_better": False,
        "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "dtype": WLABEL[args.weights] + " weights, f32 accumulate",
        "data": "synthetic (seeded random-init layers drawn on the GPU)",
        "config": {"workload": f"{cfg.name} MoE layer, decode batch 1, naive op",
                   "launches_per_call": 3 + 5 * k, "layers_rotated": L},
        "naive_GBps": round(nbytes / us_naive / 1e3, 1),
        "fused_us": round(us_fused, 2), "fused_GBps": round(nbytes / us_fused / 1e3, 1),
        "fused_speedup": round(us_naive / us_fused, 3),
    }), flush=True)
    return 0


def copy_probe(nbytes: int, iters: int) -> dict:
    """Device-to-device copy of nbytes (torch's copy kernel): the achievable
    streaming ceiling, and the calibration run for FETCH_SIZE / WRITE_SIZE."""
    import torch
    src = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda").normal_()
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(iters):
        dst.copy_(src)
    e.record()
    torch.cuda.synchronize()
    us = s.elapsed_time(e) * 1e3 / iters
    return {"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "us_per_copy": round(us, 2),
            "copy_GBps_read_plus_write": round(2 * nbytes / us / 1e3, 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--config", default="mixtral", choices=["mixtral", "deepseek", "dbrx"])
    ap.add_argument("--weights", default="fp16", choices=["fp16", "bf16", "fp8", "mxfp4", "fp32"],
                    help="expert weight format (the headline is fp16)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true")
    ap.add_argument("--read-probe", action="store_true",
                    help="time the read-only streaming ceiling over the selected experts")
    ap.add_argument("--gateup-probe", action="store_true",
                    help="time the single-token gate/up read order against the streaming "
                         "ceiling over the same bytes (16-bit weights)")
    ap.add_argument("--probe-sweep", action="store_true",
                    help="with --read-probe: sweep PROBE_SWEEP instead of PROBE_SHAPES")
    ap.add_argument("--op", default="fused", choices=["fused", "naive"],
                    help="naive: time the naive multi-kernel op (with fused beside it)")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="skip the streaming-ceiling measurement in the headline line")
    ap.add_argument("--batch", default=None,
                    help="comma-separated batch sizes: time batched decode instead")
    ap.add_argument("--throughput", action="store_true",
                    help="batched against a loop of single-token calls, Mixtral and DBRX, "
                         "top-2, B = 1..64 (or --batch)")
    ap.add_argument("--stack", type=int, default=0,
                    help="time one token through this many layers instead")
    ap.add_argument("--graph", action="store_true",
                    help="with --stack: also replay the step from a captured HIP graph")
    ap.add_argument("--timeline", type=int, default=0, metavar="N",
                    help="per-phase timeline of the single-token kernel over N calls instead "
                         "(needs the library built with WR_HIPCC_FLAGS=-DWR_TIMELINE=1)")
    ap.add_argument("--tp-shard", type=int, default=1, metavar="G",
                    help="time one GPU's share of a G-way tensor-parallel split over the "
                         "intermediate dimension (I/G rows of gate/up, I/G columns of down)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested): the MoE layer is "
              "benchmarked on a single MI355X; multi-GPU sharding is a design note, not a "
              "measured configuration.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1

    if args.copy_probe:
        print(json.dumps(copy_probe(1 << 30, 50)), flush=True)
        return 0
    if args.read_probe:
        return read_probe_bench(args)
    if args.gateup_probe:
        return gateup_probe_bench(args)
    if args.op == "naive":
        return naive_bench(args)
    if args.throughput:
        return throughput_bench(args)
    if args.batch:
        return batched_bench(args)
    if args.stack:
        return stack_bench(args)

    from warp_route import functional as F
    from warp_route.synthetic import make_config_layer

    cfg = bench_config(args)
    G = args.tp_shard
    E, h, I, k = cfg.num_experts, cfg.hidden_dim, cfg.intermediate_dim, cfg.top_k
    dev = torch.device("cuda:0")
    log(f"[bench] generating {args.layers} {cfg.name} {args.weights} layers on the GPU")
    layers = [make_config_layer(cfg, seed=s, device=dev, gen_device=dev)
              for s in range(args.layers)]
    torch.cuda.synchronize()

    # Distinct selected experts per call (always k at batch 1).
    sel_bytes = cfg.selected_bytes
    for x, gw, _ in layers:
        ids, _ = F.gate_topk(x, gw, E, h, k, cfg.renormalize)
        assert len(set(ids.tolist())) == k

    def step(i):
        x, gw, buf = layers[i % len(layers)]
        return F.fused_moe(x, gw, buf, E, h, I, k, cfg.renormalize)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    if args.timeline:
        print(json.dumps({
            "metric": "single-token kernel phase timeline (us from the first workgroup's start)",
            "config": {"workload": f"{cfg.name} MoE layer, decode batch 1"
                       + (f", one of {G} tensor-parallel shards over I" if G > 1 else ""),
                       "weight_dtype": args.weights, "layers_rotated": args.layers},
            "timeline": timeline_summary(step, args.timeline)}), flush=True)
        return 0

    # Whole timed region: K back-to-back calls between two events on the
    # stream the kernels run on (the current HIP stream).
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        step(i)
    stop.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    us = total_ms * 1e3 / args.steps

    # Per-call distribution (separate pass, events around each call).
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for i, (a, b) in enumerate(evs):
        a.record()
        step(i)
        b.record()
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
    p10, p50, p90 = (per[int(q * (len(per) - 1))] for q in (0.1, 0.5, 0.9))

    # The dominant kernel alone, for the roofline (same layers, same stream).
    kern_us = ffn_kernel_us(layers, cfg, args.steps, args.warmup)
    achieved = sel_bytes / (kern_us * 1e-6) / 1e9
    traffic = None
    suffix = "" if args.weights == "fp16" else f"_{args.weights}"
    tfile = os.path.join(ROOT, "profiles", f"traffic_{cfg.name}{suffix}.json")
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_call")

    result = {
        "metric": METRIC,
        "value": round(us, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": WLABEL[args.weights] + " weights, f32 accumulate",
        "data": "synthetic (seeded random-init layers drawn on the GPU)",
        "config": {"workload": f"{cfg.name} MoE layer, decode batch 1"
                   + (f", one of {G} tensor-parallel shards over I" if G > 1 else ""),
                   "hidden": h,
                   "intermediate": I, "experts": E, "top_k": k,
                   "renormalize": cfg.renormalize, "weight_dtype": args.weights,
                   "x_dtype": "fp32", "layers_rotated": args.layers,
                   "parallelism": "single GPU" if G == 1 else f"tp{G} shard, one GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "kernel": "k_fused_ffn",
                     "kernel_us": round(kern_us, 2),
                     "layer_GBps": round(sel_bytes / us / 1e3, 1),
                     "layer_frac": round(sel_bytes / us / 1e3 / HBM_PEAK_GBPS, 4)},
        "per_call_us": {"p10": round(p10, 2), "p50": round(p50, 2), "p90": round(p90, 2)},
        "selected_bytes_per_call": sel_bytes,
    }
    if not args.no_ceiling:
        ceil = read_ceiling(selected_ranges(layers, cfg), args.steps)
        result["roofline"]["read_ceiling"] = {
            "GBps": ceil["GBps"], "us": ceil["us"], "shape": ceil["shape"],
            "kernel_frac_of_ceiling": round(achieved / ceil["GBps"], 4),
            "what": "best read-only streaming kernel (libwr_probe.so) over exactly the "
                    "selected experts' bytes of the same rotated layers"}
    if not args.no_cpu_baseline:
        x, gw, buf = layers[0]
        log(f"[bench] cpu baseline ({args.cpu_seconds:.0f} s sample)")
        result["cpu_baseline"] = cpu_baseline(x, gw, buf, cfg, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
