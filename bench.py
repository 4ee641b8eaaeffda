#!/usr/bin/env python3
"""MoE-layer decode µs/token and achieved HBM GB/s at W4A16 on one MI355X.

Workload (default, ``moe_decode``): one Kimi-Linear MoE layer decoding one
token: hidden 2304, 256 routed experts + 1 shared, moe_intermediate 1024,
sigmoid top-8 router (routed_scaling_factor 2.446) on logits ~N(0, 1), W4A16
weights drawn from N(0, 0.02) and quantised at group 128 on the GPU. A step is
router + gate/up + SwiGLU + W2 + weighted combine + shared expert for one
token. 26 distinct layer banks (24.4 GB) are rotated so every step reads its
weights from HBM, not from the 256 MB MALL. Steps are captured in a HIP graph
and replayed; inputs are resident in HBM before the timed region.

``--workload dense_decode``: x [1, 2304] x W [9216, 2304] at group 128, 40
rotated weight copies (439 MB).

``--workload klinear_decode``: the model-slice caller of the same layer
(``local_kimi_amd.klinear.KLinearMoE``: the router logits ``x Wg^T`` in fp32
from bf16 router weights, then the MoE block), 26 layers with their own
router weights, one token per layer step, captured in one HIP graph.

Prints ONE JSON line. ``roofline`` is for the dominant kernel (gate/up +
SwiGLU, or the dense GEMV), timed with HIP events on the stream it runs on;
``cpu_baseline`` times the numpy oracle of the same step on the host (one
thread, a bounded sample of tokens).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
H, E_ROUTED, INTER, TOP_K, G, SCALING = 2304, 256, 1024, 8, 128, 2.446
DENSE_N = 9216


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def w4a16_bytes(n: int, k: int, g: int = G) -> int:
    return n * k // 2 + n * (k // g) * 2


EXPERT_BYTES = 2 * w4a16_bytes(INTER, H) + w4a16_bytes(H, INTER)       # 3,649,536
GATEUP_EXPERT_BYTES = 2 * w4a16_bytes(INTER, H)                         # 2,433,024
TOKEN_IO_BYTES = H * 2 + E_ROUTED * 4 + H * 2                           # x + logits + y


def measured_traffic(kernel: str) -> tuple[int | None, str | None]:
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/traffic.json)."""
    import json as _json

    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        data = _json.load(open(path))
        return int(data["kernels"][kernel]["traffic_bytes"]), "profiles/traffic.json"
    except (OSError, KeyError, ValueError):
        return None, None


def make_bank(rows: int, cols: int, experts: int, gen: torch.Generator, dev):
    from local_kimi_amd.quant import quantise

    packed = torch.empty((experts, rows, cols // 2), dtype=torch.uint8, device=dev)
    scales = torch.empty((experts, rows, cols // G), dtype=torch.bfloat16, device=dev)
    for e in range(experts):
        w = (torch.randn((rows, cols), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        enc = quantise(w, group_size=G)
        packed[e].copy_(enc.packed)
        scales[e].copy_(enc.scales)
    return packed, scales


def time_graph(graph: torch.cuda.CUDAGraph, replays: int, stream: torch.cuda.Stream) -> float:
    """Milliseconds for `replays` graph replays, HIP events on the replay stream."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def capture(fn, stream: torch.cuda.Stream) -> torch.cuda.CUDAGraph:
    with torch.cuda.stream(stream):
        fn()  # warm-up outside the graph (allocations, library load)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    torch.cuda.synchronize()
    return graph


def cpu_baseline_moe(banks_l0, xs, logits, sample: int) -> dict:
    """Oracle decode of `sample` tokens on one host thread (layer-0 weights)."""
    from threadpoolctl import threadpool_limits

    from oracle import moe as OM

    host = [t.cpu().numpy() if t.dtype == torch.uint8 else
            t.cpu().view(torch.int16).numpy().view(np.uint16) for t in banks_l0]
    times = []
    with threadpool_limits(1):
        for i in range(sample):
            x = xs[i].cpu().view(torch.int16).numpy().view(np.uint16)
            lg = logits[i].cpu().numpy()
            t0 = time.perf_counter()
            OM.moe_block(x, lg, None, *host, top_k=TOP_K, routed_scaling_factor=SCALING, group_size=G)
            times.append(time.perf_counter() - t0)
    us = float(np.median(times)) * 1e6
    return {"value": round(us, 1), "unit": "us/token", "cores": 1, "kind": "port",
            "sample": f"numpy oracle of the full MoE decode step (router, dequantise 9 experts, "
                      f"gate/up, SwiGLU, W2, combine) for {sample} tokens on one host thread, median"}


def cpu_baseline_dense(packed, scales, x, sample: int) -> dict:
    from threadpoolctl import threadpool_limits

    from oracle import w4a16 as OW

    p = packed.cpu().numpy()
    s = scales.cpu().view(torch.int16).numpy().view(np.uint16)
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    times = []
    with threadpool_limits(1):
        for _ in range(sample):
            t0 = time.perf_counter()
            OW.dense(xb, p, s, G)
            times.append(time.perf_counter() - t0)
    us = float(np.median(times)) * 1e6
    return {"value": round(us, 1), "unit": "us/token", "cores": 1, "kind": "port",
            "sample": f"numpy oracle dense GEMV (dequantise + matmul) x{sample}, one host thread, median"}


def run_moe(args, dev) -> dict:
    from local_kimi_amd.kernels import w4a16_moe_block, w4a16_moe_gateup

    layers = args.layers
    gen = torch.Generator(device=dev).manual_seed(20260729)
    t0 = time.time()
    master = (*make_bank(INTER, H, E_ROUTED + 1, gen, dev), *make_bank(INTER, H, E_ROUTED + 1, gen, dev),
              *make_bank(H, INTER, E_ROUTED + 1, gen, dev))
    banks = [master] + [tuple(t.clone() for t in master) for _ in range(layers - 1)]
    xs = [(torch.randn((1, H), device=dev, generator=gen)).to(torch.bfloat16) for _ in range(layers)]
    logits = [torch.randn((1, E_ROUTED), device=dev, generator=gen) for _ in range(layers)]
    torch.cuda.synchronize()
    log(f"[bench] {layers} layer banks ready in {time.time() - t0:.1f}s "
        f"({layers * (E_ROUTED + 1) * EXPERT_BYTES / 1e9:.1f} GB)")

    stream = torch.cuda.Stream(device=dev)

    def block_all():
        for l in range(layers):
            w4a16_moe_block(xs[l], logits[l], None, *banks[l], TOP_K, SCALING)

    def gateup_all():
        for l in range(layers):
            w1p, w1s, w3p, w3s = banks[l][:4]
            w4a16_moe_gateup(xs[l], logits[l], None, w1p, w1s, w3p, w3s, TOP_K, SCALING)

    g_block = capture(block_all, stream)
    g_gateup = capture(gateup_all, stream)

    steps = max(layers, (args.steps + layers - 1) // layers * layers)
    warm = max(1, (args.warmup + layers - 1) // layers)
    for _ in range(warm):
        g_block.replay()
        g_gateup.replay()
    torch.cuda.synchronize()
    log(f"[bench] warm-up done ({warm * layers} steps); timing {steps} steps")
    block_ms = time_graph(g_block, steps // layers, stream)
    gateup_ms = time_graph(g_gateup, steps // layers, stream)
    us_per_token = block_ms * 1000.0 / steps
    gateup_us = gateup_ms * 1000.0 / steps
    block_bytes = (TOP_K + 1) * EXPERT_BYTES + TOKEN_IO_BYTES
    gateup_bytes = (TOP_K + 1) * GATEUP_EXPERT_BYTES + H * 2 + E_ROUTED * 4 + (TOP_K + 1) * INTER * 2
    log(f"[bench] block {us_per_token:.2f} us/token, gate/up kernel {gateup_us:.2f} us/launch")

    result = {
        "metric": "MoE-layer decode us/token + achieved HBM GB/s (% of peak) at W4A16",
        "value": round(us_per_token, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm * layers,
        "ms_per_step": round(block_ms / steps, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,0.02) weights quantised W4A16 g128 on the GPU, N(0,1) x and logits",
        "config": {"workload": "moe_decode_batch1", "hidden": H, "routed_experts": E_ROUTED,
                   "shared_experts": 1, "moe_intermediate": INTER, "top_k": TOP_K, "group_size": G,
                   "tokens_per_step": 1, "layer_banks_rotated": layers, "launches_per_step": 2},
        "achieved_gbps": round(block_bytes / (us_per_token * 1e3), 1),
        "pct_hbm_peak": round(100.0 * block_bytes / (us_per_token * 1e3) / HBM_PEAK_GBPS, 2),
        "algorithmic_bytes_per_step": block_bytes,
        "roofline": {"kernel": "moe_gateup_ksplit_kernel (router + gate/up + SwiGLU, 9 routes)",
                     "bound": "hbm",
                     "achieved": round(gateup_bytes / (gateup_us * 1e3), 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s",
                     "frac": round(gateup_bytes / (gateup_us * 1e3) / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic("moe_gateup_ksplit_kernel")[0],
                     "traffic_source": measured_traffic("moe_gateup_ksplit_kernel")[1],
                     "bytes_per_launch": gateup_bytes,
                     "avg_launch_us": round(gateup_us, 3)},
    }
    if args.cpu_sample > 0:
        log(f"[bench] timing the CPU oracle on {args.cpu_sample} tokens")
        result["cpu_baseline"] = cpu_baseline_moe(banks[0], xs, logits, args.cpu_sample)
    return result


def run_klinear_decode(args, dev) -> dict:
    from local_kimi_amd.checkpoint import MoeBanks
    from local_kimi_amd.klinear import KLinearMoE

    layers = args.layers
    gen = torch.Generator(device=dev).manual_seed(20260729)
    t0 = time.time()
    master = (*make_bank(INTER, H, E_ROUTED + 1, gen, dev), *make_bank(INTER, H, E_ROUTED + 1, gen, dev),
              *make_bank(H, INTER, E_ROUTED + 1, gen, dev))
    mods = []
    for l in range(layers):
        b = master if l == 0 else tuple(t.clone() for t in master)
        gate = (torch.randn((E_ROUTED, H), device=dev, generator=gen) * (1.0 / H ** 0.5)).to(torch.bfloat16)
        bias = torch.randn((E_ROUTED,), device=dev, generator=gen) * 0.01
        mods.append(KLinearMoE(gate, bias, MoeBanks(*b), top_k=TOP_K, routed_scaling_factor=SCALING))
    xs = [(torch.randn((1, H), device=dev, generator=gen)).to(torch.bfloat16) for _ in range(layers)]
    torch.cuda.synchronize()
    log(f"[bench] {layers} KLinearMoE layers ready in {time.time() - t0:.1f}s")
    stream = torch.cuda.Stream(device=dev)

    def all_layers():
        for l in range(layers):
            mods[l](xs[l])

    graph = capture(all_layers, stream)
    steps = max(layers, (args.steps + layers - 1) // layers * layers)
    warm = max(1, (args.warmup + layers - 1) // layers)
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    ms = time_graph(graph, steps // layers, stream)
    us = ms * 1000.0 / steps
    router_bytes = E_ROUTED * H * 2
    step_bytes = (TOP_K + 1) * EXPERT_BYTES + TOKEN_IO_BYTES + router_bytes
    log(f"[bench] KLinearMoE decode {us:.2f} us/token")
    return {
        "metric": "MoE-layer decode us/token + achieved HBM GB/s (% of peak) at W4A16",
        "value": round(us, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm * layers,
        "ms_per_step": round(ms / steps, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,0.02) weights quantised W4A16 g128 on the GPU, N(0,1) x, "
                "N(0,1/H) bf16 router weights",
        "config": {"workload": "klinear_moe_decode_batch1", "hidden": H, "routed_experts": E_ROUTED,
                   "shared_experts": 1, "moe_intermediate": INTER, "top_k": TOP_K, "group_size": G,
                   "tokens_per_step": 1, "layer_banks_rotated": layers,
                   "router": "lk_router_logits (bf16 x, bf16 Wg [256, 2304], fp32 sums), then the MoE block"},
        "achieved_gbps": round(step_bytes / (us * 1e3), 1),
        "pct_hbm_peak": round(100.0 * step_bytes / (us * 1e3) / HBM_PEAK_GBPS, 2),
        "algorithmic_bytes_per_step": step_bytes,
    }


def run_dense(args, dev) -> dict:
    from local_kimi_amd.kernels import w4a16_dense
    from local_kimi_amd.quant import quantise

    copies = args.copies
    gen = torch.Generator(device=dev).manual_seed(20260729)
    w = (torch.randn((DENSE_N, H), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
    enc = quantise(w, group_size=G)
    weights = [(enc.packed.clone(), enc.scales.clone()) for _ in range(copies)]
    x = torch.randn((1, H), device=dev, generator=gen).to(torch.bfloat16)
    stream = torch.cuda.Stream(device=dev)

    def all_copies():
        for p, s in weights:
            w4a16_dense(x, p, s)

    graph = capture(all_copies, stream)
    steps = max(copies, (args.steps + copies - 1) // copies * copies)
    warm = max(1, (args.warmup + copies - 1) // copies)
    for _ in range(warm):
        graph.replay()
    ms = time_graph(graph, steps // copies, stream)
    us = ms * 1000.0 / steps
    nbytes = w4a16_bytes(DENSE_N, H) + H * 2 + DENSE_N * 2
    result = {
        "metric": "Dense W4A16 GEMV decode us/token + achieved HBM GB/s (% of peak)",
        "value": round(us, 3), "unit": "us/token", "n_gpus": 1, "steps": steps,
        "warmup": warm * copies, "ms_per_step": round(ms / steps, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,0.02) weights quantised W4A16 g128 on the GPU, N(0,1) x",
        "config": {"workload": "dense_gemv_decode", "m": 1, "n": DENSE_N, "k": H, "group_size": G,
                   "weight_copies_rotated": copies},
        "achieved_gbps": round(nbytes / (us * 1e3), 1),
        "pct_hbm_peak": round(100.0 * nbytes / (us * 1e3) / HBM_PEAK_GBPS, 2),
        "roofline": {"kernel": "dense_ksplit_kernel", "bound": "hbm",
                     "achieved": round(nbytes / (us * 1e3), 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(nbytes / (us * 1e3) / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic("dense_ksplit_kernel")[0],
                     "traffic_source": measured_traffic("dense_ksplit_kernel")[1],
                     "bytes_per_launch": nbytes, "avg_launch_us": round(us, 3)},
    }
    if args.cpu_sample > 0:
        result["cpu_baseline"] = cpu_baseline_dense(weights[0][0], weights[0][1], x, args.cpu_sample)
    return result


def make_mx_bank(rows: int, cols: int, experts: int, gen: torch.Generator, dev):
    from local_kimi_amd.quant import quantize_mxfp4

    packed = torch.empty((experts, rows, cols // 2), dtype=torch.uint8, device=dev)
    scale = torch.empty((experts, rows, cols // 32), dtype=torch.uint8, device=dev)
    for e in range(experts):
        w = (torch.randn((rows, cols), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        p, sc = quantize_mxfp4(w)
        packed[e].copy_(p)
        scale[e].copy_(sc)
    return packed, scale


MX_EXPERT_BYTES = 3 * (INTER * H // 2 + INTER * (H // 32))   # 3,760,128


def _layer_banks(layers: int, gen: torch.Generator, dev, weights: str = "w4a16"):
    mk = make_mx_bank if weights == "mxfp4" else make_bank
    master = (*mk(INTER, H, E_ROUTED + 1, gen, dev), *mk(INTER, H, E_ROUTED + 1, gen, dev),
              *mk(H, INTER, E_ROUTED + 1, gen, dev))
    return [master] + [tuple(t.clone() for t in master) for _ in range(layers - 1)]


def _block_fn(weights: str, path: str = "expert"):
    from local_kimi_amd.kernels import mxfp4_moe_block, w4a16_moe_decode, w4a16_moe_forward

    if weights == "mxfp4":
        return mxfp4_moe_block
    return w4a16_moe_forward if path == "expert" else w4a16_moe_decode


def cpu_baseline_block(banks_l0, xs, logits, tokens: int, weights: str) -> dict:
    """Oracle block for `tokens` tokens of the step on one host thread."""
    from threadpoolctl import threadpool_limits

    from oracle import moe as OM
    from oracle import mxfp4 as OX

    host = [t.cpu().numpy() if t.dtype == torch.uint8 else
            t.cpu().view(torch.int16).numpy().view(np.uint16) for t in banks_l0]
    x = xs[:tokens].cpu().view(torch.int16).numpy().view(np.uint16)
    lg = logits[:tokens].cpu().numpy()
    with threadpool_limits(1):
        t0 = time.perf_counter()
        if weights == "mxfp4":
            OX.moe_block(x, lg, None, *host, top_k=TOP_K, routed_scaling_factor=SCALING)
        else:
            OM.moe_block(x, lg, None, *host, top_k=TOP_K, routed_scaling_factor=SCALING, group_size=G)
        dt = time.perf_counter() - t0
    return {"value": round(dt * 1e6 / tokens, 1), "unit": "us/token", "cores": 1, "kind": "port",
            "sample": f"numpy oracle of the MoE block ({weights}: router, dequantise the routed "
                      f"experts, gate/up, SwiGLU, W2, combine) for {tokens} tokens of the step "
                      "on one host thread"}


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
EXPERT_FLOPS = 2 * 3 * INTER * H  # gate, up and down projections per routed row


def run_moe_batched(args, dev) -> dict:
    """Batched decode: M tokens per step, Zipf(1.1)-skewed routing (the block's path by default)."""
    from local_kimi_amd.workloads import zipf_router_logits
    from oracle import moe as OM

    from local_kimi_amd.kernels.moe import MOE_EXPERT_MAJOR_MIN_TOKENS

    m, layers = args.tokens, args.layers
    path = args.moe_path
    if path == "auto":  # the block's own choice
        path = "expert" if m >= MOE_EXPERT_MAJOR_MIN_TOKENS or args.weights == "mxfp4" else "token"
    gen = torch.Generator(device=dev).manual_seed(20260729)
    rng = np.random.default_rng(20260729)
    t0 = time.time()
    banks = _layer_banks(layers, gen, dev, args.weights)
    block = _block_fn(args.weights, path)
    xs = [(torch.randn((m, H), device=dev, generator=gen)).to(torch.bfloat16) for _ in range(layers)]
    host_logits = [zipf_router_logits(rng, m, E_ROUTED) for _ in range(layers)]
    logits = [torch.from_numpy(lg).to(dev) for lg in host_logits]
    unions = [len(np.unique(OM.route(lg, None, TOP_K)[0])) for lg in host_logits]
    torch.cuda.synchronize()
    log(f"[bench] {layers} layer banks ready in {time.time() - t0:.1f}s; distinct routed "
        f"experts per layer: mean {np.mean(unions):.1f} (min {min(unions)}, max {max(unions)})")
    stream = torch.cuda.Stream(device=dev)

    def all_layers():
        for l in range(layers):
            block(xs[l], logits[l], None, *banks[l], TOP_K, SCALING)

    graph = capture(all_layers, stream)
    reps = max(1, args.steps // layers)
    warm = max(1, args.warmup // layers)
    for _ in range(warm):
        graph.replay()
    ms = time_graph(graph, reps, stream)
    steps = reps * layers
    us_step = ms * 1000.0 / steps
    ebytes = MX_EXPERT_BYTES if args.weights == "mxfp4" else EXPERT_BYTES
    step_bytes = float(np.mean([(u + 1) * ebytes for u in unions])) + m * TOKEN_IO_BYTES
    step_flops = m * (TOP_K + 1) * EXPERT_FLOPS
    gbps = step_bytes / (us_step * 1e3)
    result = {
        "metric": f"Batched MoE decode us/step + achieved HBM GB/s (% of peak) at {args.weights.upper()}",
        "value": round(us_step, 3), "unit": "us/step", "n_gpus": 1, "steps": steps,
        "warmup": warm * layers, "ms_per_step": round(ms / steps, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": f"synthetic: N(0,0.02) weights quantised {_weights_desc(args.weights)} on the GPU, "
                "N(0,1) x, Zipf(1.1) router logits (log p + Gumbel)",
        "config": {"workload": f"moe_batched_decode_m{m}", "weights": args.weights,
                   "path": f"{path}-major", "tokens_per_step": m, "hidden": H,
                   "routed_experts": E_ROUTED, "shared_experts": 1, "moe_intermediate": INTER,
                   "top_k": TOP_K, "layer_banks_rotated": layers,
                   "mean_distinct_routed_experts": round(float(np.mean(unions)), 2)},
        "us_per_token": round(us_step / m, 3),
        "achieved_gbps": round(gbps, 1),
        "pct_hbm_peak": round(100.0 * gbps / HBM_PEAK_GBPS, 2),
        "algorithmic_bytes_per_step": int(step_bytes),
        "roofline": {"kernel": (("whole block (router + schedule, gate/up GEMM, W2 + combine GEMV)"
                                 if args.weights == "w4a16" and m <= 4 else
                                 "whole block (router, schedule, gate/up GEMM, down GEMM, combine)")
                                if path == "expert" else
                                "whole block (router + gate/up GEMV, W2 + combine GEMV)"),
                     "bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "mfma_tflops": round(step_flops / (us_step * 1e6), 2)},
    }
    if args.cpu_sample > 0:
        log(f"[bench] timing the CPU oracle on {min(args.cpu_sample, m)} tokens")
        result["cpu_baseline"] = cpu_baseline_block(banks[0], xs[0], logits[0], min(args.cpu_sample, m),
                                                    args.weights)
    return result


def _weights_desc(weights: str) -> str:
    return "OCP MXFP4 (E2M1, E8M0 per 32)" if weights == "mxfp4" else "W4A16 g128"


def run_moe_prefill(args, dev) -> dict:
    """Prefill: 2048 tokens x top-8 (+ shared) through one layer, N(0,1) logits."""
    m = args.prefill_tokens
    gen = torch.Generator(device=dev).manual_seed(20260729)
    banks = _layer_banks(2, gen, dev, args.weights)
    block = _block_fn(args.weights)
    xs = [(torch.randn((m, H), device=dev, generator=gen)).to(torch.bfloat16) for _ in range(2)]
    logits = [torch.randn((m, E_ROUTED), device=dev, generator=gen) for _ in range(2)]
    stream = torch.cuda.Stream(device=dev)

    def both():
        for l in range(2):
            block(xs[l], logits[l], None, *banks[l], TOP_K, SCALING)

    graph = capture(both, stream)
    reps = max(1, args.prefill_steps // 2)
    for _ in range(3):
        graph.replay()
    ms = time_graph(graph, reps, stream)
    steps = 2 * reps
    us = ms * 1000.0 / steps
    ebytes = MX_EXPERT_BYTES if args.weights == "mxfp4" else EXPERT_BYTES
    nbytes = (E_ROUTED + 1) * ebytes + m * TOKEN_IO_BYTES
    flops = m * (TOP_K + 1) * EXPERT_FLOPS
    tflops = flops / (us * 1e6)
    gbps = nbytes / (us * 1e3)
    result = {
        "metric": f"MoE prefill us/layer + MFMA TFLOP/s and HBM GB/s at {args.weights.upper()}",
        "value": round(us, 2), "unit": "us/layer", "n_gpus": 1, "steps": steps, "warmup": 6,
        "ms_per_step": round(ms / steps, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": f"synthetic: N(0,0.02) weights quantised {_weights_desc(args.weights)} on the GPU, "
                "N(0,1) x and logits",
        "config": {"workload": f"moe_prefill_{m}", "weights": args.weights, "tokens": m, "hidden": H,
                   "routed_experts": E_ROUTED, "shared_experts": 1, "moe_intermediate": INTER,
                   "top_k": TOP_K},
        "tokens_per_s": round(m / (us * 1e-6), 1),
        "achieved_gbps": round(gbps, 1), "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "achieved_tflops": round(tflops, 1),
        "pct_mfma_peak": round(100 * tflops / MFMA_BF16_PEAK_TFLOPS, 2),
        "algorithmic_bytes_per_step": nbytes, "flops_per_step": flops,
        "roofline": {"kernel": "whole block (router, schedule, gate/up GEMM, down GEMM, combine)",
                     "bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": None, "hbm_gbps": round(gbps, 1)},
    }
    if args.cpu_sample > 0:
        n = min(args.cpu_sample, m)
        log(f"[bench] timing the CPU oracle on {n} tokens")
        result["cpu_baseline"] = cpu_baseline_block(banks[0], xs[0], logits[0], n, args.weights)
    return result


def run_qkv_prefill(args, dev) -> dict:
    """Fused QKV projection of 2048 tokens: [2048, 2304] x [2304, 3 x 4096] at W4A16."""
    from local_kimi_amd.kernels import fused_qkv_w4a16
    from local_kimi_amd.quant import quantise

    m, n = args.prefill_tokens, 4096
    gen = torch.Generator(device=dev).manual_seed(20260729)
    mats = []
    for _ in range(3):
        enc = quantise((torch.randn((n, H), device=dev, generator=gen) * 0.02).to(torch.bfloat16),
                       group_size=G)
        mats += [enc.packed, enc.scales]
    x = torch.randn((m, H), device=dev, generator=gen).to(torch.bfloat16)
    stream = torch.cuda.Stream(device=dev)
    graph = capture(lambda: fused_qkv_w4a16(x, *mats), stream)
    reps = max(1, args.prefill_steps)
    for _ in range(3):
        graph.replay()
    ms = time_graph(graph, reps, stream)
    us = ms * 1000.0 / reps
    nbytes = 3 * w4a16_bytes(n, H) + m * H * 2 + 3 * m * n * 2
    flops = 2 * m * H * 3 * n
    tflops = flops / (us * 1e6)
    result = {
        "metric": "Fused QKV prefill GEMM us + MFMA TFLOP/s at W4A16",
        "value": round(us, 2), "unit": "us/call", "n_gpus": 1, "steps": reps, "warmup": 3,
        "ms_per_step": round(ms / reps, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,0.02) weights quantised W4A16 g128 on the GPU, N(0,1) x",
        "config": {"workload": f"qkv_prefill_{m}", "m": m, "n_per_projection": n, "k": H,
                   "group_size": G},
        "achieved_tflops": round(tflops, 1),
        "pct_mfma_peak": round(100 * tflops / MFMA_BF16_PEAK_TFLOPS, 2),
        "achieved_gbps": round(nbytes / (us * 1e3), 1),
        "algorithmic_bytes_per_step": nbytes, "flops_per_step": flops,
        "roofline": {"kernel": "dense W4A16 GEMM (3 outputs, one launch)", "bound": "mfma",
                     "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None},
    }
    if args.cpu_sample > 0:
        from threadpoolctl import threadpool_limits

        from oracle import w4a16 as OW

        rows = min(args.cpu_sample, m)
        host = [t.cpu().numpy() if t.dtype == torch.uint8 else
                t.cpu().view(torch.int16).numpy().view(np.uint16) for t in mats]
        xb = x[:rows].cpu().view(torch.int16).numpy().view(np.uint16)
        with threadpool_limits(1):
            t0 = time.perf_counter()
            OW.fused_qkv(xb, *host, G)
            dt = time.perf_counter() - t0
        result["cpu_baseline"] = {
            "value": round(dt * 1e6 / rows, 1), "unit": "us/token", "cores": 1, "kind": "port",
            "sample": f"numpy oracle fused QKV (dequantise 3 x [4096, 2304] + matmul) for {rows} "
                      "rows on one host thread"}
    return result


def run_copy(args, dev) -> dict:
    """Plain device copy of a known size: calibrates the HBM byte counters."""
    nbytes = args.copy_mb << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    reps = 10
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1000.0 / reps
    return {"metric": "device copy (counter calibration)", "value": round(us, 2), "unit": "us/copy",
            "bytes_read": nbytes, "bytes_written": nbytes, "gbps": round(2 * nbytes / (us * 1e3), 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2600)
    ap.add_argument("--warmup", type=int, default=260)
    ap.add_argument("--workload", default="moe_decode",
                    choices=["moe_decode", "dense_decode", "moe_batched", "moe_prefill",
                             "qkv_prefill", "klinear_decode", "copy"])
    ap.add_argument("--tokens", type=int, default=64, help="moe_batched tokens per step")
    ap.add_argument("--moe-path", choices=["auto", "expert", "token"], default="auto",
                    help="moe_batched: the block's choice, expert-major GEMMs or token-major GEMVs")
    ap.add_argument("--weights", choices=["w4a16", "mxfp4"], default="w4a16",
                    help="moe_batched / moe_prefill expert weight format")
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--prefill-steps", type=int, default=40)
    ap.add_argument("--copy-mb", type=int, default=256, help="copy workload size (MiB)")
    ap.add_argument("--layers", type=int, default=26, help="MoE layer banks rotated")
    ap.add_argument("--copies", type=int, default=40, help="dense weight copies rotated")
    ap.add_argument("--cpu-sample", type=int, default=4, help="tokens for the CPU oracle baseline (0: skip)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path. Run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    from local_kimi_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    log(f"[bench] device {torch.cuda.get_device_name(0)}, workload {args.workload}")
    runners = {"moe_decode": run_moe, "dense_decode": run_dense, "moe_batched": run_moe_batched,
               "moe_prefill": run_moe_prefill, "qkv_prefill": run_qkv_prefill,
               "klinear_decode": run_klinear_decode, "copy": run_copy}
    result = runners[args.workload](args, dev)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
