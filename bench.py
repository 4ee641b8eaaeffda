#!/usr/bin/env python3
"""MoE-layer decode µs/token + achieved HBM GB/s (% of peak) at W4A16, one MI355X.

Default run (``--workload all``): one JSON line whose top level is the
headline, a batch-1 Kimi-Linear MoE layer decode (hidden 2304, 256 routed + 1
shared experts, moe_intermediate 1024, sigmoid top-8 router with
routed_scaling_factor 2.446 on logits ~N(0, 1), W4A16 weights ~N(0, 0.02)
quantised at group 128 on the GPU). A step is router + gate/up + SwiGLU + W2
+ weighted combine + shared expert for one token. 26 distinct layer banks
(24.4 GB) rotate so every step reads its weights from HBM, not from the
256 MB MALL; the steps of one rotation are captured in a HIP graph and
replayed; inputs are resident in HBM before the timed region. Exactly
``--steps`` steps are timed (520 by default, 20 rotations, captured as one
graph) after exactly ``--warmup`` warm-up steps (52 by default), for every
workload of the line.

The line also carries ``configs``: the other four workload shapes, each timed
the same way and each with its own ``roofline`` and ``cpu_baseline``:
config 1 dense GEMV x[1,2304] . W[9216,2304]; config 3 batched decode at
M = 4, 16, 64 with Zipf(1.1) routing; config 4 the 2048-token MoE prefill and
the fused QKV projection [2048,2304] x [2304,3 x 4096]; config 5 the MXFP4
expert banks at M = 64 and 2048 tokens. ``floor`` holds the measured memory
floors (empty-kernel launch, a streaming read of 11 MB and of one MoE layer's
33 MB in its 27 matrices) that the decode kernels are also reported against.

``roofline``: for the decode configs the dominant kernel's algorithmic bytes
per launch over its average launch time, timed with HIP events on the stream
it is launched on; for the prefill configs the whole block's (or the QKV
kernel's) FLOPs over its time. ``cpu_baseline``: a torch restatement of the
reference path on the host (dequantise to bf16, F.linear with fp32
accumulation, the bf16 SwiGLU, the fp32 weighted combine, the bf16 add of the
shared expert), all host threads the process may use, median of 10 runs after
3 warm-ups, on a bounded sample stated per config.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

import numpy as np
import torch
import torch.nn.functional as F

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

H, E_ROUTED, INTER, TOP_K, G, SCALING = 2304, 256, 1024, 8, 128, 2.446
DENSE_N, QKV_N, PREFILL_TOKENS = 9216, 4096, 2048
LAYERS, DENSE_COPIES = 26, 40
MIN_TIMED_STEPS, MIN_WARMUP_STEPS = 104, 10  # below these the timing is noisier (a warning)
DEFAULT_STEPS, DEFAULT_WARMUP = 520, 52

HBM_PEAK_GBPS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0     # dense bf16 MFMA
FP4_PEAK_TFLOPS = 10100.0     # dense fp4 MFMA

METRIC = "MoE-layer decode us/token + achieved HBM GB/s (% of peak) at W4A16"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def w4a16_bytes(n: int, k: int, g: int = G) -> int:
    return n * k // 2 + n * (k // g) * 2


def mxfp4_bytes(n: int, k: int) -> int:
    return n * k // 2 + n * (k // 32)


EXPERT_BYTES = 2 * w4a16_bytes(INTER, H) + w4a16_bytes(H, INTER)          # 3,649,536
GATEUP_EXPERT_BYTES = 2 * w4a16_bytes(INTER, H)                            # 2,433,024
MX_EXPERT_BYTES = 2 * mxfp4_bytes(INTER, H) + mxfp4_bytes(H, INTER)        # 3,760,128
TOKEN_IO_BYTES = H * 2 + E_ROUTED * 4 + H * 2                              # x + logits + y
EXPERT_FLOPS = 2 * 3 * INTER * H                                           # per routed row


# ---------------------------------------------------------------------------
# GPU timing


class Plan:
    """Exactly `steps` timed steps after exactly `warmup` warm-up steps, for
    every workload (the defaults, 520 and 52, are whole rotations of the
    26-layer banks)."""

    def __init__(self, steps: int, warmup: int):
        if steps < 1 or warmup < 0:
            raise ValueError("--steps must be at least 1 and --warmup at least 0")
        self.steps, self.warmup = steps, warmup


def capture(fn, stream: torch.cuda.Stream) -> torch.cuda.CUDAGraph:
    with torch.cuda.stream(stream):
        fn()  # outside the graph first: allocations, library load, kernel attributes
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    torch.cuda.synchronize()
    return graph


def time_steps(step, count: int, stream, plan: Plan) -> dict:
    """Time `plan.steps` steps of a rotation of `count` distinct steps.

    `step(i)` enqueues step i (0 <= i < count). The timed steps are captured as
    one HIP graph that cycles through the rotation (as a decode step captures
    all of its layers in one graph), so the region holds exactly the timed
    steps and one graph launch. Warm-ups run first; the last of them (up to
    one rotation, taken from the end of the rotation, so the timed steps,
    which start at step 0, still read their weights from HBM) are enqueued
    back to back with the start event, keeping the GPU busy while the host
    enqueues the timed graph. The events are recorded on the replay stream."""
    lead = min(plan.warmup, count)

    def span(first: int, n: int):
        return capture(lambda: [step((first + i) % count) for i in range(n)], stream)

    early = span(0, plan.warmup - lead) if plan.warmup > lead else None
    led = span(count - lead, lead) if lead else None
    timed = span(0, plan.steps)

    if early is not None:
        with torch.cuda.stream(stream):
            early.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        if led is None:
            torch.cuda._sleep(2_000_000)  # no warm-up steps: a spin kernel covers the enqueue
        else:
            led.replay()
        start.record(stream)
        timed.replay()
        end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    return {"us": ms * 1000.0 / plan.steps, "steps": plan.steps, "warmup": plan.warmup,
            "ms_total": ms}


# ---------------------------------------------------------------------------
# synthetic weights (quantised on the GPU)


def make_w4a16_bank(rows, cols, experts, gen, dev):
    from local_kimi_amd.quant import quantise

    packed = torch.empty((experts, rows, cols // 2), dtype=torch.uint8, device=dev)
    scales = torch.empty((experts, rows, cols // G), dtype=torch.bfloat16, device=dev)
    for e in range(experts):
        w = (torch.randn((rows, cols), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        enc = quantise(w, group_size=G)
        packed[e].copy_(enc.packed)
        scales[e].copy_(enc.scales)
    return packed, scales


def make_mxfp4_bank(rows, cols, experts, gen, dev):
    from local_kimi_amd.quant import quantize_mxfp4

    packed = torch.empty((experts, rows, cols // 2), dtype=torch.uint8, device=dev)
    scale = torch.empty((experts, rows, cols // 32), dtype=torch.uint8, device=dev)
    for e in range(experts):
        w = (torch.randn((rows, cols), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
        p, s = quantize_mxfp4(w)
        packed[e].copy_(p)
        scale[e].copy_(s)
    return packed, scale


def layer_banks(weights: str, gen, dev, layers: int = LAYERS):
    mk = make_mxfp4_bank if weights == "mxfp4" else make_w4a16_bank
    master = (*mk(INTER, H, E_ROUTED + 1, gen, dev), *mk(INTER, H, E_ROUTED + 1, gen, dev),
              *mk(H, INTER, E_ROUTED + 1, gen, dev))
    return [master] + [tuple(t.clone() for t in master) for _ in range(layers - 1)]


# ---------------------------------------------------------------------------
# CPU baseline: a torch restatement of the reference path on the host


def cpu_threads() -> int:
    limit = os.environ.get("OMP_NUM_THREADS")
    n = os.cpu_count() or 1
    threads = min(n, int(limit)) if limit and limit.isdigit() and int(limit) > 0 else n
    torch.set_num_threads(threads)
    return threads


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_median(fn, runs: int = 10, warm: int = 3) -> float:
    for _ in range(warm):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def cpu_dequant_w4a16(packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """bf16(q * s) (engine/quant/w4a16.py:108-129) on the host."""
    n = packed.shape[0]
    codes = torch.stack(((packed & 0xF), (packed >> 4)), dim=-1).reshape(n, -1).to(torch.int16)
    codes = torch.where(codes >= 8, codes - 16, codes).float()
    g = codes.shape[1] // scales.shape[1]
    return (codes.reshape(n, -1, g) * scales.float()[..., None]).reshape(n, -1).to(torch.bfloat16)


_E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                      -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def cpu_dequant_mxfp4(packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """e2m1 * 2^(e8m0 - 127) cast to bf16 (engine/k3ref/dequant.py:43-73)."""
    n = packed.shape[0]
    codes = torch.stack(((packed & 0xF), (packed >> 4)), dim=-1).reshape(n, -1).long()
    vals = _E2M1[codes].reshape(n, -1, 32)
    exps = torch.ldexp(torch.ones(()), scale.to(torch.int32) - 127)
    return (vals * exps[..., None]).reshape(n, -1).to(torch.bfloat16)


def cpu_linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return F.linear(x.float(), w.float()).to(torch.bfloat16)


def cpu_router(logits: torch.Tensor, top_k: int | None = None):
    """klinear/router.py:52-85 (no bias, one group)."""
    s = torch.sigmoid(logits)
    idx = torch.topk(s, TOP_K if top_k is None else top_k, dim=1).indices
    w = s.gather(1, idx)
    return idx, w / (w.sum(dim=1, keepdim=True) + 1e-20) * SCALING


class CpuMoe:
    """The block on the host for one layer's banks (W4A16 or MXFP4)."""

    def __init__(self, banks, weights: str):
        self.host = [t.cpu() for t in banks]
        self.deq = cpu_dequant_mxfp4 if weights == "mxfp4" else cpu_dequant_w4a16

    def expert(self, e: int, rows: torch.Tensor) -> torch.Tensor:
        """SwiGLU expert e on bf16 rows: kernels/__init__.py:182-197 then W2."""
        w1p, w1s, w3p, w3s, w2p, w2s = self.host
        gate = cpu_linear(rows, self.deq(w1p[e], w1s[e]))
        up = cpu_linear(rows, self.deq(w3p[e], w3s[e]))
        act = F.silu(gate) * up  # bf16 silu, bf16 multiply
        return cpu_linear(act, self.deq(w2p[e], w2s[e]))

    def routed(self, x, idx, experts, eo):
        for e in experts:
            tok, slot = torch.nonzero(idx == e, as_tuple=True)
            eo[tok, slot] = self.expert(int(e), x[tok])

    def step(self, x, logits, experts=None):
        """Router, the routed experts (all, or `experts` only), shared expert, combine."""
        idx, w = cpu_router(logits)
        eo = torch.zeros((x.shape[0], TOP_K + 1, H), dtype=torch.bfloat16)
        self.routed(x, idx, torch.unique(idx) if experts is None else experts, eo)
        eo[:, TOP_K] = self.expert(E_ROUTED, x)
        routed = eo[:, :TOP_K].float().mul(w.unsqueeze(-1)).sum(dim=1).to(torch.bfloat16)
        return routed + eo[:, TOP_K]


def cpu_baseline_block(banks, x, logits, weights: str, unit: str, per_step: float = 1.0,
                       max_experts: int = 16) -> dict:
    """The block of one step on the host. With more routed experts than
    `max_experts` in the step, a stride sample of them is timed with the router,
    shared expert and combine, and the routed part is scaled by the expert count."""
    threads = cpu_threads()
    cpu = CpuMoe(banks, weights)
    xh, lh = x.cpu(), logits.cpu()
    union = torch.unique(cpu_router(lh)[0])
    u = int(union.numel())
    if u <= max_experts:
        t = cpu_median(lambda: cpu.step(xh, lh))
        sample = f"the whole step ({xh.shape[0]} tokens, {u} routed experts + shared)"
    else:
        subset = union[:: math.ceil(u / max_experts)]
        idx = cpu_router(lh)[0]
        eo = torch.zeros((xh.shape[0], TOP_K + 1, H), dtype=torch.bfloat16)
        t_sample = cpu_median(lambda: cpu.step(xh, lh, subset))
        t_subset = cpu_median(lambda: cpu.routed(xh, idx, subset, eo))
        t = t_sample + t_subset * (u / subset.numel() - 1.0)
        sample = (f"{xh.shape[0]} tokens: router, shared expert, combine and {subset.numel()} of "
                  f"the {u} routed experts (every {math.ceil(u / max_experts)}th, their real rows) "
                  f"timed; the routed part scaled by {u}/{subset.numel()}")
    return {"value": round(t * 1e6 / per_step, 1), "unit": unit, "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"torch restatement on the host ({weights}: dequantise to bf16, F.linear "
                      f"fp32, bf16 SwiGLU, W2, fp32 combine + shared); {sample}; median of 10 "
                      "after 3 warm-ups"}


# ---------------------------------------------------------------------------
# configs


def run_moe_decode(plan: Plan, dev, banks, cpu: bool) -> dict:
    """Config 2: batch-1 decode, the headline."""
    from local_kimi_amd.kernels import w4a16_moe_block, w4a16_moe_gateup

    gen = torch.Generator(device=dev).manual_seed(20260729)
    xs = [torch.randn((1, H), device=dev, generator=gen).to(torch.bfloat16) for _ in range(LAYERS)]
    logits = [torch.randn((1, E_ROUTED), device=dev, generator=gen) for _ in range(LAYERS)]
    stream = torch.cuda.Stream(device=dev)

    def block(l):
        w4a16_moe_block(xs[l], logits[l], None, *banks[l], TOP_K, SCALING)

    def gateup(l):
        w4a16_moe_gateup(xs[l], logits[l], None, *banks[l][:4], TOP_K, SCALING)

    blk = time_steps(block, LAYERS, stream, plan)
    gu = time_steps(gateup, LAYERS, stream, plan)
    # a short timed region carries the fixed cost of its graph launch and
    # completion (about 10 us); the steady-state rate beside it, at the default count
    steady = blk if plan.steps >= DEFAULT_STEPS else time_steps(block, LAYERS, stream,
                                                                 Plan(DEFAULT_STEPS, plan.warmup))
    step_bytes = (TOP_K + 1) * EXPERT_BYTES + TOKEN_IO_BYTES
    gu_bytes = (TOP_K + 1) * GATEUP_EXPERT_BYTES + H * 2 + E_ROUTED * 4 + (TOP_K + 1) * INTER * 2
    traffic = measured_traffic("moe_gateup_ksplit_kernel")
    prof_us = rocprof_avg_us("moe_decode", "moe_gateup_ksplit_kernel")
    log(f"[bench] config 2: block {blk['us']:.2f} us/token, gate/up kernel {gu['us']:.2f} us")
    res = {
        "value": round(blk["us"], 3), "unit": "us/token", "steps": blk["steps"],
        "warmup": blk["warmup"], "ms_per_step": round(blk["us"] / 1000.0, 6),
        "achieved_gbps": round(step_bytes / (blk["us"] * 1e3), 1),
        "pct_hbm_peak": round(100.0 * step_bytes / (blk["us"] * 1e3) / HBM_PEAK_GBPS, 2),
        "algorithmic_bytes_per_step": step_bytes,
        "us_per_token_at_520_steps": round(steady["us"], 3),
        "roofline": {"kernel": "moe_gateup_ksplit_kernel (router + gate/up + SwiGLU, 9 routes)",
                     "bound": "hbm", "achieved": round(gu_bytes / (gu["us"] * 1e3), 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gu_bytes / (gu["us"] * 1e3) / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "bytes_per_launch": gu_bytes,
                     "avg_launch_us": round(gu["us"], 3),
                     # the same kernel's average dispatch in the committed rocprofv3 trace
                     "rocprof_avg_launch_us": prof_us,
                     "frac_at_rocprof_avg": (round(gu_bytes / (prof_us * 1e3) / HBM_PEAK_GBPS, 4)
                                             if prof_us else None)},
    }
    if cpu:
        log("[bench] config 2: CPU baseline")
        res["cpu_baseline"] = cpu_baseline_block(banks[0], xs[0], logits[0], "w4a16", "us/token")
    return res


def run_dense(plan: Plan, dev, cpu: bool) -> dict:
    """Config 1: dense GEMV x[1,2304] . W[9216,2304], 40 rotated copies (439 MB)."""
    from local_kimi_amd.kernels import w4a16_dense
    from local_kimi_amd.quant import quantise

    gen = torch.Generator(device=dev).manual_seed(20260730)
    enc = quantise((torch.randn((DENSE_N, H), device=dev, generator=gen) * 0.02)
                   .to(torch.bfloat16), group_size=G)
    weights = [(enc.packed.clone(), enc.scales.clone()) for _ in range(DENSE_COPIES)]
    x = torch.randn((1, H), device=dev, generator=gen).to(torch.bfloat16)
    stream = torch.cuda.Stream(device=dev)

    t = time_steps(lambda i: w4a16_dense(x, *weights[i]), DENSE_COPIES, stream, plan)
    nbytes = w4a16_bytes(DENSE_N, H) + H * 2 + DENSE_N * 2
    log(f"[bench] config 1: dense GEMV {t['us']:.2f} us")
    res = {
        "metric": "Dense W4A16 GEMV decode us/call + HBM GB/s", "value": round(t["us"], 3),
        "unit": "us/call", "steps": t["steps"], "warmup": t["warmup"],
        "config": {"workload": "dense_gemv_decode", "m": 1, "n": DENSE_N, "k": H,
                   "group_size": G, "weight_copies_rotated": DENSE_COPIES},
        "roofline": {"kernel": "dense_ksplit_kernel", "bound": "hbm",
                     "achieved": round(nbytes / (t["us"] * 1e3), 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(nbytes / (t["us"] * 1e3) / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic("dense_ksplit_kernel"),
                     "bytes_per_launch": nbytes, "avg_launch_us": round(t["us"], 3)},
    }
    if cpu:
        threads = cpu_threads()
        p, s, xh = enc.packed.cpu(), enc.scales.cpu(), x.cpu()
        sec = cpu_median(lambda: cpu_linear(xh, cpu_dequant_w4a16(p, s)))
        res["cpu_baseline"] = {
            "value": round(sec * 1e6, 1), "unit": "us/call", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": "torch restatement: dequantise W [9216, 2304] to bf16 + F.linear fp32, "
                      "the whole call, median of 10 after 3 warm-ups"}
    return res


def zipf_logits(rng, m: int):
    from local_kimi_amd.workloads import zipf_router_logits

    return zipf_router_logits(rng, m, E_ROUTED)


def run_moe_batched(plan: Plan, dev, banks, m: int, weights: str, cpu: bool) -> dict:
    """Configs 3 and 5 (M = 64): M tokens per step, Zipf(1.1)-skewed routing."""
    from local_kimi_amd.kernels import mxfp4_moe_block, w4a16_moe_block

    block = mxfp4_moe_block if weights == "mxfp4" else w4a16_moe_block
    gen = torch.Generator(device=dev).manual_seed(20260731 + m)
    rng = np.random.default_rng(20260731 + m)
    xs = [torch.randn((m, H), device=dev, generator=gen).to(torch.bfloat16) for _ in range(LAYERS)]
    logits = [torch.from_numpy(zipf_logits(rng, m)).to(dev) for _ in range(LAYERS)]
    unions = [int(torch.unique(cpu_router(lg.cpu())[0]).numel()) for lg in logits]
    stream = torch.cuda.Stream(device=dev)

    t = time_steps(lambda l: block(xs[l], logits[l], None, *banks[l], TOP_K, SCALING), LAYERS,
                   stream, plan)
    ebytes = MX_EXPERT_BYTES if weights == "mxfp4" else EXPERT_BYTES
    step_bytes = float(np.mean([(u + 1) * ebytes for u in unions])) + m * TOKEN_IO_BYTES
    gbps = step_bytes / (t["us"] * 1e3)
    log(f"[bench] batched {weights} M={m}: {t['us']:.2f} us/step ({gbps:.0f} GB/s)")
    res = {
        "metric": f"Batched MoE decode us/step + HBM GB/s at {weights.upper()}",
        "value": round(t["us"], 3), "unit": "us/step", "steps": t["steps"],
        "warmup": t["warmup"], "us_per_token": round(t["us"] / m, 3),
        "config": {"workload": f"moe_batched_decode_m{m}", "weights": weights,
                   "tokens_per_step": m, "routing": "Zipf(1.1): log p + Gumbel",
                   "mean_distinct_routed_experts": round(float(np.mean(unions)), 2)},
        "roofline": {"kernel": "whole block (router, schedule, expert GEMMs, combine)",
                     "bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(
                         f"whole block (moe_batched_decode_m{m}"
                         f"{', mxfp4' if weights == 'mxfp4' else ''})"),
                     "bytes_per_step": int(step_bytes)},
    }
    if cpu:
        log(f"[bench] batched {weights} M={m}: CPU baseline")
        res["cpu_baseline"] = cpu_baseline_block(banks[0], xs[0], logits[0], weights, "us/step")
    return res


def run_moe_prefill(plan: Plan, dev, banks, weights: str, cpu: bool) -> dict:
    """Configs 4 and 5: 2048 tokens x top-8 (+ shared) through one layer, N(0,1) logits."""
    from local_kimi_amd.kernels import mxfp4_moe_block, w4a16_moe_block

    block = mxfp4_moe_block if weights == "mxfp4" else w4a16_moe_block
    m = PREFILL_TOKENS
    layers = 4  # 4 x 0.94 GB of weights rotated: each step reads its layer from HBM
    gen = torch.Generator(device=dev).manual_seed(20260733)
    xs = [torch.randn((m, H), device=dev, generator=gen).to(torch.bfloat16) for _ in range(layers)]
    logits = [torch.randn((m, E_ROUTED), device=dev, generator=gen) for _ in range(layers)]
    stream = torch.cuda.Stream(device=dev)

    t = time_steps(lambda l: block(xs[l], logits[l], None, *banks[l], TOP_K, SCALING), layers,
                   stream, plan)
    ebytes = MX_EXPERT_BYTES if weights == "mxfp4" else EXPERT_BYTES
    nbytes = (E_ROUTED + 1) * ebytes + m * TOKEN_IO_BYTES
    flops = m * (TOP_K + 1) * EXPERT_FLOPS
    tflops = flops / (t["us"] * 1e6)
    # the default forms of both formats multiply on bf16 MFMA (MXFP4 weights
    # decoded by the scaled convert), so the bf16 peak is the bound; the fp4
    # one is also reported
    peak = BF16_PEAK_TFLOPS
    log(f"[bench] prefill {weights}: {t['us']:.1f} us/layer ({tflops:.0f} TFLOP/s)")
    res = {
        "metric": f"MoE prefill us/layer + MFMA TFLOP/s at {weights.upper()}",
        "value": round(t["us"], 2), "unit": "us/layer", "steps": t["steps"],
        "warmup": t["warmup"], "tokens_per_s": round(m / (t["us"] * 1e-6), 1),
        "config": {"workload": f"moe_prefill_{m}", "weights": weights, "tokens": m,
                   "routing": "N(0,1) logits"},
        "achieved_gbps": round(nbytes / (t["us"] * 1e3), 1),
        "pct_hbm_peak": round(100 * nbytes / (t["us"] * 1e3) / HBM_PEAK_GBPS, 2),
        "roofline": {"kernel": "whole block (router, schedule, gate/up GEMM, down GEMM, combine)",
                     "bound": "mfma", "achieved": round(tflops, 1), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(tflops / peak, 4),
                     "traffic": measured_traffic(
                         f"whole block (moe_prefill_{m}{', mxfp4' if weights == 'mxfp4' else ''})"),
                     "algorithmic_bytes_per_step": nbytes, "flops_per_step": flops,
                     "frac_of_fp4_peak": round(tflops / FP4_PEAK_TFLOPS, 4)},
    }
    if cpu:
        log(f"[bench] prefill {weights}: CPU baseline")
        res["cpu_baseline"] = cpu_baseline_block(banks[0], xs[0], logits[0], weights, "us/layer")
    return res


def run_qkv_prefill(plan: Plan, dev, cpu: bool) -> dict:
    """Config 4: fused QKV [2048, 2304] x [2304, 3 x 4096] at W4A16, one launch."""
    from local_kimi_amd.kernels import fused_qkv_w4a16
    from local_kimi_amd.quant import quantise

    m, n = PREFILL_TOKENS, QKV_N
    copies = 4
    gen = torch.Generator(device=dev).manual_seed(20260734)
    mats = []
    for _ in range(3):
        enc = quantise((torch.randn((n, H), device=dev, generator=gen) * 0.02).to(torch.bfloat16),
                       group_size=G)
        mats += [enc.packed, enc.scales]
    sets = [mats] + [[t.clone() for t in mats] for _ in range(copies - 1)]
    x = torch.randn((m, H), device=dev, generator=gen).to(torch.bfloat16)
    stream = torch.cuda.Stream(device=dev)

    t = time_steps(lambda i: fused_qkv_w4a16(x, *sets[i]), copies, stream, plan)
    flops = 2 * m * H * 3 * n
    tflops = flops / (t["us"] * 1e6)
    log(f"[bench] fused QKV: {t['us']:.1f} us ({tflops:.0f} TFLOP/s)")
    res = {
        "metric": "Fused QKV prefill GEMM us/call + MFMA TFLOP/s at W4A16",
        "value": round(t["us"], 2), "unit": "us/call", "steps": t["steps"], "warmup": t["warmup"],
        "config": {"workload": f"qkv_prefill_{m}", "m": m, "n_per_projection": n, "k": H,
                   "group_size": G},
        "roofline": {"kernel": "w4a16_stream_kernel (dense, three outputs in one launch)",
                     "bound": "mfma", "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(f"w4a16_stream_kernel (qkv_prefill_{m})"),
                     "algorithmic_bytes_per_launch": 3 * w4a16_bytes(n, H) + m * H * 2 + 3 * m * n * 2,
                     "flops_per_launch": flops, "avg_launch_us": round(t["us"], 2)},
    }
    if cpu:
        threads = cpu_threads()
        host = [a.cpu() for a in mats]
        rows = 256
        xh = x[:rows].cpu()
        deq = lambda: [cpu_dequant_w4a16(host[2 * j], host[2 * j + 1]) for j in range(3)]
        ws = deq()
        t_all = cpu_median(lambda: [cpu_linear(xh, w) for w in deq()])
        t_gemm = cpu_median(lambda: [cpu_linear(xh, w) for w in ws])
        sec = t_all + t_gemm * (m / rows - 1.0)
        res["cpu_baseline"] = {
            "value": round(sec * 1e6, 1), "unit": "us/call", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"torch restatement: dequantise the three [4096, 2304] matrices + F.linear "
                      f"fp32 for {rows} of the {m} rows, timed; the F.linear part scaled by "
                      f"{m}/{rows}; median of 10 after 3 warm-ups"}
    return res


# the reference's published isolated decode figures (L40S, G = 32,
# engine/kernels/RESULTS.md:37-40): context for the same shapes here, on other
# hardware and another group size, so never a vs_baseline ratio
REFERENCE_L40S_US = {"gate_9_routes": 29.7, "w2_9_routes": 30.1, "dense_4096x2304": 55.3,
                     "dense_2304x4096": 62.8}


def _decode_entry(name, t, nbytes, kernel, config, cpu_fn, cpu_sample, cpu):
    t_us = t["us"]
    gbps = nbytes / (t_us * 1e3)
    res = {
        "metric": f"{name} decode us/call + HBM GB/s at W4A16", "value": round(t_us, 3),
        "unit": "us/call", "steps": t["steps"], "warmup": t["warmup"], "config": config,
        "roofline": {"kernel": kernel, "bound": "hbm", "achieved": round(gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(f"{kernel} ({config['workload']})"),
                     "bytes_per_launch": nbytes, "avg_launch_us": round(t_us, 3)},
    }
    if cpu:
        threads = cpu_threads()
        sec = cpu_median(cpu_fn)
        res["cpu_baseline"] = {"value": round(sec * 1e6, 1), "unit": "us/call", "cores": threads,
                               "kind": "port", "cpu_model": cpu_model(), "sample": cpu_sample}
    return res


def run_decode_shapes(plan: Plan, dev, banks, cpu: bool) -> dict:
    """The isolated decode projections whose times the reference publishes
    (engine/kernels/RESULTS.md:37-40): gate alone over 9 routes (N = 1024, K =
    2304), W2 over 9 routes (N = 2304, K = 1024; x [9, 1024], one route per
    row, as moe.py:317-326 calls it), dense N = 4096 x K = 2304 (a KDA q/k/v
    projection) and dense N = 2304 x K = 4096 (o_proj); each call timed alone
    in a graph of calls that rotate the 26 layer banks or 60 dense copies, so
    every call reads HBM."""
    from local_kimi_amd.kernels import grouped_w4a16_gemv, w4a16_dense
    from local_kimi_amd.quant import quantise

    out = {}
    gen = torch.Generator(device=dev).manual_seed(20260737)
    rng = np.random.default_rng(20260737)
    stream = torch.cuda.Stream(device=dev)
    idx = [torch.tensor(np.append(rng.choice(E_ROUTED, TOP_K, replace=False), E_ROUTED)[None],
                        dtype=torch.int64, device=dev) for _ in range(LAYERS)]
    x = torch.randn((1, H), device=dev, generator=gen).to(torch.bfloat16)
    act = (torch.randn((TOP_K + 1, INTER), device=dev, generator=gen) * 0.1).to(torch.bfloat16)
    w2_idx = [i.reshape(TOP_K + 1, 1).contiguous() for i in idx]
    per_route = w4a16_bytes(INTER, H)
    host = [t.cpu() for t in banks[0]]
    hidx = idx[0].cpu()[0]

    t = time_steps(lambda l: grouped_w4a16_gemv(x, idx[l], banks[l][0], banks[l][1]), LAYERS,
                   stream, plan)
    out["gate_9_routes"] = _decode_entry(
        "Grouped gate projection (9 routes)", t,
        (TOP_K + 1) * per_route + H * 2 + (TOP_K + 1) * INTER * 2, "grouped_ksplit_kernel",
        {"workload": "grouped_gate_decode_9_routes", "n": INTER, "k": H, "routes": TOP_K + 1,
         "group_size": G, "reference_l40s_g32_us": REFERENCE_L40S_US["gate_9_routes"]},
        lambda: [cpu_linear(x.cpu(), cpu_dequant_w4a16(host[0][e], host[1][e])) for e in hidx],
        "torch restatement: 9 x (dequantise W1[e] to bf16 + F.linear fp32), median of 10", cpu)
    t = time_steps(lambda l: grouped_w4a16_gemv(act, w2_idx[l], banks[l][4], banks[l][5]),
                   LAYERS, stream, plan)
    out["w2_9_routes"] = _decode_entry(
        "Grouped W2 projection (9 routes)", t,
        (TOP_K + 1) * w4a16_bytes(H, INTER) + (TOP_K + 1) * (INTER + H) * 2,
        "grouped_ksplit_kernel",
        {"workload": "grouped_w2_decode_9_routes", "n": H, "k": INTER, "routes": TOP_K + 1,
         "group_size": G, "reference_l40s_g32_us": REFERENCE_L40S_US["w2_9_routes"]},
        lambda: [cpu_linear(act.cpu()[r:r + 1], cpu_dequant_w4a16(host[4][e], host[5][e]))
                 for r, e in enumerate(hidx)],
        "torch restatement: 9 x (dequantise W2[e] to bf16 + F.linear fp32), median of 10", cpu)
    for n, k in ((4096, H), (H, 4096)):
        enc = quantise((torch.randn((n, k), device=dev, generator=gen) * 0.02).to(torch.bfloat16),
                       group_size=G)
        copies = [(enc.packed.clone(), enc.scales.clone()) for _ in range(60)]
        xk = torch.randn((1, k), device=dev, generator=gen).to(torch.bfloat16)
        t = time_steps(lambda i: w4a16_dense(xk, *copies[i]), len(copies), stream, plan)
        key = f"dense_{n}x{k}"
        hp, hs, hx = enc.packed.cpu(), enc.scales.cpu(), xk.cpu()
        out[key] = _decode_entry(
            f"Dense GEMV N={n} K={k}", t, w4a16_bytes(n, k) + k * 2 + n * 2,
            "dense_ksplit_kernel",
            {"workload": f"dense_gemv_decode_{n}x{k}", "m": 1, "n": n, "k": k, "group_size": G,
             "weight_copies_rotated": len(copies), "reference_l40s_g32_us": REFERENCE_L40S_US[key]},
            lambda: cpu_linear(hx, cpu_dequant_w4a16(hp, hs)),
            f"torch restatement: dequantise W [{n}, {k}] to bf16 + F.linear fp32, median of 10",
            cpu)
        del copies
    log("[bench] decode shapes: " + ", ".join(f"{k} {v['value']:.2f} us" for k, v in out.items()))
    return out


def run_qkv_decode(plan: Plan, dev, cpu: bool) -> dict:
    """Fused QKV at decode: x [1, 2304] . 3 x [4096, 2304] at W4A16 G = 128, one
    launch; 20 weight sets (292 MB) rotated."""
    from local_kimi_amd.kernels import fused_qkv_w4a16
    from local_kimi_amd.quant import quantise

    n, copies = QKV_N, 20
    gen = torch.Generator(device=dev).manual_seed(20260738)
    mats = []
    for _ in range(3):
        enc = quantise((torch.randn((n, H), device=dev, generator=gen) * 0.02).to(torch.bfloat16),
                       group_size=G)
        mats += [enc.packed, enc.scales]
    sets = [mats] + [[t.clone() for t in mats] for _ in range(copies - 1)]
    x = torch.randn((1, H), device=dev, generator=gen).to(torch.bfloat16)
    stream = torch.cuda.Stream(device=dev)
    t = time_steps(lambda i: fused_qkv_w4a16(x, *sets[i]), copies, stream, plan)
    host = [a.cpu() for a in mats]
    hx = x.cpu()
    log(f"[bench] fused QKV decode: {t['us']:.2f} us")
    res = _decode_entry(
        "Fused QKV (one launch)", t, 3 * w4a16_bytes(n, H) + H * 2 + 3 * n * 2,
        "dense_ksplit_kernel",
        {"workload": "qkv_decode", "m": 1, "n_per_projection": n, "k": H, "group_size": G,
         "weight_sets_rotated": copies, "launches": 1},
        lambda: [cpu_linear(hx, cpu_dequant_w4a16(host[2 * j], host[2 * j + 1])) for j in range(3)],
        "torch restatement: dequantise the three [4096, 2304] matrices + F.linear fp32, "
        "median of 10", cpu)
    return res


def run_norm_decode(plan: Plan, dev, cpu: bool) -> dict:
    """The decode norms (next 4): the residual add + RMSNorm of one token's
    hidden state (hidden 2304), the gated RMSNorm of one KDA output (32 heads
    of 128, fp32 values rounded to bf16 in the same launch), and the residual
    add + RMSNorm of a 2048-token prefill (HBM-bound: 37.7 MB moved)."""
    from local_kimi_amd.kernels import add_rms_norm, rms_gated_norm

    gen = torch.Generator(device=dev).manual_seed(20260739)
    stream = torch.cuda.Stream(device=dev)
    bf = torch.bfloat16

    def rnd(shape, dtype=bf, std=1.0):
        return (torch.randn(shape, device=dev, generator=gen) * std).to(dtype)

    w = (1 + rnd((H,), torch.float32, 0.1)).to(bf)
    gw = (1 + rnd((128,), torch.float32, 0.1)).to(bf)
    tok = [(rnd((1, H)), rnd((1, H))) for _ in range(LAYERS)]
    kda = [(rnd((1, 32, 128), torch.float32), rnd((1, 32, 128))) for _ in range(LAYERS)]
    pre = [(rnd((PREFILL_TOKENS, H)), rnd((PREFILL_TOKENS, H))) for _ in range(8)]
    t_add = time_steps(lambda l: add_rms_norm(*tok[l], w, 1e-5), LAYERS, stream, plan)
    t_gated = time_steps(lambda l: rms_gated_norm(*kda[l], gw, 1e-5, input_dtype=bf), LAYERS,
                         stream, plan)
    t_pre = time_steps(lambda l: add_rms_norm(*pre[l], w, 1e-5), len(pre), stream, plan)
    pre_bytes = 4 * PREFILL_TOKENS * H * 2 + H * 2
    gbps = pre_bytes / (t_pre["us"] * 1e3)
    log(f"[bench] norms: add+rmsnorm {t_add['us']:.2f} us, gated {t_gated['us']:.2f} us, "
        f"prefill add+rmsnorm {t_pre['us']:.2f} us ({gbps:.0f} GB/s)")
    res = {
        "metric": "Decode add + RMSNorm us/call (hidden 2304, batch 1)",
        "value": round(t_add["us"], 3), "unit": "us/call", "steps": t_add["steps"],
        "warmup": t_add["warmup"], "higher_is_better": False,
        "config": {"workload": "norm_decode", "hidden": H, "launches": 1},
        "gated_norm_us": round(t_gated["us"], 3),
        "prefill_add_rms_norm_us": round(t_pre["us"], 3),
        "roofline": {"kernel": "norm_kernel (add + RMSNorm, 2048 x 2304 prefill rows)",
                     "bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(
                         "norm_kernel (add + RMSNorm, 2048 x 2304 prefill rows)"),
                     "bytes_per_launch": pre_bytes, "avg_launch_us": round(t_pre["us"], 3)},
    }
    if cpu:
        threads = cpu_threads()
        r, d = (a.cpu() for a in tok[0])
        wh = w.cpu()

        def cpu_add_norm():
            hidden = r + d
            v = hidden.float()
            return hidden, wh * (v * torch.rsqrt(v.square().mean(-1, keepdim=True) + 1e-5)).to(bf)

        sec = cpu_median(cpu_add_norm)
        res["cpu_baseline"] = {"value": round(sec * 1e6, 1), "unit": "us/call", "cores": threads,
                               "kind": "port", "cpu_model": cpu_model(),
                               "sample": "torch restatement of layer.py:156-160 on one token "
                                         "(bf16 add, rms_norm), median of 10"}
    return res


def run_floor(plan: Plan, dev, banks) -> dict:
    """Memory floors: empty-kernel launches, a streaming read of one dense
    weight (11 MB), of one batch-1 MoE layer's 27 matrices (33 MB), and of
    the gate/up weights the batched-decode expert GEMMs read at 16 and 64
    tokens (the mean distinct experts of the Zipf routing, plus the shared
    expert; one contiguous region, four copies rotated)."""
    lib = load_probe_library()
    stream = torch.cuda.Stream(device=dev)
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    s_ptr = stream.cuda_stream

    def checked(rc):
        if rc != 0:
            raise RuntimeError(f"probe failed ({rc}): {lib.lk_probe_last_error().decode()}")

    def probe(regions):
        ptrs = (ctypes.c_void_p * len(regions))(*[r.data_ptr() for r in regions])
        sizes = (ctypes.c_int64 * len(regions))(*[r.numel() * r.element_size() for r in regions])
        checked(lib.lk_probe_stream_read(ptrs, sizes, len(regions), sink.data_ptr(), s_ptr))

    empty = time_steps(lambda i: checked(lib.lk_probe_empty(s_ptr)), 100, stream, plan)
    # one MoE layer's matrices: 9 experts x (gate, up, down) packed weights + scales, per layer
    rng = np.random.default_rng(5)
    layer_sets = []
    for l in range(LAYERS):
        experts = list(rng.choice(E_ROUTED, TOP_K, replace=False)) + [E_ROUTED]
        regions = []
        for e in experts:
            for j in (0, 2, 4):
                regions.append(banks[l][j][e])
        layer_sets.append(regions)  # 27 packed matrices (scales are 3 % more)
    layer_bytes = sum(r.numel() for r in layer_sets[0])
    moe = time_steps(lambda l: probe(layer_sets[l]), LAYERS, stream, plan)
    dense = [torch.empty(w4a16_bytes(DENSE_N, H), dtype=torch.uint8, device=dev).fill_(3)
             for _ in range(DENSE_COPIES)]
    den = time_steps(lambda i: probe([dense[i]]), DENSE_COPIES, stream, plan)
    d_bytes = dense[0].numel()
    del dense
    gateup = {}
    for m in (16, 64):
        rng_m = np.random.default_rng(20260731 + m)
        unions = [int(torch.unique(cpu_router(torch.from_numpy(zipf_logits(rng_m, m)))[0]).numel())
                  for _ in range(LAYERS)]
        nbytes = int(np.mean(unions) + 1) * (EXPERT_BYTES * 2 // 3) // 16 * 16
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(3) for _ in range(4)]
        t = time_steps(lambda i: probe([bufs[i]]), 4, stream, plan)
        gateup[m] = (nbytes, t["us"])
        del bufs
    log(f"[bench] floor: empty {empty['us']:.2f} us, 11 MB {den['us']:.2f} us, "
        f"{layer_bytes / 1e6:.1f} MB in 27 regions {moe['us']:.2f} us, "
        + ", ".join(f"M={m} gate/up {b / 1e6:.0f} MB {u:.2f} us ({b / (u * 1e3):.0f} GB/s)"
                    for m, (b, u) in gateup.items()))
    return {"empty_kernel_us": round(empty["us"], 3),
            **{f"read_gateup_m{m}_{k}": v for m, (b, u) in gateup.items()
               for k, v in (("bytes", b), ("us", round(u, 3)),
                            ("gbps", round(b / (u * 1e3), 1)))},
            "read_11MB_us": round(den["us"], 3), "read_11MB_bytes": d_bytes,
            "read_11MB_gbps": round(d_bytes / (den["us"] * 1e3), 1),
            "read_moe_layer_us": round(moe["us"], 3), "read_moe_layer_bytes": layer_bytes,
            "read_moe_layer_gbps": round(layer_bytes / (moe["us"] * 1e3), 1),
            "kernel": "stream_read_kernel (16-byte non-temporal loads, one launch per step)"}


def load_probe_library() -> ctypes.CDLL:
    """The measurement probes (local_kimi_amd/liblkprobe.so, include/lk_probe.h),
    built beside the product library but not part of it."""
    path = os.path.join(ROOT, "local_kimi_amd", "liblkprobe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run python -m local_kimi_amd._build")
    lib = ctypes.CDLL(path)
    P = ctypes.c_void_p
    lib.lk_probe_stream_read.argtypes = [P, P, ctypes.c_int, P, P]
    lib.lk_probe_stream_read.restype = ctypes.c_int
    lib.lk_probe_empty.argtypes = [P]
    lib.lk_probe_empty.restype = ctypes.c_int
    lib.lk_probe_last_error.argtypes = []
    lib.lk_probe_last_error.restype = ctypes.c_char_p
    return lib


def measured_traffic(kernel: str):
    """HBM bytes per launch (or per step, for a whole block) from rocprofv3
    FETCH_SIZE + WRITE_SIZE, copy-calibrated (profiles/traffic.json)."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return int(json.load(f)["kernels"][kernel]["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def rocprof_avg_us(run: str, kernel: str, grid: str | None = None):
    """Average dispatch duration of a kernel in the committed rocprofv3 trace
    of a bench run (profiles/kernel_times.json), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "kernel_times.json")) as f:
            rows = json.load(f)["runs"][run]["kernels"]
    except (OSError, KeyError, ValueError):
        return None
    hits = [r for r in rows if kernel in r["kernel"] and (grid is None or r["grid"] == grid)]
    return hits[0]["avg_us"] if len(hits) == 1 else None


def run_copy(dev) -> dict:
    """Plain device copy of a known size: calibrates the HBM byte counters."""
    nbytes = 256 << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(10):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 100.0
    return {"metric": "device copy (counter calibration)", "value": round(us, 2),
            "unit": "us/copy", "bytes_read": nbytes, "bytes_written": nbytes}


# ---------------------------------------------------------------------------


def headline(plan: Plan, res: dict) -> dict:
    out = {
        "metric": METRIC, "value": res["value"], "unit": "us/token", "n_gpus": 1,
        "steps": res["steps"], "warmup": res["warmup"], "ms_per_step": res["ms_per_step"],
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,0.02) weights quantised W4A16 g128 on the GPU, N(0,1) x and logits",
        "config": {"workload": "moe_decode_batch1", "hidden": H, "routed_experts": E_ROUTED,
                   "shared_experts": 1, "moe_intermediate": INTER, "top_k": TOP_K,
                   "group_size": G, "tokens_per_step": 1, "layer_banks_rotated": LAYERS,
                   "launches_per_step": 2},
    }
    for key in ("achieved_gbps", "pct_hbm_peak", "algorithmic_bytes_per_step",
                "us_per_token_at_520_steps", "roofline", "cpu_baseline"):
        if key in res:
            out[key] = res[key]
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=DEFAULT_STEPS)
    ap.add_argument("--warmup", type=int, default=DEFAULT_WARMUP)
    ap.add_argument("--workload", default="all",
                    choices=["all", "moe_decode", "dense_decode", "moe_batched", "moe_prefill",
                             "qkv_prefill", "stream_floor", "klinear_decode", "kda_decode",
                             "norm_decode", "qkv_decode", "decode_shapes", "copy"])
    ap.add_argument("--tokens", type=int, default=64, help="moe_batched tokens per step")
    ap.add_argument("--weights", choices=["w4a16", "mxfp4"], default="w4a16",
                    help="moe_batched / moe_prefill expert weight format")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--path", action="append", default=[], metavar="KNOB=CHOICE",
                    help="force one of the library's kernel forms (lk_set_path), e.g. "
                         "mxfp4_mfma=bf16; repeatable")
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
    forced = {}
    for item in args.path:
        knob, sep, choice = item.partition("=")
        if not sep or knob not in _lib.PATH_KNOBS or choice not in _lib.PATH_KNOBS[knob]:
            print(f"--path takes KNOB=CHOICE with a knob and choice of {_lib.PATH_KNOBS}; "
                  f"got {item!r}", file=sys.stderr)
            return 2
        _lib.set_path(knob, choice)
        forced[knob] = choice
    dev = torch.device("cuda:0")
    try:
        plan = Plan(args.steps, args.warmup)
    except ValueError as err:
        print(err, file=sys.stderr)
        return 2
    if args.steps < MIN_TIMED_STEPS or args.warmup < MIN_WARMUP_STEPS:
        log(f"[bench] note: fewer than {MIN_TIMED_STEPS} timed or {MIN_WARMUP_STEPS} warm-up "
            f"steps; the figures are noisier than at the defaults")
    cpu = not args.no_cpu
    log(f"[bench] device {torch.cuda.get_device_name(0)}, workload {args.workload}, "
        f"steps requested {args.steps}, warm-up requested {args.warmup}")
    t0 = time.time()
    w4 = None
    needs_w4a16 = args.workload in ("all", "moe_decode", "stream_floor", "klinear_decode",
                                    "decode_shapes") or (
        args.workload in ("moe_batched", "moe_prefill") and args.weights == "w4a16")
    if needs_w4a16:
        w4 = layer_banks("w4a16", torch.Generator(device=dev).manual_seed(20260729), dev)
        torch.cuda.synchronize()
        log(f"[bench] {LAYERS} W4A16 layer banks ready in {time.time() - t0:.1f}s")

    if args.workload == "all":
        res = headline(plan, run_moe_decode(plan, dev, w4, cpu))
        configs = {"1_dense_gemv": run_dense(plan, dev, cpu)}
        for m in (4, 16, 64):
            configs[f"3_batched_m{m}"] = run_moe_batched(plan, dev, w4, m, "w4a16", cpu)
        configs["4_moe_prefill"] = run_moe_prefill(plan, dev, w4, "w4a16", cpu)
        configs["4_qkv_prefill"] = run_qkv_prefill(plan, dev, cpu)
        configs["qkv_decode"] = run_qkv_decode(plan, dev, cpu)
        for key, entry in run_decode_shapes(plan, dev, w4, cpu).items():
            configs[f"iso_{key}"] = entry
        configs["next1_klinear_decode"] = run_klinear_decode(plan, dev, w4)
        configs["next4_kda_decode"] = run_kda_decode(plan, dev, cpu)
        configs["next4_norm_decode"] = run_norm_decode(plan, dev, cpu)
        res["floor"] = run_floor(plan, dev, w4)
        del w4
        torch.cuda.empty_cache()
        mx = layer_banks("mxfp4", torch.Generator(device=dev).manual_seed(20260735), dev)
        configs["5_mxfp4_batched_m64"] = run_moe_batched(plan, dev, mx, 64, "mxfp4", cpu)
        configs["5_mxfp4_prefill"] = run_moe_prefill(plan, dev, mx, "mxfp4", cpu)
        # the scaled fp4 MFMA form of the same two workloads (the default is bf16 MFMA)
        with _lib.forced_path("mxfp4_mfma", "fp4"):
            for key, fn in (("5_mxfp4_batched_m64_fp4_mfma",
                             lambda: run_moe_batched(plan, dev, mx, 64, "mxfp4", False)),
                            ("5_mxfp4_prefill_fp4_mfma",
                             lambda: run_moe_prefill(plan, dev, mx, "mxfp4", False))):
                configs[key] = fn()
                configs[key]["config"]["mfma_form"] = "fp4 (scaled f8f6f4, fp8 hi/lo activations)"
                configs[key]["roofline"]["traffic"] = None  # counted for the default form only
        res["configs"] = configs
        floor = res["floor"]
        res["roofline"]["frac_of_measured_floor"] = round(
            floor["read_moe_layer_us"] / res["value"], 4)
        configs["1_dense_gemv"]["roofline"]["frac_of_measured_floor"] = round(
            floor["read_11MB_us"] / configs["1_dense_gemv"]["value"], 4)
    elif args.workload == "moe_decode":
        res = headline(plan, run_moe_decode(plan, dev, w4, cpu))
    elif args.workload == "dense_decode":
        res = run_dense(plan, dev, cpu)
    elif args.workload == "moe_batched":
        banks = w4 if args.weights == "w4a16" else layer_banks(
            "mxfp4", torch.Generator(device=dev).manual_seed(20260735), dev)
        res = run_moe_batched(plan, dev, banks, args.tokens, args.weights, cpu)
    elif args.workload == "moe_prefill":
        banks = w4 if args.weights == "w4a16" else layer_banks(
            "mxfp4", torch.Generator(device=dev).manual_seed(20260735), dev, layers=4)
        res = run_moe_prefill(plan, dev, banks, args.weights, cpu)
    elif args.workload == "qkv_prefill":
        res = run_qkv_prefill(plan, dev, cpu)
    elif args.workload == "stream_floor":
        res = run_floor(plan, dev, w4)
    elif args.workload == "klinear_decode":
        res = run_klinear_decode(plan, dev, w4)
    elif args.workload == "kda_decode":
        res = run_kda_decode(plan, dev, cpu)
    elif args.workload == "norm_decode":
        res = run_norm_decode(plan, dev, cpu)
    elif args.workload == "qkv_decode":
        res = run_qkv_decode(plan, dev, cpu)
    elif args.workload == "decode_shapes":
        res = run_decode_shapes(plan, dev, w4, cpu)
    else:
        res = run_copy(dev)
    if forced:
        res["forced_paths"] = forced
    res["bench_seconds"] = round(time.time() - t0, 1)
    print(json.dumps(res), flush=True)
    return 0


def run_klinear_decode(plan: Plan, dev, banks) -> dict:
    """The model-slice caller: KLinearMoE (router logits x Wg^T, then the block)."""
    from local_kimi_amd.checkpoint import MoeBanks
    from local_kimi_amd.klinear import KLinearMoE

    gen = torch.Generator(device=dev).manual_seed(20260736)
    mods = []
    for l in range(LAYERS):
        gate = (torch.randn((E_ROUTED, H), device=dev, generator=gen) * H ** -0.5).to(torch.bfloat16)
        bias = torch.randn((E_ROUTED,), device=dev, generator=gen) * 0.01
        mods.append(KLinearMoE(gate, bias, MoeBanks(*banks[l]), top_k=TOP_K,
                               routed_scaling_factor=SCALING))
    xs = [torch.randn((1, H), device=dev, generator=gen).to(torch.bfloat16) for _ in range(LAYERS)]
    stream = torch.cuda.Stream(device=dev)

    t = time_steps(lambda l: mods[l](xs[l]), LAYERS, stream, plan)
    step_bytes = (TOP_K + 1) * EXPERT_BYTES + TOKEN_IO_BYTES + E_ROUTED * H * 2
    return {"metric": "KLinearMoE decode us/token (router logits + MoE block)",
            "value": round(t["us"], 3), "unit": "us/token", "steps": t["steps"],
            "warmup": t["warmup"], "achieved_gbps": round(step_bytes / (t["us"] * 1e3), 1)}


KDA_HEADS, KDA_DIM, KDA_LAYERS = 32, 128, 160


def run_kda_decode(plan: Plan, dev, cpu: bool) -> dict:
    """KDA decode, batch 1 (next 4): per layer the three short convolutions,
    the gates and the recurrence step on a 32 x 128 x 128 fp32 state; 160
    layers' states (320 MB) rotate so each step reads and writes HBM. `value`
    is the one-launch layer over 8 blocks per head (kda_decode_layer with the
    conv states double-buffered); the one-block-per-head layer and the
    reference's three-launch chain (plus torch's bf16 -> fp32 view of v) are
    timed beside it."""
    from local_kimi_amd.kernels import (fused_kda_gates, fused_short_conv_triple,
                                        kda_decode_layer, kda_decode_step)

    gen = torch.Generator(device=dev).manual_seed(20260740)
    h, d, c = KDA_HEADS, KDA_DIM, KDA_HEADS * KDA_DIM
    bf = torch.bfloat16

    def rnd(shape, std=1.0, dtype=bf):
        return (torch.randn(shape, device=dev, generator=gen) * std).to(dtype)

    ins = [rnd((1, 1, c)) for _ in range(3)]
    conv_w = [rnd((c, 1, 4), 0.3) for _ in range(3)]
    raw_decay, raw_beta = rnd((1, 1, h, d)), rnd((1, 1, h))
    dt_bias = rnd((c,), 1.0, torch.float32)
    a_log = torch.log(torch.rand((1, 1, h, 1), device=dev, generator=gen) * 15 + 1)
    conv_states = [[torch.zeros((1, c, 4), dtype=bf, device=dev) for _ in range(3)]
                   for _ in range(KDA_LAYERS)]
    # the split layer's second conv-state set (a caller alternates the two)
    conv_next = [[torch.zeros((1, c, 4), dtype=bf, device=dev) for _ in range(3)]
                 for _ in range(KDA_LAYERS)]
    rec = [rnd((1, h, d, d), 0.05, torch.float32) for _ in range(KDA_LAYERS)]
    stream = torch.cuda.Stream(device=dev)
    scale = d ** -0.5

    def layer(l):
        q, k, v = fused_short_conv_triple(*ins, *conv_states[l], *conv_w)
        decay, beta, qn, kn = fused_kda_gates(raw_decay, dt_bias, a_log, raw_beta, q, k,
                                              num_heads=h, head_dim=d, eps=1e-6)
        return kda_decode_step(rec[l], qn[:, 0], kn[:, 0], v.view(1, h, d).float(), decay[:, 0],
                               beta[:, 0], scale=scale)

    def one_launch(l):
        kda_decode_layer(*ins, *conv_states[l], *conv_w, raw_decay, dt_bias, a_log, raw_beta,
                         rec[l], num_heads=h, head_dim=d, eps=1e-6, scale=scale,
                         conv_states_out=conv_next[l])

    def one_block_per_head(l):
        kda_decode_layer(*ins, *conv_states[l], *conv_w, raw_decay, dt_bias, a_log, raw_beta,
                         rec[l], num_heads=h, head_dim=d, eps=1e-6, scale=scale)

    qn = torch.randn((1, h, d), device=dev, generator=gen)
    qn = qn / qn.norm(dim=-1, keepdim=True)
    vv = torch.randn((1, h, d), device=dev, generator=gen) * 0.2
    dd = -(0.005 + 0.075 * torch.rand((1, h, d), device=dev, generator=gen))
    bb = torch.sigmoid(torch.randn((1, h), device=dev, generator=gen))

    def step_only(l):
        kda_decode_step(rec[l], qn, qn, vv, dd, bb, scale=scale)

    one = time_steps(one_launch, KDA_LAYERS, stream, plan)
    blk = time_steps(one_block_per_head, KDA_LAYERS, stream, plan)
    t = time_steps(layer, KDA_LAYERS, stream, plan)
    st = time_steps(step_only, KDA_LAYERS, stream, plan)
    state_bytes = h * d * d * 4
    # state in and out; bf16 inputs, conv states (in and out) and weights; small gates
    layer_bytes = (2 * state_bytes + 3 * d * h * 2 * (1 + 4 + 4 + 4) + h * d * (2 + 4) + h * 6
                   + h * d * 4)
    step_bytes = 2 * state_bytes + h * (3 * d + d + 1) * 4 + h * d * 4  # state in + out, q k v decay beta, out
    log(f"[bench] KDA decode: {one['us']:.2f} us/layer in one launch (one block per head "
        f"{blk['us']:.2f} us), three-launch chain {t['us']:.2f} us, step kernel {st['us']:.2f} us")
    res = {
        "metric": "KDA decode us/layer (short convs + gates + recurrence step, batch 1)",
        "value": round(one["us"], 3), "unit": "us/layer", "steps": one["steps"],
        "warmup": one["warmup"], "higher_is_better": False,
        "dtype": "f32 state, bf16 projections",
        "config": {"workload": "kda_decode_batch1", "heads": h, "head_dim": d,
                   "layers_rotated": KDA_LAYERS, "launches_per_layer": 1},
        "one_block_per_head_us": round(blk["us"], 3),
        "three_launch_chain_us": round(t["us"], 3),
        "step_kernel_us": round(st["us"], 3),
        "roofline": {"kernel": "kda_layer_split_kernel (convs + gates + step, one launch, "
                               "8 blocks per head)",
                     "bound": "hbm",
                     "achieved": round(layer_bytes / (one["us"] * 1e3), 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s",
                     "frac": round(layer_bytes / (one["us"] * 1e3) / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic("kda_layer_split_kernel"),
                     "bytes_per_launch": layer_bytes,
                     "avg_launch_us": round(one["us"], 3),
                     "step_kernel_gbps": round(step_bytes / (st["us"] * 1e3), 1)},
    }
    if cpu:
        log("[bench] KDA decode: CPU baseline")
        res["cpu_baseline"] = cpu_kda_layer(ins, conv_states[0], conv_w, raw_decay, dt_bias,
                                            a_log, raw_beta, rec[0], scale)
    return res


def cpu_kda_layer(ins, conv_states, conv_w, raw_decay, dt_bias, a_log, raw_beta, rec, scale):
    """The reference's eager decode path for one KDA layer on the host
    (engine/klinear/attention.py:219-276 through the kda_prepare / kda_step
    reference functions), in torch on all host threads."""
    threads = cpu_threads()
    c_ins = [t.cpu() for t in ins]
    c_states = [t.cpu().clone() for t in conv_states]
    c_w = [t.cpu()[:, 0, :].float() for t in conv_w]
    c_rd, c_rb = raw_decay.cpu(), raw_beta.cpu()
    c_bias, c_alog = dt_bias.cpu(), a_log.cpu()
    c_rec = rec.cpu().clone()
    h, d = KDA_HEADS, KDA_DIM

    def layer():
        outs = []
        for x, st, w in zip(c_ins, c_states, c_w):
            shifted = torch.cat((st[:, :, 1:], x[:, 0].unsqueeze(-1)), dim=-1)
            conv = (shifted.float() * w.unsqueeze(0)).sum(dim=-1)
            outs.append(F.silu(conv).to(x.dtype))
            st.copy_(shifted)
        q, k, v = (o.view(1, h, d).float() for o in outs)
        decay = -c_alog.float().view(1, h, 1).exp() * F.softplus(
            c_rd.float().view(1, h, d) + c_bias.view(h, d))
        beta = torch.sigmoid(c_rb.float().view(1, h))
        q = q * torch.rsqrt(q.square().sum(-1, keepdim=True) + 1e-6)
        k = k * torch.rsqrt(k.square().sum(-1, keepdim=True) + 1e-6)
        cand = c_rec * torch.exp(decay).unsqueeze(-1)
        pred = (cand * k.unsqueeze(-1)).sum(dim=-2)
        cand = cand + beta.unsqueeze(-1).unsqueeze(-1) * k.unsqueeze(-1) * (v - pred).unsqueeze(-2)
        out = (cand * (q * scale).unsqueeze(-1)).sum(dim=-2)
        c_rec.copy_(cand)
        return out

    sec = cpu_median(layer)
    return {"value": round(sec * 1e6, 1), "unit": "us/layer", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": "one KDA layer, batch 1: the three short convolutions, gates and the "
                      "recurrence step in eager torch on the host (the reference's eager path); "
                      "median of 10 after 3 warm-ups"}


if __name__ == "__main__":
    sys.exit(main())
