"""Benchmark of TinyEngine's attention step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--ctx 8192] [--no-cpu-baseline]

Workload (the config the metric is quoted on):
Qwen2.5-Coder-3B-shaped decode attention across all 36 layers at context 8K --
16 query heads, 2 KV heads, head_dim 128, batch 1, fp16 KV cache.  One step =
one decode token through the attention step of all 36 layers:
    RoPE(q, k) + fp16 append of k/v at position L   (1 launch, all layers)
    split-K GQA decode attention over positions 0..L (1 launch, all layers)
    combine of the split-K partials                  (1 launch)
Inputs are synthetic (torch N(0,1) on the GPU, seed 42; Q scaled by 1/sqrt(128))
and resident in HBM before timing.  Four distinct KV caches (~1.2 GB total) are
rotated across steps so the 256 MB MALL cannot serve a step from the previous
one.

Reported: value = microseconds per layer for the whole step; the split-K
kernel's achieved HBM GB/s against the 8 TB/s peak from HIP events on the
launch stream; prefill TFLOP/s (config 3, L=4096, one layer per launch) against
the 2.5 PFLOP/s fp16 dense MFMA peak; and the reference CPU decode attention
(the reference's own ops.c te_attention_decode_f32 when it was built into
oracle/_ref, else this repository's C restatement) timed on one host core.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode-attn µs/layer + HBM GB/s (% peak) at Qwen2.5-3B, ctx 8K; prefill TFLOP/s"
HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0

H, KV, D, LAYERS = 16, 2, 128, 36
THETA = 1e6


def decode_bytes_per_layer(ctx_len: int) -> int:
    """Algorithmic HBM bytes of decode attention for one (seq, layer): fp16 K+V
    over positions 0..L plus fp32 q in and o out (BASELINE.md / SURVEY 8(d))."""
    return 2 * (ctx_len + 1) * KV * D * 2 + H * D * (4 + 4)


def prefill_flops(tokens: int, base: int = 0) -> float:
    """Causal QK^T + PV FLOPs for one layer: 4*H*D*sum_t(base+t+1)."""
    return 4.0 * H * D * (tokens * base + tokens * (tokens + 1) / 2)


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--ctx", type=int, default=8192, help="decode context length L (query at position L)")
    p.add_argument("--kv-sets", type=int, default=4, help="distinct KV caches rotated across steps")
    p.add_argument("--prefill-tokens", type=int, default=4096)
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    return p.parse_args()


def cpu_baseline(q_layer, k_layer, v_layer, ctx_len: int, seconds: float) -> dict:
    """Reference CPU decode attention on one layer, one pinned core, median of reps."""
    import numpy as np

    import oracle

    use_ref = oracle.ref_lib() is not None
    kind = "reference" if use_ref else "port"
    cpus = sorted(os.sched_getaffinity(0))
    old = set(cpus)
    os.sched_setaffinity(0, {cpus[0]})
    try:
        times = []
        t_end = time.perf_counter() + seconds
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 200):
            t0 = time.perf_counter()
            oracle.attention_decode_f32(q_layer, k_layer, v_layer, ctx_len, H, KV, D, use_ref=use_ref)
            times.append(time.perf_counter() - t0)
    finally:
        os.sched_setaffinity(0, old)
    med = statistics.median(times)
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": med * 1e6,
        "unit": "us/layer",
        "cores": 1,
        "kind": kind,
        "sample": (f"te_attention_decode_f32 ({'reference c/src/ops.c, -std=c11 -O3' if use_ref else 'oracle port'})"
                   f" on one 3B layer at L={ctx_len} (fp16 cache upcast to fp32), {len(times)} reps, median;"
                   f" x{LAYERS} layers = {med * LAYERS * 1e3:.1f} ms per decode step"),
        "cpu_model": model,
        "host_cpus_visible": len(cpus),
    }


def bench_decode(torch, A, args) -> dict:
    dev = "cuda"
    L = args.ctx
    ctx = L + 1
    g = torch.Generator(device=dev).manual_seed(42)
    sets = []
    for _ in range(args.kv_sets):
        kc = torch.randn((1, LAYERS, ctx, KV, D), generator=g, device=dev, dtype=torch.float32).half()
        vc = torch.randn((1, LAYERS, ctx, KV, D), generator=g, device=dev, dtype=torch.float32).half()
        q = torch.randn((1, LAYERS, 1, H, D), generator=g, device=dev) / math.sqrt(D)
        k = torch.randn((1, LAYERS, 1, KV, D), generator=g, device=dev)
        v = torch.randn((1, LAYERS, 1, KV, D), generator=g, device=dev)
        sets.append((q, k, v, kc, vc))
    cos, sin = A.rope_table(ctx, D, THETA)
    ws = A.decode_workspace(1, LAYERS, H, KV, D, position=L)
    out = torch.empty((1, LAYERS, H, D), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()

    def step(i, ev=None):
        q, k, v, kc, vc = sets[i % len(sets)]
        if ev is not None:
            ev[0].record(stream)
        A.rope_kv_append(q, k, v, cos, sin, kc, vc, base_position=L)
        if ev is not None:
            ev[1].record(stream)
        A.attention_decode(q, kc, vc, position=L, out=out, workspace=ws, stage="splitk")
        if ev is not None:
            ev[2].record(stream)
        A.attention_decode(q, kc, vc, position=L, out=out, workspace=ws, stage="combine")
        if ev is not None:
            ev[3].record(stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # whole-step timing: K back-to-back steps bracketed by events
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(args.steps):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    # per-kernel timing: events between the three launches of every step
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    rope_ms = [e[0].elapsed_time(e[1]) for e in evs]
    splitk_ms = [e[1].elapsed_time(e[2]) for e in evs]
    comb_ms = [e[2].elapsed_time(e[3]) for e in evs]
    splitk_avg = sum(splitk_ms) / len(splitk_ms)
    bytes_launch = decode_bytes_per_layer(L) * LAYERS
    achieved = bytes_launch / (splitk_avg * 1e-3) / 1e9
    step_gbs = bytes_launch / (ms_per_step * 1e-3) / 1e9
    q_cpu = sets[0][0][0, 0, 0].reshape(-1).float().cpu().numpy().copy()
    k_cpu = sets[0][3][0, 0].float().cpu().numpy().reshape(-1).copy()
    v_cpu = sets[0][4][0, 0].float().cpu().numpy().reshape(-1).copy()
    del sets
    torch.cuda.empty_cache()
    return dict(ms_per_step=ms_per_step, rope_ms=sum(rope_ms) / len(rope_ms), splitk_ms=splitk_avg,
                splitk_p10=sorted(splitk_ms)[len(splitk_ms) // 10], splitk_p90=sorted(splitk_ms)[(9 * len(splitk_ms)) // 10],
                combine_ms=sum(comb_ms) / len(comb_ms), bytes_per_launch=bytes_launch, achieved_gbs=achieved,
                step_gbs=step_gbs, cpu_inputs=(q_cpu, k_cpu, v_cpu))


def bench_prefill(torch, A, args) -> dict:
    dev = "cuda"
    Lp = args.prefill_tokens
    g = torch.Generator(device=dev).manual_seed(43)
    q = torch.randn((1, 1, Lp, H, D), generator=g, device=dev).half().float()
    k = torch.randn((1, 1, Lp, KV, D), generator=g, device=dev).half().float()
    v = torch.randn((1, 1, Lp, KV, D), generator=g, device=dev).half().float()
    cos, sin = A.rope_table(Lp, D, THETA)
    kc = torch.empty((1, 1, Lp, KV, D), dtype=torch.float16, device=dev)
    vc = torch.empty_like(kc)
    qh = torch.empty((1, 1, Lp, H, D), dtype=torch.float16, device=dev)
    out = torch.empty((1, 1, Lp, H, D), dtype=torch.float32, device=dev)
    q0, k0, v0 = q.clone(), k.clone(), v.clone()
    stream = torch.cuda.current_stream()
    steps = max(5, args.steps // 2)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for i in range(-3, steps):
        q.copy_(q0)
        k.copy_(k0)
        v.copy_(v0)
        e = evs[i] if i >= 0 else None
        if e:
            e[0].record(stream)
        A.rope_kv_append(q, k, v, cos, sin, kc, vc, base_position=0, q_half=qh)
        if e:
            e[1].record(stream)
        A.attention_prefill(qh, kc, vc, base_position=0, out=out)
        if e:
            e[2].record(stream)
    torch.cuda.synchronize()
    att_ms = [e[1].elapsed_time(e[2]) for e in evs]
    rope_ms = [e[0].elapsed_time(e[1]) for e in evs]
    avg = sum(att_ms) / len(att_ms)
    flops = prefill_flops(Lp)
    tflops = flops / (avg * 1e-3) / 1e12
    return dict(tokens=Lp, attention_ms=avg, rope_append_ms=sum(rope_ms) / len(rope_ms), flops=flops,
                tflops=tflops, frac=tflops / FP16_MFMA_PEAK_TFLOPS, steps=steps)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    from tinymetalagent_amd import attention as A
    from tinymetalagent_amd import runtime as R

    if not R.hip_available():
        raise SystemExit("bench.py: libtinyengine.so found no gfx950 GPU")
    name, cus = R.device_info()
    dec = bench_decode(torch, A, args)
    pre = None if args.no_prefill else bench_prefill(torch, A, args)
    cpu = None
    if not args.no_cpu_baseline:
        q_cpu, k_cpu, v_cpu = dec["cpu_inputs"]
        cpu = cpu_baseline(q_cpu, k_cpu, v_cpu, args.ctx, args.cpu_seconds)
    us_per_layer = dec["ms_per_step"] * 1e3 / LAYERS
    line = {
        "metric": METRIC,
        "value": round(us_per_layer, 4),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"Qwen2.5-3B decode attention step (RoPE + fp16 KV append + split-K GQA attention), "
                        f"all {LAYERS} layers per step, ctx {args.ctx} (BASELINE configs[1])",
            "heads": H, "kv_heads": KV, "head_dim": D, "layers": LAYERS, "context": args.ctx, "batch": 1,
            "kv_cache": "fp16", "softmax_accumulate": "f32", "kv_sets_rotated": args.kv_sets,
            "device": name, "compute_units": cus,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_splitk_f16_kernel<128>",
            "achieved": round(dec["achieved_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["achieved_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": None,
            "bytes_per_launch": dec["bytes_per_launch"],
            "launch_ms": round(dec["splitk_ms"], 5),
        },
        "decode": {
            "step_ms": round(dec["ms_per_step"], 5),
            "rope_append_ms": round(dec["rope_ms"], 5),
            "splitk_ms": round(dec["splitk_ms"], 5),
            "splitk_p10_ms": round(dec["splitk_p10"], 5),
            "splitk_p90_ms": round(dec["splitk_p90"], 5),
            "combine_ms": round(dec["combine_ms"], 5),
            "attention_us_per_layer": round((dec["splitk_ms"] + dec["combine_ms"]) * 1e3 / LAYERS, 4),
            "step_hbm_gbs": round(dec["step_gbs"], 1),
            "step_frac_hbm_peak": round(dec["step_gbs"] / HBM_PEAK_GBS, 4),
        },
    }
    if pre is not None:
        line["prefill"] = {
            "workload": f"Qwen2.5-3B causal prefill attention, L={pre['tokens']}, one layer per launch "
                        "(BASELINE configs[2])",
            "attention_ms": round(pre["attention_ms"], 5),
            "rope_append_ms": round(pre["rope_append_ms"], 5),
            "tflops": round(pre["tflops"], 2),
            "roofline": {"bound": "mfma", "kernel": "prefill_causal_f16_kernel<128>",
                         "achieved": round(pre["tflops"], 2), "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pre["frac"], 4), "flops_per_launch": pre["flops"]},
        }
    if cpu is not None:
        line["cpu_baseline"] = cpu
        line["cpu_baseline"]["gpu_speedup"] = round(cpu["value"] / us_per_layer, 1)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
