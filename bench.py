"""Benchmark of TinyEngine's attention step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--quick]

Headline workload (the config the metric is quoted
on): Qwen2.5-Coder-3B-shaped decode attention across all 36 layers at context
8K -- 16 query heads, 2 KV heads, head_dim 128, batch 1, fp16 KV cache.  One
step = one decode token through the attention step of all 36 layers, fused:
    split-K GQA decode attention over positions 0..L, whose prologue applies
    RoPE to q and appends the RoPE'd fp16 k/v at position L (1 launch, all layers)
    combine of the split-K partials                  (1 launch)
The unfused sequence (separate RoPE+append launch, split-K, combine) is timed
too and reported as decode.step_3launch_us.
Inputs are synthetic (torch N(0,1) on the GPU, seed 42; Q scaled by 1/sqrt(128))
and resident in HBM before timing.  Distinct KV caches (>= 1.2 GB in total) are
rotated across steps so the 256 MB MALL cannot serve a step from the previous
one.

Timing: after --warmup-seconds of sustained GPU load (the engine clock ramps
up over the first seconds of work) and W warm-up steps, the step is timed over
K back-to-back steps between two HIP events on the launch stream; each kernel
is also timed alone over K back-to-back launches (the per-kernel average that
rocprofv3 --kernel-trace reports).

Reported: value = microseconds per layer for the whole step; the split-K
kernel's achieved HBM GB/s against the 8 TB/s peak; prefill TFLOP/s (config 3,
L=4096, one layer per launch) against the 2.5 PFLOP/s fp16 dense MFMA peak; the
other BASELINE configs (2K/32K, 7B ragged batch, 1.5B at 128K with outlier keys,
0.5B config 1, chunked prefill) under "configs"; and the reference CPU decode
attention (the reference's own ops.c te_attention_decode_f32 when it was built
into oracle/_ref, else this repository's C restatement) on one host core.
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
INT8_MFMA_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, TOP/s
HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
THETA = 1e6


def decode_bytes(heads: int, kv: int, d: int, positions) -> int:
    """Algorithmic HBM bytes of one fused decode step summed over (seq, layer)
    units: fp16 K+V over positions 0..L (the appended slot included), fp32 q in
    and o out, the new token's fp32 k/v in and fp16 k/v out, one fp32 cos/sin row."""
    return sum(2 * (p + 1) * kv * d * 2 + heads * d * (4 + 4) + kv * d * (2 * 4 + 2 * 2) + d * 4
               for p in positions)


def prefill_flops(heads: int, d: int, tokens: int, base: int = 0) -> float:
    """Causal QK^T + PV FLOPs for one layer: 4*H*D*sum_t(base+t+1)."""
    return 4.0 * heads * d * (tokens * base + tokens * (tokens + 1) / 2)


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--ctx", type=int, default=8192, help="headline decode context length L")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    p.add_argument("--quick", action="store_true", help="headline decode + prefill only")
    p.add_argument("--warmup-seconds", type=float, default=1.0,
                   help="sustained GPU load before timing, so clocks are at their steady state")
    p.add_argument("--profile", action="store_true",
                   help="run a fixed kernel sequence for rocprofv3 (5x decode step at 3B/8K/36 layers, "
                        "5x prefill at L=4096, 3x a 512 MiB device copy for counter calibration) and exit")
    p.add_argument("--profile-layers", action="store_true",
                   help="run a fixed decode-layer sequence for rocprofv3 (10x lm_head GEMV Q4_0 and Q8_0 over "
                        "rotated weight copies, 5x a 3B decode token through 36 layers, 3x a 512 MiB device copy) "
                        "and exit")
    p.add_argument("--prefill-gemm", action="store_true",
                   help="only the prefill GEMM cases (3B gate and down, 512 rows, Q4_0); print their JSON and exit")
    p.add_argument("--phases", action="store_true",
                   help="only the prefill phase table: load the phase-instrumented library "
                        "(python -m tinymetalagent_amd.build --phases), run the causal prefill at 3B L=4096 and "
                        "L=2048 and a 1.5B 2K chunk after 128K, print per-step shader-clock cycles per phase, "
                        "and the rows kernel's wall-clock marks at L=128 and L=512, as JSON and exit")
    p.add_argument("--generate", action="store_true",
                   help="only the end-to-end te_generate_raw case on a 3B-shaped GGUF (Q4_0 and Q8_0); print its "
                        "JSON and exit")
    return p.parse_args()


def settle(torch, fn, seconds: float = 0.25) -> None:
    """Repeat fn for `seconds` of wall time: the engine clock drops while the
    host sets a case up and needs tens of milliseconds of load to recover."""
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        fn()
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def profile_sequence(torch, A) -> None:
    """Fixed launch sequence profiled by the commands recorded under profiles/.
    Each kernel first runs for 0.25 s of wall time (clock settling), so the
    traced averages are steady-state durations.  The device copy (torch's elementwise copy kernel, 512 MiB read + 512 MiB
    written) calibrates FETCH_SIZE / WRITE_SIZE against known bytes."""
    dev = "cuda"
    H, KV, D, LAYERS, L = 16, 2, 128, 36, 8192
    g = torch.Generator(device=dev).manual_seed(42)
    # four KV sets (1.2 GB) rotated as in the timed runs, so the 256 MB MALL
    # cannot serve a launch from the previous one
    sets = [(torch.randn((1, LAYERS, L + 1, KV, D), generator=g, device=dev).half(),
             torch.randn((1, LAYERS, L + 1, KV, D), generator=g, device=dev).half()) for _ in range(4)]
    q = torch.randn((1, LAYERS, 1, H, D), generator=g, device=dev) / math.sqrt(D)
    k = torch.randn((1, LAYERS, 1, KV, D), generator=g, device=dev)
    v = torch.randn((1, LAYERS, 1, KV, D), generator=g, device=dev)
    cos, sin = A.rope_table(L + 1, D, THETA)
    ws = A.decode_workspace(1, LAYERS, H, KV, D, position=L)
    out = torch.empty((1, LAYERS, H, D), dtype=torch.float32, device=dev)
    count = iter(range(1 << 30))

    def step():
        kc, vc = sets[next(count) % 4]
        A.decode_step(q, k, v, cos, sin, kc, vc, position=L, out=out, workspace=ws)

    settle(torch, step)
    for _ in range(5):
        step()
    torch.cuda.synchronize()
    del sets
    Lp = 4096
    qh = torch.randn((1, 1, Lp, H, D), generator=g, device=dev).half()
    kp = torch.randn((1, 1, Lp, KV, D), generator=g, device=dev).half()
    vp = torch.randn((1, 1, Lp, KV, D), generator=g, device=dev).half()
    po = torch.empty((1, 1, Lp, H, D), dtype=torch.float32, device=dev)
    vt = A.value_t_buffer(1, 1, Lp, KV, D)
    A.value_transpose(vp, vt)
    settle(torch, lambda: A.attention_prefill_vt(qh, kp, vt, out=po))
    for _ in range(5):
        A.attention_prefill_vt(qh, kp, vt, out=po)
    torch.cuda.synchronize()
    src = torch.ones(128 << 20, dtype=torch.float32, device=dev)  # 512 MiB
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("profile sequence done: decode step (0.25 s of steps, then 5 more; 3B, L=8192, 36 layers, "
          "4 rotated KV sets), "
          "prefill (0.25 s, then 5 more; L=4096), copy x3 (536870912 B read + written)")


def profile_layers_sequence(torch) -> None:
    """Fixed decode-layer launch sequence profiled by the commands recorded under
    profiles/: the lm_head GEMV (151936 x 2048) in Q4_0 and Q8_0, each after
    0.25 s of settling, 10 launches over weight copies rotated past the MALL;
    then 5 decode tokens through 36 layers at 3B / ctx 8K (Q4_0); then the
    512 MiB device copy that calibrates FETCH_SIZE / WRITE_SIZE."""
    from tinymetalagent_amd import layers as LY
    from tinymetalagent_amd import vecops as V
    for t in (2, 8):
        rows, cols = 151936, 2048
        nbytes = rows * V.row_bytes(t, cols)
        ws = [random_ggml(torch, t, nbytes) for _ in range(max(2, math.ceil(1.2e9 / nbytes)))]
        x = torch.randn(cols, device="cuda")
        out = torch.empty(rows, device="cuda")
        count = iter(range(1 << 30))
        settle(torch, lambda: V.matvec(ws[next(count) % len(ws)], t, x, rows, out=out))
        for i in range(10):
            V.matvec(ws[i % len(ws)], t, x, rows, out=out)
        torch.cuda.synchronize()
        del ws
        torch.cuda.empty_cache()
    decode_layers_case(torch, LY, V, 2, reps=5)
    src = torch.ones(128 << 20, dtype=torch.float32, device="cuda")  # 512 MiB
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("profile sequence done: lm_head GEMV Q4_0 / Q8_0 (0.25 s, then 10 each; rotated copies), "
          "3B decode token x5 (graph), copy x3 (536870912 B read + written)")


def gpu_warmup(torch, A, seconds: float) -> None:
    """Sustained load before any timing: the engine clock of a freshly idle GPU
    ramps up over the first seconds of work (prefill times fall by ~10 % over
    the first three seconds), and every figure here is a steady-state rate."""
    if seconds <= 0:
        return
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(3)
    L, H, KV, D = 4096, 16, 2, 128
    q = torch.randn((1, 1, L, H, D), generator=g, device=dev).half()
    k = torch.randn((1, 1, L, KV, D), generator=g, device=dev).half()
    v = torch.randn((1, 1, L, KV, D), generator=g, device=dev).half()
    out = torch.empty((1, 1, L, H, D), dtype=torch.float32, device=dev)
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(20):
            A.attention_prefill(q, k, v, out=out)
        torch.cuda.synchronize()
    del q, k, v, out


class Timer:
    """Average duration of a launch sequence over back-to-back repetitions."""

    def __init__(self, torch, settle_seconds: float = 0.25):
        self.torch = torch
        self.settle = settle_seconds

    def __call__(self, fn, reps: int, warmup: int = 3) -> float:
        torch = self.torch
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        # keep the GPU busy on this very launch sequence for a moment first
        count = iter(range(1 << 30))
        settle(torch, lambda: fn(next(count)), self.settle)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        stream = torch.cuda.current_stream()
        e0.record(stream)
        for i in range(reps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps  # ms

    def spread(self, fn, reps: int) -> dict:
        """Per-repetition durations (an event between consecutive launches of
        the back-to-back sequence): median, p10, p90 in ms."""
        torch = self.torch
        fn(0)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        ev[0].record(stream)
        for i in range(reps):
            fn(i)
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
        d = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))
        q = lambda f: d[min(reps - 1, int(round(f * (reps - 1))))]
        return {"median": q(0.5), "p10": q(0.1), "p90": q(0.9)}


def mfma_ceilings(torch, timer) -> dict:
    """fp16 MFMA rates this device sustains, measured in the same run as the
    prefill kernel: a register-operand MFMA loop (te_hip_calibrate_mfma_f16: no
    memory, no LDS) and the vendor library's dense fp16 GEMM (hipBLASLt through
    torch.matmul, 8192^3).  The prefill fraction is reported against both."""
    from tinymetalagent_amd.runtime import check, load_library

    lib = load_library()
    blocks, iters = 512, 1000
    sink = torch.empty(blocks * 512, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    check(lib.te_hip_calibrate_mfma_f16(blocks, iters, sink.data_ptr(), stream))
    loop_ms = timer(lambda i: lib.te_hip_calibrate_mfma_f16(blocks, iters, sink.data_ptr(), stream), 10)
    loop_flop = blocks * 8 * iters * 8 * 16 * 16 * 32 * 2
    n = 8192
    a = torch.randn(n, n, device="cuda", dtype=torch.float16)
    b = torch.randn(n, n, device="cuda", dtype=torch.float16)
    c = torch.empty(n, n, device="cuda", dtype=torch.float16)
    gemm_ms = timer(lambda i: torch.matmul(a, b, out=c), 10)
    del a, b, c, sink
    return {"register_mfma_loop_tflops": round(loop_flop / (loop_ms * 1e-3) / 1e12, 1),
            "hipblaslt_fp16_gemm_8192_tflops": round(2.0 * n ** 3 / (gemm_ms * 1e-3) / 1e12, 1)}


def cpu_baseline(sample: dict, heads, kv, d, ctx_len: int, layers: int, seconds: float) -> dict:
    """Reference CPU decode attention on one layer, one pinned core, median of
    reps; and the GPU fused step's output for that layer checked against it.

    The reference step at position ctx_len (qwen.c's per-layer order): rotate q
    and k with te_rope_f32, store k and v at row ctx_len of the cache as fp16,
    then te_attention_decode_f32 over rows 0..ctx_len.  The GPU's layer-0 output
    of the same fused step (sample["out"]) must agree with it to fp16-cache
    rounding: max_abs_err_vs_reference is reported beside the timing."""
    import numpy as np

    import oracle

    use_ref = oracle.ref_lib() is not None
    q_layer = oracle.rope_f32(sample["q"], heads, d, ctx_len, THETA, use_ref=use_ref)
    k_row = oracle.rope_f32(sample["k"], kv, d, ctx_len, THETA, use_ref=use_ref)
    k_layer = sample["kc"].copy()
    v_layer = sample["vc"].copy()
    k_layer[ctx_len] = k_row.astype(np.float16).astype(np.float32)
    v_layer[ctx_len] = sample["v"].astype(np.float16).astype(np.float32)
    want = oracle.attention_decode_f32(q_layer, k_layer, v_layer, ctx_len, heads, kv, d, use_ref=use_ref)
    err = float(np.abs(sample["out"] - want).max())
    # the cache row the GPU appended, against the reference's rotated fp16 k and v
    row_err = max(float(np.abs(sample["kc"][ctx_len] - k_layer[ctx_len]).max()),
                  float(np.abs(sample["vc"][ctx_len] - v_layer[ctx_len]).max()))
    cpus = sorted(os.sched_getaffinity(0))
    old = set(cpus)
    os.sched_setaffinity(0, {cpus[0]})
    try:
        times = []
        t_end = time.perf_counter() + seconds
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 200):
            t0 = time.perf_counter()
            oracle.attention_decode_f32(q_layer, k_layer, v_layer, ctx_len, heads, kv, d, use_ref=use_ref)
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
        "value": round(med * 1e6, 1),
        "unit": "us/layer",
        "cores": 1,
        "kind": "reference" if use_ref else "port",
        "sample": (f"te_attention_decode_f32 ({'reference c/src/ops.c, -std=c11 -O3' if use_ref else 'oracle port'})"
                   f" on one 3B layer at L={ctx_len} (fp16 cache upcast to fp32), {len(times)} reps on one pinned"
                   f" core, median; x{layers} layers = {med * layers * 1e3:.1f} ms per decode step"),
        "cpu_model": model,
        "host_cpus_visible": len(cpus),
        "max_abs_err_vs_reference": err,
        "appended_row_max_abs_err_vs_reference": row_err,
    }


def cpu_prefill_baseline(heads: int, kv: int, d: int, lengths=(512, 2048)) -> dict:
    """Reference CPU causal prefill (the per-token loop: row t = decode at
    position t) for one 3B layer at each length, one pinned core, timed once."""
    import numpy as np

    import oracle

    use_ref = oracle.ref_lib() is not None
    rng = np.random.default_rng(42)
    cpus = sorted(os.sched_getaffinity(0))
    old = set(cpus)
    os.sched_setaffinity(0, {cpus[0]})
    res = {}
    try:
        for L in lengths:
            q = (rng.standard_normal((L, heads * d)) / math.sqrt(d)).astype(np.float32)
            k = rng.standard_normal((L, kv * d)).astype(np.float16).astype(np.float32)
            v = rng.standard_normal((L, kv * d)).astype(np.float16).astype(np.float32)
            t0 = time.perf_counter()
            for t in range(L):
                oracle.attention_decode_f32(q[t], k, v, t, heads, kv, d, use_ref=use_ref)
            res[L] = time.perf_counter() - t0
    finally:
        os.sched_setaffinity(0, old)
    flops = {L: prefill_flops(heads, d, L) for L in lengths}
    last = max(lengths)
    return {
        "value": round(flops[last] / res[last] / 1e9, 3),
        "unit": "GFLOP/s",
        "cores": 1,
        "kind": "reference" if use_ref else "port",
        "sample": (f"causal prefill as the reference runs it (qwen.c:810-824: te_attention_decode_f32 at position t "
                   f"for every row t, {'reference c/src/ops.c' if use_ref else 'oracle port'}), one 3B layer, "
                   + ", ".join(f"L={L}: {res[L]:.2f} s" for L in lengths) + ", one pinned core, timed once"),
    }


def decode_case(torch, A, timer, *, heads, kv, d, layers, positions, reps, min_set_bytes=1.2e9, outliers=False,
                keep_cpu_sample=False, warmup=3, per_layer=False):
    """Decode step over `layers` layers of len(positions) sequences; returns timings."""
    dev = "cuda"
    seqs = len(positions)
    ctx = max(positions) + 1
    cache_bytes = 2 * seqs * layers * ctx * kv * d * 2
    nsets = max(1, min(4, math.ceil(min_set_bytes / cache_bytes)))
    g = torch.Generator(device=dev).manual_seed(42)
    sets = []
    for _ in range(nsets):
        shape = (seqs, layers, ctx, kv, d)
        kc = torch.randn(shape, generator=g, device=dev, dtype=torch.float32)
        if outliers:
            # fixed 2% of channels per KV head carry +-20 spikes (random sign per element)
            nch = max(1, round(0.02 * d))
            gen_cpu = torch.Generator().manual_seed(7)
            for h in range(kv):
                ch = torch.randperm(d, generator=gen_cpu)[:nch].to(dev)
                sign = torch.randint(0, 2, (seqs, layers, ctx, nch), generator=g, device=dev) * 2 - 1
                kc[:, :, :, h, ch] += 20.0 * sign
        kc = kc.half()
        vc = torch.randn(shape, generator=g, device=dev, dtype=torch.float32).half()
        q = torch.randn((seqs, layers, 1, heads, d), generator=g, device=dev) / math.sqrt(d)
        k = torch.randn((seqs, layers, 1, kv, d), generator=g, device=dev)
        v = torch.randn((seqs, layers, 1, kv, d), generator=g, device=dev)
        sets.append((q, k, v, kc, vc))
    cos, sin = A.rope_table(ctx, d, THETA)
    ws = A.decode_workspace(seqs, layers, heads, kv, d, positions=positions)
    out = torch.empty((seqs, layers, heads, d), dtype=torch.float32, device=dev)
    ns = len(sets)

    def rope(i):
        q, k, v, kc, vc = sets[i % ns]
        A.rope_kv_append(q, k, v, cos, sin, kc, vc, base_positions=positions)

    def splitk(i):
        q, k, v, kc, vc = sets[i % ns]
        A.attention_decode(q, kc, vc, positions=positions, out=out, workspace=ws, stage="splitk")

    def combine(i):
        q, k, v, kc, vc = sets[i % ns]
        A.attention_decode(q, kc, vc, positions=positions, out=out, workspace=ws, stage="combine")

    def step_3launch(i):
        rope(i)
        splitk(i)
        combine(i)

    def step_fused(i):
        q, k, v, kc, vc = sets[i % ns]
        A.decode_step(q, k, v, cos, sin, kc, vc, positions=positions, out=out, workspace=ws)

    def step_splitk(i):
        q, k, v, kc, vc = sets[i % ns]
        A.decode_step(q, k, v, cos, sin, kc, vc, positions=positions, workspace=ws, stage="splitk")

    step_ms = timer(step_fused, reps, warmup=warmup)
    spread = timer.spread(step_fused, reps)
    sample = None
    if keep_cpu_sample:
        # The fused step leaves q, k, v in place: one more step on set 0 and its
        # layer-0 output, with the inputs that made it, for the reference check.
        step_fused(0)
        torch.cuda.synchronize()
        q, k, v, kc, vc = sets[0]
        sample = dict(q=q[0, 0, 0].reshape(-1).float().cpu().numpy().copy(),
                      k=k[0, 0, 0].reshape(-1).float().cpu().numpy().copy(),
                      v=v[0, 0, 0].reshape(-1).float().cpu().numpy().copy(),
                      kc=kc[0, 0].float().cpu().numpy().reshape(ctx, -1).copy(),
                      vc=vc[0, 0].float().cpu().numpy().reshape(ctx, -1).copy(),
                      out=out[0, 0].reshape(-1).cpu().numpy().copy())
    fsplitk_ms = timer(step_splitk, reps)
    step3_ms = timer(step_3launch, reps)
    splitk_ms = timer(splitk, reps)
    rope_ms = timer(rope, reps)
    combine_ms = timer(combine, reps)
    nbytes = decode_bytes(heads, kv, d, [p for p in positions for _ in range(layers)])
    res = dict(step_ms=step_ms, step3_ms=step3_ms, fsplitk_ms=fsplitk_ms, splitk_ms=splitk_ms,
               rope_append_ms=rope_ms, combine_ms=combine_ms, bytes_per_step=nbytes, spread=spread,
               splitk_gbs=nbytes / (fsplitk_ms * 1e-3) / 1e9, step_gbs=nbytes / (step_ms * 1e-3) / 1e9)
    if per_layer and seqs == 1:
        # The same step as `layers` separate fused launches (one layer each, as a
        # runtime that finishes layer l before layer l+1 would issue them), eager
        # and captured in one HIP graph.
        ws1 = A.decode_workspace(1, 1, heads, kv, d, positions=positions)
        views = []
        for q, k, v, kc, vc in sets:
            views.append([(q[:, l:l + 1], k[:, l:l + 1], v[:, l:l + 1], kc[:, l:l + 1], vc[:, l:l + 1],
                           out[:, l:l + 1]) for l in range(layers)])

        def layer_by_layer(i):
            for ql, kl, vl, kcl, vcl, ol in views[i % ns]:
                A.decode_step(ql, kl, vl, cos, sin, kcl, vcl, positions=positions, out=ol, workspace=ws1)

        res["per_layer_ms"] = timer(layer_by_layer, max(5, reps // 5))
        layer_by_layer(0)
        torch.cuda.synchronize()
        eager = out.clone()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                layer_by_layer(0)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        same = True
        for _ in range(3):  # every replay must reproduce the eager result
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            same = same and torch.equal(out, eager)
        res["per_layer_graph_ms"] = timer(lambda i: graph.replay(), max(5, reps // 5))
        res["per_layer_graph_matches_eager"] = same
        del graph
    if sample is not None:
        res["cpu_sample"] = sample
    del sets
    torch.cuda.empty_cache()
    return res


def prefill_case(torch, A, timer, *, heads, kv, d, tokens, base=0, chunks=1, reps=10, split=False,
                 check_rows=None):
    """Causal prefill of `chunks` chunks of `tokens` tokens starting at position
    `base` (one layer).  The prefix (positions < base) and every chunk's K/V are
    in the cache, and V^T of the whole cache is built once beforehand, as a
    caller that keeps V^T current has it.  Timed per chunk sequence:
      attention  te_hip_attention_prefill_vt_f16, one split (the headline kernel)
      split      the same with the library's key split (partials + merge launch)
      step       te_hip_attention_prefill_step_vt_f16: bias + RoPE + fp16 append
                 of the chunk's k/v, its V^T, and the attention (the whole
                 BASELINE config-3 step)
      plain      te_hip_attention_prefill_f16, which builds V^T of the prefix
                 itself on every call
      rope       te_hip_rope_kv_append_f16 of q, k, v (the unfused step's first half)
    With check_rows, also the largest difference of those rows of the last chunk
    from the reference decode at position base + t (the oracle)."""
    dev = "cuda"
    ctx = base + chunks * tokens
    g = torch.Generator(device=dev).manual_seed(43)
    kc = torch.randn((1, 1, ctx, kv, d), generator=g, device=dev).half()  # prefix (positions < base)
    vc = torch.randn((1, 1, ctx, kv, d), generator=g, device=dev).half()
    q0 = torch.randn((chunks, 1, 1, tokens, heads, d), generator=g, device=dev).half().float()
    k0 = torch.randn((chunks, 1, 1, tokens, kv, d), generator=g, device=dev).half().float()
    v0 = torch.randn((chunks, 1, 1, tokens, kv, d), generator=g, device=dev).half().float()
    cos, sin = A.rope_table(ctx, d, THETA)
    q, k, v = q0.clone(), k0.clone(), v0.clone()
    qh = torch.empty((chunks, 1, 1, tokens, heads, d), dtype=torch.float16, device=dev)
    out = torch.empty((1, 1, tokens, heads, d), dtype=torch.float32, device=dev)
    for c in range(chunks):
        A.rope_kv_append(q[c], k[c], v[c], cos, sin, kc, vc, base_position=base + c * tokens, q_half=qh[c])
    vt = A.value_t_buffer(1, 1, ctx, kv, d)
    A.value_transpose(vc, vt)
    bases = [base + c * tokens for c in range(chunks)]
    ws = [A.prefill_vt_workspace(1, 1, tokens, heads, kv, d, base_position=b, context_tokens=ctx) for b in bases]

    def attn(i):
        for c in range(chunks):
            A.attention_prefill_vt(qh[c], kc, vt, base_position=bases[c], out=out)

    def attn_split(i):
        for c in range(chunks):
            A.attention_prefill_vt(qh[c], kc, vt, base_position=bases[c], out=out, workspace=ws[c])

    def step_vt(i):
        for c in range(chunks):
            A.prefill_step_vt(q0[c], k0[c], v0[c], cos, sin, kc, vc, vt, base_position=bases[c], out=out,
                              workspace=ws[c])

    def plain(i):
        for c in range(chunks):
            A.attention_prefill(qh[c], kc, vc, base_position=bases[c], out=out)

    def rope(i):
        for c in range(chunks):
            A.rope_kv_append(q[c], k[c], v[c], cos, sin, kc, vc, base_position=bases[c], q_half=qh[c])

    attn_ms = timer(attn, reps, warmup=2)
    res = dict(attention_ms=attn_ms)
    if check_rows:
        import numpy as np

        import oracle

        attn(0)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(tokens, heads, d)
        kb = kc[0, 0].cpu().view(torch.int16).numpy().view(np.uint16)
        vb = vc[0, 0].cpu().view(torch.int16).numpy().view(np.uint16)
        qf = qh[chunks - 1].float().cpu().numpy().reshape(tokens, heads, d)
        worst = 0.0
        for t in check_rows:
            want = oracle.attention_decode_f16kv(qf[t].reshape(1, 1, heads, d).copy(), kb, vb, None,
                                                 bases[-1] + t, 1, 1, ctx, heads, kv, d)
            worst = max(worst, float(np.abs(got[t] - want.reshape(heads, d)).max()))
        # every row against the split-K decode kernel at its position (the
        # same fp16 queries; that kernel is checked against the oracle)
        dec = torch.empty((1, 1, heads, d), dtype=torch.float32, device=dev)
        qd = qh[chunks - 1].float()
        worst_all = torch.zeros((), dtype=torch.float32, device=dev)
        for t in range(tokens):
            A.attention_decode(qd[:, :, t].contiguous(), kc, vc, position=bases[-1] + t, out=dec)
            worst_all = torch.maximum(worst_all, (dec[0, 0] - out[0, 0, t]).abs().max())
        res["check"] = dict(max_abs_err=worst, rows=len(check_rows),
                            max_abs_err_all_rows_vs_decode_kernel=float(worst_all), all_rows=tokens)
    res["step_ms"] = timer(step_vt, reps, warmup=2)
    res["plain_ms"] = timer(plain, reps, warmup=1)
    res["rope_append_ms"] = timer(rope, reps, warmup=1)
    flops = sum(prefill_flops(heads, d, tokens, b) for b in bases)
    res.update(flops=flops, tflops=flops / (attn_ms * 1e-3) / 1e12)
    if split:
        res["split_ms"] = timer(attn_split, reps, warmup=2)
        res["split_tflops"] = flops / (res["split_ms"] * 1e-3) / 1e12
        res["splits"] = [1 if w is None else w.numel() // (tokens * heads * (d + 2) * 4) for w in ws]
    del kc, vc, vt, ws, q0, k0, v0, q, k, v, qh, out
    torch.cuda.empty_cache()
    return res


def prefill_graph_us(torch, A, *, heads, kv, d, tokens, base=0, kernel=None, launches=20, reps=20) -> float:
    """te_hip_attention_prefill_vt_f16 (one split, V^T resident) per launch,
    `launches` launches captured in one HIP graph and replayed: the kernel
    time without the host's launch cost.  kernel "rows" / "tile" forces that
    kernel (TE_HIP_PREFILL_ROWS), None takes the library's choice."""
    ctx = base + tokens
    g = torch.Generator(device="cuda").manual_seed(44)
    kc = torch.randn((1, 1, ctx, kv, d), generator=g, device="cuda").half()
    vc = torch.randn((1, 1, ctx, kv, d), generator=g, device="cuda").half()
    qh = torch.randn((1, 1, tokens, heads, d), generator=g, device="cuda").half()
    vt = A.value_t_buffer(1, 1, ctx, kv, d)
    A.value_transpose(vc, vt)
    out = torch.empty((1, 1, tokens, heads, d), device="cuda")
    old = os.environ.pop("TE_HIP_PREFILL_ROWS", None)
    if kernel is not None:
        os.environ["TE_HIP_PREFILL_ROWS"] = "1" if kernel == "rows" else "0"
    try:
        us = graph_time_us(torch, [lambda s: A.attention_prefill_vt(qh, kc, vt, base_position=base, out=out,
                                                                    stream=s)] * launches, reps)
    finally:
        os.environ.pop("TE_HIP_PREFILL_ROWS", None)
        if old is not None:
            os.environ["TE_HIP_PREFILL_ROWS"] = old
    del kc, vc, qh, vt, out
    torch.cuda.empty_cache()
    return us


def graph_time_us(torch, launches, reps: int) -> float:
    """Mean microseconds per launch of `launches` (a list of callables taking a
    stream), captured once into a HIP graph and replayed: no host launch cost."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    for f in launches:
        f(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for f in launches:
            f(s)
    torch.cuda.synchronize()
    settle(torch, g.replay, 0.25)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * len(launches))


def random_ggml(torch, ggml_type: int, nbytes: int):
    """Random GGUF block bytes on the GPU with every block scale set to a small
    finite fp16 (0x2000 = 2^-7), so no NaN / inf reaches the sums."""
    w = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda")
    blocks = w[: nbytes // (18 if ggml_type == 2 else 34) * (18 if ggml_type == 2 else 34)]
    blocks = blocks.view(-1, 18 if ggml_type == 2 else 34)
    blocks[:, 0] = 0
    blocks[:, 1] = 0x20
    return w


def gemv_case(torch, V, ggml_type: int, rows: int, cols: int, reps: int = 100) -> dict:
    """te_hip_matvec_f32 on a [rows][cols] tensor: weight copies rotated so that
    >= 1.2 GB is streamed per replay round (no MALL reuse), graph-replayed."""
    nbytes = rows * V.row_bytes(ggml_type, cols)
    copies = max(2, min(64, math.ceil(1.2e9 / nbytes)))
    ws = [random_ggml(torch, ggml_type, nbytes) for _ in range(copies)]
    x = torch.randn(cols, device="cuda")
    out = torch.empty(rows, device="cuda")
    us = graph_time_us(torch, [lambda s, w=w: V.matvec(w, ggml_type, x, rows, out=out, stream=s) for w in ws],
                       max(1, reps // copies))
    moved = nbytes + 4 * (cols + rows)
    del ws
    torch.cuda.empty_cache()
    return {"us": r(us, 2), "gbs": round(moved / us / 1e3, 1), "frac": r(moved / us / 1e3 / HBM_PEAK_GBS),
            "bytes_per_launch": moved}


def decode_layers_case(torch, LY, V, ggml_type: int, *, layers=36, heads=16, kv_heads=2, d=128, ffn=11008,
                       vocab=151936, ctx=8192, reps=30) -> dict:
    """One decode token through every layer (te_hip_decode_all_layers_f16) at
    Qwen2.5-3B shapes: position ctx-1, random weights of the given GGUF type (one
    set: at 1.7 / 3.3 GB it exceeds the MALL by itself), greedy head + argmax."""
    hidden, kv = heads * d, kv_heads * d
    rb = lambda cols: V.row_bytes(ggml_type, cols)
    shapes = [("q", hidden, hidden), ("k", kv, hidden), ("v", kv, hidden), ("output", hidden, hidden),
              ("gate", ffn, hidden), ("up", ffn, hidden), ("down", hidden, ffn)]
    offsets, cur, regions = {n: [] for n, _, _ in shapes}, 0, []
    for _ in range(layers):
        for n, rows, cols in shapes:
            offsets[n].append(cur)
            regions.append((cur, rows * rb(cols)))
            cur += (rows * rb(cols) + 255) // 256 * 256
    head_off = cur
    regions.append((cur, vocab * rb(hidden)))
    cur += (vocab * rb(hidden) + 255) // 256 * 256
    mapping = torch.randint(0, 256, (cur,), dtype=torch.uint8, device="cuda")
    bb = 18 if ggml_type == 2 else 34
    for off, n in regions:
        blk = mapping[off:off + n].view(-1, bb)
        blk[:, 0] = 0
        blk[:, 1] = 0x20
    g = torch.Generator(device="cuda").manual_seed(42)
    ones = lambda *shape: torch.ones(*shape, device="cuda")
    an, fn, on = ones(layers, hidden), ones(layers, hidden), ones(hidden)
    qb, kb, vb = (torch.randn(layers, n, generator=g, device="cuda") * 0.1 for n in (hidden, kv, kv))
    from tinymetalagent_amd import attention as A
    cos_t, sin_t = A.rope_table(ctx, d, THETA)
    kc = torch.randn(layers, ctx, kv, generator=g, device="cuda").half()
    vc = torch.randn(layers, ctx, kv, generator=g, device="cuda").half()
    x = torch.randn(hidden, generator=g, device="cuda")
    out, tok = torch.empty_like(x), torch.empty(1, dtype=torch.int32, device="cuda")
    pos = ctx - 1
    wsp = LY.workspace(pos, hidden, kv, heads, kv_heads, d, ffn, vocab)

    def step(s):
        LY.decode_all_layers(mapping, offsets, layers, ggml_type, x, an, fn, qb, kb, vb, cos_t, sin_t, kc, vc, pos,
                             ctx, heads, kv_heads, d, ffn, 1e-6, out=out, head=(head_off, ggml_type), output_norm=on,
                             vocab=vocab, token_out=tok, ws=wsp, stream=s)
    us = graph_time_us(torch, [step], reps)
    wbytes = sum(n for _, n in regions)
    kvbytes = layers * (pos + 1) * kv * 2 * 2
    del mapping, kc, vc
    torch.cuda.empty_cache()
    return {"us_per_token": r(us, 1), "tokens_per_s": round(1e6 / us, 1), "weight_bytes": wbytes,
            "kv_bytes": kvbytes, "gbs": round((wbytes + kvbytes) / us / 1e3, 1),
            "frac": r((wbytes + kvbytes) / us / 1e3 / HBM_PEAK_GBS), "launches_per_token": 6 * layers + 2}


def gemm_case(torch, ggml_type: int, rows: int, n: int, k: int, pre: int = 0, reps: int = 20) -> dict:
    """te_hip_gemm_q_f32 (the batched-prefill projection: activation digits +
    int8-MFMA GEMM) at one prompt-chunk shape, graph-replayed over weight
    copies rotated past the MALL.  Algorithmic work: rows * n * k multiply-adds,
    priced against the dense int8 MFMA peak at two int8 products per
    multiply-add (two activation digits) and, as `frac_algorithmic`, at one."""
    from tinymetalagent_amd import runtime as R
    lib = R.load_library()
    rb = k // 32 * (18 if ggml_type == 2 else 34)
    copies = max(1, int(math.ceil(1.2e9 / (n * rb))))
    ws = [random_ggml(torch, ggml_type, n * rb) for _ in range(copies)]
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(rows, k, generator=g, device="cuda")
    x2 = torch.randn(rows, k, generator=g, device="cuda")
    nw = torch.ones(k, device="cuda")
    out = torch.empty(rows, n, device="cuda")
    act = torch.empty(lib.te_hip_gemm_act_bytes(rows, k), dtype=torch.uint8, device="cuda")
    part = torch.empty(8 * rows * n, device="cuda")
    state = {"i": 0}

    def launch(s):
        w = ws[state["i"] % copies]
        state["i"] += 1
        R.check(lib.te_hip_gemm_q_f32(w.data_ptr(), ggml_type, x.data_ptr(), x2.data_ptr(), nw.data_ptr(), 1e-6, pre,
                                      rows, n, k, out.data_ptr(), None, act.data_ptr(), part.data_ptr(),
                                      part.numel() * 4, s.cuda_stream))
    us = graph_time_us(torch, [launch] * copies, reps)
    macs = rows * n * k
    tops = 2 * macs / us / 1e6
    del ws
    torch.cuda.empty_cache()
    return {"rows": rows, "n": n, "k": k, "us": r(us, 2), "algorithmic_tops": round(tops, 1),
            "int8_mfma_tops": round(2 * tops, 1), "frac": r(2 * tops / INT8_MFMA_PEAK_TOPS),
            "frac_algorithmic": r(tops / INT8_MFMA_PEAK_TOPS)}


def write_3b_gguf(path: str, ggml_type: int, *, layers=36, heads=16, kv_heads=2, d=128, ffn=11008,
                  vocab=151936) -> int:
    """A Qwen2.5-3B-shaped GGUF with random weights (block scales 2^-7, random
    codes), unit norms, small biases and a byte-level vocabulary of `vocab`
    tokens (256 byte symbols, filler tokens, the chat specials), written in
    streaming fashion.  Returns the file size."""
    sys.path.insert(0, str(ROOT / "tests"))
    import numpy as np
    import _gguf as G
    hidden, kv = heads * d, kv_heads * d
    bb = {2: 18, 8: 34}[ggml_type]
    syms = G.gpt2_byte_symbols()
    tokens = syms + [f"tok{i}" for i in range(vocab - 256 - 3)] + G.SPECIALS
    w = G.GGUFWriter(3, 32)
    w.kv("general.architecture", G.STR, "qwen2").kv("general.name", G.STR, "synthetic-qwen2.5-3b")
    for k, v in (("context_length", 32768), ("embedding_length", hidden), ("block_count", layers),
                 ("feed_forward_length", ffn), ("attention.head_count", heads),
                 ("attention.head_count_kv", kv_heads)):
        w.kv(f"qwen2.{k}", G.U32, v)
    w.kv("qwen2.attention.layer_norm_rms_epsilon", G.F32, 1e-6).kv("qwen2.rope.freq_base", G.F32, THETA)
    w.kv("tokenizer.ggml.model", G.STR, "gpt2").kv("tokenizer.ggml.pre", G.STR, "qwen2")
    w.kv("tokenizer.ggml.tokens", G.ARR, (G.STR, tokens))
    w.kv("tokenizer.ggml.token_type", G.ARR, (G.I32, [1] * (vocab - 3) + [3] * 3))
    w.kv("tokenizer.ggml.merges", G.ARR, (G.STR, []))
    w.kv("tokenizer.ggml.eos_token_id", G.U32, vocab - 1).kv("tokenizer.ggml.padding_token_id", G.U32, vocab - 3)
    plan = []  # (name, dims, type, kind, nbytes)
    mats = [("attn_q", hidden, hidden), ("attn_k", kv, hidden), ("attn_v", kv, hidden), ("attn_output", hidden, hidden),
            ("ffn_gate", ffn, hidden), ("ffn_up", ffn, hidden), ("ffn_down", hidden, ffn)]
    for l in range(layers):
        for n, rows, cols in mats:
            plan.append((f"blk.{l}.{n}.weight", (cols, rows), ggml_type, "q", rows * cols // 32 * bb))
        for n, size, kind in (("attn_norm.weight", hidden, "one"), ("ffn_norm.weight", hidden, "one"),
                              ("attn_q.bias", hidden, "small"), ("attn_k.bias", kv, "small"),
                              ("attn_v.bias", kv, "small")):
            plan.append((f"blk.{l}.{n}", (size,), 0, kind, size * 4))
    plan.append(("output_norm.weight", (hidden,), 0, "one", hidden * 4))
    plan.append(("token_embd.weight", (hidden, vocab), ggml_type, "q", vocab * hidden // 32 * bb))
    plan.append(("output.weight", (hidden, vocab), ggml_type, "q", vocab * hidden // 32 * bb))
    off = 0
    for name, dims, t, _, nb in plan:
        w.tensor(name, dims, t, b"", offset=off)
        off = (off + nb + 31) // 32 * 32
    head = w.header()
    rng = np.random.default_rng(7)
    with open(path, "wb") as f:
        f.write(head + b"\0" * ((-len(head)) % 32))
        for name, dims, t, kind, nb in plan:
            if kind == "q":
                blk = rng.integers(0, 256, size=(nb // bb, bb), dtype=np.uint8)
                blk[:, 0], blk[:, 1] = 0, 0x20
                data = blk.tobytes()
            elif kind == "one":
                data = np.ones(nb // 4, np.float32).tobytes()
            else:
                data = (rng.standard_normal(nb // 4) * 0.1).astype(np.float32).tobytes()
            f.write(data + b"\0" * ((-nb) % 32))
    return os.path.getsize(path)


def generate_case(ggml_type: int, prompt_tokens: int = 512, new_tokens: int = 128, ctx: int = 1024) -> dict:
    """End-to-end te_generate_raw on a 3B-shaped GGUF through the public C ABI
    (the reference's own entry point, qwen.c:261-400): load, a prompt of
    `prompt_tokens` byte tokens through the batched prefill (int8-MFMA prompt
    GEMMs and causal attention over 512-row chunks,
    te_hip_prefill_all_layers_f16), then greedy decode with every token
    streamed to the callback.  Times: load (parse + upload of
    the file to HBM on first use), prompt (to the first generated token) and
    decode (tokens after the first, per second)."""
    import ctypes
    import tempfile
    from tinymetalagent_amd import runtime as R
    from tinymetalagent_amd.model import Model, RuntimeOptions
    tmp = os.environ.get("TMPDIR", tempfile.gettempdir())
    path = os.path.join(tmp, f"te_bench_3b_{ggml_type}.gguf")
    t0 = time.perf_counter()
    size = write_3b_gguf(path, ggml_type)
    write_s = time.perf_counter() - t0
    os.environ["TINYENGINE_TEMPERATURE"] = "0"
    os.environ["TINYENGINE_IGNORE_EOS"] = "1"
    out = {"file_bytes": size, "write_s": r(write_s, 2), "prompt_tokens": prompt_tokens, "new_tokens": new_tokens,
           "context_tokens": ctx}
    try:
        m = Model(path, RuntimeOptions(context_tokens=ctx))
        lib = R.load_library()
        for rep in range(2):  # the first run also uploads the file and builds the context state
            stamps = []
            cb = R._TOKEN_CALLBACK(lambda s, i, u: stamps.append(time.perf_counter()))
            hctx = ctypes.c_void_p()
            opts = RuntimeOptions(context_tokens=ctx)._to_c()
            R.check(lib.te_context_create(m.handle, ctypes.byref(opts), ctypes.byref(hctx)))
            t0 = time.perf_counter()
            R.check(lib.te_generate_raw(hctx, b"a" * prompt_tokens, new_tokens, cb, None))
            lib.te_context_free(hctx)
            assert len(stamps) == new_tokens
            key = "first_run" if rep == 0 else "steady"
            out[key] = {"to_first_token_ms": r((stamps[0] - t0) * 1e3, 2),
                        "prompt_tokens_per_s": round(prompt_tokens / (stamps[0] - t0), 1),
                        "decode_tokens_per_s": round((new_tokens - 1) / (stamps[-1] - stamps[0]), 1),
                        "decode_ms_per_token": r((stamps[-1] - stamps[0]) * 1e3 / (new_tokens - 1), 3)}
        # the reference's default sampling (T 0.3, top-k 40): logits come back per token
        os.environ.pop("TINYENGINE_TEMPERATURE")
        stamps = []
        cb = R._TOKEN_CALLBACK(lambda s, i, u: stamps.append(time.perf_counter()))
        hctx = ctypes.c_void_p()
        opts = RuntimeOptions(context_tokens=ctx)._to_c()
        R.check(lib.te_context_create(m.handle, ctypes.byref(opts), ctypes.byref(hctx)))
        R.check(lib.te_generate_raw(hctx, b"a" * prompt_tokens, new_tokens, cb, None))
        lib.te_context_free(hctx)
        out["sampled_t0.3_top40"] = {"decode_tokens_per_s": round((len(stamps) - 1) / (stamps[-1] - stamps[0]), 1),
                                     "decode_ms_per_token": r((stamps[-1] - stamps[0]) * 1e3 / (len(stamps) - 1), 3)}
        os.environ["TINYENGINE_TEMPERATURE"] = "0"
        # a second turn on the same context: the first turn's prompt plus 64
        # new tokens, with the cache reused (default) and recomputed
        for mode in ("1", "0"):
            os.environ["TINYENGINE_KV_REUSE"] = mode
            stamps = []
            cb = R._TOKEN_CALLBACK(lambda s, i, u: stamps.append(time.perf_counter()))
            hctx = ctypes.c_void_p()
            opts = RuntimeOptions(context_tokens=ctx)._to_c()
            R.check(lib.te_context_create(m.handle, ctypes.byref(opts), ctypes.byref(hctx)))
            R.check(lib.te_generate_raw(hctx, b"a" * prompt_tokens, 8, cb, None))
            stamps.clear()
            t0 = time.perf_counter()
            R.check(lib.te_generate_raw(hctx, b"a" * prompt_tokens + b"b" * 64, 8, cb, None))
            lib.te_context_free(hctx)
            key = "second_turn_kv_reuse" if mode == "1" else "second_turn_recomputed"
            out[key] = {"prompt_tokens": prompt_tokens + 64, "to_first_token_ms": r((stamps[0] - t0) * 1e3, 2)}
        os.environ.pop("TINYENGINE_KV_REUSE", None)
        m.close()
    finally:
        os.remove(path)
    return out


def split_fields(p) -> dict:
    """The key-split entry point's figures of a prefill_case(split=True) result."""
    return dict(attention_us=r(p["split_ms"] * 1e3, 2), tflops=round(p["split_tflops"], 1),
                frac=r(p["split_tflops"] / FP16_MFMA_PEAK_TFLOPS), splits=p["splits"])


def r(x, n=4):
    return round(x, n)


def measured_traffic(ctx_len: int):
    """HBM bytes per split-K launch measured with rocprofv3 counters for the
    headline workload (recorded in profiles/), or None for other contexts."""
    import re

    if ctx_len != 8192:
        return None
    path = ROOT / "profiles" / "decode_splitk_3b_ctx8k.md"
    try:
        m = re.search(r"^TRAFFIC_BYTES_PER_LAUNCH=(\d+)$", path.read_text(), re.M)
    except OSError:
        return None
    return int(m.group(1)) if m else None


PHASE_NAMES = ["step start (DMA plan, clamped loads)", "QK^T + weights (with the next step's DMA pieces)",
               "merge: to the exchange + barrier", "reference checks + PV", "merge: normalise + output stores",
               "DMA wait", "barrier", "merge: last barrier", "steps", "prologue"]


def phase_table() -> dict:
    """Per-phase shader-clock cycles of prefill_causal_f16_kernel<128>, from the
    -DTE_PREFILL_PHASES build: every wave sums s_memtime deltas per phase of
    its step loop; reported as the mean over waves, per step (the merge and
    the prologue as totals per wave)."""
    import ctypes

    import torch

    from tinymetalagent_amd import attention as A
    from tinymetalagent_amd import build as B
    from tinymetalagent_amd import runtime as R

    lib = R.load_library()
    if not hasattr(lib, "te_hip_prefill_phase_log_set"):
        raise SystemExit("bench.py --phases: set TINYENGINE_LIBRARY to the phases build "
                         f"({B.PHASE_LIBRARY}; python -m tinymetalagent_amd.build --phases)")
    waves, nph = 8, len(PHASE_NAMES)
    out = {}
    for (h, kv, d, L, base) in [(16, 2, 128, 4096, 0), (16, 2, 128, 2048, 0), (16, 2, 128, 512, 0),
                                (12, 2, 128, 2048, 131072)]:
        ctx = base + L
        g = torch.Generator(device="cuda").manual_seed(1)
        kc = torch.randn((1, 1, ctx, kv, d), generator=g, device="cuda").half()
        vc = torch.randn((1, 1, ctx, kv, d), generator=g, device="cuda").half()
        qh = torch.randn((1, 1, L, h, d), generator=g, device="cuda").half()
        vt = A.value_t_buffer(1, 1, ctx, kv, d)
        A.value_transpose(vc, vt)
        o = torch.empty((1, 1, L, h, d), device="cuda")
        log = torch.zeros(4096 * waves * nph, dtype=torch.int32, device="cuda")
        for _ in range(3):
            A.attention_prefill_vt(qh, kc, vt, base_position=base, out=o)
        torch.cuda.synchronize()
        lib.te_hip_prefill_phase_log_set(ctypes.c_void_p(log.data_ptr()))
        A.attention_prefill_vt(qh, kc, vt, base_position=base, out=o)
        torch.cuda.synchronize()
        lib.te_hip_prefill_phase_log_set(ctypes.c_void_p(0))
        x = log.view(-1, waves, nph).cpu().numpy().astype("float64")
        x = x[x[:, :, 8].sum(axis=1) > 0]
        steps = float(x[:, :, 8].mean())
        case = {"workgroups": int(x.shape[0]), "steps_per_wave": round(steps, 1),
                "cycles_per_wave": round(float(x[:, :, [i for i, nm in enumerate(PHASE_NAMES) if nm not in ("-", "steps")]]
                                         .sum(axis=2).mean()))}
        for i, nm in enumerate(PHASE_NAMES):
            if nm in ("-", "steps"):
                continue
            if i in (2, 4, 7, 9):
                case[nm + " (per wave, total)"] = round(float(x[:, :, i].mean()))
            else:
                case[nm] = round(float(x[:, :, i].mean()) / max(steps, 1.0))
        out[f"H{h}_L{L}_base{base}"] = case
        del kc, vc, qh, vt, o
        torch.cuda.empty_cache()
    return out


ROWS_MARKS = ["start", "first block's weights", "block loop done", "(m, l) exchanged", "rows staged",
              "rows stored"]


def rows_phase_table() -> dict:
    """Wall-clock marks of prefill_rows_f16_kernel<128> (forced on), from the
    -DTE_PREFILL_PHASES build: each wave records s_memrealtime (100 MHz) at
    the marks of ROWS_MARKS; reported in us from the launch's first wave start:
    the slowest workgroup's range over its waves, and the median over
    workgroups of each phase."""
    import ctypes

    import numpy as np
    import torch

    from tinymetalagent_amd import attention as A
    from tinymetalagent_amd import runtime as R

    lib = R.load_library()
    waves, nph = 8, len(PHASE_NAMES)
    out = {}
    os.environ["TE_HIP_PREFILL_ROWS"] = "1"
    try:
        for (h, kv, d, L, base) in [(16, 2, 128, 128, 0), (16, 2, 128, 512, 0)]:
            ctx = base + L
            g = torch.Generator(device="cuda").manual_seed(1)
            kc = torch.randn((1, 1, ctx, kv, d), generator=g, device="cuda").half()
            vc = torch.randn((1, 1, ctx, kv, d), generator=g, device="cuda").half()
            qh = torch.randn((1, 1, L, h, d), generator=g, device="cuda").half()
            vt = A.value_t_buffer(1, 1, ctx, kv, d)
            A.value_transpose(vc, vt)
            o = torch.empty((1, 1, L, h, d), device="cuda")
            nwg = (L + 31) // 32 * h
            log = torch.zeros(nwg * waves * nph, dtype=torch.int32, device="cuda")
            for _ in range(20):
                A.attention_prefill_vt(qh, kc, vt, base_position=base, out=o)
            torch.cuda.synchronize()
            lib.te_hip_prefill_phase_log_set(ctypes.c_void_p(log.data_ptr()))
            A.attention_prefill_vt(qh, kc, vt, base_position=base, out=o)
            torch.cuda.synchronize()
            lib.te_hip_prefill_phase_log_set(ctypes.c_void_p(0))
            t = log.cpu().numpy().view(np.uint32).astype(np.int64).reshape(nwg, waves, nph)[:, :, :len(ROWS_MARKS)]
            us = np.where(t > 0, (t - t[:, :, 0].min()) * 0.01, np.nan)  # a wave without a block has no mark 1
            first = us[:, :, 1]
            crit = int(np.argmax(us[:, :, 5].max(axis=1)))
            case = {"workgroups": nwg, "span_us": round(float(us[:, :, 5].max()), 2),
                    "slowest_workgroup_us": {nm: [round(float(np.nanmin(us[crit, :, i])), 2),
                                                  round(float(np.nanmax(us[crit, :, i])), 2)]
                                             for i, nm in enumerate(ROWS_MARKS)},
                    "median_us": {
                        "start -> first block's weights": round(float(np.nanmedian(first - us[:, :, 0])), 2),
                        "block loop done -> rows staged": round(float(np.median(us[:, :, 4] - us[:, :, 2])), 2),
                        "rows staged -> stored": round(float(np.median(us[:, :, 5] - us[:, :, 4])), 2)}}
            out[f"H{h}_L{L}_base{base}"] = case
            del kc, vc, qh, vt, o
            torch.cuda.empty_cache()
    finally:
        os.environ.pop("TE_HIP_PREFILL_ROWS", None)
    return out


def main():
    args = parse_args()
    if args.phases:
        from tinymetalagent_amd import build as B

        os.environ["TINYENGINE_LIBRARY"] = str(B.PHASE_LIBRARY)
        os.environ["TE_HIP_PREFILL_ROWS"] = "0"
        tile = phase_table()
        print(json.dumps({"prefill_phases_cycles": tile, "prefill_rows_phases_us": rows_phase_table()}))
        return
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
    if args.profile:
        gpu_warmup(torch, A, args.warmup_seconds)
        profile_sequence(torch, A)
        return
    if args.profile_layers:
        gpu_warmup(torch, A, args.warmup_seconds)
        profile_layers_sequence(torch)
        return
    if args.prefill_gemm:
        print(json.dumps({"prefill_gemm_gate_q4_0": gemm_case(torch, 2, 512, 11008, 2048, pre=1, reps=5),
                          "prefill_gemm_down_q4_0": gemm_case(torch, 2, 512, 2048, 11008, pre=2, reps=5)}))
        return
    if args.generate:
        print(json.dumps({"generate": {"q4_0": generate_case(2), "q8_0": generate_case(8),
                                       "prefill_gemm_gate_q4_0": gemm_case(torch, 2, 512, 11008, 2048, pre=1),
                                       "prefill_gemm_down_q4_0": gemm_case(torch, 2, 512, 2048, 11008, pre=2)}}))
        return
    timer = Timer(torch)
    H, KV, D, LAYERS = 16, 2, 128, 36
    K = args.steps
    gpu_warmup(torch, A, args.warmup_seconds)
    dec = decode_case(torch, A, timer, heads=H, kv=KV, d=D, layers=LAYERS, positions=[args.ctx], reps=K,
                      keep_cpu_sample=not args.no_cpu_baseline, warmup=args.warmup, per_layer=True)
    pre = prefill_case(torch, A, timer, heads=H, kv=KV, d=D, tokens=4096, reps=max(5, K // 5),
                       check_rows=None if args.no_cpu_baseline else (0, 1, 63, 64, 1000, 2047, 4000, 4095))
    ceil = mfma_ceilings(torch, timer)
    us_per_layer = dec["step_ms"] * 1e3 / LAYERS
    line = {
        "metric": METRIC,
        "value": r(us_per_layer),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": r(dec["step_ms"], 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"Qwen2.5-3B decode attention step (fused RoPE + fp16 KV append + split-K GQA attention, "
                        f"then combine), "
                        f"all {LAYERS} layers per step, ctx {args.ctx} (BASELINE configs[1])",
            "heads": H, "kv_heads": KV, "head_dim": D, "layers": LAYERS, "context": args.ctx, "batch": 1,
            "kv_cache": "fp16", "softmax_accumulate": "f32", "device": name, "compute_units": cus,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_splitk_f16_kernel<128, FUSED=true>",
            "achieved": round(dec["splitk_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": r(dec["splitk_gbs"] / HBM_PEAK_GBS),
            "traffic": measured_traffic(args.ctx),
            "traffic_source": "profiles/decode_splitk_3b_ctx8k.md: rocprofv3 FETCH_SIZE x2.000 + WRITE_SIZE, "
                              "calibrated on a 512 MiB device copy",
            "bytes_per_launch": dec["bytes_per_step"],
            "launch_us": r(dec["fsplitk_ms"] * 1e3, 2),
        },
        "decode": {
            "step_us": r(dec["step_ms"] * 1e3, 2),
            # per-step distribution, an event recorded between consecutive steps
            "step_us_evented_median_p10_p90": [r(dec["spread"][k] * 1e3, 2) for k in ("median", "p10", "p90")],
            "per_layer_launches_step_us": r(dec["per_layer_ms"] * 1e3, 2),
            "per_layer_launches_graph_step_us": r(dec["per_layer_graph_ms"] * 1e3, 2),
            "per_layer_graph_matches_eager": dec["per_layer_graph_matches_eager"],
            "fused_splitk_us": r(dec["fsplitk_ms"] * 1e3, 2),
            "step_3launch_us": r(dec["step3_ms"] * 1e3, 2),
            "rope_append_us": r(dec["rope_append_ms"] * 1e3, 2),
            "splitk_us": r(dec["splitk_ms"] * 1e3, 2),
            "combine_us": r(dec["combine_ms"] * 1e3, 2),
            "step_hbm_gbs": round(dec["step_gbs"], 1),
            "step_frac_hbm_peak": r(dec["step_gbs"] / HBM_PEAK_GBS),
        },
        "prefill": {
            "workload": "Qwen2.5-3B causal prefill attention, L=4096, one layer per launch (BASELINE configs[2]); "
                        "K and V^T (the transposed value copy the engine keeps) resident",
            "attention_us": r(pre["attention_ms"] * 1e3, 2),
            "rope_append_us": r(pre["rope_append_ms"] * 1e3, 2),
            # the whole prefill step (bias + RoPE + fp16 K/V append + V^T of the
            # chunk + attention), as the engine runs it per layer
            "step_fused_us": r(pre["step_ms"] * 1e3, 2),
            # te_hip_attention_prefill_f16 (plain V layout: builds V^T itself per call)
            "plain_entry_us": r(pre["plain_ms"] * 1e3, 2),
            "tflops": round(pre["tflops"], 1),
            "roofline": {"bound": "mfma", "kernel": "prefill_causal_f16_kernel (V^T operand layout)",
                         "achieved": round(pre["tflops"], 1), "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": r(pre["tflops"] / FP16_MFMA_PEAK_TFLOPS), "flops_per_launch": pre["flops"]},
            # achievable fp16 MFMA rates measured in this run (see mfma_ceilings)
            "ceilings": dict(ceil, frac_of_register_mfma_loop=r(pre["tflops"] / ceil["register_mfma_loop_tflops"]),
                             frac_of_hipblaslt_gemm=r(pre["tflops"] / ceil["hipblaslt_fp16_gemm_8192_tflops"])),
        },
    }
    if "check" in pre:
        line["prefill"]["max_abs_err_vs_reference"] = pre["check"]["max_abs_err"]
        line["prefill"]["reference_check"] = (f"{pre['check']['rows']} rows of the L=4096 output against the "
                                              "oracle's per-token decode over the fp16 cache (row t = decode at t)")
        line["prefill"]["max_abs_err_all_rows_vs_decode_kernel"] = pre["check"][
            "max_abs_err_all_rows_vs_decode_kernel"]
        line["prefill"]["all_rows_check"] = (f"all {pre['check']['all_rows']} rows x 16 heads against the split-K "
                                             "decode kernel at position t (same fp16 queries)")
    if not args.quick:
        cfgs = {}
        reps = max(10, K // 2)
        for L in (2048, 32768):
            c = decode_case(torch, A, timer, heads=16, kv=2, d=128, layers=36, positions=[L], reps=reps)
            cfgs[f"3b_decode_ctx{L}"] = dict(us_per_layer=r(c["step_ms"] * 1e3 / 36), splitk_gbs=round(c["splitk_gbs"], 1),
                                             splitk_frac=r(c["splitk_gbs"] / HBM_PEAK_GBS), step_us=r(c["step_ms"] * 1e3, 2))
        g = torch.Generator().manual_seed(42)
        ragged = [int(x) for x in torch.randint(1024, 16385, (8,), generator=g)]
        c = decode_case(torch, A, timer, heads=28, kv=4, d=128, layers=28, positions=ragged, reps=reps)
        cfgs["7b_decode_ragged8"] = dict(positions=ragged, us_per_layer=r(c["step_ms"] * 1e3 / 28),
                                         splitk_gbs=round(c["splitk_gbs"], 1),
                                         splitk_frac=r(c["splitk_gbs"] / HBM_PEAK_GBS), step_us=r(c["step_ms"] * 1e3, 2))
        c = decode_case(torch, A, timer, heads=12, kv=2, d=128, layers=28, positions=[131072], reps=max(5, reps // 2),
                        outliers=True)
        cfgs["1p5b_decode_128k_outliers"] = dict(us_per_layer=r(c["step_ms"] * 1e3 / 28),
                                                 splitk_gbs=round(c["splitk_gbs"], 1),
                                                 splitk_frac=r(c["splitk_gbs"] / HBM_PEAK_GBS),
                                                 step_us=r(c["step_ms"] * 1e3, 2))
        c = decode_case(torch, A, timer, heads=14, kv=2, d=64, layers=1, positions=[512], reps=reps)
        cfgs["0p5b_decode_pos512_1layer"] = dict(step_us=r(c["step_ms"] * 1e3, 2), splitk_us=r(c["splitk_ms"] * 1e3, 2))
        for L in (512, 2048):
            p = prefill_case(torch, A, timer, heads=16, kv=2, d=128, tokens=L, reps=20, split=True)
            gus = prefill_graph_us(torch, A, heads=16, kv=2, d=128, tokens=L)
            cfgs[f"3b_prefill_L{L}"] = dict(attention_us=r(p["attention_ms"] * 1e3, 2), tflops=round(p["tflops"], 1),
                                            frac=r(p["tflops"] / FP16_MFMA_PEAK_TFLOPS),
                                            attention_graph_us=r(gus, 2),
                                            step_fused_us=r(p["step_ms"] * 1e3, 2),
                                            split_entry=split_fields(p))
        # prompts of at most 256 keys take the rows kernel; both kernels timed
        for L in (128, 256):
            rows_us = prefill_graph_us(torch, A, heads=16, kv=2, d=128, tokens=L)
            tile_us = prefill_graph_us(torch, A, heads=16, kv=2, d=128, tokens=L, kernel="tile")
            fl = prefill_flops(16, 128, L, 0)
            cfgs[f"3b_prefill_L{L}"] = dict(kernel="prefill_rows_f16_kernel", attention_graph_us=r(rows_us, 2),
                                            tflops=round(fl / rows_us / 1e6, 1),
                                            tile_kernel_graph_us=r(tile_us, 2))
        p = prefill_case(torch, A, timer, heads=12, kv=2, d=128, tokens=2048, base=0, chunks=8, reps=3, split=True)
        cfgs["1p5b_chunked_prefill_16k_from0"] = dict(chunks=8, chunk_tokens=2048, attention_ms=r(p["attention_ms"], 3),
                                                     step_fused_ms=r(p["step_ms"], 3),
                                                     tflops=round(p["tflops"], 1),
                                                     frac=r(p["tflops"] / FP16_MFMA_PEAK_TFLOPS),
                                                     split_entry=split_fields(p))
        p = prefill_case(torch, A, timer, heads=12, kv=2, d=128, tokens=2048, base=131072, chunks=8, reps=2,
                         split=True)
        cfgs["1p5b_chunked_prefill_16k_after128k"] = dict(chunks=8, chunk_tokens=2048, base=131072,
                                                         attention_ms=r(p["attention_ms"], 3),
                                                         step_fused_ms=r(p["step_ms"], 3),
                                                         tflops=round(p["tflops"], 1),
                                                         frac=r(p["tflops"] / FP16_MFMA_PEAK_TFLOPS),
                                                         split_entry=split_fields(p))
        line["configs"] = cfgs
        # the decode-layer slot around attention: quantized projections and the
        # whole token through every layer (one GPU, batch 1, greedy head)
        from tinymetalagent_amd import layers as LY
        from tinymetalagent_amd import vecops as V
        line["decode_layers"] = {
            "workload": "Qwen2.5-3B decode token: 36 x (RMSNorm + QKV GEMV, fused decode step, Wo + residual, "
                        "RMSNorm + gate/up GEMV, SwiGLU + down GEMV + residual), then RMSNorm + lm_head + argmax; "
                        "ctx 8K, random GGUF weights",
            "gemv_lm_head_q4_0": gemv_case(torch, V, 2, 151936, 2048),
            "gemv_lm_head_q8_0": gemv_case(torch, V, 8, 151936, 2048),
            "gemv_gate_q4_0": gemv_case(torch, V, 2, 11008, 2048),
            "gemv_down_q4_0": gemv_case(torch, V, 2, 2048, 11008),
            "token_q4_0": decode_layers_case(torch, LY, V, 2),
            "token_q8_0": decode_layers_case(torch, LY, V, 8),
        }
        # generation through the public C ABI on a 3B-shaped GGUF
        line["generate"] = {
            "workload": "te_generate_raw on a Qwen2.5-3B-shaped GGUF (random weights, 151936-token byte-level "
                        "vocabulary): 512 prompt tokens through the batched int8-MFMA prefill (512-row chunks), "
                        "then 128 greedy tokens; ctx 1024",
            "q4_0": generate_case(2),
            "prefill_gemm_gate_q4_0": gemm_case(torch, 2, 512, 11008, 2048, pre=1),
            "prefill_gemm_down_q4_0": gemm_case(torch, 2, 512, 2048, 11008, pre=2),
        }
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(dec["cpu_sample"], H, KV, D, args.ctx, LAYERS, args.cpu_seconds)
        cpu["gpu_speedup"] = round(cpu["value"] / us_per_layer, 1)
        line["decode"]["max_abs_err_vs_reference"] = cpu.pop("max_abs_err_vs_reference")
        line["decode"]["appended_row_max_abs_err_vs_reference"] = cpu.pop("appended_row_max_abs_err_vs_reference")
        line["decode"]["reference_check"] = (
            f"layer 0 of the fused step at position {args.ctx} against {cpu['kind']} te_rope_f32 + fp16 store + "
            f"te_attention_decode_f32 on the host")
        line["cpu_baseline"] = cpu
        if not args.quick:
            cp = cpu_prefill_baseline(H, KV, D)
            cp["gpu_speedup_L4096"] = round(pre["tflops"] * 1e3 / cp["value"], 1)
            line["cpu_baseline_prefill"] = cp
    print(json.dumps(line))


if __name__ == "__main__":
    main()
