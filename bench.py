#!/usr/bin/env python3
"""Benchmark: Qwen3-4B-shaped native-INT4 decode-layer MLP on one MI355X.

Workload: hidden 2560, intermediate 9728; per layer
the fused gate+up projection with SwiGLU (TrySwiGLUVector, one kernel) then the
down projection (Int4Linear), 36 layers with independent seeds, batch 1.  A
"step" is one token through the 36 layers, the output of layer l feeding layer
l+1.  Weights are bf16 N(0, 0.02) (truncated from fp32 as SingleToBF16 does)
packed with QuickNN's INT4 algorithm; activations fp32 N(0,1) RMS-normalised
with unit gamma.  The 36-layer weight set (1.68 GB) exceeds the 256 MB MALL,
so every step streams its weights from HBM.

value = algorithmic bytes per step (packed weights + activations read once +
outputs written once) / measured time per step, in GB/s.

Also reported: us/layer and tokens/s; the dominant kernel's roofline (the
fused gate/up SwiGLU matvec: algorithmic bytes per launch over its average
launch time, from HIP events on the context stream around 36-launch runs of
it); batch-8 figures; and the reference's CPU SIMD path (an AVX2 restatement in
the CPU oracle) timed on this host on the same packed weights.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HIDDEN, INTER, LAYERS = 2560, 9728, 36
HBM_PEAK_GBS = 8000.0


def make_layer(seed: int, hip):
    rng = np.random.default_rng(seed)

    def mat(n, k):
        w = rng.standard_normal((n, k), dtype=np.float32)
        w *= np.float32(0.02)
        b = (w.view(np.uint32) >> 16).astype(np.uint16)  # SingleToBF16 truncation
        return hip.quantize_int4(b)

    return mat(INTER, HIDDEN), mat(INTER, HIDDEN), mat(HIDDEN, INTER)


def layer_bytes(m: int, hip) -> tuple[int, int]:
    """(weight bytes, activation bytes) per layer at batch m."""
    w = 2 * INTER * hip.int4_row_bytes(HIDDEN) + HIDDEN * hip.int4_row_bytes(INTER)
    act = 4 * m * (HIDDEN + INTER + INTER + HIDDEN)  # x in, h out, h in, y out
    return w, act


def cpu_baseline(packed, x0: np.ndarray, budget_s: float, wbytes: int, abytes: int) -> dict:
    """The reference's CPU direct-matvec path (TCPUProjection.Linear with the
    AVX2 Int4VectorDot, QwenHybrid.CPU.pas:238-248 composition), restated in
    the oracle, at the reference default of min(8, nproc) worker threads."""
    import oracle

    pool = oracle.Pool(0)
    layers_done, t0 = 0, time.perf_counter()
    x = x0.copy()
    while True:
        g, u, d = packed[layers_done % LAYERS]
        x = oracle.cpu_mlp(g, u, d, oracle.ENC_INT4, x, HIDDEN, INTER, pool)[0]
        layers_done += 1
        el = time.perf_counter() - t0
        if el >= budget_s and layers_done >= LAYERS:
            break
    us_layer = el / layers_done * 1e6
    return {"value": round((wbytes + abytes) / (us_layer * 1e-6) / 1e9, 2), "unit": "GB/s",
            "cores": pool.threads, "kind": "port",
            "sample": f"{layers_done} INT4 MLP layers at batch 1 ({el:.1f} s), same packed weights; "
                      f"{us_layer:.0f} us/layer; nproc={os.cpu_count()}"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(sharding the path over several GPUs is a design note, not built)", file=sys.stderr)
        return 2

    from quicknn_amd import hip

    t0 = time.perf_counter()
    packed = [make_layer(1000 + l, hip) for l in range(LAYERS)]
    gen_s = time.perf_counter() - t0
    blocks = [tuple(hip.MemoryBlock.int4(p) for p in lay) for lay in packed]
    rng = np.random.default_rng(7)
    raw = rng.standard_normal((8, HIDDEN)).astype(np.float32)
    x8 = raw / np.sqrt(np.mean(raw.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6).astype(np.float32)
    x1 = x8[0].copy()

    wbytes, abytes1 = layer_bytes(1, hip)
    _, abytes8 = layer_bytes(8, hip)

    ctx = hip.GPUContext(0)
    x = ctx.UploadRaw(x1)
    h = ctx.NewTensor(INTER)
    ya, yb = ctx.NewTensor(HIDDEN), ctx.NewTensor(HIDDEN)

    def step():
        src, outs = x, (ya, yb)
        for l, (g, u, d) in enumerate(blocks):
            ctx.TrySwiGLUVector(h, src, g, u, HIDDEN, INTER)
            y = outs[l & 1]
            ctx.Int4Linear(y, h, d, 1, INTER, HIDDEN)
            src = y

    for b in blocks:  # weights resident before timing (first use uploads them)
        ctx.PreloadWeights(list(b))
    for _ in range(args.warmup):
        step()
    ctx.Flush()

    # Timed region: exactly K steps between two synchronisations.
    ctx.EventRecord(0)
    for _ in range(args.steps):
        step()
    ctx.EventRecord(1)
    ctx.Flush()
    total_ms = ctx.EventElapsedMs(0, 1)
    ms_step = total_ms / args.steps
    us_layer = ms_step * 1000 / LAYERS
    value = (wbytes + abytes1) * LAYERS / (ms_step * 1e-3) / 1e9

    # Dominant kernel (the fused gate/up SwiGLU matvec, 62% of the layer's
    # bytes): HIP events on the context stream around its 36 launches over the
    # 36 layers, back to back, repeated; average per launch.
    reps = max(3, args.steps // 5)
    ctx.EventRecord(6)
    for _ in range(reps):
        for (g, u, d) in blocks:
            ctx.TrySwiGLUVector(h, x, g, u, HIDDEN, INTER)
    ctx.EventRecord(7)
    ctx.Flush()
    gu_us = ctx.EventElapsedMs(6, 7) * 1000 / (reps * LAYERS)
    gu_bytes = 2 * INTER * hip.int4_row_bytes(HIDDEN) + 4 * (HIDDEN + INTER)  # weights + x in + h out
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9

    # Batch 8: gate and up as Int4Linear (8 rows), GO_SWIGLU, then down (the
    # engine's multi-row path, LLM.pas:594-601).
    x8t = ctx.UploadRaw(x8)
    g8, u8, hh8 = ctx.NewTensor(8 * INTER), ctx.NewTensor(8 * INTER), ctx.NewTensor(8 * INTER)
    y8a, y8b = ctx.NewTensor(8 * HIDDEN), ctx.NewTensor(8 * HIDDEN)

    def step8():
        src = x8t
        for l, (g, u, d) in enumerate(blocks):
            ctx.Int4Linear(g8, src, g, 8, HIDDEN, INTER)
            ctx.Int4Linear(u8, src, u, 8, HIDDEN, INTER)
            ctx.Kernel(hip.GO_SWIGLU, 8 * INTER, hh8, g8, u8, None, [INTER, 0])
            y = (y8a, y8b)[l & 1]
            ctx.Int4Linear(y, hh8, d, 8, INTER, HIDDEN)
            src = y

    step8()
    ctx.Flush()
    n8 = max(5, args.steps // 5)
    ctx.EventRecord(4)
    for _ in range(n8):
        step8()
    ctx.EventRecord(5)
    ms8 = ctx.EventElapsedMs(4, 5) / n8

    # Traffic calibration for rocprofv3 --pmc runs: one device-to-device copy
    # of a known 64 MiB (FETCH_SIZE / WRITE_SIZE of this copy give the
    # counter's bytes-per-KiB factor).
    cal_a, cal_b = ctx.NewTensor(16 << 20), ctx.NewTensor(16 << 20)
    ctx.Copy(cal_b, cal_a, 16 << 20)
    ctx.Flush()

    traffic = None  # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    tpath = os.path.join(ROOT, "profiles", "int4_swiglu_gateup_qwen3_4b_traffic.json")
    if os.path.exists(tpath):
        try:
            traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    ctx.close()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(packed, x1, args.cpu_seconds, wbytes, abytes1)

    line = {
        "metric": "quant matvec HBM GB/s (% of 8 TB/s) + decode us/layer, Qwen3-4B-shape INT4",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-w/fp32-acc",
        "data": "synthetic (seeded N(0,0.02) bf16 weights packed to QuickNN INT4; N(0,1) RMS-normalised activations)",
        "config": {"workload": "configs[1]: Qwen3-4B MLP, hidden 2560, intermediate 9728, fused gate+up SwiGLU "
                               "then down, native INT4, 36 layers, batch 1",
                   "global_batch": 1, "layers": LAYERS, "hidden": HIDDEN, "intermediate": INTER},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "us_per_layer": round(us_layer, 3),
        "tokens_per_s": round(1000.0 / ms_step, 1),
        "batch8": {"us_per_layer": round(ms8 * 1000 / LAYERS, 3),
                   "GBps": round((wbytes + abytes8) * LAYERS / (ms8 * 1e-3) / 1e9, 1),
                   "tokens_per_s": round(8000.0 / ms8, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "k_int4_matvec (I4_SWIGLU: fused gate+up SwiGLU, 9728x2560 pair)",
                     "kernel_us": round(gu_us, 3), "bytes_per_launch": gu_bytes,
                     "timing": f"HIP events around {reps}x{LAYERS} back-to-back launches on the context stream"},
        "cpu_baseline": cpu,
        "setup_s": round(gen_s, 1),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
