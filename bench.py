#!/usr/bin/env python3
"""Benchmark: QuickNN's quantized-weight decode path on one MI355X.

Default (`--config 2`, the headline): Qwen3-4B-shaped native-INT4 decode-layer
MLP.  hidden 2560, intermediate 9728; per layer the gate+up projection with
SwiGLU (TrySwiGLUVector) then the down projection (Int4Linear), which the
backend runs as one fused launch; 36 layers with independent seeds, batch 1.  A "step" is one token
through the 36 layers, the output of layer l feeding layer l+1.  Weights are
bf16 N(0, 0.02) (truncated from fp32 as SingleToBF16 does) packed with
QuickNN's INT4 algorithm; activations fp32 N(0,1) RMS-normalised with unit
gamma.  The 36-layer weight set (1.68 GB) exceeds the 256 MB MALL, so every
step streams its weights from HBM.

value = algorithmic bytes per step (packed weights + activations read once +
outputs written once) / measured time per step, in GB/s.

Also reported: us/layer and tokens/s; the dominant kernel's roofline (the
fused decode MLP, one launch per layer: algorithmic bytes per launch over its
average launch time, from HIP events on the context stream around 36-launch
runs of it); batch-8 figures; and the reference's CPU SIMD path (an AVX2
restatement in the CPU oracle) timed on this host on the same packed weights.

The other workloads of the benchmark definition are measured with
`--config 1|3|4|5|6` (one JSON line each, same fields), and the default run
also times each of them briefly and reports them under `other_configs`:
  1  one INT4 matvec 6144x2048 (Qwen3-1.7B gate shape), batch 1;
  3  Gemma-2-9B-shaped GGUF K-quant decode layer (Q4_K q/o, Q3_K k/v, Q2_K
     gate/up + GEGLU, Q6_K down) and the Q6_K output head;
  4  Qwen3-30B-A3B-shaped MoE expert layer (128 INT4 experts, top-8) at batch
     1 and 16, routed on the device;
  5  Q8_0 prefill GEMM 512x3072x12288;
  6  the rest of the decode layer at the Qwen3-4B shape: cached attention
     over 4096 and 32768 keys, token sampling over 151936 tokens, RoPE.
Each rotates over enough distinct weight copies (> 256 MB) that the weights
come from HBM, not from the MALL.
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
FP16_MFMA_PEAK_TFLOPS = 2500.0
INT8_MFMA_PEAK_TOPS = 5000.0
METRIC = "quant matvec HBM GB/s (% of 8 TB/s) + decode us/layer, Qwen3-4B-shape INT4"


def bf16_trunc(w: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits by truncation (SingleToBF16)."""
    return (w.view(np.uint32) >> 16).astype(np.uint16)


def make_layer(seed: int, hip):
    rng = np.random.default_rng(seed)

    def mat(n, k):
        w = rng.standard_normal((n, k), dtype=np.float32)
        w *= np.float32(0.02)
        return hip.quantize_int4(bf16_trunc(w))

    return mat(INTER, HIDDEN), mat(INTER, HIDDEN), mat(HIDDEN, INTER)


def layer_bytes(m: int, hip) -> tuple[int, int]:
    """(weight bytes, activation bytes) per layer at batch m."""
    w = 2 * INTER * hip.int4_row_bytes(HIDDEN) + HIDDEN * hip.int4_row_bytes(INTER)
    act = 4 * m * (HIDDEN + INTER + INTER + HIDDEN)  # x in, h out, h in, y out
    return w, act


def timed_ms(ctx, fn, reps: int) -> float:
    """Average ms of fn() over `reps` back-to-back runs, HIP events on the context stream."""
    ctx.EventRecord(2)
    for _ in range(reps):
        fn()
    ctx.EventRecord(3)
    ctx.Flush()
    return ctx.EventElapsedMs(2, 3) / reps


def gguf_matrix(hip, enc: int, n: int, k: int, seed: int, max_rows: int = 16384) -> np.ndarray:
    """N(0, 0.02) fp32 [n, k] encoded to GGML blocks; rows beyond max_rows repeat the first max_rows
    (same statistics, bounded generation time)."""
    rng = np.random.default_rng(seed)
    base = min(n, max_rows)
    w = rng.standard_normal(base * k, dtype=np.float32)
    w *= np.float32(0.02)
    b = hip.gguf_quantize(enc, w).reshape(base, -1)
    if base < n:
        b = np.concatenate([b] * ((n + base - 1) // base))[:n]
    return np.ascontiguousarray(b).reshape(-1)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def traffic_calibration_copy(ctx) -> None:
    """For rocprofv3 --pmc runs: one device-to-device copy of a known 64 MiB
    (its FETCH_SIZE / WRITE_SIZE give the counters' bytes-per-KiB factors)."""
    a, b = ctx.NewTensor(16 << 20), ctx.NewTensor(16 << 20)
    ctx.Copy(b, a, 16 << 20)
    ctx.Flush()
    ctx.Recycle(a)
    ctx.Recycle(b)


def base_line(args, metric, value, unit, ms_step, dtype, data, config, **extra) -> dict:
    line = {"metric": metric, "value": round(value, 2), "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": data, "config": config}
    line.update(extra)
    return line


# ---------------------------------------------------------------------------
# cfg2 (default): Qwen3-4B INT4 MLP, 36 layers
# ---------------------------------------------------------------------------
def cpu_baseline_mlp(packed, x0: np.ndarray, budget_s: float, wbytes: int, abytes: int) -> dict:
    """The reference's CPU direct-matvec path (TCPUProjection.Linear with the
    AVX2 Int4VectorDot, QwenHybrid.CPU.pas:238-248 composition), restated in
    the oracle, at the reference default of min(8, nproc) worker threads."""
    import oracle

    def timed(pool, budget):
        layers_done, t0 = 0, time.perf_counter()
        x = x0.copy()
        while True:
            g, u, d = packed[layers_done % LAYERS]
            x = oracle.cpu_mlp(g, u, d, oracle.ENC_INT4, x, HIDDEN, INTER, pool)[0]
            layers_done += 1
            el = time.perf_counter() - t0
            if el >= budget and layers_done >= LAYERS:
                return layers_done, el

    pool = oracle.Pool(0)  # the reference default: min(8, nproc) threads (CPU.Inference.pas:112-115)
    n8, el8 = timed(pool, budget_s)
    us8 = el8 / n8 * 1e6
    allc = oracle.Pool(min(64, os.cpu_count() or 1))  # every core this process may use (the pool's cap is 64)
    na, ela = timed(allc, budget_s / 2)
    usa = ela / na * 1e6
    gbs = lambda us: round((wbytes + abytes) / (us * 1e-6) / 1e9, 2)
    return {"value": gbs(us8), "unit": "GB/s", "cores": pool.threads, "kind": "port",
            "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "all_cores": {"value": gbs(usa), "cores": allc.threads, "us_per_layer": round(usa, 1)},
            "sample": f"{n8} INT4 MLP layers at batch 1 ({el8:.1f} s) with {pool.threads} threads, {us8:.0f} us/layer; "
                      f"{na} layers ({ela:.1f} s) with {allc.threads} threads; same packed weights"}


def run_cfg2(args, hip) -> dict:
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

    # Dominant kernel: the fused decode MLP (k_int4_mlp, one launch per layer:
    # the gate/up SwiGLU recorded by TrySwiGLUVector runs together with the
    # Int4Linear that reads its output).  HIP events on the context stream
    # around 36-launch runs over the 36 layers, back to back, repeated;
    # average per launch.  With QNN_FUSE_MLP=0 the pair runs as two launches
    # and the figure is per pair.
    reps = max(3, args.steps // 5)
    fused0 = ctx.status().mlp_fused
    ctx.EventRecord(6)
    for _ in range(reps):
        for (g, u, d) in blocks:
            ctx.TrySwiGLUVector(h, x, g, u, HIDDEN, INTER)
            ctx.Int4Linear(ya, h, d, 1, INTER, HIDDEN)
    ctx.EventRecord(7)
    ctx.Flush()
    fused = ctx.status().mlp_fused - fused0 == reps * LAYERS
    k_us = ctx.EventElapsedMs(6, 7) * 1000 / (reps * LAYERS)
    k_bytes = wbytes + abytes1  # the layer's weights + x in, h out and in, y out
    achieved = k_bytes / (k_us * 1e-6) / 1e9

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

    # The engine's call order (LLM.pas:588-598, QwenHybrid.pas:692-702): each
    # layer's outputs are created right before the projection that writes them
    # and released afterwards (its TGPUWorkspace).  Same launches (the fused
    # MLP per layer); the figure adds this host's per-call overhead.
    def step_engine():
        src = x
        for (g, u, d) in blocks:
            hh = ctx.NewTensor(INTER)
            ctx.TrySwiGLUVector(hh, src, g, u, HIDDEN, INTER)
            yy = ctx.NewTensor(HIDDEN)
            ctx.Int4Linear(yy, hh, d, 1, INTER, HIDDEN)
            ctx.Recycle(hh)
            if src is not x:
                ctx.Recycle(src)
            src = yy
        ctx.Recycle(src)

    step_engine()
    ctx.Flush()
    fused1 = ctx.status().mlp_fused
    ne = max(5, args.steps // 5)
    ctx.EventRecord(8)
    for _ in range(ne):
        step_engine()
    ctx.EventRecord(9)
    engine_us = ctx.EventElapsedMs(8, 9) * 1000 / (ne * LAYERS)
    engine_fused = ctx.status().mlp_fused - fused1 == ne * LAYERS

    traffic_calibration_copy(ctx)

    traffic = None  # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    tpath = os.path.join(ROOT, "profiles", "int4_mlp_fused_qwen3_4b_traffic.json")
    if os.path.exists(tpath):
        try:
            traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    ctx.close()

    cpu = None if args.no_cpu else cpu_baseline_mlp(packed, x1, args.cpu_seconds, wbytes, abytes1)
    return base_line(
        args, METRIC, value, "GB/s", ms_step, "int4-w/x16-fixed-act/fp32-acc",
        "synthetic (seeded N(0,0.02) bf16 weights packed to QuickNN INT4; N(0,1) RMS-normalised activations)",
        {"workload": "configs[1]: Qwen3-4B MLP, hidden 2560, intermediate 9728, fused gate+up SwiGLU "
                     "then down, native INT4, 36 layers, batch 1",
         "global_batch": 1, "layers": LAYERS, "hidden": HIDDEN, "intermediate": INTER},
        pct_of_hbm_peak=round(100 * value / HBM_PEAK_GBS, 2),
        us_per_layer=round(us_layer, 3),
        tokens_per_s=round(1000.0 / ms_step, 1),
        engine_order={"us_per_layer": round(engine_us, 3), "fused_every_layer": engine_fused,
                      "note": "NewTensor before and Recycle after each projection, as the engine's workspace does"},
        arithmetic="weights INT4 exact; activations per 32-group 16-bit fixed point (two int8 planes) into "
                   "v_dot4_i32_i8, exact integer group sums, fp32 scale and accumulation",
        batch8={"us_per_layer": round(ms8 * 1000 / LAYERS, 3),
                "GBps": round((wbytes + abytes8) * LAYERS / (ms8 * 1e-3) / 1e9, 1),
                "tokens_per_s": round(8000.0 / ms8, 1)},
        roofline={"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic if fused else None,
                  "kernel": ("k_int4_mlp (fused decode MLP: gate/up SwiGLU 2x9728x2560 + down 2560x9728, "
                             "one launch per layer)") if fused else
                            "k_int4_matvec I4_SWIGLU + I4_STORE (two launches per layer, fusion off)",
                  "kernel_us": round(k_us, 3), "bytes_per_launch": k_bytes,
                  "timing": f"HIP events around {reps}x{LAYERS} back-to-back launches on the context stream"},
        cpu_baseline=cpu,
        setup_s=round(gen_s, 1))


# ---------------------------------------------------------------------------
# cfg1: one INT4 matvec 6144 x 2048
# ---------------------------------------------------------------------------
def run_cfg1(args, hip) -> dict:
    N, K, R = 6144, 2048, 64  # 64 distinct copies: 503 MB, beyond the MALL
    rng = np.random.default_rng(11)
    w = rng.standard_normal((N, K), dtype=np.float32)
    w *= np.float32(0.02)
    packed = hip.quantize_int4(bf16_trunc(w))
    x = rng.standard_normal(K).astype(np.float32)
    ctx = hip.GPUContext(0)
    blocks = [hip.MemoryBlock.int4(packed) for _ in range(R)]  # distinct identities, same bytes
    ctx.PreloadWeights(blocks)
    xt, yt = ctx.UploadRaw(x), ctx.NewTensor(N)

    def step():
        for b in blocks:
            ctx.Int4Linear(yt, xt, b, 1, K, N)

    for _ in range(args.warmup):
        step()
    ms_step = timed_ms(ctx, step, args.steps)
    traffic_calibration_copy(ctx)
    ctx.close()
    nbytes = packed.size + 4 * (K + N)
    us = ms_step * 1000 / R
    achieved = nbytes / (us * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle

        pool = oracle.Pool(0)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds or n < 3:
            oracle.cpu_linear(packed, oracle.ENC_INT4, x, K, N, pool)
            n += 1
        el = time.perf_counter() - t0
        cpu = {"value": round(nbytes * n / el / 1e9, 2), "unit": "GB/s", "cores": pool.threads, "kind": "port",
               "sample": f"{n} matvecs ({el:.1f} s), {el / n * 1e6:.0f} us each; nproc={os.cpu_count()}"}
    return base_line(
        args, "INT4 matvec HBM GB/s, 6144x2048", achieved, "GB/s", ms_step, "int4-w/x16-fixed-act/fp32-acc",
        f"synthetic (seeded N(0,0.02) bf16 packed to QuickNN INT4; x N(0,1)); {R} distinct weight copies rotated",
        {"workload": "configs[0]: native INT4 matvec, N 6144, K 2048, batch 1", "global_batch": 1},
        us_per_matvec=round(us, 3), pct_of_hbm_peak=round(100 * achieved / HBM_PEAK_GBS, 2),
        roofline={"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                  "kernel": "k_int4_matvec (I4_STORE)", "kernel_us": round(us, 3), "bytes_per_launch": nbytes,
                  "timing": f"HIP events around {args.steps}x{R} back-to-back launches"},
        cpu_baseline=cpu)


# ---------------------------------------------------------------------------
# cfg3: Gemma-2-9B GGUF decode layer + Q6_K head
# ---------------------------------------------------------------------------
def run_cfg3(args, hip) -> dict:
    H, I, Q, KV, V, L = 3584, 14336, 4096, 2048, 256000, 8
    t0 = time.perf_counter()
    shapes = {"q": (hip.WE_Q4_K, Q, H), "k": (hip.WE_Q3_K, KV, H), "v": (hip.WE_Q3_K, KV, H),
              "o": (hip.WE_Q4_K, H, Q), "gate": (hip.WE_Q2_K, I, H), "up": (hip.WE_Q2_K, I, H),
              "down": (hip.WE_Q6_K, H, I)}
    data = {nm: gguf_matrix(hip, e, n, k, 300 + i) for i, (nm, (e, n, k)) in enumerate(shapes.items())}
    head = gguf_matrix(hip, hip.WE_Q6_K, V, H, 399)
    gen_s = time.perf_counter() - t0
    layers = [{nm: hip.MemoryBlock.gguf(data[nm], n, k, e) for nm, (e, n, k) in shapes.items()} for _ in range(L)]
    head_b = hip.MemoryBlock.gguf(head, V, H, hip.WE_Q6_K)
    wbytes = {nm: d.size for nm, d in data.items()}
    rng = np.random.default_rng(13)
    x = rng.standard_normal(H).astype(np.float32)
    ctx = hip.GPUContext(0)
    for lay in layers:
        ctx.PreloadWeights(list(lay.values()))
    ctx.PreloadWeights([head_b])
    xt = ctx.UploadRaw(x)
    q, k_, v_, o = ctx.NewTensor(Q), ctx.NewTensor(KV), ctx.NewTensor(KV), ctx.NewTensor(H)
    g, u, hh, y, logits = ctx.NewTensor(I), ctx.NewTensor(I), ctx.NewTensor(I), ctx.NewTensor(H), ctx.NewTensor(V)
    # Gemma2's layer (Gemma2.pas:142-198): q, k, v, o, gate, up, GEGLU, down.
    # Attention itself is outside the path; o reads q's output.
    # Each op on a given weight (o reads q's output).
    opw = {
        "q": lambda w: ctx.Linear(q, xt, w, None, None, 1, H, Q),
        "k": lambda w: ctx.Linear(k_, xt, w, None, None, 1, H, KV),
        "v": lambda w: ctx.Linear(v_, xt, w, None, None, 1, H, KV),
        "o": lambda w: ctx.Linear(o, q, w, None, None, 1, Q, H),
        "gate": lambda w: ctx.Linear(g, xt, w, None, None, 1, H, I),
        "up": lambda w: ctx.Linear(u, xt, w, None, None, 1, H, I),
        "down": lambda w: ctx.Linear(y, hh, w, None, None, 1, I, H),
    }
    ops = {nm: (lambda lay, nm=nm: opw[nm](lay[nm])) for nm in opw}
    ops["geglu"] = lambda lay: ctx.Kernel(hip.GO_GEGLU, I, hh, g, u, None, [I, 0])
    order = ("q", "k", "v", "o", "gate", "up", "geglu", "down")

    def step():
        for lay in layers:
            for nm in order:
                ops[nm](lay)

    for _ in range(max(1, args.warmup)):
        step()
    ms_step = timed_ms(ctx, step, args.steps)
    us_layer = ms_step * 1000 / L
    act = 4 * (H * 6 + Q * 2 + KV * 2 + I * 5 + H)  # activation reads and writes of the 8 ops
    layer_b = sum(wbytes.values()) + act
    # Per op: its own launches back to back over copies of its weight totalling
    # more than 512 MB, so every launch streams from HBM (the layer rotation
    # above holds 8 copies, 25-135 MB per op, which the MALL could serve).
    per_op, multi_row = {}, {}
    for nm in ("q", "k", "v", "o", "gate", "up", "down"):
        e, n, kk = shapes[nm]
        ncopy = max(L, -(-600_000_000 // wbytes[nm]))
        copies = [lay[nm] for lay in layers] + [hip.MemoryBlock.gguf(data[nm], n, kk, e) for _ in range(ncopy - L)]
        ctx.PreloadWeights(copies[L:])
        run = lambda: [opw[nm](w) for w in copies]  # noqa: E731
        run()  # first launches of this shape outside the timed region
        ctx.Flush()
        t = timed_ms(ctx, run, max(2, args.steps // 10)) * 1000 / ncopy
        per_op[nm] = {"us": round(t, 2), "GBps": round(wbytes[nm] / (t * 1e-6) / 1e9, 1), "copies": ncopy,
                      "rotation_MB": round(ncopy * wbytes[nm] / 1e6)}
        if nm == "q":
            # Eight rows through one Linear (the multi-token matvec, all eight
            # per pass over the weight), over the same cold rotation.
            x8, y8 = ctx.UploadRaw(rng.standard_normal((8, H)).astype(np.float32)), ctx.NewTensor(8 * Q)
            run8 = lambda: [ctx.Linear(y8, x8, w, None, None, 8, H, Q) for w in copies]  # noqa: E731
            run8()
            ctx.Flush()
            t8 = timed_ms(ctx, run8, max(2, args.steps // 10)) * 1000 / ncopy
            multi_row["q_8_rows"] = {"us": round(t8, 2), "GBps": round(wbytes[nm] / (t8 * 1e-6) / 1e9, 1),
                                     "copies": ncopy, "path": "k_gguf_matvec_mt: 8 rows per pass over the weight"}
            ctx.Recycle(x8)
            ctx.Recycle(y8)
        del copies
    ctx.Linear(logits, xt, head_b, None, None, 1, H, V)  # first launch of the head's shape, untimed
    ctx.Flush()
    head_us = timed_ms(ctx, lambda: ctx.Linear(logits, xt, head_b, None, None, 1, H, V), 20) * 1000
    # A 512-row prefill through q (the fp16-copy GEMM over each weight's
    # cached fp16 copy, made by the first, untimed call), over the layer copies.
    x512, y512 = ctx.UploadRaw(rng.standard_normal((512, H)).astype(np.float32)), ctx.NewTensor(512 * Q)
    run512 = lambda: [ctx.Linear(y512, x512, lay["q"], None, None, 512, H, Q) for lay in layers]  # noqa: E731
    run512()
    ctx.Flush()
    t512 = timed_ms(ctx, run512, max(2, args.steps // 5)) * 1000 / L
    multi_row["q_512_rows"] = {"us": round(t512, 2), "TFLOPs": round(2 * 512 * H * Q / (t512 * 1e-6) / 1e12, 1),
                               "path": "k_h16_gemm over the cached fp16 copy (K split over 2 slices, summed by "
                                       "k_sum_kslices), after k_act_prep"}
    traffic_calibration_copy(ctx)
    ctx.close()
    dom = max(per_op, key=lambda nm: per_op[nm]["us"])
    value = layer_b / (us_layer * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle

        pool = oracle.Pool(0)
        encs = {hip.WE_Q4_K: oracle.ENC_Q4_K, hip.WE_Q3_K: oracle.ENC_Q3_K, hip.WE_Q2_K: oracle.ENC_Q2_K,
                hip.WE_Q6_K: oracle.ENC_Q6_K}
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds or n < 1:
            outs = {}
            for nm in ("q", "k", "v", "o", "gate", "up", "down"):
                e, nn, kk = shapes[nm]
                src = x
                if nm == "o":
                    src = outs["q"]
                elif nm == "down":
                    gg, uu = outs["gate"], outs["up"]
                    c = np.float32(0.7978845608)
                    src = (0.5 * gg * (1 + np.tanh(c * (gg + np.float32(0.044715) * gg ** 3))) * uu).astype(np.float32)
                outs[nm] = oracle.cpu_linear(data[nm], encs[e], src, kk, nn, pool)
            n += 1
        el = time.perf_counter() - t0
        cpu = {"value": round(layer_b * n / el / 1e9, 2), "unit": "GB/s", "cores": pool.threads, "kind": "port",
               "sample": f"{n} Gemma layers ({el:.1f} s, {el / n * 1e6:.0f} us/layer): TCPUProjection.Linear "
                         f"with the direct PackedDot paths (Q2_K block decode + VectorDot); nproc={os.cpu_count()}"}
    return base_line(
        args, "GGUF K-quant decode HBM GB/s + us/layer, Gemma-2-9B shape", value, "GB/s", ms_step,
        "gguf-w/x16-fixed-act/fp32-acc",
        "synthetic (N(0,0.02) fp32 encoded to GGML blocks; rows past 16384 repeat; x N(0,1)); "
        f"{L} layer copies rotated ({L * sum(wbytes.values()) / 1e6:.0f} MB); per-op figures over > 512 MB of "
        "copies of each op's weight",
        {"workload": "configs[2]: Gemma-2-9B layer, hidden 3584, q/o Q4_K, k/v Q3_K, gate/up Q2_K + GEGLU, "
                     "down Q6_K, batch 1; head Q6_K 256000x3584", "global_batch": 1},
        us_per_layer=round(us_layer, 2), pct_of_hbm_peak=round(100 * value / HBM_PEAK_GBS, 2), per_op=per_op,
        head={"us": round(head_us, 2), "GBps": round(head.size / (head_us * 1e-6) / 1e9, 1)},
        multi_row_linear=multi_row,
        roofline={"bound": "hbm", "achieved": per_op[dom]["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(per_op[dom]["GBps"] / HBM_PEAK_GBS, 4), "traffic": None,
                  "kernel": f"k_gguf_matvec ({dom}: {shapes[dom][1]}x{shapes[dom][2]})",
                  "kernel_us": per_op[dom]["us"], "bytes_per_launch": wbytes[dom],
                  "timing": f"HIP events around back-to-back launches over {per_op[dom]['copies']} copies "
                            f"({per_op[dom]['rotation_MB']} MB) of the op's weight"},
        cpu_baseline=cpu, setup_s=round(gen_s, 1))


# ---------------------------------------------------------------------------
# cfg4: Qwen3-30B-A3B MoE expert layer
# ---------------------------------------------------------------------------
def run_cfg4(args, hip) -> dict:
    E, H, I, K, L = 128, 2048, 768, 8, 4
    t0 = time.perf_counter()
    rng = np.random.default_rng(17)

    def mat(n, k):
        w = rng.standard_normal((n, k), dtype=np.float32)
        w *= np.float32(0.02)
        return hip.quantize_int4(bf16_trunc(w))

    gates = [mat(I, H) for _ in range(E)]
    ups = [mat(I, H) for _ in range(E)]
    downs = [mat(H, I) for _ in range(E)]
    gen_s = time.perf_counter() - t0
    per_expert = 2 * I * hip.int4_row_bytes(H) + H * hip.int4_row_bytes(I)
    ctx = hip.GPUContext(0)
    sets = [ctx.CreateExpertSet([hip.MemoryBlock.int4(w) for w in gates], [hip.MemoryBlock.int4(w) for w in ups],
                                [hip.MemoryBlock.int4(w) for w in downs], H, I) for _ in range(L)]
    res = {}
    for rows in (1, 16):
        x = rng.standard_normal((rows, H)).astype(np.float32)
        xt = ctx.UploadRaw(x)
        # Batch 1: each layer copy gets E/K router outputs whose top-8 are the
        # disjoint expert groups 8j..8j+7 (those logits raised by 10), so one
        # rotation reads every expert of every copy (L x 128 experts, 1.5 GB)
        # and no step finds its experts in the MALL.  Batch 16: one random
        # router output per copy (about 80 distinct experts each, 950 MB).
        nr = E // K if rows == 1 else 1
        routes, logit_t, distinct, first_logits = [], [], 0, None
        for l in range(L):
            for j in range(nr):
                lg = rng.standard_normal((rows, E)).astype(np.float32)
                if rows == 1:
                    lg[:, K * j:K * (j + 1)] += np.float32(10.0)
                first_logits = lg if first_logits is None else first_logits
                lt = ctx.UploadRaw(lg)
                rt = ctx.NewTensor(2 * rows * K)
                ctx.Kernel(hip.GO_MOE_ROUTE, 2 * rows * K, rt, lt, None, None, [rows, E, K, 1])
                routes.append((sets[l], rt))
                logit_t.append(lt)
                distinct += len(set(ctx.Download(rt)[:rows * K].view(np.uint32).tolist()))
        calls = len(routes)
        out = ctx.NewTensor(rows * H)

        def step():
            for st, rt in routes:
                ctx.MoEExperts(st, out, xt, rt, rows, K)

        def route_step():  # GO_MOE_ROUTE again on the same logits: the same routes
            for (st, rt), lt in zip(routes, logit_t):
                ctx.Kernel(hip.GO_MOE_ROUTE, 2 * rows * K, rt, lt, None, None, [rows, E, K, 1])

        def layer_step():  # route then experts, as a decode layer issues them
            for (st, rt), lt in zip(routes, logit_t):
                ctx.Kernel(hip.GO_MOE_ROUTE, 2 * rows * K, rt, lt, None, None, [rows, E, K, 1])
                ctx.MoEExperts(st, out, xt, rt, rows, K)

        for _ in range(args.warmup):
            step()
            route_step()
        layer_step()
        ctx.Flush()
        ms = timed_ms(ctx, step, args.steps)
        us_route = timed_ms(ctx, route_step, args.steps) * 1000 / calls
        us_both = timed_ms(ctx, layer_step, args.steps) * 1000 / calls
        us_layer = ms * 1000 / calls
        nbytes = distinct / calls * per_expert + 4 * rows * (2 * H + 2 * K)
        res[rows] = {"ms_step": ms, "us_per_layer": round(us_layer, 2), "distinct_experts": round(distinct / calls, 1),
                     "rotation_MB": round(distinct * per_expert / 1e6),
                     "GBps": round(nbytes / (us_layer * 1e-6) / 1e9, 1), "bytes": nbytes, "x": x,
                     "logits": first_logits, "route_us": round(us_route, 2), "route_plus_experts_us": round(us_both, 2)}
    traffic_calibration_copy(ctx)
    ctx.close()
    r1 = res[1]
    cpu = None
    if not args.no_cpu:
        import oracle

        pool = oracle.Pool(0)
        ids, probs = oracle.moe_route(r1["logits"], K, True)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds or n < 3:
            oracle.cpu_moe(gates, ups, downs, r1["x"], ids, probs, H, I, pool)
            n += 1
        el = time.perf_counter() - t0
        cpu = {"value": round(r1["bytes"] * n / el / 1e9, 2), "unit": "GB/s", "cores": pool.threads, "kind": "port",
               "sample": f"{n} composed batch-1 MoE layers ({el:.1f} s, {el / n * 1e6:.0f} us each): 8 experts x "
                         f"(gate, up, down) TCPUProjection.Linear + weighted sum; nproc={os.cpu_count()}"}
    return base_line(
        args, "MoE routed-expert HBM GB/s + us/layer, Qwen3-30B-A3B shape INT4", r1["GBps"], "GB/s", r1["ms_step"],
        "int4-w/x16-fixed-act/fp32-acc",
        "synthetic (N(0,0.02) bf16 experts packed to INT4; router logits N(0,1), top-8 renormalised); "
        f"{L} expert-set copies x {E // K} disjoint top-8 routes rotated at batch 1 ({r1['rotation_MB']} MB of "
        "distinct experts per rotation, beyond the MALL)",
        {"workload": "configs[3]: 128 experts, hidden 2048, expert inter 768, top-8, batch 1 (batch 16 below)",
         "global_batch": 1},
        us_per_layer=r1["us_per_layer"], distinct_experts=r1["distinct_experts"],
        route_us=r1["route_us"], route_plus_experts_us=r1["route_plus_experts_us"],
        pct_of_hbm_peak=round(100 * r1["GBps"] / HBM_PEAK_GBS, 2),
        batch16={k: v for k, v in res[16].items()
                 if k in ("us_per_layer", "distinct_experts", "GBps", "route_us", "route_plus_experts_us",
                          "rotation_MB")},
        rotation_MB=r1["rotation_MB"],
        roofline={"bound": "hbm", "achieved": r1["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(r1["GBps"] / HBM_PEAK_GBS, 4), "traffic": None,
                  "kernel": "k_moe_decode (one qnn_moe_experts call for one token: a single launch)",
                  "kernel_us": r1["us_per_layer"], "bytes_per_launch": round(r1["bytes"]),
                  "timing": f"HIP events around {args.steps}x{L * E // K} calls, each on experts no earlier call "
                            "of the rotation read"},
        cpu_baseline=cpu, setup_s=round(gen_s, 1))


# ---------------------------------------------------------------------------
# cfg5: Q8_0 prefill GEMM
# ---------------------------------------------------------------------------
def vendor_fp16_gemm_us(M: int, K: int, N: int, R: int, steps: int):
    """torch.matmul (hipBLASLt) on the cfg5 product in fp16 (fp16 out), R weight
    copies rotated as run_cfg5 does: a comparison figure for the fp16 Linear,
    not this library's code.  `bench.py --vendor-gemm` runs it alone, before
    this library is loaded (torch's HIP runtime is not shared with it).  None
    without a GPU torch."""
    try:
        import torch
    except ImportError:
        return None
    if not torch.cuda.is_available():
        return None
    g = torch.Generator(device="cuda").manual_seed(5)
    a = torch.randn(M, K, device="cuda", dtype=torch.float16, generator=g)
    ws = [torch.randn(N, K, device="cuda", dtype=torch.float16, generator=g) for _ in range(R)]
    for _ in range(2):
        for w in ws:
            torch.matmul(a, w.t())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        for w in ws:
            torch.matmul(a, w.t())
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000 / (steps * R)
    del a, ws
    torch.cuda.empty_cache()
    return {"us_per_gemm": round(us, 2), "TFLOPs": round(2.0 * M * N * K / us / 1e6, 1),
            "what": "torch.matmul fp16 x fp16 -> fp16 (hipBLASLt), same shape, same weight rotation"}


def run_cfg5(args, hip) -> dict:
    """the activations are quantised per 32-element block to int8
    for the MFMA path (qnn_q8_gemm_int8: int8 matrix cores, per-block fp32
    epilogue); Linear's fp16-MFMA product (within 1e-3 of the reference's fp32
    path) is timed beside it."""
    M, K, N, R = 512, 3072, 12288, 8  # 8 weight copies: 321 MB
    wq = gguf_matrix(hip, hip.WE_Q8_0, N, K, 500)
    rng = np.random.default_rng(19)
    a = rng.standard_normal((M, K)).astype(np.float32)
    ctx = hip.GPUContext(0)
    ws = [hip.MemoryBlock.gguf(wq, N, K, hip.WE_Q8_0) for _ in range(R)]
    ctx.PreloadWeights(ws)
    at, ct = ctx.UploadRaw(a), ctx.NewTensor(M * N)

    def step_int8():
        for w in ws:
            ctx.Q8GemmInt8(ct, at, w, M, K, N)

    def step_fp16():
        for w in ws:
            ctx.Linear(ct, at, w, None, None, M, K, N)

    for _ in range(max(1, args.warmup)):
        step_int8()
        step_fp16()
    ms_step = timed_ms(ctx, step_int8, args.steps)
    ms_fp16 = timed_ms(ctx, step_fp16, args.steps)
    traffic_calibration_copy(ctx)
    ctx.close()
    us = ms_step * 1000 / R
    us16 = ms_fp16 * 1000 / R
    ops = 2.0 * M * N * K
    tops = ops / (us * 1e-6) / 1e12
    tflops16 = ops / (us16 * 1e-6) / 1e12
    nbytes = wq.size + 4 * M * K + 4 * M * N
    cpu = None
    if not args.no_cpu:
        import oracle

        pool = oracle.Pool(0)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds or n < 4:
            oracle.cpu_linear(wq, oracle.ENC_Q8_0, a[n % M], K, N, pool)
            n += 1
        el = time.perf_counter() - t0
        cpu = {"value": round(ops / M * n / el / 1e12, 4), "unit": "TOP/s", "cores": pool.threads,
               "kind": "port", "cpu_model": cpu_model(), "nproc": os.cpu_count(),
               "sample": f"{n} of the 512 rows as SIMD per-row PackedDotQ8 matvecs (fp32 activations, {el:.1f} s)"}
    return base_line(
        args, "Q8_0 prefill GEMM TOP/s, 512x3072x12288, int8 activations", tops, "TOP/s", ms_step,
        "int8-act(per-32)/q8_0-w/int32-block/fp32-acc",
        f"synthetic (N(0,0.02) fp32 encoded to Q8_0; A N(0,1) quantised per 32-element block to int8); "
        f"{R} weight copies rotated",
        {"workload": "configs[4]: Q8_0 GEMM M 512, K 3072, N 12288, activations int8 per 32-element block",
         "global_batch": M},
        us_per_gemm=round(us, 2), hbm_GBps=round(nbytes / (us * 1e-6) / 1e9, 1),
        fp16_linear={"us_per_gemm": round(us16, 2), "TFLOPs": round(tflops16, 1),
                     "frac_of_fp16_peak": round(tflops16 / FP16_MFMA_PEAK_TFLOPS, 4),
                     "note": "qnn_linear: from 128 rows over a cached fp16 copy of the weight (k_h16_gemm); fp32 "
                             "activations scaled per row by a power of two and rounded to fp16; within 1e-3 of "
                             "the reference's fp32 path"},
        roofline={"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_MFMA_PEAK_TOPS, "unit": "TOP/s",
                  "frac": round(tops / INT8_MFMA_PEAK_TOPS, 4), "traffic": None,
                  "kernel": "k_q8_gemm_i8 (+ k_q8_act_quant, the per-32 int8 activation quantiser)",
                  "kernel_us": round(us, 2), "ops_per_launch": int(ops),
                  "bound_note": "per output and 32-element block: convert and fma on the VALU (1.2 G "
                                "lane-ops at this shape); the scale products on the fp32 matrix cores",
                  "timing": f"HIP events around {args.steps}x{R} back-to-back calls"},
        cpu_baseline=cpu)


# ---------------------------------------------------------------------------
# cfg6: the rest of the decode layer (cached attention, sampling, RoPE)
# ---------------------------------------------------------------------------
def run_cfg6(args, hip) -> dict:
    """Decode-layer ops around the quantized matvecs, at the Qwen3-4B shape
    (32 query heads, 8 KV heads, head dim 128, vocabulary 151936):
    CachedAttention for one query row over 4096 keys (one cache per layer,
    36 layers: 1.21 GB, so the caches come from HBM) and over 32768 keys
    (4 caches of 268 MB), SampleToken (top-k 1 and 40) and GO_LLM_ROPE on
    the query heads.  value = K and V bytes read per 4096-key call over its
    average time."""
    heads, kvh, dim, vocab = 32, 8, 128, 151936
    rng = np.random.default_rng(23)
    ctx = hip.GPUContext(0)

    def cache_set(keys, count):
        one = rng.standard_normal(2 * keys * kvh * dim).astype(np.float32)
        return [ctx.UploadRaw(one) for _ in range(count)]

    def attn_us(keys, caches):
        def step():
            for c in caches:
                ctx.CachedAttention(o, q, c, 1, keys, heads, kvh, dim, keys - 1)
        for _ in range(max(1, args.warmup)):
            step()
        return timed_ms(ctx, step, args.steps) * 1000 / len(caches)

    q = ctx.UploadRaw(rng.standard_normal(heads * dim).astype(np.float32))
    o = ctx.NewTensor(heads * dim)
    t0 = time.perf_counter()
    caches = cache_set(4096, LAYERS)
    us4k = attn_us(4096, caches)
    for c in caches:
        ctx.Recycle(c)
    caches = cache_set(32768, 4)
    us32k = attn_us(32768, caches)
    for c in caches:
        ctx.Recycle(c)
    gen_s = time.perf_counter() - t0
    bytes4k = 2 * 4096 * kvh * dim * 4
    bytes32k = 2 * 32768 * kvh * dim * 4
    gbs = bytes4k / (us4k * 1e-6) / 1e9

    logits = ctx.UploadRaw(rng.standard_normal(vocab).astype(np.float32))
    seen = ctx.UploadRaw(np.zeros(vocab, np.float32))
    tok = ctx.NewTensor(1)
    sample = {}
    for k, temp in ((1, 0.0), (40, 0.7)):
        def s_step(k=k, temp=temp):
            ctx.SampleToken(tok, logits, seen, vocab, k, temp, 0.9, 1.1, 0.5)
        for _ in range(max(1, args.warmup)):
            s_step()
        sample[f"top_k_{k}_us"] = round(timed_ms(ctx, s_step, args.steps * 4) * 1000, 2)

    def r_step():
        ctx.Kernel(hip.GO_LLM_ROPE, heads * dim // 2, q, q, None, None, [heads, dim, 4000, hip.float_bits(1e6)])
    for _ in range(max(1, args.warmup)):
        r_step()
    rope_us = timed_ms(ctx, r_step, args.steps * 4) * 1000
    ctx.close()

    cpu = None
    if not args.no_cpu:
        import oracle

        qh = rng.standard_normal(heads * dim).astype(np.float32)
        ch = rng.standard_normal(2 * 4096 * kvh * dim).astype(np.float32)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds or n < 2:
            oracle.cached_attention(qh, ch, 1, 4096, heads, kvh, dim, 4095)
            n += 1
        el = time.perf_counter() - t0
        cpu = {"value": round(bytes4k * n / el / 1e9, 2), "unit": "GB/s", "cores": 1, "kind": "port",
               "cpu_model": cpu_model(), "nproc": os.cpu_count(),
               "sample": f"{n} CachedAttention calls over 4096 keys, the oracle's scalar restatement "
                         f"in double ({el:.1f} s)"}
    return base_line(
        args, "cached attention GB/s (K and V read once), Qwen3-4B shape, 4096 keys", gbs, "GB/s", us4k / 1000,
        "f32", "synthetic (N(0,1) queries and caches); one cache per layer, 36 layers",
        {"workload": "decode-layer ops: CachedAttention 32x8 heads dim 128 over 4096 and 32768 keys, "
                     "SampleToken over 151936 tokens, GO_LLM_ROPE", "global_batch": 1},
        attention_32k={"us": round(us32k, 2), "GBps": round(bytes32k / (us32k * 1e-6) / 1e9, 1),
                       "frac_of_hbm_peak": round(bytes32k / (us32k * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        sample=sample, rope_us=round(rope_us, 2), setup_s=round(gen_s, 1),
        roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                  "kernel": "k_attn_dma + k_attn_merge (one qnn_cached_attention call; 64-key chunks streamed "
                            "into LDS; the 32768-key calls take k_attn)",
                  "kernel_us": round(us4k, 2), "bytes_per_launch": bytes4k,
                  "timing": f"HIP events around {args.steps}x{LAYERS} calls"},
        cpu_baseline=cpu)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5, 6])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-others", action="store_true", help="config 2 only: skip the other configs' summaries")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only time torch.matmul (hipBLASLt) on the cfg5 shape in fp16, for comparison")
    args = ap.parse_args()
    if args.vendor_gemm:
        print(json.dumps({"vendor_fp16_gemm": vendor_fp16_gemm_us(512, 3072, 12288, 8, args.steps)}))
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(sharding the path over several GPUs is a design note, not built)", file=sys.stderr)
        return 2

    from quicknn_amd import hip

    runs = {1: run_cfg1, 2: run_cfg2, 3: run_cfg3, 4: run_cfg4, 5: run_cfg5, 6: run_cfg6}
    line = runs[args.config](args, hip)
    if args.config == 2 and not args.no_others:
        # The other workloads of the benchmark definition, in the same run (so
        # the driver's clock covers them): short timings, no CPU legs.
        sub = argparse.Namespace(**vars(args))
        sub.steps, sub.warmup, sub.no_cpu = max(5, args.steps // 5), max(2, args.warmup), True
        others = {}
        for c in (1, 3, 4, 5, 6):
            t0 = time.perf_counter()
            r = runs[c](sub, hip)
            rf = r["roofline"]
            others[f"cfg{c}"] = {
                "workload": r["config"]["workload"], "metric": r["metric"], "value": r["value"], "unit": r["unit"],
                "dtype": r["dtype"], "kernel": rf["kernel"], "kernel_us": rf["kernel_us"],
                "roofline_frac": rf["frac"], "roofline_bound": rf["bound"], "roofline_peak": rf["peak"],
                **{k: r[k] for k in ("us_per_matvec", "us_per_layer", "us_per_gemm", "head", "batch16", "per_op",
                                     "route_plus_experts_us", "hbm_GBps", "fp16_linear", "attention_32k", "sample",
                                     "rope_us") if k in r},
                "steps": sub.steps, "wall_s": round(time.perf_counter() - t0, 1)}
        line["other_configs"] = others
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
