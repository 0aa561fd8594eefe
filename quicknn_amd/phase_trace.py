"""Where the time of one fused decode-MLP launch goes, and the HBM stream floor.

    python -m quicknn_amd.phase_trace [--runs N] [--no-stream]

Loads libqnn_hip_trace.so (the library built with QNN_PHASE_TRACE: the same
kernels, with thread 0 of every workgroup storing the device real-time
counter, 100 MHz, at each phase) and runs the Qwen3-4B MLP of
`bench.py --config 2`: 36 independently seeded INT4 layers (1.68 GB, beyond
the 256 MB MALL), one fused launch per layer, batch 1.  The timestamps of the
last launch of a run are read back; for each phase it prints, over the
workgroups that reached it, the earliest, median and latest time in
microseconds after the launch's first workgroup started, taking the median of
each over several runs.

Phases of k_int4_mlp:
  0 start, 1 x slice staged, 2 gate/up parts in LDS, 3 gate/up partial sum
  exchanged (every item), 4 h block and flag published (last arrival of the
  block), 5 h flags of the slice seen, 6 h slice staged, 7 down parts in LDS,
  8 y stored (last arrival of the tile).

The stream floor: one plain streaming read (qnn_stream_read: non-temporal
16-byte loads, every piece requested at once, as the weight loads of the
matvec kernels) of 16, 32 and 46.8 MB, rotating over enough distinct buffers
(> 512 MB) that every read comes from HBM; HIP events around back-to-back
reads, per read.
"""
from __future__ import annotations

import argparse
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HIDDEN, INTER, LAYERS = 2560, 9728, 36
PHASES = ["start", "x staged", "gate/up parts", "gate/up exchanged", "h published", "h slice seen", "h staged",
          "down parts", "y stored"]


def layers(hip, rng):
    out = []
    for _ in range(LAYERS):
        mats = []
        for n, k in ((INTER, HIDDEN), (INTER, HIDDEN), (HIDDEN, INTER)):
            w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
            mats.append(hip.MemoryBlock.int4(hip.quantize_int4((w.view(np.uint32) >> 16).astype(np.uint16))))
        out.append(tuple(mats))
    return out


def timeline(ctx, hip, blocks, runs: int):
    x = ctx.UploadRaw(np.random.default_rng(3).standard_normal(HIDDEN).astype(np.float32))
    h, ya, yb = ctx.NewTensor(INTER), ctx.NewTensor(HIDDEN), ctx.NewTensor(HIDDEN)
    for b in blocks:
        ctx.PreloadWeights(list(b))

    def step():
        src = x
        for l, (g, u, d) in enumerate(blocks):
            ctx.TrySwiGLUVector(h, src, g, u, HIDDEN, INTER)
            ctx.Int4Linear((ya, yb)[l & 1], h, d, 1, INTER, HIDDEN)
            src = (ya, yb)[l & 1]

    for _ in range(3):
        step()
    ctx.Flush()
    ctx.PhaseTrace()  # clear
    per_run, us_layer = [], []
    for _ in range(runs):
        ctx.EventRecord(0)
        step()
        ctx.EventRecord(1)
        ctx.Flush()
        us_layer.append(ctx.EventElapsedMs(0, 1) * 1000 / LAYERS)
        ts = ctx.PhaseTrace().astype(np.int64)  # the last layer's launch
        starts = ts[:, 0][ts[:, 0] > 0]
        t0 = starts.min()
        row = {}
        for k in range(9):
            v = ts[:, k]
            v = v[v >= t0]  # every workgroup rewrites phase 0; earlier values are an earlier launch's
            if v.size:
                us = (v - t0) / 100.0
                row[k] = (float(us.min()), float(np.median(us)), float(us.max()), int(v.size))
        per_run.append(row)
    out = {}
    for k in range(9):
        vals = [r[k] for r in per_run if k in r]
        if vals:
            a = np.array([v[:3] for v in vals])
            out[k] = {"first_us": round(float(np.median(a[:, 0])), 2), "median_us": round(float(np.median(a[:, 1])), 2),
                      "last_us": round(float(np.median(a[:, 2])), 2), "workgroups": vals[0][3]}
    return out, float(np.median(us_layer))


def stream_floor(ctx, hip, sizes_mb=(16.0, 32.0, 46.8), total_mb=600.0, reps=3):
    res = {}
    dst = ctx.NewTensor(4)
    for mb in sizes_mb:
        count = int(mb * 1e6 / 4) // 4 * 4
        nbuf = max(2, int(np.ceil(total_mb / mb)))
        bufs = [ctx.NewTensor(count) for _ in range(nbuf)]
        for b in bufs:
            ctx.Kernel(hip.GO_FILL, count, b, None, None, None, [0])
        for b in bufs:  # warm-up pass
            ctx.StreamRead(b, count, dst)
        ctx.Flush()
        ctx.EventRecord(2)
        for _ in range(reps):
            for b in bufs:
                ctx.StreamRead(b, count, dst)
        ctx.EventRecord(3)
        ctx.Flush()
        us = ctx.EventElapsedMs(2, 3) * 1000 / (reps * nbuf)
        res[f"{mb:g} MB"] = {"us": round(us, 2), "GBps": round(count * 4 / (us * 1e-6) / 1e9, 1),
                             "buffers": nbuf}
        for b in bufs:
            ctx.Recycle(b)
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--runs", type=int, default=5)
    ap.add_argument("--no-stream", action="store_true")
    args = ap.parse_args()
    from quicknn_amd import build, hip

    if not os.path.exists(build.TRACE_LIB):
        raise SystemExit(f"{build.TRACE_LIB} is not built: run __graft_entry__.build()")
    hip.LIB_PATH = build.TRACE_LIB
    rng = np.random.default_rng(2024)
    blocks = layers(hip, rng)
    ctx = hip.GPUContext(0)
    s0 = ctx.status()
    phases, us_layer = timeline(ctx, hip, blocks, args.runs)
    if ctx.status().mlp_fused - s0.mlp_fused < LAYERS:
        raise SystemExit("the decode MLP did not run as one fused launch per layer")
    ran, names = "k_int4_mlp", PHASES
    print(f"kernel {ran}: {us_layer:.2f} us/layer (HIP events, 36-layer runs, median of {args.runs})")
    print(f"{'phase':<20s} {'first':>8s} {'median':>8s} {'last':>8s} {'workgroups':>11s}")
    for k, v in phases.items():
        if names[k]:
            print(f"{k} {names[k]:<18s} {v['first_us']:8.2f} {v['median_us']:8.2f} {v['last_us']:8.2f} "
                  f"{v['workgroups']:11d}")
    out = {"kernel": ran, "us_per_layer": round(us_layer, 2),
           "phases": {names[k]: v for k, v in phases.items() if names[k]}}
    if not args.no_stream:
        out["stream_floor"] = stream_floor(ctx, hip)
        for k, v in out["stream_floor"].items():
            print(f"stream {k}: {v['us']:.2f} us, {v['GBps']:.0f} GB/s ({v['buffers']} buffers rotated)")
    print(json.dumps(out))
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
