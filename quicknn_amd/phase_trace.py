"""Where the time of one fused decode-MLP launch goes, and the HBM stream floor.

    python -m quicknn_amd.phase_trace [--runs N] [--no-stream] [--moe | --attn]

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
  8 y stored (last arrival of the tile); 9 down partial stored and ticket
  taken (every down item), 10 the tile's down partials loaded and summed and
  11 a block's gate/up partials loaded and summed (last arrivals).

--moe times the one-token routed-expert launch (k_moe_decode) of
`bench.py --config 4` instead: 128 INT4 experts of 2048 -> 2 x 768 -> 2048 in
4 expert sets, top-8 routes whose experts are the disjoint groups 8j..8j+7,
so that each rotation reads every expert of every set (1.5 GB) and no launch
finds its experts in the MALL.  Its phases are those of the MLP kernel, with
an expert slot's gate/up tiles and blocks of h in place of the layer's.

--attn times the 4096-key cached attention of `bench.py --config 6` (32
query heads, 8 KV heads, head dim 128, one f32 cache per layer, 36 layers):
phases of k_attn_dma 0 start, 1 q and K landed, 2 scores and softmax, 3 V
landed, 4 values accumulated, 5 key lanes summed, 6 chunk output stored (the
chunk merge is a second launch).

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
          "down parts", "y stored", "down ticket taken", "down partials summed", "gate/up partials summed"]


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
        per_run.append(phases_of(ctx.PhaseTrace()))  # the last layer's launch
    return summarise(per_run), float(np.median(us_layer))


def summarise(per_run, nphases=None):
    out = {}
    for k in range(nphases or len(PHASES)):
        vals = [r[k] for r in per_run if k in r]
        if vals:
            a = np.array([v[:3] for v in vals])
            out[k] = {"first_us": round(float(np.median(a[:, 0])), 2), "median_us": round(float(np.median(a[:, 1])), 2),
                      "last_us": round(float(np.median(a[:, 2])), 2), "workgroups": vals[0][3]}
    return out


def phases_of(ts, nphases=None):
    """{phase: (earliest, median, latest us after the first start, workgroups)} of one launch's stamps."""
    ts = ts.astype(np.int64)
    starts = ts[:, 0][ts[:, 0] > 0]
    t0 = starts.min()
    row = {}
    for k in range(nphases or len(PHASES)):
        v = ts[:, k]
        v = v[v >= t0]  # every workgroup rewrites phase 0; earlier values are an earlier launch's
        if v.size:
            us = (v - t0) / 100.0
            row[k] = (float(us.min()), float(np.median(us)), float(us.max()), int(v.size))
    return row


MOE_E, MOE_H, MOE_I, MOE_K, MOE_SETS = 128, 2048, 768, 8, 4
ATTN_PHASES = ["start", "q and K landed", "scores and softmax", "V landed", "values accumulated",
               "key lanes summed", "chunk output stored"]
A_HEADS, A_KV, A_DIM, A_KEYS, A_LAYERS = 32, 8, 128, 4096, 36


def attn_timeline(ctx, hip, runs: int):
    """One decode query over 4096 cached keys per layer, one cache per layer (bench.py --config 6)."""
    rng = np.random.default_rng(5)
    caches = [ctx.UploadRaw(rng.standard_normal(2 * A_KEYS * A_KV * A_DIM).astype(np.float32))
              for _ in range(A_LAYERS)]
    q = ctx.UploadRaw((rng.standard_normal(A_HEADS * A_DIM) * 0.3).astype(np.float32))
    o = ctx.NewTensor(A_HEADS * A_DIM)

    def step():
        for c in caches:
            ctx.CachedAttention(o, q, c, 1, A_KEYS, A_HEADS, A_KV, A_DIM, A_KEYS - 1)

    for _ in range(3):
        step()
    ctx.Flush()
    ctx.PhaseTrace("attn")  # clear
    per_run, us_call = [], []
    for _ in range(runs):
        ctx.EventRecord(0)
        step()
        ctx.EventRecord(1)
        ctx.Flush()
        us_call.append(ctx.EventElapsedMs(0, 1) * 1000 / A_LAYERS)
        per_run.append(phases_of(ctx.PhaseTrace("attn"), len(ATTN_PHASES)))  # the last call's launch
    return summarise(per_run, len(ATTN_PHASES)), float(np.median(us_call))


def moe_timeline(ctx, hip, runs: int):
    rng = np.random.default_rng(17)

    def mat(n, k):
        w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
        return hip.MemoryBlock.int4(hip.quantize_int4((w.view(np.uint32) >> 16).astype(np.uint16)))

    sets = [ctx.CreateExpertSet([mat(MOE_I, MOE_H) for _ in range(MOE_E)], [mat(MOE_I, MOE_H) for _ in range(MOE_E)],
                                [mat(MOE_H, MOE_I) for _ in range(MOE_E)], MOE_H, MOE_I) for _ in range(MOE_SETS)]
    x = ctx.UploadRaw(rng.standard_normal(MOE_H).astype(np.float32))
    out = ctx.NewTensor(MOE_H)
    routes = []
    for st in sets:
        for j in range(MOE_E // MOE_K):
            lg = rng.standard_normal((1, MOE_E)).astype(np.float32)
            lg[:, MOE_K * j:MOE_K * (j + 1)] += np.float32(10.0)
            lt, rt = ctx.UploadRaw(lg), ctx.NewTensor(2 * MOE_K)
            ctx.Kernel(hip.GO_MOE_ROUTE, 2 * MOE_K, rt, lt, None, None, [1, MOE_E, MOE_K, 1])
            routes.append((st, rt))

    def step():
        for st, rt in routes:
            ctx.MoEExperts(st, out, x, rt, 1, MOE_K)

    for _ in range(3):
        step()
    ctx.Flush()
    ctx.PhaseTrace("moe")  # clear
    per_run, us_call = [], []
    for _ in range(runs):
        ctx.EventRecord(0)
        step()
        ctx.EventRecord(1)
        ctx.Flush()
        us_call.append(ctx.EventElapsedMs(0, 1) * 1000 / len(routes))
        per_run.append(phases_of(ctx.PhaseTrace("moe")))  # the last call's launch
    return summarise(per_run), float(np.median(us_call))


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
    ap.add_argument("--moe", action="store_true", help="the one-token routed-expert launch instead")
    ap.add_argument("--attn", action="store_true", help="the 4096-key cached-attention launch instead")
    args = ap.parse_args()
    from quicknn_amd import build, hip

    if not os.path.exists(build.TRACE_LIB):
        raise SystemExit(f"{build.TRACE_LIB} is not built: run __graft_entry__.build()")
    hip.LIB_PATH = build.TRACE_LIB
    if args.attn:
        ctx = hip.GPUContext(0)
        phases, us_call = attn_timeline(ctx, hip, args.runs)
        print(f"kernel k_attn_dma (+ k_attn_merge): {us_call:.2f} us per call (HIP events, 36-call runs, "
              f"median of {args.runs})")
        print(f"{'phase':<22s} {'first':>8s} {'median':>8s} {'last':>8s} {'workgroups':>11s}")
        for k, v in phases.items():
            print(f"{k} {ATTN_PHASES[k]:<20s} {v['first_us']:8.2f} {v['median_us']:8.2f} {v['last_us']:8.2f} "
                  f"{v['workgroups']:11d}")
        print(json.dumps({"kernel": "k_attn_dma", "us_per_call": round(us_call, 2),
                          "phases": {ATTN_PHASES[k]: v for k, v in phases.items()}}))
        ctx.close()
        return 0
    if args.moe:
        ctx = hip.GPUContext(0)
        s0 = ctx.status()
        phases, us_call = moe_timeline(ctx, hip, args.runs)
        if ctx.status().moe_fused == s0.moe_fused:
            raise SystemExit("the one-token experts did not run as one launch")
        print(f"kernel k_moe_decode: {us_call:.2f} us per call (HIP events, 64-call runs over 4 expert sets, "
              f"median of {args.runs})")
        print(f"{'phase':<20s} {'first':>8s} {'median':>8s} {'last':>8s} {'workgroups':>11s}")
        for k, v in phases.items():
            print(f"{k} {PHASES[k]:<18s} {v['first_us']:8.2f} {v['median_us']:8.2f} {v['last_us']:8.2f} "
                  f"{v['workgroups']:11d}")
        print(json.dumps({"kernel": "k_moe_decode", "us_per_call": round(us_call, 2),
                          "phases": {PHASES[k]: v for k, v in phases.items()}}))
        ctx.close()
        return 0
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
