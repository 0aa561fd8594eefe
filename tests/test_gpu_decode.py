"""GPU parity of the rest of the decode layer against the CPU oracle.

* GO_LLM_ROPE: within 1 ulp of the oracle's double-precision statement
  (QwenHybrid.CPU.pas:51-67); both round a double result once.
* GO_LLM_CACHE_WRITE, GO_LLM_SEEN, GO_SCALE: bit-exact (data movement, flags,
  one multiply and one add).
* CachedAttention: normwise relative error <= 1e-4 against the oracle's
  double-precision attention (the decode path's fp bar is 1e-3).
* SampleToken: the greedy token and the whole ranked top-k exactly (each
  candidate drawn by a uniform in the middle of its probability interval), and
  the oracle's token for random uniforms that are not within 1e-4 of an
  interval boundary (where 1-ulp differences of exp may legitimately flip).
"""
import numpy as np
import pytest

import oracle
from quicknn_amd import hip
from tests.conftest import normwise_rel_err

pytestmark = pytest.mark.gpu


def up(ctx, a):
    return ctx.UploadRaw(np.ascontiguousarray(a).view(np.float32).reshape(-1))


def ulp_diff(a: np.ndarray, b: np.ndarray) -> int:
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return int(np.max(np.abs(ia - ib))) if a.size else 0


# ---------------------------------------------------------------- RoPE
@pytest.mark.parametrize("rows,heads,dim,pos,theta", [
    (1, 32, 128, 0, 1e6), (1, 32, 128, 4095, 1e6), (1, 8, 128, 100000, 1e4), (5, 16, 256, 37, 1e4),
    (3, 4, 64, 1000, 5e5), (1, 1, 2, 123456, 1e4)])
def test_rope_matches_cpu_statement(ctx, rng, rows, heads, dim, pos, theta):
    x = rng.standard_normal(rows * heads * dim).astype(np.float32)
    t = up(ctx, x)
    n = rows * heads * dim // 2
    ctx.Kernel(hip.GO_LLM_ROPE, n, t, t, None, None, [heads, dim, pos, hip.float_bits(theta)])
    got = ctx.Download(t)
    want = oracle.rope(x, rows, heads, dim, pos, theta)
    assert ulp_diff(got, want) <= 1
    # Out of place: the source is left as it was.
    src, dst = up(ctx, x), ctx.NewTensor(x.size)
    ctx.Kernel(hip.GO_LLM_ROPE, n, dst, src, None, None, [heads, dim, pos, hip.float_bits(theta)])
    assert np.array_equal(ctx.Download(dst), got) and np.array_equal(ctx.Download(src), x)
    for z in (t, src, dst):
        ctx.Recycle(z)


# ---------------------------------------------------------------- cache, seen, scale
def test_cache_write_bit_exact(ctx, rng):
    kvh, dim, cap = 8, 128, 300
    cache_ref = np.zeros(2 * cap * kvh * dim, np.float32)
    cache = ctx.UploadRaw(cache_ref)
    for pos, rows in ((0, 1), (1, 7), (8, 1), (299, 1)):
        k = rng.standard_normal((rows, kvh, dim)).astype(np.float32)
        v = rng.standard_normal((rows, kvh, dim)).astype(np.float32)
        tk, tv = up(ctx, k), up(ctx, v)
        ctx.Kernel(hip.GO_LLM_CACHE_WRITE, rows * kvh * dim, cache, tk, tv, None, [rows, kvh, dim, cap, pos])
        oracle.cache_write(cache_ref, k, v, rows, kvh, dim, cap, pos)
        ctx.Recycle(tk)
        ctx.Recycle(tv)
    assert np.array_equal(ctx.Download(cache), cache_ref)
    with pytest.raises(hip.EArgumentException):  # past the capacity
        tk = ctx.NewTensor(2 * kvh * dim)
        ctx.Kernel(hip.GO_LLM_CACHE_WRITE, 2 * kvh * dim, cache, tk, tk, None, [2, kvh, dim, cap, 299])
    ctx.Recycle(cache)


def test_seen_flags_and_scale(ctx, rng):
    vocab = 1000
    flags = np.zeros(vocab, np.uint32)
    flags[[5, 9]] = 0xFFFFFFFF
    ids = np.array([3, 5, 999, 1000, 70000, 3, 42], np.uint32)
    tf, ti = up(ctx, flags), up(ctx, ids)
    ctx.Kernel(hip.GO_LLM_SEEN, ids.size, tf, ti, None, None, [vocab])
    want = flags.copy()
    for t in ids:
        if t < vocab:
            want[t] |= 1
    assert np.array_equal(ctx.Download(tf).view(np.uint32), want)
    x = rng.standard_normal(5000).astype(np.float32)
    tx = up(ctx, x)
    ctx.Kernel(hip.GO_SCALE, x.size, tx, tx, None, None, [hip.float_bits(1.7)])
    assert np.array_equal(ctx.Download(tx), x * np.float32(1.7))
    ctx.Kernel(hip.GO_SCALE, x.size, tx, tx, None, None, [hip.float_bits(0.5), hip.float_bits(-3.0)])
    assert np.array_equal(ctx.Download(tx), (x * np.float32(1.7)) * np.float32(0.5) + np.float32(-3.0))
    ty = up(ctx, x * 10)
    ctx.Kernel(hip.GO_SOFTCAP, x.size, ty, ty, None, None, [hip.float_bits(30.0)])
    want = 30.0 * np.tanh(np.clip(x.astype(np.float64) * 10 / 30.0, -20, 20))
    assert np.max(np.abs(ctx.Download(ty) - want)) <= 4e-6 * 30
    for z in (tf, ti, tx, ty):
        ctx.Recycle(z)


# ---------------------------------------------------------------- attention
ATTN = [
    # rows, heads, kvh, dim, cap, pos, window, softcap, scale, masked
    (1, 32, 8, 128, 64, 0, 0, 0.0, 0.0, False),
    (1, 32, 8, 128, 300, 5, 0, 0.0, 0.0, False),
    (1, 32, 8, 128, 300, 255, 0, 0.0, 0.0, False),
    (1, 32, 8, 128, 300, 256, 0, 0.0, 0.0, False),
    (1, 32, 8, 128, 4096, 4095, 0, 0.0, 0.0, False),      # Qwen3-4B shape, 16 key chunks
    (1, 32, 4, 128, 2048, 1500, 0, 0.0, 0.0, False),      # Qwen3-30B-A3B: 8 heads per KV head
    (1, 16, 8, 256, 5200, 5100, 4096, 50.0, 0.0625, False),  # Gemma-2-9B: window, softcap, scale
    (1, 16, 1, 64, 900, 800, 0, 0.0, 0.0, False),         # 16 heads per KV head (two workgroups)
    (1, 12, 2, 80, 700, 650, 0, 0.0, 0.0, False),         # 6 heads per KV head, dim 80
    (1, 4, 4, 576, 600, 520, 0, 0.0, 0.0, False),         # MHA, dim 576 (three channels per thread)
    (1, 2, 1, 1152, 400, 333, 0, 0.0, 0.0, False),        # the largest dim
    (7, 32, 8, 128, 1024, 300, 0, 0.0, 0.0, False),       # prefill rows
    (3, 8, 2, 128, 700, 600, 0, 0.0, 0.0, True),          # masked
    (2, 8, 8, 64, 40, 10, 3, 0.0, 0.0, False),            # short window
    (1, 32, 8, 128, 40000, 39000, 0, 0.0, 0.0, False),    # several sub-chunks per workgroup
    (1, 16, 2, 1152, 300, 290, 0, 0.0, 0.0, False),       # 8 heads per workgroup, two float4 groups per lane
    (2, 8, 4, 66, 200, 150, 0, 0.0, 0.0, False),          # dim not a multiple of 4
    (2, 8, 2, 128, 3000, 2500, 1000, 30.0, 0.0, True),    # window and mask together
    (1, 32, 8, 128, 5000, 4999, 4096, 0.0, 0.0, False),   # window, 64-key chunks from key 904
    (1, 32, 8, 128, 8192, 2047, 0, 20.0, 0.125, False),   # softcap and scale on 64-key chunks
]


@pytest.mark.parametrize("case", ATTN, ids=[f"r{c[0]}h{c[1]}k{c[2]}d{c[3]}p{c[5]}w{c[6]}m{int(c[9])}" for c in ATTN])
def test_cached_attention_matches_oracle(ctx, rng, tune, case):
    """Against the oracle within 1e-4 per head row.  At dim 128 with 64-key chunks whose starts are
    multiples of 4 the call takes the kernel that streams each chunk into LDS; it must give the same
    bits as the general kernel (QNN_ATTN_DMA=0), which every other shape takes."""
    rows, heads, kvh, dim, cap, pos, window, softcap, scale, masked = case
    n = pos + rows
    size = 2 * cap * kvh * dim + (rows * cap if masked else 0)
    cache_ref = np.zeros(size, np.float32)
    k = rng.standard_normal((n, kvh, dim)).astype(np.float32)
    v = rng.standard_normal((n, kvh, dim)).astype(np.float32)
    oracle.cache_write(cache_ref, k, v, n, kvh, dim, cap, 0)
    if masked:
        m = (rng.random((rows, cap)) < 0.6).astype(np.uint32) * rng.integers(1, 9, (rows, cap)).astype(np.uint32)
        m[:, 0] = 1
        cache_ref.view(np.uint32)[2 * cap * kvh * dim:] = m.reshape(-1)
    q = (rng.standard_normal(rows * heads * dim) * 0.3).astype(np.float32)
    want = oracle.cached_attention(q, cache_ref, rows, cap, heads, kvh, dim, pos, window, softcap, scale, masked)
    tq, tc, to = up(ctx, q), up(ctx, cache_ref), ctx.NewTensor(rows * heads * dim)
    ctx.CachedAttention(to, tq, tc, rows, cap, heads, kvh, dim, pos, window, softcap, scale, masked)
    got = ctx.Download(to).reshape(rows * heads, dim)
    w = want.reshape(rows * heads, dim)
    for i in range(rows * heads):
        assert normwise_rel_err(got[i], w[i]) <= 1e-4, i
    tune("QNN_ATTN_DMA", "0")
    ctx.CachedAttention(to, tq, tc, rows, cap, heads, kvh, dim, pos, window, softcap, scale, masked)
    general = ctx.Download(to).reshape(rows * heads, dim)
    assert np.array_equal(got.view(np.uint32), general.view(np.uint32))
    for z in (tq, tc, to):
        ctx.Recycle(z)


def test_decode_step_through_the_device_cache(ctx, rng):
    """RoPE of q and k, cache append and attention, all on the device, step by step."""
    heads, kvh, dim, cap, theta = 16, 4, 128, 64, 1e6
    cache = ctx.UploadRaw(np.zeros(2 * cap * kvh * dim, np.float32))
    cache_ref = np.zeros(2 * cap * kvh * dim, np.float32)
    for pos in range(0, 40, 13):
        q = rng.standard_normal(heads * dim).astype(np.float32)
        k = rng.standard_normal(kvh * dim).astype(np.float32)
        v = rng.standard_normal(kvh * dim).astype(np.float32)
        tq, tk, tv, to = up(ctx, q), up(ctx, k), up(ctx, v), ctx.NewTensor(heads * dim)
        ctx.Kernel(hip.GO_LLM_ROPE, heads * dim // 2, tq, tq, None, None, [heads, dim, pos, hip.float_bits(theta)])
        ctx.Kernel(hip.GO_LLM_ROPE, kvh * dim // 2, tk, tk, None, None, [kvh, dim, pos, hip.float_bits(theta)])
        ctx.Kernel(hip.GO_LLM_CACHE_WRITE, kvh * dim, cache, tk, tv, None, [1, kvh, dim, cap, pos])
        ctx.CachedAttention(to, tq, cache, 1, cap, heads, kvh, dim, pos)
        qr, kr = oracle.rope(q, 1, heads, dim, pos, theta), oracle.rope(k, 1, kvh, dim, pos, theta)
        oracle.cache_write(cache_ref, kr, v, 1, kvh, dim, cap, pos)
        want = oracle.cached_attention(qr, cache_ref, 1, cap, heads, kvh, dim, pos)
        assert normwise_rel_err(ctx.Download(to), want) <= 1e-4, pos
        for z in (tq, tk, tv, to):
            ctx.Recycle(z)
    ctx.Recycle(cache)


def test_attention_argument_errors(ctx):
    q, c, o = ctx.NewTensor(4 * 64), ctx.NewTensor(2 * 8 * 64), ctx.NewTensor(4 * 64)
    bad = [dict(heads=3, kv_heads=2), dict(position=8), dict(dim=2000), dict(window=-1), dict(softcap=float("nan"))]
    for b in bad:
        kw = dict(query_rows=1, capacity=8, heads=4, kv_heads=1, dim=64, position=0, window=0, softcap=0.0,
                  scale=0.0)
        kw.update(b)
        with pytest.raises(hip.EArgumentException):
            ctx.CachedAttention(o, q, c, **kw)
    for z in (q, c, o):
        ctx.Recycle(z)


# ---------------------------------------------------------------- sampling
def sample(ctx, logits, seen, k, temp, top_p, penalty, u, tl=None, ts=None):
    own = tl is None
    tl = tl or up(ctx, logits)
    ts = ts or up(ctx, seen)
    td = ctx.NewTensor(1)
    ctx.SampleToken(td, tl, ts, logits.size, k, temp, top_p, penalty, u)
    tok = int(ctx.Download(td).view(np.uint32)[0])
    ctx.Recycle(td)
    if own:
        ctx.Recycle(tl)
        ctx.Recycle(ts)
    return tok


def intervals(scores, k, temp, top_p):
    """float64 cumulative probability intervals of the kept candidates."""
    w = np.exp((scores[:k].astype(np.float64) - scores[0]) / temp)
    c = np.cumsum(w)
    keep = int(np.searchsorted(c, top_p * c[-1] * (1 - 1e-12)) + 1)
    keep = min(keep, k)
    c = c[:keep] / c[keep - 1]
    return np.concatenate([[0.0], c])


@pytest.mark.parametrize("vocab", [100, 4096, 4097, 151936, 256000, 300000])
def test_sampling_matches_oracle(ctx, rng, vocab):
    logits = (rng.standard_normal(vocab) * 3).astype(np.float32)
    logits[rng.integers(0, vocab, vocab // 50)] = logits.max()  # ties at the top
    seen = np.zeros(vocab, np.uint32)
    seen[rng.random(vocab) < 0.1] = 1
    seen[rng.random(vocab) < 0.02] = 0xFFFFFFFF
    tl, ts = up(ctx, logits), up(ctx, seen)
    # Greedy: the best token after the penalty, lower id first among ties.
    assert sample(ctx, logits, seen, 40, 0.0, 0.9, 1.3, 0.5, tl, ts) == oracle.sample_token(
        logits, seen, 40, 0.0, 0.9, 1.3, 0.5)
    for k, temp, top_p in ((64, 1.0, 1.0), (40, 0.7, 0.9), (5, 0.2, 1.0)):
        kk = min(k, vocab)
        s, ids = oracle.sample_topk(logits, seen, kk, 1.3)
        edges = intervals(s, kk, temp, top_p)
        # Every kept candidate, in rank order, from the middle of its interval.
        for j in range(len(edges) - 1):
            u = float((edges[j] + edges[j + 1]) / 2)
            if edges[j + 1] - edges[j] < 1e-6:
                continue
            assert sample(ctx, logits, seen, k, temp, top_p, 1.3, u, tl, ts) == int(ids[j]), (k, j)
        for u in rng.random(30):
            if np.min(np.abs(edges - u)) < 1e-4:
                continue
            assert sample(ctx, logits, seen, k, temp, top_p, 1.3, float(u), tl, ts) == oracle.sample_token(
                logits, seen, k, temp, top_p, 1.3, float(u))
    ctx.Recycle(tl)
    ctx.Recycle(ts)


def test_sampling_excluded_tokens_and_errors(ctx):
    vocab = 9000
    logits = np.zeros(vocab, np.float32)
    logits[8999] = 5.0
    seen = np.full(vocab, 0xFFFFFFFF, np.uint32)
    seen[[3, 8000]] = 0
    # Only tokens 3 and 8000 remain; equal scores rank the lower id first.
    assert sample(ctx, logits, seen, 10, 0.0, 1.0, 1.0, 0.3) == 3
    assert sample(ctx, logits, seen, 10, 1.0, 1.0, 1.0, 0.99) == 8000
    # Everything excluded: no token (0xffffffff), as the reference's kernel leaves it.
    assert sample(ctx, logits, np.full(vocab, 0xFFFFFFFF, np.uint32), 10, 0.0, 1.0, 1.0, 0.3) == 0xFFFFFFFF
    tl, ts, td = up(ctx, logits), up(ctx, seen), ctx.NewTensor(1)
    for args in ((0, 1.0, 1.0, 1.0, 0.5), (65, 1.0, 1.0, 1.0, 0.5), (10, -1.0, 1.0, 1.0, 0.5),
                 (10, 1.0, 0.0, 1.0, 0.5), (10, 1.0, 1.0, 0.0, 0.5), (10, 1.0, 1.0, 1.0, 1.0)):
        with pytest.raises(hip.EArgumentException):
            ctx.SampleToken(td, tl, ts, vocab, *args)
    with pytest.raises(hip.EArgumentException):
        ctx.SampleToken(tl, tl, ts, vocab, 10, 1.0, 1.0, 1.0, 0.5)
    for z in (tl, ts, td):
        ctx.Recycle(z)


# ---------------------------------------------------------------- gather
@pytest.mark.parametrize("kind", ["f32", "bf16", "s8", "q4_k", "q6_k", "q8_0", "q5_k", "iq4_xs", "q2_0", "iq2_xxs",
                                  "iq3_s"])
def test_gather_embedding_rows(ctx, rng, kind):
    """Gather: token rows of the table, bit-exact; ids at or past the vocabulary give zeros."""
    vocab, dim = 1000, 512
    table = (rng.standard_normal((vocab, dim)) * 0.05).astype(np.float32)
    scales = None
    if kind == "f32":
        w, rows_f = hip.MemoryBlock.matrix(table), table
    elif kind == "bf16":
        bits = (table.view(np.uint32) >> 16).astype(np.uint16)
        w, rows_f = hip.MemoryBlock.matrix(bits), (bits.astype(np.uint32) << 16).view(np.float32)
    elif kind == "s8":
        q = rng.integers(-127, 128, (vocab, dim)).astype(np.int8)
        s = (rng.random(vocab) * 0.01).astype(np.float32)
        w = hip.MemoryBlock(q, q.shape, hip.DT_S8)
        scales = hip.MemoryBlock.vector(s)
        rows_f = q.astype(np.float32) * s[:, None]
    else:
        enc = {"q4_k": hip.WE_Q4_K, "q6_k": hip.WE_Q6_K, "q8_0": hip.WE_Q8_0, "q5_k": hip.WE_Q5_K,
               "iq4_xs": hip.WE_IQ4_XS, "q2_0": hip.WE_Q2_0, "iq2_xxs": hip.WE_IQ2_XXS, "iq3_s": hip.WE_IQ3_S}[kind]
        blocks = hip.gguf_quantize(enc, table)
        w = hip.MemoryBlock.gguf(blocks, vocab, dim, enc)
        rows_f = oracle.gguf_dequant_scalar(blocks, enc, vocab * dim).reshape(vocab, dim)
    ids = np.array([0, 999, 5, 1000, 123, 0xFFFFFFFF, 5], np.uint32)
    ti, td = up(ctx, ids), ctx.NewTensor(ids.size * dim)
    ctx.Gather(td, ti, w, scales, ids.size, dim, vocab)
    got = ctx.Download(td).reshape(ids.size, dim)
    for r, t in enumerate(ids):
        want = rows_f[t] if t < vocab else np.zeros(dim, np.float32)
        assert np.array_equal(got[r], want), (kind, r)
    with pytest.raises(hip.ENotSupportedException):
        ctx.Gather(td, ti, w, scales, ids.size, dim, vocab, 1)
    ctx.Recycle(ti)
    ctx.Recycle(td)
