"""Pins for the oracle's decode-layer restatements (RoPE, KV-cache append,
cached attention, token sampling), against closed forms, invariants and brute
force -- each chosen so that a plausible slip (a flipped sign, adjacent instead
of half-split pairs, a wrong GQA head map, an off-by-one key range, a transposed
cache, a top-k tie broken the wrong way) fails one of them.
"""
import math

import numpy as np
import pytest

import oracle


# ---------------------------------------------------------------- RoPE
def test_rope_position_zero_is_identity():
    x = np.random.default_rng(0).standard_normal(3 * 4 * 16).astype(np.float32)
    assert np.array_equal(oracle.rope(x, 3, 4, 16, 0, 10000.0)[:4 * 16], x[:4 * 16])


def test_rope_single_pair_closed_form():
    # dim 2: one pair, angle = position exactly; (1, 0) -> (cos p, sin p): the sign of the rotation.
    for p in (1, 7, 1000):
        y = oracle.rope(np.array([1.0, 0.0], np.float32), 1, 1, 2, p, 10000.0)
        assert y[0] == np.float32(math.cos(p)) and y[1] == np.float32(math.sin(p))


def test_rope_pairs_are_half_split():
    # dim 4: element 0 pairs with element 2 (j + dim/2), not with element 1.
    y = oracle.rope(np.array([1.0, 0.0, 0.0, 0.0], np.float32), 1, 1, 4, 3, 10000.0)
    assert y[1] == 0.0 and y[3] == 0.0
    assert y[0] == np.float32(math.cos(3.0)) and y[2] == np.float32(math.sin(3.0))
    # The second pair turns at theta^(-1/2) per position.
    y = oracle.rope(np.array([0.0, 1.0, 0.0, 0.0], np.float32), 1, 1, 4, 3, 100.0)
    assert abs(y[1] - math.cos(0.3)) < 1e-7 and abs(y[3] - math.sin(0.3)) < 1e-7


def test_rope_rows_norms_and_composition():
    rng = np.random.default_rng(1)
    rows, heads, dim = 3, 2, 64
    x = rng.standard_normal(rows * heads * dim).astype(np.float32)
    y = oracle.rope(x, rows, heads, dim, 17, 10000.0).reshape(rows, heads, 2, dim // 2)
    x4 = x.reshape(rows, heads, 2, dim // 2)
    assert np.allclose(np.hypot(y[:, :, 0], y[:, :, 1]), np.hypot(x4[:, :, 0], x4[:, :, 1]), rtol=1e-6, atol=1e-7)
    # Row r sits at position + r: rotating row 0 by 17 + 2 equals row 2 of the call at 17.
    one = oracle.rope(x.reshape(rows, heads * dim)[2], 1, heads, dim, 19, 10000.0)
    assert np.array_equal(one, y[2].reshape(-1))
    # Rotations compose: 17 then 40 equals 57 (to rounding).
    a = oracle.rope(oracle.rope(x[:heads * dim], 1, heads, dim, 17, 10000.0), 1, heads, dim, 40, 10000.0)
    b = oracle.rope(x[:heads * dim], 1, heads, dim, 57, 10000.0)
    assert np.max(np.abs(a - b)) < 1e-5


# ---------------------------------------------------------------- cache + attention
def cache_of(rng, kvh, dim, cap, n, masked_rows=0):
    cache = np.zeros(2 * cap * kvh * dim + masked_rows * cap, np.float32)
    k = rng.standard_normal((n, kvh, dim)).astype(np.float32)
    v = rng.standard_normal((n, kvh, dim)).astype(np.float32)
    oracle.cache_write(cache, k, v, n, kvh, dim, cap, 0)
    return cache, k, v


def test_cache_layout_is_transposed_k_then_head_major_v():
    rng = np.random.default_rng(2)
    kvh, dim, cap = 2, 3, 5
    cache, k, v = cache_of(rng, kvh, dim, cap, 4)
    kt = cache[:cap * kvh * dim].reshape(kvh, dim, cap)
    vv = cache[cap * kvh * dim:].reshape(kvh, cap, dim)
    assert np.array_equal(kt[:, :, :4], k.transpose(1, 2, 0)) and not kt[:, :, 4].any()
    assert np.array_equal(vv[:, :4], v.transpose(1, 0, 2)) and not vv[:, 4].any()
    # Appending at position 4 fills the last slot only.
    oracle.cache_write(cache, k[:1], v[:1], 1, kvh, dim, cap, 4)
    assert np.array_equal(cache.reshape(2, kvh, -1)[0].reshape(kvh, dim, cap)[:, :, 4], k[0])


def test_attention_single_key_returns_its_value():
    rng = np.random.default_rng(3)
    cache, k, v = cache_of(rng, 1, 8, 4, 1)
    q = rng.standard_normal(8).astype(np.float32)
    assert np.array_equal(oracle.cached_attention(q, cache, 1, 4, 1, 1, 8, 0), v[0, 0])


def test_attention_uniform_scores_average_the_window():
    rng = np.random.default_rng(4)
    cap, dim = 10, 6
    cache, k, v = cache_of(rng, 1, dim, cap, 9)
    q = np.zeros(dim, np.float32)
    got = oracle.cached_attention(q, cache, 1, cap, 1, 1, dim, 8)
    assert np.allclose(got, v[:9, 0].astype(np.float64).mean(0), atol=1e-6)
    # A window of 3 keeps keys 6..8; a window of 1 only the newest.
    got = oracle.cached_attention(q, cache, 1, cap, 1, 1, dim, 8, window=3)
    assert np.allclose(got, v[6:9, 0].astype(np.float64).mean(0), atol=1e-6)
    assert np.array_equal(oracle.cached_attention(q, cache, 1, cap, 1, 1, dim, 8, window=1), v[8, 0])
    # Query row r of a multi-row call ends at key position + r.
    q2 = np.zeros(3 * dim, np.float32)
    got = oracle.cached_attention(q2, cache, 3, cap, 1, 1, dim, 6).reshape(3, dim)
    for r in range(3):
        assert np.allclose(got[r], v[:7 + r, 0].astype(np.float64).mean(0), atol=1e-6)


def test_attention_two_keys_closed_form_scale_and_softcap():
    dim, cap = 4, 2
    cache = np.zeros(2 * cap * dim, np.float32)
    k = np.array([[[1, 0, 0, 0]], [[0, 1, 0, 0]]], np.float32)
    v = np.array([[[1, 2, 3, 4]], [[5, 6, 7, 8]]], np.float32)
    oracle.cache_write(cache, k, v, 2, 1, dim, cap, 0)
    q = np.array([2.0, -1.0, 0, 0], np.float32)
    a, b = 2.0 / 2.0, -1.0 / 2.0  # scores scaled by 1/sqrt(4)
    pa = math.exp(a) / (math.exp(a) + math.exp(b))
    want = pa * v[0, 0] + (1 - pa) * v[1, 0]
    assert np.allclose(oracle.cached_attention(q, cache, 1, cap, 1, 1, dim, 1), want, atol=1e-6)
    assert np.allclose(oracle.cached_attention(q, cache, 1, cap, 1, 1, dim, 1, scale=0.5), want, atol=1e-6)
    # softcap c: scores c * tanh(s / c).
    c = 0.3
    ca, cb = c * math.tanh(a / c), c * math.tanh(b / c)
    pc = math.exp(ca) / (math.exp(ca) + math.exp(cb))
    want = pc * v[0, 0] + (1 - pc) * v[1, 0]
    assert np.allclose(oracle.cached_attention(q, cache, 1, cap, 1, 1, dim, 1, softcap=c), want, atol=1e-6)


def test_attention_gqa_head_map_and_mask():
    # 4 query heads over 2 KV heads: heads 0,1 read KV head 0, heads 2,3 read KV head 1.
    rng = np.random.default_rng(5)
    dim, cap = 4, 3
    cache, k, v = cache_of(rng, 2, dim, cap, 1)
    q = rng.standard_normal(4 * dim).astype(np.float32)
    got = oracle.cached_attention(q, cache, 1, cap, 4, 2, dim, 0).reshape(4, dim)
    assert np.array_equal(got[0], v[0, 0]) and np.array_equal(got[1], v[0, 0])
    assert np.array_equal(got[2], v[0, 1]) and np.array_equal(got[3], v[0, 1])
    # Masked: only the key with a non-zero word counts.
    cache, k, v = cache_of(rng, 1, dim, cap, 3, masked_rows=1)
    words = cache.view(np.uint32)
    words[2 * cap * dim:] = [0, 7, 0]
    got = oracle.cached_attention(q[:dim], cache, 1, cap, 1, 1, dim, 2, masked=True)
    assert np.array_equal(got, v[1, 0])


# ---------------------------------------------------------------- sampling
def brute_topk(logits, seen, k, penalty):
    items = []
    for t, (s, f) in enumerate(zip(logits.tolist(), seen.tolist())):
        if f == 0xFFFFFFFF or math.isnan(s) or s == -math.inf:
            continue
        s = np.float32(s)
        if f:
            s = np.float32(s * np.float32(penalty)) if s < 0 else np.float32(s / np.float32(penalty))
        items.append((float(s), t))
    items.sort(key=lambda it: (-it[0], it[1]))
    return items[:k]


@pytest.mark.parametrize("vocab,k", [(1, 1), (7, 7), (100, 10), (5000, 64), (20000, 40)])
def test_topk_matches_brute_force_with_ties_bans_and_penalty(vocab, k):
    rng = np.random.default_rng(vocab)
    logits = rng.integers(-20, 20, vocab).astype(np.float32) / 4  # many ties
    seen = np.zeros(vocab, np.uint32)
    seen[rng.random(vocab) < 0.2] = 1
    seen[rng.random(vocab) < 0.05] = 0xFFFFFFFF
    s, ids = oracle.sample_topk(logits, seen, k, 1.3)
    want = brute_topk(logits, seen, k, 1.3)
    got = [(float(a), int(b)) for a, b in zip(s, ids) if b != 0xFFFFFFFF]
    assert got == want


def test_sampling_closed_forms():
    rng = np.random.default_rng(7)
    logits = rng.standard_normal(300).astype(np.float32)
    seen = np.zeros(300, np.uint32)
    best = int(np.argmax(logits))
    assert oracle.sample_token(logits, seen, 40, 0.0, 0.9, 1.0, 0.7) == best   # greedy
    assert oracle.sample_token(logits, seen, 40, 0.8, 0.9, 1.0, 0.0) == best   # uniform 0 -> rank 0
    assert oracle.sample_token(logits, seen, 40, 0.8, 1e-9, 1.0, 0.99) == best  # nucleus of one
    assert oracle.sample_token(logits, seen, 1, 0.8, 1.0, 1.0, 0.99) == best   # k = 1
    # Ties rank the lower id first.
    tie = np.zeros(5, np.float32)
    assert oracle.sample_token(tie, np.zeros(5, np.uint32), 5, 0.0, 1.0, 1.0, 0.5) == 0


def test_sampling_draws_the_softmax_of_the_top_k():
    # Over a fine grid of uniforms the draws reproduce exp((v - v0)/T) / sum within the grid step.
    rng = np.random.default_rng(8)
    logits = rng.standard_normal(50).astype(np.float32) * 2
    seen = np.zeros(50, np.uint32)
    k, temp = 8, 0.7
    s, ids = oracle.sample_topk(logits, seen, k, 1.0)
    w = np.exp((s.astype(np.float64) - s[0]) / temp)
    p = w / w.sum()
    grid = (np.arange(4000) + 0.5) / 4000
    draws = [oracle.sample_token(logits, seen, k, temp, 1.0, 1.0, float(u)) for u in grid]
    freq = np.array([draws.count(int(t)) for t in ids]) / len(grid)
    assert np.max(np.abs(freq - p)) <= 1.5 / len(grid)
    # top_p keeps the shortest prefix reaching top_p of the mass.
    keep = int(np.searchsorted(np.cumsum(p), 0.5) + 1)
    draws = {oracle.sample_token(logits, seen, k, temp, 0.5, 1.0, float(u)) for u in grid}
    assert draws == {int(t) for t in ids[:keep]}
