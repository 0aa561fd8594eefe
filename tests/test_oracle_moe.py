"""Pins the MoE part of the oracle.

The reference has no CPU MoE; the oracle restates the route op (moe.comp:25-50:
fp32 softmax, k rounds of argmax over the probabilities with ties to the
lower id, optional renormalisation by the top-k sum; exp correctly rounded,
the denominator in the shader's 256-partial order) and the expert accumulation of
TLLMMoE.forward (LLM.MoE.pas:376-448: experts in ascending id, out += y*p,
moe.comp:70 and :125-126).  Pins: route invariants, a brute-force stable sort
on small and tied inputs, and a float64 brute-force composition of the expert
layer over bit-exact dequantised weights.
"""
import numpy as np
import pytest

import oracle
from tests.conftest import rand_int4


def softmax64(l):
    l = np.asarray(l, np.float64)
    e = np.exp(l - l.max())
    return e / e.sum()


@pytest.mark.parametrize("rows,experts,k", [(1, 128, 8), (16, 128, 8), (3, 512, 64), (2, 8, 8), (5, 3, 1)])
@pytest.mark.parametrize("normalize", [True, False])
def test_route_invariants(rng, rows, experts, k, normalize):
    logits = rng.standard_normal((rows, experts)).astype(np.float32)
    ids, probs = oracle.moe_route(logits, k, normalize)
    for r in range(rows):
        assert len(set(ids[r].tolist())) == k
        sm = softmax64(logits[r])
        # brute force: stable sort on -logit == (value desc, id asc)
        assert np.array_equal(ids[r], np.argsort(-logits[r].astype(np.float64), kind="stable")[:k])
        want = sm[ids[r]] / (sm[ids[r]].sum() if normalize else 1.0)
        assert np.allclose(probs[r], want, rtol=2e-6, atol=0)
        assert np.all(np.diff(probs[r]) <= 0)
        if normalize:
            assert abs(float(probs[r].astype(np.float64).sum()) - 1.0) < 1e-5


def test_route_ties_take_lower_id():
    logits = np.array([[0.5, 2.0, 2.0, -1.0, 2.0, 0.5]], np.float32)
    ids, probs = oracle.moe_route(logits, 4, True)
    assert ids[0].tolist() == [1, 2, 4, 0]
    assert probs[0][0] == probs[0][1] == probs[0][2]


def test_route_exp_is_correctly_rounded_and_sum_is_close():
    """v = exp(l - max) rounded once: p * denominator reproduces the float64
    exponential to within half an ulp plus the division's rounding, and the
    denominator is within the float32 summation bound of the float64 sum."""
    logits = np.linspace(-30, 3, 300).astype(np.float32)[None, :]
    ids, probs = oracle.moe_route(logits, 64, False)
    e64 = np.exp(logits[0].astype(np.float64) - float(logits.max()))
    den = e64.sum()
    rel = np.abs(probs[0].astype(np.float64) * den - e64[ids[0]]) / e64[ids[0]]
    assert np.all(rel < 3 * 2.0 ** -24 + 300 * 2.0 ** -24)


def test_route_equal_probabilities_of_distinct_logits_tie_to_lower_id():
    """moe.comp:36-46 compares probabilities: exp(-1e-8) rounds to 1.0f, so ids
    3 (logit -1e-8) and 7 (logit 0) have equal probability and 3 ranks first.
    Ranking by logit would put 7 first."""
    logits = np.full((1, 128), -4.0, np.float32)
    logits[0, 7], logits[0, 3] = 0.0, -1e-8
    assert np.float32(np.exp(np.float64(np.float32(-1e-8)))) == np.float32(1.0)
    ids, probs = oracle.moe_route(logits, 2, True)
    assert ids[0].tolist() == [3, 7] and probs[0, 0] == probs[0, 1] == np.float32(0.5)
    by_logit, _ = oracle.moe_route(logits, 2, True, select_on_logits=True)
    assert by_logit[0].tolist() == [7, 3]


def test_route_denominator_equal_terms():
    """All experts equal: every v is 1, the partial sums and the tree are exact,
    so p = 1/E exactly, whatever E (here beyond the 256 partials)."""
    for E in (5, 256, 300, 1000):
        ids, probs = oracle.moe_route(np.zeros((1, E), np.float32), 4, False)
        assert ids[0].tolist() == [0, 1, 2, 3]
        assert np.all(probs == np.float32(1.0) / np.float32(E))


def test_route_logit_and_probability_selection_agree_without_ties(rng):
    logits = rng.standard_normal((32, 128)).astype(np.float32)
    a = oracle.moe_route(logits, 8, True, select_on_logits=True)
    b = oracle.moe_route(logits, 8, True, select_on_logits=False)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def _mlp64(g, u, d, x, hidden, inter):
    wg = oracle.int4_dequant(g, hidden).astype(np.float64)
    wu = oracle.int4_dequant(u, hidden).astype(np.float64)
    wd = oracle.int4_dequant(d, inter).astype(np.float64)
    a = wg @ x
    h = np.where(a >= 20, a, np.where(a <= -20, 0.0, a / (1.0 + np.exp(-a)))) * (wu @ x)
    return wd @ h


def test_cpu_moe_brute_force(rng):
    E, hidden, inter, k, rows = 6, 96, 64, 3, 4
    gs = [rand_int4(rng, inter, hidden) for _ in range(E)]
    us = [rand_int4(rng, inter, hidden) for _ in range(E)]
    ds = [rand_int4(rng, hidden, inter) for _ in range(E)]
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    ids, probs = oracle.moe_route(rng.standard_normal((rows, E)).astype(np.float32), k, True)
    got = oracle.cpu_moe(gs, us, ds, x, ids, probs, hidden, inter)
    for r in range(rows):
        want = sum(float(probs[r, j]) * _mlp64(gs[e], us[e], ds[e], x[r].astype(np.float64), hidden, inter)
                   for j, e in enumerate(ids[r]))
        assert np.max(np.abs(got[r] - want)) <= 1e-5 * np.max(np.abs(want))
