"""Pins the oracle's int8-activation Q8_0 GEMM (the benchmark's configs[4]
prefill path: activations quantised per 32-element block to int8).

The reference has no such path, so the pins come from what the mathematics
fixes:
* quantiser: |q| <= 127, the block's largest magnitude maps to +-127, an
  all-zero block gives d = 0 and q = 0, and every value reconstructs to within
  half a step (|x - q d| <= d/2);
* GEMM: an all-integer case (d = 1 on both sides) is exact and equals the
  integer matmul; random cases equal a float64 sum of dx * dw * S_b within
  fp32 rounding; a transposed operand or a wrong block index fails both;
* against the reference's fp32 product (qo_gguf_gemm_scalar) the int8 path is
  within 1e-2 normwise for N(0, 1) activations: the cost of the quantisation.
"""
import numpy as np
import pytest

import oracle
from tests.conftest import normwise_rel_err


def q8_0_blocks(rng, n, k, scale=0.02):
    from quicknn_amd import hip

    return hip.gguf_quantize(hip.WE_Q8_0, (rng.standard_normal((n, k)) * scale).astype(np.float32))


def decode_q8_0(w, n, k):
    b = np.frombuffer(np.ascontiguousarray(w).tobytes(), np.uint8).reshape(n, k // 32, 34)
    d = b[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float64)
    q = b[:, :, 2:].view(np.int8).astype(np.int64)
    return q, d


@pytest.mark.parametrize("m,k", [(1, 32), (5, 96), (17, 3072)])
def test_act_quant_invariants(rng, m, k):
    a = (rng.standard_normal((m, k)) * rng.uniform(0.1, 10, (m, 1))).astype(np.float32)
    a[0, :32] = 0.0  # an all-zero block
    q, d = oracle.q8_act_quant(a)
    assert d[0, 0] == 0 and np.all(q[0, :32] == 0)
    blocks = a.reshape(m, k // 32, 32)
    qb = q.reshape(m, k // 32, 32).astype(np.int64)
    assert np.all(np.abs(qb) <= 127)
    nz = d > 0
    assert np.all(np.abs(qb).max(axis=2)[nz] == 127)
    assert np.allclose(d, np.abs(blocks).max(axis=2) / np.float32(127), rtol=1e-7, atol=0)
    err = np.abs(blocks.astype(np.float64) - qb * d[..., None].astype(np.float64))
    assert np.all(err <= d[..., None].astype(np.float64) * (0.5 + 1e-5))


def test_gemm_integer_case_is_exact(rng):
    """d = 1 on both sides (activations whose block maximum is 127, weights with
    fp16 scale 1.0): every block sum is an exact integer, so C is the integer
    matmul exactly."""
    m, k, n = 7, 96, 40
    a = rng.integers(-127, 128, (m, k)).astype(np.float32)
    a.reshape(m, k // 32, 32)[:, :, 0] = 127.0  # block maxima 127: d = 1 exactly
    q, d = oracle.q8_act_quant(a)
    assert np.all(d == 1.0) and np.array_equal(q.astype(np.float32), a)
    wq = rng.integers(-127, 128, (n, k // 32, 32)).astype(np.int8)
    blocks = np.zeros((n, k // 32, 34), np.uint8)
    blocks[:, :, :2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blocks[:, :, 2:] = wq.view(np.uint8)
    c = oracle.q8_gemm_i8(blocks.reshape(-1), q, d, n)
    want = a.astype(np.int64) @ wq.reshape(n, k).astype(np.int64).T
    assert np.array_equal(c.astype(np.int64), want)
    # a transposed weight or a shifted block would not reproduce it
    assert not np.array_equal(c.astype(np.int64), a.astype(np.int64) @ np.roll(wq.reshape(n, k), 32, axis=1).astype(np.int64).T)


@pytest.mark.parametrize("m,k,n", [(3, 64, 50), (9, 288, 33), (4, 3072, 64)])
def test_gemm_matches_float64_block_sum(rng, m, k, n):
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = q8_0_blocks(rng, n, k)
    q, d = oracle.q8_act_quant(a)
    c = oracle.q8_gemm_i8(w, q, d, n)
    wq, wd = decode_q8_0(w, n, k)
    s = np.einsum("rbi,obi->rob", q.reshape(m, k // 32, 32).astype(np.int64), wq)
    want = np.einsum("rob,rb,ob->ro", s.astype(np.float64), d.astype(np.float64), wd)
    assert normwise_rel_err(c, want) < 2e-6


def test_int8_path_costs_about_the_quantisation_against_fp32(rng):
    m, k, n = 6, 3072, 96
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = q8_0_blocks(rng, n, k)
    q, d = oracle.q8_act_quant(a)
    c = oracle.q8_gemm_i8(w, q, d, n)
    ref = oracle.gguf_gemm_scalar(w, oracle.ENC_Q8_0, a, n)
    e = normwise_rel_err(c, ref)
    assert 1e-4 < e < 1e-2
