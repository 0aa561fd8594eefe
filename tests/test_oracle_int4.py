"""Pins the INT4 part of the oracle (src/core/QuickNN.Quantization.Int4.pas and
Int4VectorDot, src/backends/cpu/QuickNN.CPU.Inference.AVX2.inc:210-285) with
known answers, invariants and brute force, and checks the product packer
(qnn_quantize_int4) against it bit for bit."""
import struct

import numpy as np
import pytest

import oracle
from tests.conftest import bf16_bits, bf16_to_f32


def f32(v):
    return struct.unpack("<f", struct.pack("<f", v))[0]


def unpack(packed: np.ndarray, cols: int):
    """Split a packed row matrix into (scales [N,G], nibbles [N,G*32])."""
    rows = packed.shape[0]
    g = (cols + 31) // 32
    blk = packed.reshape(rows, g, 20)
    scales = blk[:, :, :4].copy().view(np.float32).reshape(rows, g)
    b = blk[:, :, 4:]
    nib = np.empty((rows, g, 32), np.uint8)
    nib[:, :, 0::2] = b & 15
    nib[:, :, 1::2] = b >> 4
    return scales, nib.reshape(rows, g * 32)


def test_row_bytes_known_answers():
    assert [oracle.int4_row_bytes(k) for k in (2048, 2560, 9728, 768, 1, 32, 33)] == [1280, 1600, 6080, 480, 20, 20, 40]
    assert oracle.int4_row_bytes(0) == -1


def test_exact_multiples_reconstruct_exactly():
    # c*k with c a power of two: max/7 = c exactly, the refit keeps c, nibbles are k+8.
    k = np.array([-7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6, 7] * 2 + [7, -7], np.float32)
    w = (0.125 * k).reshape(1, 32)
    p = oracle.quantize_int4(w)
    s, n = unpack(p, 32)
    assert s[0, 0] == np.float32(0.125)
    assert np.array_equal(n[0].astype(int) - 8, k.astype(int))
    assert np.array_equal(oracle.int4_dequant(p, 32), w)


def test_zero_group_and_tail():
    w = np.zeros((2, 40), np.float32)
    w[1, :35] = np.linspace(-1, 1, 35)
    p = oracle.quantize_int4(w)
    assert p.shape == (2, 40)
    s, n = unpack(p, 40)
    assert s[0, 0] == 0 and s[0, 1] == 0 and np.all(n[0] == 8)  # all-zero group: scale 0, nibbles 8
    assert np.all(n[1, 35:] == 8)  # tail elements beyond K store 8 (Int4.pas:85-89)
    assert s[1, 1] > 0


def test_round_half_even_then_refit():
    # values [7, 2.5, 0...]: first scale 1, Round(2.5) = 2 (half-to-even), refit
    # s = (7*7 + 2.5*2) / (49 + 4) = 54/53; final q = Round(v/s) -> [7, 2].
    w = np.zeros((1, 32), np.float32)
    w[0, 0], w[0, 1] = 7.0, 2.5
    p = oracle.quantize_int4(w)
    s, n = unpack(p, 32)
    assert s[0, 0] == np.float32(54.0 / 53.0)
    assert n[0, 0] == 15 and n[0, 1] == 10 and np.all(n[0, 2:] == 8)


def test_invariants_and_least_squares(rng):
    w = (rng.standard_normal((64, 300)) * 0.02).astype(np.float32)
    w[3, :] = 0.0
    w[5, 7] = 1e-3  # one outlier
    p = oracle.quantize_int4(w)
    s, n = unpack(p, 300)
    assert np.all(s >= 0)
    real = n[:, :300]
    nz = s.repeat(32, axis=1)[:, :300] > 0
    assert np.all((real[nz] >= 1) & (real[nz] <= 15))  # q in [-7, 7]
    # The refit minimises sum (v - s q0)^2 over s for the first-pass levels
    # q0 = Round(v / (max|v|/7)) (Int4.pas:62-76): the gradient
    # sum q0 (v - s q0) vanishes up to the fp32 rounding of s.
    q = n.astype(np.float64).reshape(64, -1, 32) - 8
    v = np.zeros((64, q.shape[1] * 32))
    v[:, :300] = w
    v = v.reshape(64, -1, 32)
    first = (np.max(np.abs(v), axis=2) / 7).astype(np.float32).astype(np.float64)
    with np.errstate(invalid="ignore", divide="ignore"):
        q0 = np.clip(np.round(np.where(first[:, :, None] > 0, v / first[:, :, None], 0)), -7, 7)
    grad = np.sum(q0 * (v - s[:, :, None].astype(np.float64) * q0), axis=2)
    qq = np.sum(q0 * q0, axis=2)
    bound = qq * np.abs(s) * 2.0 ** -23 + 1e-30
    assert np.all(np.abs(grad) <= bound)
    # Each stored nibble is the nearest level for the refitted scale.
    recon = s[:, :, None] * q
    err = np.abs(v - recon)
    ok = err <= 0.5 * s[:, :, None] * (1 + 1e-6) + 1e-30
    clamped = np.abs(v) > 7 * s[:, :, None]
    assert np.all(ok | clamped)


def test_non_finite_raises():
    w = np.ones((1, 32), np.float32)
    w[0, 3] = np.nan
    with pytest.raises(ValueError):
        oracle.quantize_int4(w)
    w[0, 3] = np.inf
    with pytest.raises(ValueError):
        oracle.quantize_int4(w)


def test_bf16_path_matches_f32_on_bf16_values(rng):
    b = bf16_bits(rng.standard_normal((8, 96)) * 0.02)
    assert np.array_equal(oracle.quantize_int4(b), oracle.quantize_int4(bf16_to_f32(b)))


def test_dequant_is_single_rounding(rng):
    b = bf16_bits(rng.standard_normal((16, 64)) * 0.02)
    p = oracle.quantize_int4(b)
    s, n = unpack(p, 64)
    want = ((n.astype(np.float64) - 8) * s.repeat(32, axis=1).astype(np.float64)).astype(np.float32)
    assert np.array_equal(oracle.int4_dequant(p, 64).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("k", [32, 64, 2048, 2560, 40, 33, 7])
def test_int4_vector_dot_brute_force(rng, k):
    b = bf16_bits(rng.standard_normal((4, k)) * 0.02)
    p = oracle.quantize_int4(b)
    x = rng.standard_normal(k).astype(np.float32)
    deq = oracle.int4_dequant(p, k).astype(np.float64)
    for r in range(4):
        got = oracle.int4_vector_dot(x, p[r])
        want = float(deq[r] @ x.astype(np.float64))
        assert abs(got - want) <= 2e-6 * float(np.abs(deq[r]) @ np.abs(x)) + 1e-12


@pytest.mark.parametrize("n", [1, 7, 8, 31, 32, 33, 100, 2048])
def test_vector_dot_brute_force(rng, n):
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    got = oracle.vector_dot(a, b)
    want = float(a.astype(np.float64) @ b.astype(np.float64))
    assert abs(got - want) <= 2e-6 * float(np.abs(a) @ np.abs(b))


def test_cpu_linear_threads_bit_identical(rng):
    # Rows are independent, so the pool split cannot change any output bit
    # (CPU.Inference.pas:378-389).  K*N >= 1M engages the pool.
    b = bf16_bits(rng.standard_normal((1024, 1024)) * 0.02)
    p = oracle.quantize_int4(b)
    x = rng.standard_normal(1024).astype(np.float32)
    one = oracle.Pool(1)
    many = oracle.Pool(8)
    y1 = oracle.cpu_linear(p, oracle.ENC_INT4, x, 1024, 1024, one)
    y8 = oracle.cpu_linear(p, oracle.ENC_INT4, x, 1024, 1024, many)
    assert np.array_equal(y1.view(np.uint32), y8.view(np.uint32))
    rows = np.array([oracle.int4_vector_dot(x, p[r]) for r in range(0, 1024, 97)], np.float32)
    assert np.array_equal(y1[::97].view(np.uint32), rows.view(np.uint32))


def test_product_packer_matches_oracle(rng):
    """qnn_quantize_int4 (product, multithreaded) == oracle restatement, bit for bit."""
    from quicknn_amd import hip

    for shape in [(1, 1), (3, 33), (64, 2048), (130, 2560), (17, 768)]:
        w = rng.standard_normal(shape).astype(np.float32) * 0.02
        w[0, 0] = 0.0
        b = bf16_bits(w)
        assert np.array_equal(hip.quantize_int4(b), oracle.quantize_int4(b))
        assert np.array_equal(hip.quantize_int4(w), oracle.quantize_int4(w))
    with pytest.raises(hip.EArgumentException):
        bad = np.ones((2, 32), np.float32)
        bad[1, 1] = np.nan
        hip.quantize_int4(bad)
