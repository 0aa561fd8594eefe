"""Pins the oracle's decode-layer composites and its multi-row GGUF product.

Functions pinned here (each by something the mathematics fixes, not by
retyping the oracle's formula):
  - rmsnorm (QwenHybrid.CPU.pas:110-120): exact power-of-two scale invariance,
    unit mean square, the closed form c/sqrt(c^2+eps) for constant rows, gamma
    per column and the add-one form.
  - silu (QwenHybrid.CPU.pas:78-82, :242-246): x*sigmoid(x) in float64 to one
    rounding, the reflection silu(-x) = silu(x) - x, and the +-20 clamps.
  - cpu_mlp (QwenHybrid.CPU.pas:238-248): float64 brute force over bit-exact
    dequantised INT4 and K-quant weights (gate and up are not interchangeable
    because silu is not symmetric).
  - gguf_gemm_scalar (QuickNN.Quantization.pas:247-258): float64 matmul over
    the dequantised rows, then one rounding to fp32; row ranges compose.
"""
import numpy as np
import pytest
from scipy.special import expit

import oracle
from tests.conftest import normwise_rel_err, rand_int4


def ulp32(x):
    return np.spacing(np.abs(np.asarray(x, np.float32))).astype(np.float64)


def test_rmsnorm_scale_invariance_and_unit_mean_square(rng):
    x = rng.standard_normal((5, 2560)).astype(np.float32)
    gamma = np.ones(2560, np.float32)
    y = oracle.rmsnorm(x, gamma, eps=0.0)
    for a in (0.25, 8.0, 1024.0):  # powers of two: sum scales by a^2 and the root by a, exactly
        assert np.array_equal(oracle.rmsnorm(x * np.float32(a), gamma, eps=0.0), y)
    ms = np.mean(y.astype(np.float64) ** 2, axis=1)
    assert np.allclose(ms, 1.0, rtol=1e-6)
    # a dropped 1/dim or a square root in the wrong place fails here
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=1, keepdims=True))
    assert np.all(np.abs(y - ref) <= 3 * ulp32(ref))


@pytest.mark.parametrize("c,eps", [(3.0, 1e-6), (1e-3, 1e-6), (0.5, 0.25), (0.0, 1e-6)])
def test_rmsnorm_constant_rows_closed_form(c, eps):
    x = np.full((2, 64), c, np.float32)
    y = oracle.rmsnorm(x, np.ones(64, np.float32), eps=eps)
    want = np.float64(np.float32(c)) / np.sqrt(np.float64(np.float32(c)) ** 2 + np.float64(np.float32(eps)))
    assert np.all(np.isfinite(y))
    assert np.all(np.abs(y - want) <= 2 * ulp32(want))


def test_rmsnorm_gamma_and_add_one(rng):
    x = rng.standard_normal((3, 256)).astype(np.float32)
    g = rng.standard_normal(256).astype(np.float32)
    base = oracle.rmsnorm(x, np.ones(256, np.float32), eps=1e-6)
    y = oracle.rmsnorm(x, g, eps=1e-6)
    assert np.all(np.abs(y - base * g) <= 2 * ulp32(base * g))
    # Gemma's (1 + gamma) form equals passing gamma + 1 (exact when gamma + 1 is exact)
    gi = rng.integers(-4, 4, 256).astype(np.float32)
    assert np.array_equal(oracle.rmsnorm(x, gi, eps=1e-6, add_one=True), oracle.rmsnorm(x, gi + 1, eps=1e-6))


def test_silu_against_float64_and_reflection(rng):
    xs = np.concatenate([rng.uniform(-19.9, 19.9, 4000), [-1e-30, 0.0, 1e-30, 0.5, -0.5, 19.99, -19.99]])
    xs = xs.astype(np.float32)
    got = np.array([oracle.silu(float(v)) for v in xs], np.float32)
    ref = xs.astype(np.float64) * expit(xs.astype(np.float64))
    assert np.all(np.abs(got - ref) <= 2 * ulp32(ref) + 1e-45)
    refl = np.array([oracle.silu(float(-v)) for v in xs], np.float64)
    assert np.all(np.abs(refl - (got.astype(np.float64) - xs)) <= 4 * ulp32(xs) + 4 * ulp32(got))
    assert oracle.silu(0.0) == 0.0


def test_silu_clamps():
    for v in (20.0, 25.0, 1e30, 1e38):
        assert oracle.silu(v) == np.float32(v)
    for v in (-20.0, -25.0, -1e30):
        assert oracle.silu(v) == 0.0
    assert 0 < oracle.silu(10.0) < 10.0  # sigmoid(10) = 1 - 4.5e-5 is below 1 in fp32
    assert -1e-6 < oracle.silu(-19.5) < 0  # just inside the clamp: x * sigmoid(x), not 0


def _mlp64(wg, wu, wd, x):
    g = wg @ x
    u = wu @ x
    h = g * expit(g) * u
    return wd @ h


@pytest.mark.parametrize("hidden,inter,rows", [(256, 512, 1), (320, 160, 3)])
def test_cpu_mlp_int4_brute_force(rng, hidden, inter, rows):
    wg, wu = rand_int4(rng, inter, hidden), rand_int4(rng, inter, hidden)
    wd = rand_int4(rng, hidden, inter)
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    y = oracle.cpu_mlp(wg, wu, wd, oracle.ENC_INT4, x, hidden, inter)
    dg, du = oracle.int4_dequant(wg, hidden).astype(np.float64), oracle.int4_dequant(wu, hidden).astype(np.float64)
    dd = oracle.int4_dequant(wd, inter).astype(np.float64)
    for r in range(rows):
        ref = _mlp64(dg, du, dd, x[r].astype(np.float64))
        assert normwise_rel_err(y[r], ref) < 1e-5
        swapped = _mlp64(du, dg, dd, x[r].astype(np.float64))  # the planted mistake: gate and up swapped
        assert normwise_rel_err(y[r], swapped) > 1e-2


@pytest.mark.parametrize("enc", [oracle.ENC_Q4_K, oracle.ENC_Q6_K])
def test_cpu_mlp_gguf_brute_force(rng, enc):
    from quicknn_amd import hip

    hidden, inter = 512, 256

    def mat(n, k):
        return hip.gguf_quantize(enc, (rng.standard_normal(n * k) * 0.02).astype(np.float32)).reshape(n, -1)

    wg, wu, wd = mat(inter, hidden), mat(inter, hidden), mat(hidden, inter)
    x = rng.standard_normal(hidden).astype(np.float32)
    y = oracle.cpu_mlp(wg, wu, wd, enc, x, hidden, inter)[0]
    deq = lambda w, n, k: oracle.gguf_dequantize(w.ravel(), enc, n * k).reshape(n, k).astype(np.float64)
    ref = _mlp64(deq(wg, inter, hidden), deq(wu, inter, hidden), deq(wd, hidden, inter), x.astype(np.float64))
    assert normwise_rel_err(y, ref) < 1e-5


@pytest.mark.parametrize("enc", [oracle.ENC_Q8_0, oracle.ENC_Q4_K, oracle.ENC_Q2_K])
def test_gguf_gemm_scalar_brute_force(rng, enc):
    from quicknn_amd import hip

    m, k, n = 6, 512, 40
    w = hip.gguf_quantize(enc, (rng.standard_normal(n * k) * 0.02).astype(np.float32))
    a = rng.standard_normal((m, k)).astype(np.float32)
    c = oracle.gguf_gemm_scalar(w, enc, a, n)
    wd = oracle.gguf_dequantize(w, enc, n * k).reshape(n, k).astype(np.float64)
    ref = a.astype(np.float64) @ wd.T
    # one rounding of a float64 sum (whose own error is far below fp32's half ulp)
    assert np.all(np.abs(c - ref) <= ulp32(ref) + 1e-30)
    # row ranges compose: rows [2, 5) alone equal the same rows of the full product
    part = oracle.gguf_gemm_scalar(w, enc, a, n, 2, 5)
    assert np.array_equal(part[2:5], c[2:5])
    assert not part[:2].any() and not part[5:].any()
