"""GPU parity of the GGUF path (Q8_0, Q4_K, Q5_K, Q6_K, Q3_K, Q2_K, IQ4_NL, IQ4_XS, Q2_0, IQ2_XXS, IQ2_S, IQ3_XXS,
IQ3_S) against the CPU oracle.

Dequantised weights must equal GGUFValue (GGUF.Quantization.pas:136-253) bit
for bit (as floats: +0 == -0, the reference's own decoders differ there);
matvec and fused gate/up outputs must match the reference CPU path
(TCPUProjection.Linear, CPU.Inference.pas:316-428, packed AVX2 dots) within a
normwise relative error of 1e-3 (max|y-r| / max|r|).
"""
import numpy as np
import pytest

import oracle
from oracle import (BLOCK_BYTES, BLOCK_ELEMENTS, ENC_IQ2_S, ENC_IQ2_XXS, ENC_IQ3_S, ENC_IQ3_XXS, ENC_IQ4_NL, ENC_IQ4_XS,
                    ENC_Q2_0, ENC_Q2_K, ENC_Q3_K, ENC_Q4_K, ENC_Q5_K, ENC_Q6_K, ENC_Q8_0)
from quicknn_amd import hip
from tests.conftest import normwise_rel_err
from tests.test_oracle_gguf import random_blocks

pytestmark = pytest.mark.gpu
TOL = 1e-3
FMTS = [ENC_Q8_0, ENC_Q4_K, ENC_Q6_K, ENC_Q3_K, ENC_Q2_K, ENC_Q5_K, ENC_IQ4_NL, ENC_IQ4_XS, ENC_Q2_0, ENC_IQ2_XXS, ENC_IQ2_S,
        ENC_IQ3_XXS, ENC_IQ3_S]
NAMES = {ENC_Q8_0: "q8_0", ENC_Q4_K: "q4_k", ENC_Q6_K: "q6_k", ENC_Q3_K: "q3_k", ENC_Q2_K: "q2_k", ENC_Q5_K: "q5_k",
         ENC_IQ4_NL: "iq4_nl", ENC_IQ4_XS: "iq4_xs", ENC_Q2_0: "q2_0", ENC_IQ2_XXS: "iq2_xxs", ENC_IQ2_S: "iq2_s",
         ENC_IQ3_XXS: "iq3_xxs", ENC_IQ3_S: "iq3_s"}


def quantized(rng, enc, n, k, scale=0.02):
    """Library-encoded blocks of N(0, scale) weights (the benchmark's weight recipe)."""
    return hip.gguf_quantize(enc, (rng.standard_normal((n, k)) * scale).astype(np.float32))


def equal_as_floats(a, b):
    return bool(np.all(a == b)) and not np.any(np.isnan(a))


@pytest.mark.parametrize("enc", FMTS, ids=NAMES.get)
@pytest.mark.parametrize("n,kb", [(1, 1), (33, 3), (64, 2), (100, 5), (257, 14)])
def test_dequant_bit_exact_random_blocks(ctx, rng, enc, n, kb):
    k = kb * BLOCK_ELEMENTS[enc]
    data = random_blocks(rng, enc, n * kb)
    out = ctx.NewTensor(n * k)
    ctx.Dequantize(out, hip.MemoryBlock.gguf(data, n, k, enc), n, k)
    got = ctx.Download(out)
    want = oracle.gguf_dequant_scalar(data, enc, n * k)
    assert equal_as_floats(got, want)
    ctx.Recycle(out)


@pytest.mark.parametrize("enc", FMTS, ids=NAMES.get)
def test_dequant_bit_exact_encoded_weight(ctx, rng, enc):
    n, k = 300, 3584 if enc != ENC_Q8_0 else 3072
    data = quantized(rng, enc, n, k)
    out = ctx.NewTensor(n * k)
    ctx.Dequantize(out, hip.MemoryBlock.gguf(data, n, k, enc), n, k)
    assert equal_as_floats(ctx.Download(out), oracle.gguf_dequant_scalar(data, enc, n * k))


def test_dequant_offset_slice(ctx, rng):
    """GGUFWeightPointer (GGUF.Quantization.pas:115-121): an element offset selects whole blocks."""
    enc, n, k = ENC_Q4_K, 40, 512
    data = random_blocks(rng, enc, 3 * n * k // 256)
    off = n * k  # the second of three [n, k] matrices packed back to back
    w = hip.MemoryBlock(data, (3 * n, k), hip.DT_U8, enc, off, 3 * n * k)
    out = ctx.NewTensor(n * k)
    ctx.Dequantize(out, w, n, k)
    full = oracle.gguf_dequant_scalar(data, enc, 3 * n * k)
    assert equal_as_floats(ctx.Download(out), full[off:off + n * k])


@pytest.mark.parametrize("enc,n,k", [
    (ENC_Q4_K, 4096, 3584), (ENC_Q3_K, 2048, 3584), (ENC_Q2_K, 14336, 3584), (ENC_Q6_K, 3584, 14336),
    (ENC_Q8_0, 6144, 2048), (ENC_Q8_0, 12288, 3072),
    (ENC_Q4_K, 5, 256), (ENC_Q6_K, 70, 768), (ENC_Q3_K, 129, 1280), (ENC_Q2_K, 63, 512), (ENC_Q8_0, 33, 96),
    (ENC_Q5_K, 4096, 3584), (ENC_IQ4_XS, 4096, 4096), (ENC_IQ4_NL, 2048, 3584), (ENC_Q5_K, 5, 256),
    (ENC_IQ4_XS, 70, 768), (ENC_IQ4_NL, 33, 96), (ENC_IQ4_NL, 129, 1312),
    (ENC_Q2_0, 4096, 3584), (ENC_Q2_0, 14336, 3584), (ENC_Q2_0, 33, 192), (ENC_Q2_0, 129, 1344), (ENC_Q2_0, 7, 64),
    (ENC_IQ2_XXS, 4096, 3584), (ENC_IQ2_S, 4096, 3584), (ENC_IQ3_XXS, 4096, 4096), (ENC_IQ3_S, 3584, 14336),
    (ENC_IQ2_XXS, 5, 256), (ENC_IQ2_S, 70, 768), (ENC_IQ3_XXS, 129, 1280), (ENC_IQ3_S, 63, 512),
])
def test_linear_m1(ctx, rng, enc, n, k):
    data = quantized(rng, enc, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    ctx.Linear(dst, src, hip.MemoryBlock.gguf(data, n, k, enc), None, None, 1, k, n)
    got = ctx.Download(dst)
    want = oracle.cpu_linear(data, enc, x, k, n)
    assert normwise_rel_err(got, want) <= TOL
    ctx.Recycle(src)
    ctx.Recycle(dst)


@pytest.mark.parametrize("enc", FMTS, ids=NAMES.get)
def test_linear_m1_random_blocks(ctx, rng, enc):
    """Arbitrary block bytes (every scale/min/quant pattern), not just encoder output."""
    n, kb = 200, 6 if enc != ENC_Q8_0 else 40
    k = kb * BLOCK_ELEMENTS[enc]
    data = random_blocks(rng, enc, n * kb)
    x = rng.standard_normal(k).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    ctx.Linear(dst, src, hip.MemoryBlock.gguf(data, n, k, enc), None, None, 1, k, n)
    assert normwise_rel_err(ctx.Download(dst), oracle.cpu_linear(data, enc, x, k, n)) <= TOL


@pytest.mark.parametrize("enc", FMTS, ids=NAMES.get)
def test_linear_rows_and_bias(ctx, rng, enc):
    n, k, rows = 300, 1024, 3
    data = quantized(rng, enc, n, k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(rows * n)
    ctx.Linear(dst, src, hip.MemoryBlock.gguf(data, n, k, enc), None, hip.MemoryBlock.vector(bias), rows, k, n)
    got = ctx.Download(dst).reshape(rows, n)
    for r in range(rows):
        want = oracle.cpu_linear(data, enc, x[r], k, n) + bias
        assert normwise_rel_err(got[r], want) <= TOL, r


@pytest.mark.parametrize("enc", FMTS, ids=NAMES.get)
def test_linear_multi_token_equals_per_row(ctx, rng, tune, enc):
    """2 to 127 rows run up to 8 rows per pass over the weight (k_gguf_matvec_mt): every row equals
    the one-row matvec bit for bit (QNN_GG_MT=0 runs one launch per row) and is within 1e-3 of the
    CPU path; ragged shapes (n not a multiple of 64, K not a multiple of 1024)."""
    n, k = 200, 1280 if BLOCK_ELEMENTS[enc] == 256 else 1344
    data = quantized(rng, enc, n, k)
    w = hip.MemoryBlock.gguf(data, n, k, enc)
    for rows in (2, 8, 11):
        x = rng.standard_normal((rows, k)).astype(np.float32)
        src, dst = ctx.UploadRaw(x), ctx.NewTensor(rows * n)
        ctx.Linear(dst, src, w, None, None, rows, k, n)
        got = ctx.Download(dst).reshape(rows, n)
        tune("QNN_GG_MT", "0")
        ctx.Linear(dst, src, w, None, None, rows, k, n)
        per_row = ctx.Download(dst).reshape(rows, n)
        tune("QNN_GG_MT", "1")
        assert np.array_equal(got.view(np.uint32), per_row.view(np.uint32)), rows
        for r in range(rows):
            assert normwise_rel_err(got[r], oracle.cpu_linear(data, enc, x[r], k, n)) <= TOL, (rows, r)
        ctx.Recycle(src)
        ctx.Recycle(dst)


# Two 256-element units per wave (k_gguf_matvec<ENC, 2>), which the planner no
# longer picks by itself: QNN_GG_BW=2 forces it at small ragged shapes,
# including launches with fewer units than waves (and at the Q6_K head below).
@pytest.mark.parametrize("enc", FMTS, ids=NAMES.get)
@pytest.mark.parametrize("n,k", [(1, 256), (37, 768), (64, 2048), (130, 2304), (300, 512), (65, 3584)])
def test_linear_two_units_per_wave_forced(ctx, rng, tune, enc, n, k):
    if enc in (ENC_Q8_0, ENC_IQ4_NL):
        k = k - 32 if k > 256 else 96  # rows of 32-element blocks need not fill their last 256-element unit
    if enc == ENC_Q2_0:
        k = k - 64 if k > 256 else 192  # likewise for 64-element blocks
    data = quantized(rng, enc, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    tune("QNN_GG_BW", "2")
    ctx.Linear(dst, src, hip.MemoryBlock.gguf(data, n, k, enc), None, None, 1, k, n)
    got = ctx.Download(dst)
    assert normwise_rel_err(got, oracle.cpu_linear(data, enc, x, k, n)) <= TOL
    ctx.Recycle(src)
    ctx.Recycle(dst)


@pytest.mark.parametrize("eg,eu,n,k", [(ENC_Q2_K, ENC_Q2_K, 700, 1024), (ENC_Q6_K, ENC_Q6_K, 33, 512),
                                       (ENC_Q4_K, ENC_Q4_K, 96, 3584)])
def test_swiglu_two_units_per_wave_forced(ctx, rng, tune, eg, eu, n, k):
    pg, pu = quantized(rng, eg, n, k), quantized(rng, eu, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    tune("QNN_GG_BW", "2")
    assert ctx.TrySwiGLUVector(dst, src, hip.MemoryBlock.gguf(pg, n, k, eg), hip.MemoryBlock.gguf(pu, n, k, eu), k, n)
    assert normwise_rel_err(ctx.Download(dst), _swiglu_want(pg, eg, pu, eu, x, k, n)) <= TOL
    ctx.Recycle(src)
    ctx.Recycle(dst)


def test_q6k_output_head_256000x3584(ctx, rng, tune):
    """configs[2]'s Q6_K output head at full size.  The planner runs it at one
    unit per wave (4000 tiles x 4 K-slices of 4, 4, 4 and 2 units); the result
    equals a forced QNN_GG_BW=1 launch bit for bit, and a forced QNN_GG_BW=2
    launch (2 slices of 8 and 6 units: other sums, other last bits) is within
    the bar too.  Rows are encoded from a prime period of 4099 rows (so no
    tile or unit index lines up with the repetition); a spread of 640 rows,
    the first and last 64 included, is checked against the CPU path on those
    rows."""
    enc, n, k, period = ENC_Q6_K, 256000, 3584, 4099
    base = quantized(rng, enc, period, k).reshape(period, -1)
    data = np.tile(base, (n // period + 1, 1))[:n]
    x = rng.standard_normal(k).astype(np.float32)
    w = hip.MemoryBlock.gguf(data, n, k, enc)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    ctx.Linear(dst, src, w, None, None, 1, k, n)
    auto = ctx.Download(dst)
    tune("QNN_GG_BW", "1")
    ctx.Linear(dst, src, w, None, None, 1, k, n)
    forced = ctx.Download(dst)
    assert np.array_equal(auto.view(np.uint32), forced.view(np.uint32))
    tune("QNN_GG_BW", "2")
    ctx.Linear(dst, src, w, None, None, 1, k, n)
    two = ctx.Download(dst)
    rows = np.unique(np.concatenate([np.arange(64), rng.choice(n, 512, replace=False), np.arange(n - 64, n)]))
    want = oracle.cpu_linear(np.ascontiguousarray(base[rows % period]), enc, x, k, len(rows))
    assert normwise_rel_err(auto[rows], want) <= TOL
    assert normwise_rel_err(two[rows], want) <= TOL
    ctx.Recycle(src)
    ctx.Recycle(dst)


def test_linear_deterministic(ctx, rng):
    enc, n, k = ENC_Q6_K, 3584, 14336
    w = hip.MemoryBlock.gguf(quantized(rng, enc, n, k), n, k, enc)
    src, dst = ctx.UploadRaw(rng.standard_normal(k).astype(np.float32)), ctx.NewTensor(n)
    outs = []
    for _ in range(3):
        ctx.Linear(dst, src, w, None, None, 1, k, n)
        outs.append(ctx.Download(dst).view(np.uint32).copy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def _swiglu_want(pg, eg, pu, eu, x, k, n):
    g = oracle.cpu_linear(pg, eg, x, k, n)
    u = oracle.cpu_linear(pu, eu, x, k, n)
    return np.array([oracle.silu(float(a)) for a in g], np.float32) * u


@pytest.mark.parametrize("eg,eu,n,k", [
    (ENC_Q2_K, ENC_Q2_K, 14336, 3584), (ENC_Q4_K, ENC_Q4_K, 1000, 768), (ENC_Q8_0, ENC_Q8_0, 96, 64),
    (ENC_Q6_K, ENC_Q6_K, 33, 256), (ENC_Q3_K, ENC_Q3_K, 257, 512), (ENC_Q4_K, ENC_Q6_K, 500, 512),
    (ENC_Q5_K, ENC_Q5_K, 1000, 768), (ENC_IQ4_XS, ENC_IQ4_XS, 300, 512), (ENC_IQ4_NL, ENC_IQ4_NL, 96, 160),
    (ENC_IQ4_NL, ENC_IQ4_XS, 200, 512), (ENC_Q2_0, ENC_Q2_0, 300, 448), (ENC_Q2_0, ENC_Q2_0, 9728, 2560),
    (ENC_Q2_0, ENC_Q4_K, 200, 512), (ENC_IQ2_XXS, ENC_IQ2_XXS, 1000, 768), (ENC_IQ2_S, ENC_IQ2_S, 96, 3584),
    (ENC_IQ3_XXS, ENC_IQ3_XXS, 257, 512), (ENC_IQ3_S, ENC_IQ3_S, 4096, 2560), (ENC_IQ2_S, ENC_IQ3_XXS, 200, 512),
])
def test_swiglu_vector(ctx, rng, eg, eu, n, k):
    pg, pu = quantized(rng, eg, n, k), quantized(rng, eu, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    assert ctx.TrySwiGLUVector(dst, src, hip.MemoryBlock.gguf(pg, n, k, eg), hip.MemoryBlock.gguf(pu, n, k, eu), k, n)
    assert normwise_rel_err(ctx.Download(dst), _swiglu_want(pg, eg, pu, eu, x, k, n)) <= TOL


def test_gguf_argument_errors(ctx, rng):
    enc, n, k = ENC_Q4_K, 16, 512
    data = quantized(rng, enc, n, k)
    src, dst = ctx.NewTensor(k), ctx.NewTensor(n)
    with pytest.raises(hip.EArgumentException):  # width not a whole number of blocks
        ctx.Linear(dst, src, hip.MemoryBlock.gguf(data, n, 500, enc), None, None, 1, 500, n)
    with pytest.raises(hip.EArgumentException):  # more rows than the block holds
        ctx.Linear(ctx.NewTensor(2 * n), src, hip.MemoryBlock.gguf(data, n, k, enc), None, None, 1, k, 2 * n)
    with pytest.raises(hip.ENotSupportedException):  # an encoding outside TQNNWeightEncoding
        ctx.Linear(dst, src, hip.MemoryBlock.gguf(data, n, k, 14), None, None, 1, k, n)
