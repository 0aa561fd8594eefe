"""GPU parity of the multi-row GGUF projection (prefill GEMM on fp16 MFMA): Q8_0, and every
other encoding over the weight's fp16 copy.

TQNNGPUContext.Linear with Rows > 1 on a Q8_0 weight (Context.Implementation.inc:852-883,
gemm.comp) must match the reference CPU paths within a normwise relative error of 1e-3
(max|y-r| / max|r|, per output row): the per-row AVX2 projection (TCPUProjection.Linear,
CPU.Inference.pas:316-428, PackedDotQ8) and the scalar double-accumulated GGUF GEMM
(QuickNN.Quantization.pas:247-258).  The device rounds both operands once to fp16
(after exact power-of-two row scaling) and accumulates in fp32.
"""
import numpy as np
import pytest

import oracle
from oracle import (ENC_IQ2_S, ENC_IQ2_XXS, ENC_IQ3_S, ENC_IQ3_XXS, ENC_IQ4_NL, ENC_IQ4_XS, ENC_Q2_0, ENC_Q2_K, ENC_Q3_K,
                    ENC_Q4_K, ENC_Q5_K, ENC_Q6_K, ENC_Q8_0)
from quicknn_amd import hip
from tests.conftest import normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def q8(rng, n, k, scale=0.02):
    return hip.gguf_quantize(ENC_Q8_0, (rng.standard_normal((n, k)) * scale).astype(np.float32))


def run_linear(ctx, w, a, n, bias=None, enc=ENC_Q8_0):
    m, k = a.shape
    src, dst = ctx.UploadRaw(a), ctx.NewTensor(m * n)
    ctx.Linear(dst, src, hip.MemoryBlock.gguf(w, n, k, enc), None,
               None if bias is None else hip.MemoryBlock.vector(bias), m, k, n)
    out = ctx.Download(dst).reshape(m, n)
    ctx.Recycle(src)
    ctx.Recycle(dst)
    return out


def test_prefill_shape_matches_cpu_paths(ctx, rng):
    """cfg5: A [512, 3072] x Q8_0 W [12288, 3072] (FLUX / Qwen-Image MLP)."""
    m, k, n = 512, 3072, 12288
    w = q8(rng, n, k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    got = run_linear(ctx, w, a, n)
    for r in [0, 1, 255, 256, 300, 511]:
        assert normwise_rel_err(got[r], oracle.cpu_linear(w, ENC_Q8_0, a[r], k, n)) <= TOL, r
    want = oracle.gguf_gemm_scalar(w, ENC_Q8_0, a, n, row_begin=137, row_end=139)
    for r in (137, 138):
        assert normwise_rel_err(got[r], want[r]) <= TOL, r


# K = 9216 and 10240: rows longer than the activation preparation holds in
# registers (8192 columns), whose last groups it reads twice.
@pytest.mark.parametrize("m,k,n", [(512, 3072, 12288), (128, 3072, 12288), (257, 1024, 97), (300, 640, 200),
                                   (130, 96, 1000), (1000, 4096, 385), (130, 9216, 96), (128, 10240, 200)])
def test_fp16_copy_equals_decoding_kernel(ctx, rng, tune, m, k, n):
    """From QNN_GEMM_H16 rows (default 128) the product runs over a pre-expanded fp16 copy
    of the weight (k_h16_gemm, qnn_status.gemm_h16), made once and cached: every output equals
    the kernel that decodes the Q8_0 blocks per K-tile (k_q8_gemm), bit for bit, including
    ragged M, N and K; the second call reuses the copy."""
    w = q8(rng, n, k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    h0 = ctx.status().gemm_h16
    fast = run_linear(ctx, w, a, n)
    again = run_linear(ctx, w, a, n)
    assert ctx.status().gemm_h16 - h0 == 2
    tune("QNN_GEMM_H16", "0")
    dec = run_linear(ctx, w, a, n)
    assert ctx.status().gemm_h16 - h0 == 2
    assert np.array_equal(fast.view(np.uint32), dec.view(np.uint32))
    assert np.array_equal(again.view(np.uint32), fast.view(np.uint32))
    for r in (0, m // 2, m - 1):
        assert normwise_rel_err(fast[r], oracle.cpu_linear(w, ENC_Q8_0, a[r], k, n)) <= TOL, r


@pytest.mark.parametrize("enc", [ENC_Q8_0, ENC_Q4_K])
def test_rows_in_several_gemm_launches(ctx, rng, tune, enc):
    """Rows beyond one launch's limit run as consecutive launches (the limit keeps the activation
    fragments below 4 GiB; QNN_GEMM_MAX_ROWS lowers it): 300 rows as 128 + 128 + 44.  Q8_0 takes
    its fp16 copy for the two full launches and decodes its tiles for the last, both the same bits
    as one launch over all rows; Q4_K takes its copy for all three."""
    m, k, n = 300, 1024, 200
    w = hip.gguf_quantize(enc, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    a = rng.standard_normal((m, k)).astype(np.float32)
    whole = run_linear(ctx, w, a, n, enc=enc)
    tune("QNN_GEMM_MAX_ROWS", "128")
    h0 = ctx.status().gemm_h16
    parts = run_linear(ctx, w, a, n, enc=enc)
    assert ctx.status().gemm_h16 - h0 == (2 if enc == ENC_Q8_0 else 3)
    if enc == ENC_Q8_0:
        assert np.array_equal(parts.view(np.uint32), whole.view(np.uint32))
    for r in (0, 127, 128, 255, 256, 299):
        assert normwise_rel_err(parts[r], oracle.cpu_linear(w, enc, a[r], k, n)) <= TOL, r
        assert normwise_rel_err(parts[r], whole[r]) <= TOL, r


@pytest.mark.parametrize("m,k,n", [(4, 96, 100), (5, 32, 64), (257, 1024, 97), (300, 640, 200), (33, 4096, 4096),
                                   (16, 2048, 6144)])
def test_ragged_shapes(ctx, rng, m, k, n):
    w = q8(rng, n, k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    got = run_linear(ctx, w, a, n)
    rows = min(m, 40)
    want = oracle.gguf_gemm_scalar(w, ENC_Q8_0, a, n, row_end=rows)
    for r in range(rows):
        assert normwise_rel_err(got[r], want[r]) <= TOL, r
    # Element-wise: one fp16 rounding of each operand bounds every output by
    # 2^-10 * sum_k |w x| (plus fp32 accumulation, far smaller).
    wd = oracle.gguf_dequant_scalar(w, ENC_Q8_0, n * k).reshape(n, k).astype(np.float64)
    bound = np.abs(a[:rows].astype(np.float64)) @ np.abs(wd).T * 2.0 ** -10
    assert np.all(np.abs(got[:rows] - want[:rows]) <= bound)


def test_operand_range_scaling(ctx, rng):
    """Rows far outside fp16's range and weight blocks with large scales (|d*q| > 65504)."""
    m, k, n = 8, 512, 192
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wf[3] *= 5e4    # |w| up to ~4e3, d up to ~30
    wf[100] *= 1e6  # |d*q| beyond fp16
    wf[7] *= 1e-3   # d in the fp16 subnormal range
    w = hip.gguf_quantize(ENC_Q8_0, wf)
    a = rng.standard_normal((m, k)).astype(np.float32)
    a[1] *= 1e8
    a[2] *= 1e-8
    a[5, ::3] = 0.0
    got = run_linear(ctx, w, a, n)
    want = oracle.gguf_gemm_scalar(w, ENC_Q8_0, a, n)
    for r in range(m):
        assert np.all(np.isfinite(got[r]))
        assert normwise_rel_err(got[r], want[r]) <= TOL, r
    # columns far below the row's largest are still right (per-row weight scale, per-element fp16)
    assert np.max(np.abs(got[:, 7] - want[:, 7])) <= 1e-3 * np.max(np.abs(want[:, 7])) * 10


def test_bias_and_determinism(ctx, rng):
    m, k, n = 64, 1024, 512
    w = q8(rng, n, k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    g1 = run_linear(ctx, w, a, n, bias)
    g2 = run_linear(ctx, w, a, n, bias)
    assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32))
    want = oracle.gguf_gemm_scalar(w, ENC_Q8_0, a, n, row_end=8) + bias
    for r in range(8):
        assert normwise_rel_err(g1[r], want[r]) <= TOL, r


def test_small_rows_use_matvec_and_agree(ctx, rng):
    """Rows below the GEMM threshold take the per-row matvec; both paths agree."""
    k, n = 1024, 300
    w = q8(rng, n, k)
    a = rng.standard_normal((6, k)).astype(np.float32)
    full = run_linear(ctx, w, a, n)        # GEMM (6 rows)
    two = run_linear(ctx, w, a[:2], n)     # matvec per row
    for r in range(2):
        assert normwise_rel_err(full[r], two[r]) <= TOL


# ---------------------------------------------------------------------------
# The other encodings (Context.Implementation.inc:852-883: gemm.comp decodes any
# of them through readGGUF).  From QNN_GGUF_GEMM_ROWS rows (default 12) the
# product runs over the weight's fp16 copy, whose values are RNE(W * 2^-e) with
# e from the row's largest |value| (k_gguf_rowexp, k_gguf_expand_h16), then
# k_h16_gemm (grids under 128 tiles split K over up to 8 workgroups per tile,
# summed in slice order); fewer rows run the matvec, up to 8 rows per pass.
# Both within 1e-3 of the CPU paths.
# ---------------------------------------------------------------------------
GEMM_FMTS = [ENC_Q4_K, ENC_Q5_K, ENC_Q6_K, ENC_Q3_K, ENC_Q2_K, ENC_IQ4_NL, ENC_IQ4_XS, ENC_Q2_0, ENC_IQ2_XXS, ENC_IQ2_S,
             ENC_IQ3_XXS, ENC_IQ3_S]


@pytest.mark.parametrize("enc", GEMM_FMTS)
# (16, 4352, 96): 68 K-tiles over 8 slices of 8 or 9 (uneven K-slices).
@pytest.mark.parametrize("m,k,n", [(128, 1024, 300), (200, 768, 97), (32, 1024, 130), (64, 3584, 512),
                                   (16, 10240, 64), (16, 4352, 96)])
def test_other_encodings_fp16_copy_gemm(ctx, rng, tune, enc, m, k, n):
    w = hip.gguf_quantize(enc, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    a = rng.standard_normal((m, k)).astype(np.float32)
    h0 = ctx.status().gemm_h16
    got = run_linear(ctx, w, a, n, enc=enc)
    again = run_linear(ctx, w, a, n, enc=enc)  # the cached copy
    assert ctx.status().gemm_h16 - h0 == 2
    assert np.array_equal(again.view(np.uint32), got.view(np.uint32))
    for r in (0, m // 2, m - 1):
        assert normwise_rel_err(got[r], oracle.cpu_linear(w, enc, a[r], k, n)) <= TOL, r
    want = oracle.gguf_gemm_scalar(w, enc, a, n, row_begin=m - 2, row_end=m)
    for r in (m - 2, m - 1):
        assert normwise_rel_err(got[r], want[r]) <= TOL, r
    tune("QNN_GGUF_GEMM_ROWS", "0")
    per_row = run_linear(ctx, w, a, n, enc=enc)
    assert ctx.status().gemm_h16 - h0 == 2
    for r in range(0, m, 7):
        assert normwise_rel_err(got[r], per_row[r]) <= TOL, r


def test_other_encoding_prefill_shape(ctx, rng):
    """The Gemma-2-9B q projection (Q4_K 4096 x 3584) over a 512-token prefill, one GEMM."""
    m, k, n = 512, 3584, 4096
    w = hip.gguf_quantize(ENC_Q4_K, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    a = rng.standard_normal((m, k)).astype(np.float32)
    h0 = ctx.status().gemm_h16
    got = run_linear(ctx, w, a, n, enc=ENC_Q4_K)
    assert ctx.status().gemm_h16 - h0 == 1
    for r in (0, 1, 255, 256, 511):
        assert normwise_rel_err(got[r], oracle.cpu_linear(w, ENC_Q4_K, a[r], k, n)) <= TOL, r


# ---------------------------------------------------------------------------
# The int8-activation GEMM (qnn_q8_gemm_int8): activations quantised per
# 32-element block to int8 (K7), int32 block sums on the int8 matrix cores,
# fma(float(S_b), dx * dw, acc) in block order (K8).  Bit-identical to the
# oracle's restatement of the same rule; its distance from the reference's
# fp32-activation product is the quantisation's (about 5e-3 normwise).
# ---------------------------------------------------------------------------
def run_int8(ctx, w, a, n):
    m, k = a.shape
    src, dst = ctx.UploadRaw(a), ctx.NewTensor(m * n)
    ctx.Q8GemmInt8(dst, src, hip.MemoryBlock.gguf(w, n, k, ENC_Q8_0), m, k, n)
    out = ctx.Download(dst).reshape(m, n)
    ctx.Recycle(src)
    ctx.Recycle(dst)
    return out


# K = 32 .. 3072: block counts 1, 2, 3, 5, 7, 8, 9, 10, 32 and 96 (the kernel
# takes blocks in pairs and groups of four, so every remainder is covered).
@pytest.mark.parametrize("m,k,n", [(1, 32, 32), (9, 64, 96), (3, 96, 100), (5, 160, 70), (7, 224, 64),
                                   (33, 256, 257), (64, 288, 64), (2, 320, 33), (100, 1024, 130),
                                   (130, 3072, 128)])
def test_int8_gemm_bit_identical_to_oracle(ctx, rng, m, k, n):
    a = rng.standard_normal((m, k)).astype(np.float32)
    a[0, :32] = 0.0  # a zero block: d = 0
    w = q8(rng, n, k)
    got = run_int8(ctx, w, a, n)
    q, d = oracle.q8_act_quant(a)
    want = oracle.q8_gemm_i8(w, q, d, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_int8_gemm_prefill_shape(ctx, rng):
    """cfg5: A [512, 3072] x Q8_0 W [12288, 3072]; 12 rows spread over A (its
    quantisation is per row) checked bit for bit against the oracle, and the
    whole product against the fp32 path."""
    m, k, n = 512, 3072, 12288
    w = q8(rng, n, k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    got = run_int8(ctx, w, a, n)
    rows = np.array([0, 1, 31, 32, 63, 64, 200, 255, 256, 384, 510, 511])
    q, d = oracle.q8_act_quant(a[rows])
    want = oracle.q8_gemm_i8(w, q, d, n)
    assert np.array_equal(got[rows].view(np.uint32), want.view(np.uint32))
    fp = run_linear(ctx, w, a, n)  # the fp32-level path (fp16 MFMA, within 1e-3 of the reference)
    e = normwise_rel_err(got, fp)
    assert 1e-4 < e < 1e-2, e
