"""GPU parity of the native INT4 path against the CPU oracle.

Dequantised weights must match bit for bit; matvec / SwiGLU / accumulate
outputs must match the reference CPU path (TCPUProjection.Linear,
src/backends/cpu/QuickNN.CPU.Inference.pas:316-428) within a normwise relative
error of 1e-3 (max|y-r| / max|r|), the benchmark definition's bar; the kernels
accumulate in fp32 in a different order, so they are not bit-identical.
"""
import threading

import numpy as np
import pytest

import oracle
from quicknn_amd import hip
from tests.conftest import bf16_bits, normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def make_int4(rng, n, k, scale=0.02):
    b = bf16_bits(rng.standard_normal((n, k)) * scale)
    return hip.quantize_int4(b)


@pytest.mark.parametrize("n,k", [(64, 32), (100, 40), (6144, 2048), (2560, 9728), (768, 2048), (2048, 768),
                                 (33, 7), (130, 2600)])
def test_dequant_bit_exact(ctx, rng, n, k):
    p = make_int4(rng, n, k)
    w = hip.MemoryBlock.int4(p)
    out = ctx.NewTensor(n * k)
    ctx.Dequantize(out, w, n, k)
    got = ctx.Download(out).reshape(n, k)
    want = oracle.int4_dequant(p, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ctx.Recycle(out)


@pytest.mark.parametrize("n,k", [(6144, 2048), (9728, 2560), (2560, 9728), (64, 32), (100, 40), (33, 7),
                                 (130, 2600), (2048, 768), (1, 5000)])
def test_int4_linear_m1(ctx, rng, n, k):
    p = make_int4(rng, n, k)
    w = hip.MemoryBlock.int4(p)
    x = rng.standard_normal(k).astype(np.float32)
    src = ctx.UploadRaw(x)
    dst = ctx.NewTensor(n)
    ctx.Int4Linear(dst, src, w, 1, k, n)
    got = ctx.Download(dst)
    want = oracle.cpu_linear(p, oracle.ENC_INT4, x, k, n)
    assert normwise_rel_err(got, want) <= TOL
    ctx.Recycle(src)
    ctx.Recycle(dst)


@pytest.mark.parametrize("rows", [2, 3, 8, 16, 17, 128])
def test_int4_linear_rows(ctx, rng, rows):
    n, k = 1000, 2560
    p = make_int4(rng, n, k)
    w = hip.MemoryBlock.int4(p)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    src = ctx.UploadRaw(x)
    dst = ctx.NewTensor(rows * n)
    ctx.Int4Linear(dst, src, w, rows, k, n)
    got = ctx.Download(dst).reshape(rows, n)
    for r in range(rows):
        want = oracle.cpu_linear(p, oracle.ENC_INT4, x[r], k, n)
        assert normwise_rel_err(got[r], want) <= TOL, r


def test_int4_linear_deterministic(ctx, rng):
    n, k = 2560, 9728
    p = make_int4(rng, n, k)
    w = hip.MemoryBlock.int4(p)
    x = rng.standard_normal(k).astype(np.float32)
    src = ctx.UploadRaw(x)
    dst = ctx.NewTensor(n)
    outs = []
    for _ in range(3):
        ctx.Int4Linear(dst, src, w, 1, k, n)
        outs.append(ctx.Download(dst).view(np.uint32).copy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("n,k", [(9728, 2560), (768, 2048), (100, 40), (96, 64)])
def test_swiglu_vector(ctx, rng, n, k):
    pg, pu = make_int4(rng, n, k), make_int4(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    src = ctx.UploadRaw(x)
    dst = ctx.NewTensor(n)
    assert ctx.TrySwiGLUVector(dst, src, hip.MemoryBlock.int4(pg), hip.MemoryBlock.int4(pu), k, n)
    got = ctx.Download(dst)
    g = oracle.cpu_linear(pg, oracle.ENC_INT4, x, k, n)
    u = oracle.cpu_linear(pu, oracle.ENC_INT4, x, k, n)
    want = np.array([oracle.silu(float(a)) for a in g], np.float32) * u
    assert normwise_rel_err(got, want) <= TOL


def silu64(g: np.ndarray) -> np.ndarray:
    """Clamped SiLU (tensor.comp:22, QwenHybrid.CPU.pas:242-246) in float64."""
    g = np.asarray(g, np.float64)
    return np.where(g >= 20.0, g, np.where(g <= -20.0, 0.0, g / (1.0 + np.exp(-np.clip(g, -20.0, 20.0)))))


@pytest.mark.parametrize("n,k", [(9728, 2560), (768, 2048), (100, 40), (37, 1001)])
@pytest.mark.parametrize("gt,ut", [("f32", "f32"), ("bf16", "bf16"), ("f32", "bf16"), ("bf16", "f32")])
def test_swiglu_vector_dense_pairs(ctx, rng, n, k, gt, ut):
    """F32 / BF16 gate and up weights, in any mix, run fused as the reference's op 66
    (Implementation.inc:1017-1023, tensor.comp:38-48): QNN_OK, within 1e-3 of a float64
    silu(Wg x) * (Wu x) over the same (bf16-widened) weights, including rows that are not
    whole 16-byte pieces (K = 40, 1001)."""
    def weight(kind):
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        if kind == "bf16":
            b = bf16_bits(w)
            return hip.MemoryBlock.matrix(b), (b.astype(np.uint32) << 16).view(np.float32)
        return hip.MemoryBlock.matrix(w), w
    (mg, wg), (mu, wu) = weight(gt), weight(ut)
    x = rng.standard_normal(k).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    assert ctx.TrySwiGLUVector(dst, src, mg, mu, k, n) is True
    x64 = x.astype(np.float64)
    want = silu64(wg.astype(np.float64) @ x64) * (wu.astype(np.float64) @ x64)
    assert normwise_rel_err(ctx.Download(dst), want) <= TOL
    ctx.Recycle(src)
    ctx.Recycle(dst)


def test_swiglu_unsupported_mix_not_handled(ctx, rng):
    """Pairs outside ops 66-68 (Implementation.inc:1019-1022) are not handled: an INT4 gate
    with an F32 up, and an F32 gate with a native INT4 up."""
    x = ctx.UploadRaw(np.ones(64, np.float32))
    dst = ctx.NewTensor(8)
    f = hip.MemoryBlock(np.ones((8, 64), np.float32), (8, 64), hip.DT_F32)
    i4 = hip.MemoryBlock.int4(make_int4(rng, 8, 64))
    assert ctx.TrySwiGLUVector(dst, x, i4, f, 64, 8) is False
    assert ctx.TrySwiGLUVector(dst, x, f, i4, 64, 8) is False


def test_int4_accumulate(ctx, rng):
    n, k = 2048, 768
    p = make_int4(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    y0 = rng.standard_normal(n).astype(np.float32)
    probs = np.array([0.0, 0.25, 0.7, 0.05], np.float32)
    src, dst, pt = ctx.UploadRaw(x), ctx.UploadRaw(y0), ctx.UploadRaw(probs)
    ctx.Int4LinearAccumulate(dst, src, pt, hip.MemoryBlock.int4(p), k, n, 2)
    got = ctx.Download(dst)
    want = y0 + oracle.cpu_linear(p, oracle.ENC_INT4, x, k, n) * np.float32(0.7)
    assert normwise_rel_err(got, want) <= TOL


def test_mlp_layer_matches_cpu_path(ctx, rng):
    """One Qwen3-4B-shaped MLP: fused gate/up SwiGLU, then down (QwenHybrid.CPU.pas:238-248)."""
    hidden, inter = 2560, 9728
    pg, pu, pd = make_int4(rng, inter, hidden), make_int4(rng, inter, hidden), make_int4(rng, hidden, inter)
    x = oracle.rmsnorm(rng.standard_normal((1, hidden)).astype(np.float32), None, 1e-6, add_one=True)[0]
    src, h, y = ctx.UploadRaw(x), ctx.NewTensor(inter), ctx.NewTensor(hidden)
    assert ctx.TrySwiGLUVector(h, src, hip.MemoryBlock.int4(pg), hip.MemoryBlock.int4(pu), hidden, inter)
    ctx.Int4Linear(y, h, hip.MemoryBlock.int4(pd), 1, inter, hidden)
    got = ctx.Download(y)
    want = oracle.cpu_mlp(pg, pu, pd, oracle.ENC_INT4, x, hidden, inter)[0]
    assert normwise_rel_err(got, want) <= TOL


def test_argument_errors(ctx, rng):
    p = make_int4(rng, 64, 64)
    w = hip.MemoryBlock.int4(p)
    src, dst = ctx.NewTensor(64), ctx.NewTensor(64)
    with pytest.raises(hip.EArgumentException):
        ctx.Int4Linear(dst, src, w, 1, 96, 64)  # shape[1] != Int4RowBytes(96)
    with pytest.raises(hip.EArgumentException):
        ctx.Int4Linear(dst, dst, w, 1, 64, 64)  # aliasing
    with pytest.raises(hip.EArgumentException):
        ctx.Int4Linear(dst, src, w, 129, 64, 64)  # rows > 128
    with pytest.raises(hip.EArgumentException):
        ctx.Int4Linear(dst, src, w, 2, 64, 64)  # src too small


def test_wrong_thread_is_invalid_op(ctx):
    err = []

    def other():
        try:
            ctx.NewTensor(4)
        except Exception as e:  # noqa: BLE001
            err.append(e)

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert err and isinstance(err[0], hip.EInvalidOp)


def test_non_finite_raises_at_download(ctx):
    t = ctx.UploadRaw(np.array([1.0, np.nan, 2.0], np.float32))
    ctx.CheckFinite(t)
    with pytest.raises(hip.EInvalidOp):
        ctx.Download(t)
    ctx.Download(t)  # the flag is cleared once reported


@pytest.mark.parametrize("lanes,tpw", [(2, 1), (4, 2), (16, 4), (8, 2)])
def test_lane_layouts_and_tile_groupings(ctx, rng, tune, lanes, tpw):
    """Rows spread over L lanes (QNN_I4_LANES, read when a weight is uploaded) and T tiles per
    workgroup (QNN_I4_TPW) compute the same projections."""
    tune("QNN_I4_LANES", str(lanes))
    tune("QNN_I4_TPW", str(tpw))
    for n, k in [(2560, 9728), (1000, 2560), (100, 40)]:
        p = make_int4(rng, n, k)
        w = hip.MemoryBlock.int4(p)
        x = rng.standard_normal(k).astype(np.float32)
        src, dst, deq = ctx.UploadRaw(x), ctx.NewTensor(n), ctx.NewTensor(n * k)
        ctx.Int4Linear(dst, src, w, 1, k, n)
        assert normwise_rel_err(ctx.Download(dst), oracle.cpu_linear(p, oracle.ENC_INT4, x, k, n)) <= TOL
        ctx.Dequantize(deq, w, n, k)
        assert np.array_equal(ctx.Download(deq).view(np.uint32), oracle.int4_dequant(p, k).reshape(-1).view(np.uint32))
    pg, pu = make_int4(rng, 768, 2048), make_int4(rng, 768, 2048)
    x = rng.standard_normal(2048).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(768)
    assert ctx.TrySwiGLUVector(dst, src, hip.MemoryBlock.int4(pg), hip.MemoryBlock.int4(pu), 2048, 768)
    g = oracle.cpu_linear(pg, oracle.ENC_INT4, x, 2048, 768)
    u = oracle.cpu_linear(pu, oracle.ENC_INT4, x, 2048, 768)
    want = np.array([oracle.silu(float(a)) for a in g], np.float32) * u
    assert normwise_rel_err(ctx.Download(dst), want) <= TOL
    x8 = rng.standard_normal((8, 2048)).astype(np.float32)
    src8, dst8 = ctx.UploadRaw(x8), ctx.NewTensor(8 * 768)
    ctx.Int4Linear(dst8, src8, hip.MemoryBlock.int4(pg), 8, 2048, 768)
    got8 = ctx.Download(dst8).reshape(8, 768)
    for r in range(8):
        assert normwise_rel_err(got8[r], oracle.cpu_linear(pg, oracle.ENC_INT4, x8[r], 2048, 768)) <= TOL, r


@pytest.mark.parametrize("n,k", [(6144, 2048), (1000, 1024), (130, 2040), (70, 2048), (300, 2560)])
def test_one_token_wide_workgroups_match_slices(ctx, rng, tune, n, k):
    """One token whose K-range splits evenly into 2 or 4 four-wave slices runs as one 8- or
    16-wave workgroup per tile (no cross-workgroup exchange): bit-identical to the split-K
    launch (QNN_I4_WIDE=0) and within tolerance of the CPU path, including a ragged last
    group (K = 2040), a partial last block of rows and a K-range (2560: five slices) that
    keeps the split-K launch."""
    p = make_int4(rng, n, k)
    w = hip.MemoryBlock.int4(p)
    x = rng.standard_normal(k).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    got = {}
    for wide in ("1", "0"):
        tune("QNN_I4_WIDE", wide)
        ctx.Int4Linear(dst, src, w, 1, k, n)
        got[wide] = ctx.Download(dst)
    assert np.array_equal(got["1"].view(np.uint32), got["0"].view(np.uint32)), (n, k)
    assert normwise_rel_err(got["1"], oracle.cpu_linear(p, oracle.ENC_INT4, x, k, n)) <= TOL
    ctx.Recycle(src)
    ctx.Recycle(dst)


@pytest.mark.parametrize("rows,tpw", [(4, 1), (5, 1), (8, 1), (8, 2), (6, 4)])
def test_multi_token_matrix_cores_match_dot4(ctx, rng, tune, rows, tpw):
    """4-8 tokens over one-lane rows with 4 steps per wave run the inner product on the int8
    matrix cores: bit-identical to the v_dot4 path (QNN_I4_MFMA=0) and within tolerance of the
    CPU path, including a partial last block of rows, a slice shorter than a wave's steps and
    2 or 4 tiles per workgroup (QNN_I4_TPW)."""
    tune("QNN_I4_SPS", "4")
    tune("QNN_I4_TPW", str(tpw))
    for n, k in [(2560, 9728), (1000, 2560), (200, 96)]:
        p = make_int4(rng, n, k)
        w = hip.MemoryBlock.int4(p)
        x = rng.standard_normal((rows, k)).astype(np.float32)
        src, dst = ctx.UploadRaw(x), ctx.NewTensor(rows * n)
        got = {}
        for mf in ("1", "0"):
            tune("QNN_I4_MFMA", mf)
            ctx.Int4Linear(dst, src, w, rows, k, n)
            got[mf] = ctx.Download(dst).reshape(rows, n)
        assert np.array_equal(got["1"].view(np.uint32), got["0"].view(np.uint32)), (n, k)
        for r in range(rows):
            want = oracle.cpu_linear(p, oracle.ENC_INT4, x[r], k, n)
            assert normwise_rel_err(got["1"][r], want) <= TOL, (n, k, r)
        ctx.Recycle(src)
        ctx.Recycle(dst)


def test_sixteen_token_chunks_on_matrix_cores(ctx, rng):
    """Rows in 16-token chunks run on the matrix cores too (4 steps per wave at shapes that fill
    the chip): each row is bit-identical to the same rows computed as two 8-token calls, and
    within tolerance of the CPU path."""
    n, k, rows = 9728, 2560, 16
    p = make_int4(rng, n, k)
    w = hip.MemoryBlock.int4(p)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(rows * n)
    ctx.Int4Linear(dst, src, w, rows, k, n)
    got16 = ctx.Download(dst).reshape(rows, n)
    halves = []
    for h in range(2):
        s8, d8 = ctx.UploadRaw(x[8 * h:8 * h + 8]), ctx.NewTensor(8 * n)
        ctx.Int4Linear(d8, s8, w, 8, k, n)
        halves.append(ctx.Download(d8).reshape(8, n))
        ctx.Recycle(s8)
        ctx.Recycle(d8)
    assert np.array_equal(got16.view(np.uint32), np.concatenate(halves).view(np.uint32))
    for r in (0, 7, 15):
        assert normwise_rel_err(got16[r], oracle.cpu_linear(p, oracle.ENC_INT4, x[r], k, n)) <= TOL, r
    ctx.Recycle(src)
    ctx.Recycle(dst)
