"""GPU parity of the F32 / BF16 projections: VectorLinear
(Context.Implementation.inc:969-1001) and Linear with an F32 or BF16 weight
(Implementation.inc:852-883), as the engine uses them for the MoE router
(LLM.MoE.pas:363-374) and native-precision layers (QwenHybrid.pas:540-551,
Gemma2.pas:142-148).

These are floating-point kernels (fp32 products and sums, bf16 widened
exactly), checked against a float64 matmul of the same fp32 / bf16 values with
a normwise relative error max|y-r| / max|r| <= 1e-5: a dropped term, a wrong
row or a transposed weight moves it by orders of magnitude more.
"""
import numpy as np
import pytest

from quicknn_amd import hip
from tests.conftest import bf16_bits, bf16_to_f32, normwise_rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def weight(rng, n, k, bf16):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    if bf16:
        b = bf16_bits(w)
        return hip.MemoryBlock.matrix(b), bf16_to_f32(b).astype(np.float64)
    return hip.MemoryBlock.matrix(w), w.astype(np.float64)


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("n,k", [(128, 2048), (1, 1), (7, 3), (130, 100), (64, 8), (1000, 2560), (33, 4100)])
def test_vector_linear(ctx, rng, bf16, n, k):
    w, w64 = weight(rng, n, k, bf16)
    x = rng.standard_normal(k).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    ctx.VectorLinear(dst, src, w, k, n)
    assert normwise_rel_err(ctx.Download(dst), w64 @ x.astype(np.float64)) <= TOL
    ctx.Recycle(src)
    ctx.Recycle(dst)


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("rows,n,k", [(1, 128, 2048), (2, 128, 2048), (16, 128, 2048), (17, 65, 33),
                                      (128, 128, 2048), (5, 300, 1000), (3, 1, 7)])
def test_linear_dense_rows(ctx, rng, bf16, rows, n, k):
    w, w64 = weight(rng, n, k, bf16)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(rows * n)
    ctx.Linear(dst, src, w, None, hip.MemoryBlock.vector(bias), rows, k, n)
    got = ctx.Download(dst).reshape(rows, n)
    want = x.astype(np.float64) @ w64.T + bias
    for r in range(rows):
        assert normwise_rel_err(got[r], want[r]) <= TOL, r
    ctx.Recycle(src)
    ctx.Recycle(dst)


def test_linear_dense_weight_offset_and_residency(ctx, rng):
    """A slice of a larger F32 block (Offset in elements) is its own cache
    entry; RetainWeight accepts F32/BF16 matrices (RetainRouters, LLM.MoE.pas:190-194)."""
    n, k = 40, 96
    full = (rng.standard_normal((3 * n, k)) * 0.02).astype(np.float32)
    w = hip.MemoryBlock(full, (3 * n, k), hip.DT_F32, offset=n * k, size=3 * n * k)
    ctx.RetainWeight(w, n, k)
    assert ctx.IsWeightResident(w, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(n)
    ctx.VectorLinear(dst, src, w, k, n)
    want = full[n:2 * n].astype(np.float64) @ x.astype(np.float64)
    assert normwise_rel_err(ctx.Download(dst), want) <= TOL


def test_dense_argument_errors(ctx, rng):
    src, dst = ctx.NewTensor(64), ctx.NewTensor(64)
    packed = hip.MemoryBlock.int4(np.zeros((64, 40), np.uint8))
    with pytest.raises(hip.EArgumentException):  # VectorLinear takes F32/BF16 only (Implementation.inc:982-985)
        ctx.VectorLinear(dst, src, packed, 64, 64)
    w = hip.MemoryBlock.matrix(np.zeros((64, 64), np.float32))
    with pytest.raises(hip.EArgumentException):  # aliasing
        ctx.VectorLinear(src, src, w, 64, 64)
    with pytest.raises(hip.EArgumentException):  # more elements than the block holds
        ctx.VectorLinear(ctx.NewTensor(65), src, w, 64, 65)
    with pytest.raises(hip.ENotSupportedException):  # native INT4 goes through Int4Linear
        ctx.Linear(dst, src, packed, None, None, 1, 64, 64)
