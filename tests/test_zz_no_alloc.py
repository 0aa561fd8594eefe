"""qnn_int4_linear_noalloc, the INT4 projection that allocates no device
memory (fixed static scratch), through the C ABI.

* Two calls in a row, the second with a smaller input: each output is
  bit-identical to qnn_int4_linear's on the same input (same kernel and plan,
  another workspace address).
* No allocation: weight, activation and upload counters are unchanged.
* Its limits fail loudly: a weight that is not resident (it does not upload),
  an input width that is not a multiple of 4, a workspace beyond the scratch.
"""
import numpy as np
import pytest

from quicknn_amd import hip
from tests.conftest import rand_int4

pytestmark = pytest.mark.gpu


def test_noalloc_matches_int4_linear_twice_second_smaller(ctx, rng):
    shapes = [(16, 2560, 9728), (3, 1024, 640)]  # (rows, in, out): the second call is smaller
    ws = [hip.MemoryBlock.int4(rand_int4(rng, n, k)) for _, k, n in shapes]
    xs = [rng.standard_normal((r, k)).astype(np.float32) for r, k, _ in shapes]
    srcs = [ctx.UploadRaw(x) for x in xs]
    want = []
    for (r, k, n), w, src in zip(shapes, ws, srcs):
        y = ctx.NewTensor(r * n)
        ctx.Int4Linear(y, src, w, r, k, n)  # also makes the weight resident
        want.append(ctx.Download(y))
    outs = [ctx.NewTensor(r * n) for r, _, n in shapes]
    ctx.Flush()
    s0 = ctx.status()
    for (r, k, n), w, src, out in zip(shapes, ws, srcs, outs):
        ctx.Int4LinearNoAlloc(out, src, w, r, k, n)
    got = [ctx.Download(out) for out in outs]
    s1 = ctx.status()
    for g, wv in zip(got, want):
        assert np.array_equal(g.view(np.uint32), wv.view(np.uint32))
    assert s1.weight_uploads == s0.weight_uploads and s1.weight_bytes == s0.weight_bytes
    assert s1.activation_bytes == s0.activation_bytes
    # and again, the scratch holding the previous call's tickets and sums
    ctx.Int4LinearNoAlloc(outs[1], srcs[1], ws[1], *shapes[1])
    assert np.array_equal(ctx.Download(outs[1]).view(np.uint32), want[1].view(np.uint32))
    for t in srcs + outs:
        ctx.Recycle(t)


def test_noalloc_limits(ctx, rng):
    k, n = 1024, 256
    w = hip.MemoryBlock.int4(rand_int4(rng, n, k))
    src, dst = ctx.UploadRaw(rng.standard_normal(k).astype(np.float32)), ctx.NewTensor(n)
    with pytest.raises(hip.EInvalidOp):  # not resident: it does not upload
        ctx.Int4LinearNoAlloc(dst, src, w, 1, k, n)
    ctx.RetainWeight(w, n, w.shape[1])
    ctx.Int4LinearNoAlloc(dst, src, w, 1, k, n)
    y = ctx.NewTensor(n)
    ctx.Int4Linear(y, src, w, 1, k, n)
    assert np.array_equal(ctx.Download(dst), ctx.Download(y))
    # an input width that is not a multiple of 4 (102: rows of four 32-element groups)
    w2 = hip.MemoryBlock.int4(hip.quantize_int4((rng.standard_normal((8, 102)) * 0.02).astype(np.float32)))
    ctx.RetainWeight(w2, 8, w2.shape[1])
    with pytest.raises(hip.EArgumentException):
        ctx.Int4LinearNoAlloc(ctx.NewTensor(8), ctx.NewTensor(102), w2, 1, 102, 8)
    big_n, big_k = 16384, 8192  # 16 rows: 256 tiles x 16 slices x 16 x 64 floats = 16 MiB of partial sums
    wb = hip.MemoryBlock.int4(rand_int4(rng, big_n, big_k))
    xb = ctx.UploadRaw(rng.standard_normal((16, big_k)).astype(np.float32))
    yb = ctx.NewTensor(16 * big_n)
    ctx.Int4Linear(yb, xb, wb, 16, big_k, big_n)  # resident
    with pytest.raises(hip.ERangeError):
        ctx.Int4LinearNoAlloc(yb, xb, wb, 16, big_k, big_n)
    ctx.Int4LinearNoAlloc(yb, xb, wb, 1, big_k, big_n)  # one row fits
    ctx.Flush()
