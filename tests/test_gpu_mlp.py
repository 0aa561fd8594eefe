"""GPU tests of the fused decode MLP (qnn_mlp.hip).

TrySwiGLUVector followed by the Int4Linear that reads its output runs as one
launch.  The work items, their order and the slice order are those
of the two per-op launches, so h and y must be bit-identical to the per-op path
(QNN_FUSE_MLP=0), and within 1e-3 normwise of the reference CPU path
(QwenHybrid.CPU.pas:238-248).  A recorded SwiGLU that is not followed by its
down projection is launched on its own by the next call.
"""
import numpy as np
import pytest

import oracle
from tests.conftest import normwise_rel_err, rand_int4

pytestmark = pytest.mark.gpu


def mlp(ctx, hip, layers, x0, hidden, inter):
    x = ctx.UploadRaw(x0)
    h = ctx.NewTensor(inter)
    ys = [ctx.NewTensor(hidden), ctx.NewTensor(hidden)]
    hs, outs, src = [], [], x
    for i, (g, u, d) in enumerate(layers):
        assert ctx.TrySwiGLUVector(h, src, g, u, hidden, inter)
        y = ys[i & 1]
        ctx.Int4Linear(y, h, d, 1, inter, hidden)
        hs.append(ctx.Download(h))
        outs.append(ctx.Download(y))
        src = y
    for t in [x, h] + ys:
        ctx.Recycle(t)
    return hs, outs


@pytest.mark.parametrize("hidden,inter,nl", [(2560, 9728, 3), (1024, 3072, 2), (2048, 768, 2), (512, 1536, 1)])
def test_fused_equals_per_op(ctx, rng, monkeypatch, hidden, inter, nl):
    from quicknn_amd import hip

    layers = [(hip.MemoryBlock.int4(rand_int4(rng, inter, hidden)), hip.MemoryBlock.int4(rand_int4(rng, inter, hidden)),
               hip.MemoryBlock.int4(rand_int4(rng, hidden, inter))) for _ in range(nl)]
    x0 = rng.standard_normal(hidden).astype(np.float32)
    before = ctx.status().mlp_fused
    h_f, y_f = mlp(ctx, hip, layers, x0, hidden, inter)
    fused = ctx.status().mlp_fused - before
    monkeypatch.setenv("QNN_FUSE_MLP", "0")
    h_p, y_p = mlp(ctx, hip, layers, x0, hidden, inter)
    assert ctx.status().mlp_fused - before == fused  # nothing fused with the switch off
    for i in range(nl):
        assert np.array_equal(h_f[i], h_p[i]), ("h", i)
        assert np.array_equal(y_f[i], y_p[i]), ("y", i)
    g, u, d = layers[0]
    want = oracle.cpu_mlp(g.data, u.data, d.data, oracle.ENC_INT4, x0, hidden, inter)[0]
    assert normwise_rel_err(y_f[0], want) < 1e-3
    if (hidden, inter) == (2560, 9728):
        assert fused == nl  # the benchmark shape runs fused


def test_recorded_swiglu_settles_on_other_calls(ctx, rng):
    """The recorded SwiGLU is launched before any other call: Download of h,
    an Int4Linear on another input, a second SwiGLU, events."""
    from quicknn_amd import hip

    hidden, inter = 1024, 3072
    g, u = hip.MemoryBlock.int4(rand_int4(rng, inter, hidden)), hip.MemoryBlock.int4(rand_int4(rng, inter, hidden))
    d = hip.MemoryBlock.int4(rand_int4(rng, hidden, inter))
    x0 = rng.standard_normal(hidden).astype(np.float32)
    x, h, y = ctx.UploadRaw(x0), ctx.NewTensor(inter), ctx.NewTensor(hidden)
    other = ctx.UploadRaw(rng.standard_normal(inter).astype(np.float32))
    ref_h = None
    for case in ("download", "other_input", "second_swiglu", "event"):
        ctx.Kernel(hip.GO_FILL, inter, h, None, None, None, [0])
        assert ctx.TrySwiGLUVector(h, x, g, u, hidden, inter)
        if case == "download":
            ref_h = ctx.Download(h)
            got = ref_h
        elif case == "other_input":
            ctx.Int4Linear(y, other, d, 1, inter, hidden)  # not h: no fusion
            got = ctx.Download(h)
            yo = ctx.Download(y)
            want_o = oracle.cpu_linear(d.data, oracle.ENC_INT4, ctx.Download(other), inter, hidden)
            assert normwise_rel_err(yo, want_o) < 1e-3
        elif case == "second_swiglu":
            h2 = ctx.NewTensor(inter)
            assert ctx.TrySwiGLUVector(h2, x, g, u, hidden, inter)
            got = ctx.Download(h)
            assert np.array_equal(ctx.Download(h2), ref_h)
            ctx.Recycle(h2)
        else:
            ctx.EventRecord(20)
            ctx.EventRecord(21)
            ctx.EventElapsedMs(20, 21)
            got = ctx.Download(h)
        assert np.array_equal(got, ref_h), case
    gg = oracle.int4_dequant(g.data, hidden).astype(np.float64) @ x0.astype(np.float64)
    uu = oracle.int4_dequant(u.data, hidden).astype(np.float64) @ x0.astype(np.float64)
    from scipy.special import expit
    assert normwise_rel_err(ref_h, gg * expit(gg) * uu) < 1e-3
    for t in (x, h, y, other):
        ctx.Recycle(t)


def test_fused_error_in_down_still_runs_swiglu(ctx, rng):
    """A failing Int4Linear (bad weight shape) raises, and the recorded SwiGLU still runs."""
    from quicknn_amd import hip

    hidden, inter = 512, 1536
    g, u = hip.MemoryBlock.int4(rand_int4(rng, inter, hidden)), hip.MemoryBlock.int4(rand_int4(rng, inter, hidden))
    bad = hip.MemoryBlock.int4(rand_int4(rng, hidden, inter + 32))  # wrong row width
    x, h, y = ctx.UploadRaw(rng.standard_normal(hidden).astype(np.float32)), ctx.NewTensor(inter), ctx.NewTensor(hidden)
    ctx.Kernel(hip.GO_FILL, inter, h, None, None, None, [0])
    assert ctx.TrySwiGLUVector(h, x, g, u, hidden, inter)
    with pytest.raises(hip.EArgumentException):
        ctx.Int4Linear(y, h, bad, 1, inter, hidden)
    assert np.any(ctx.Download(h) != 0)
    for t in (x, h, y):
        ctx.Recycle(t)
