"""Asynchronous layer prefetch (Context.API.inc:88-95, Context.Prefetch.inc:92-456)
on a context whose weight cache holds only a few layers.

The model's own sequence (QwenHybrid.pas:485-538, :706-707) streams every
layer through the two slots: ActivatePrefetchedWeights before a layer (else
PrefetchLayer + Activate), the layer's ops, then PrefetchLayer(next) =
BeginWeightPrefetch, PrefetchWeights(deferred), StageWeightPrefetch(the one
after), CompleteWeightPrefetch; SealWeightPrefetch at the end.  Results must
equal a fully resident run bit for bit (same kernels), with one asynchronous
batch per streamed layer.  Misuse raises the reference's exception classes.
"""
import numpy as np
import pytest

from tests.conftest import rand_int4

pytestmark = pytest.mark.gpu

H, I, L = 1024, 3072, 10
ROW_H, ROW_I = 640, 1920  # Int4RowBytes(1024), Int4RowBytes(3072)
LAYER = 2 * I * ROW_H + H * ROW_I  # 5.9 MB per layer
CACHE = 4 * LAYER                  # room for the two prefetch slots' layers and a little more


@pytest.fixture(scope="module")
def model():
    from quicknn_amd import hip

    rng = np.random.default_rng(44)
    layers = [tuple(hip.MemoryBlock.int4(rand_int4(rng, n, k)) for n, k in ((I, H), (I, H), (H, I))) for _ in range(L)]
    x0 = rng.standard_normal(H).astype(np.float32)
    # fully resident reference run (its own context, closed before the streaming one)
    with hip.GPUContext(0) as c:
        want = run_layers(c, layers, x0)
    return layers, x0, want


def run_layers(ctx, layers, x0, step_hook=None):
    x = ctx.UploadRaw(x0)
    h = ctx.NewTensor(I)
    ys = [ctx.NewTensor(H) for _ in layers]
    src = x
    for l, (g, u, d) in enumerate(layers):
        if step_hook:
            step_hook(l, "before")
        assert ctx.TrySwiGLUVector(h, src, g, u, H, I)
        ctx.Int4Linear(ys[l], h, d, 1, I, H)
        src = ys[l]
        if step_hook:
            step_hook(l, "after")
    out = [ctx.Download(y) for y in ys]
    return out


@pytest.fixture(scope="module")
def small(model):  # after the resident run's context is closed: one context at a time
    from quicknn_amd import hip

    c = hip.GPUContext(0, CACHE)
    yield c
    c.close()


def test_streamed_layers_equal_resident_run(small, model):
    ctx = small
    layers, x0, want = model
    assert ctx.EnableWeightPrefetch(LAYER)
    s0 = ctx.status()

    def prefetch_layer(l):
        ctx.BeginWeightPrefetch()
        ctx.PrefetchWeights(list(layers[l]), True)
        if l + 1 < L:
            ctx.StageWeightPrefetch(list(layers[l + 1]))
        ctx.CompleteWeightPrefetch()

    def hook(l, when):
        if when == "before":
            if not ctx.ActivatePrefetchedWeights(list(layers[l])):
                prefetch_layer(l)
                assert ctx.ActivatePrefetchedWeights(list(layers[l]))
        elif l + 1 < L:
            prefetch_layer(l + 1)

    got = run_layers(ctx, layers, x0, hook)
    ctx.SealWeightPrefetch()
    ctx.Flush()
    s1 = ctx.status()
    for a, b in zip(got, want):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert s1.async_weight_batches - s0.async_weight_batches == L
    assert s1.weight_evictions > s0.weight_evictions  # the model did not fit: layers were streamed
    assert s1.weight_bytes <= CACHE
    ctx.EndWeightPrefetch()


def test_prefetch_state_errors(small, model):
    from quicknn_amd import hip

    ctx = small
    layers, _, _ = model
    assert not ctx.EnableWeightPrefetch(1 << 40)  # larger than the slots (and than 512 MiB)
    assert ctx.EnableWeightPrefetch(LAYER)        # already enabled at this size
    with pytest.raises(hip.EInvalidOp):           # nothing queued to stage after
        ctx.StageWeightPrefetch(list(layers[0]))
    ctx.PrefetchWeights(list(layers[0]), True)
    with pytest.raises(hip.EInvalidOp):           # one batch queued already
        ctx.PrefetchWeights(list(layers[1]), True)
    assert not ctx.ActivatePrefetchedWeights(list(layers[1]))  # not the queued layer
    with pytest.raises(hip.EInvalidOp):           # a queued, unused layer at forward completion
        ctx.SealWeightPrefetch()
    assert ctx.ActivatePrefetchedWeights(list(layers[0]))
    ctx.CompleteWeightPrefetch()
    with pytest.raises(hip.ERangeError):          # beyond the double-buffer budget
        ctx.PrefetchWeights([w for lay in layers[:3] for w in lay], True)
    g = layers[1][0]
    part = hip.MemoryBlock(g.data, g.shape, g.dtype, g.encoding, offset=0, size=g.size - 1)
    with pytest.raises(hip.EArgumentException):   # not a complete matrix
        ctx.PrefetchWeights([part], True)
    ctx.EndWeightPrefetch()


def test_prefetched_gguf_and_dense_weights_are_joined_by_any_op(small):
    """A prefetched GGUF or F32 matrix used by an op without ActivatePrefetchedWeights:
    the op's compute still waits for the copy stream (the entry's event)."""
    from quicknn_amd import hip

    ctx = small
    rng = np.random.default_rng(3)
    n, k = 512, 1024
    wq = hip.gguf_quantize(hip.WE_Q4_K, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    wg = hip.MemoryBlock.gguf(wq, n, k, hip.WE_Q4_K)
    wf = hip.MemoryBlock.matrix((rng.standard_normal((64, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal(k).astype(np.float32)
    xt, yg, yf = ctx.UploadRaw(x), ctx.NewTensor(n), ctx.NewTensor(64)
    ctx.PrefetchWeights([wg, wf], True)
    ctx.Linear(yg, xt, wg, None, None, 1, k, n)
    ctx.VectorLinear(yf, xt, wf, k, 64)
    got_g, got_f = ctx.Download(yg), ctx.Download(yf)
    assert ctx.ActivatePrefetchedWeights([wg, wf])
    ctx.CompleteWeightPrefetch()
    ctx.EndWeightPrefetch()
    import oracle

    from tests.conftest import normwise_rel_err
    assert normwise_rel_err(got_g, oracle.cpu_linear(wq, hip.WE_Q4_K, x, k, n)) < 1e-3
    assert normwise_rel_err(got_f, wf.data.astype(np.float64) @ x.astype(np.float64)) < 1e-5
