"""Weight residency of the context on a small cache (QuickNN.Vulkan.pas:551-740,
Context.Implementation.inc:361-430), on a context of its own.

* WeightKey identity: the same identity hits, a new identity uploads again.
* LRU eviction of unpinned entries when the cache is full; evicted weights
  upload again on their next use and give the same results.
* PreloadWeights pins until the next Flush/Download (Context.API.inc:85-86):
  an acquisition that could only fit by evicting them raises ERangeError.
* RetainWeight pins for the context's lifetime, retaining twice keeps one pin,
  and WeightBatchCapacity is the limit less the retained bytes.
* A weight larger than the whole cache raises ERangeError.
"""
import numpy as np
import pytest

from tests.conftest import rand_int4

pytestmark = pytest.mark.gpu

N, K = 1024, 4096  # one matrix: 1024 x 2560 B = 2.5 MiB packed (device copy the same size)
CACHE = 9 << 20    # room for three matrices, not four


@pytest.fixture(scope="module")
def small():
    from quicknn_amd import hip

    c = hip.GPUContext(0, CACHE)
    yield c
    c.close()


def mats(rng, n):
    from quicknn_amd import hip

    return [hip.MemoryBlock.int4(rand_int4(rng, N, K)) for _ in range(n)]


def run(ctx, w, xt, yt):
    ctx.Int4Linear(yt, xt, w, 1, K, N)
    return ctx.Download(yt)


def test_lru_eviction_and_reupload(small, rng):
    ctx = small
    ws = mats(rng, 4)
    xt, yt = ctx.UploadRaw(rng.standard_normal(K).astype(np.float32)), ctx.NewTensor(N)
    s0 = ctx.status()
    first = [run(ctx, w, xt, yt) for w in ws[:3]]
    assert all(ctx.IsWeightResident(w, N, w.shape[1]) for w in ws[:3])
    s1 = ctx.status()
    assert s1.weight_uploads - s0.weight_uploads == 3
    run(ctx, ws[0], xt, yt)  # hit: ws[0] becomes the most recent
    assert ctx.status().weight_cache_hits > s1.weight_cache_hits
    run(ctx, ws[3], xt, yt)  # needs room: evicts the least recently used, ws[1]
    assert not ctx.IsWeightResident(ws[1], N, ws[1].shape[1])
    assert ctx.IsWeightResident(ws[0], N, ws[0].shape[1])
    assert ctx.status().weight_evictions - s1.weight_evictions == 1
    assert np.array_equal(run(ctx, ws[1], xt, yt), first[1])  # uploaded again, same result
    ctx.Recycle(xt)
    ctx.Recycle(yt)


def test_preload_pins_until_flush(small, rng):
    from quicknn_amd import hip

    ctx = small
    ws = mats(rng, 4)
    xt, yt = ctx.UploadRaw(rng.standard_normal(K).astype(np.float32)), ctx.NewTensor(N)
    ctx.Flush()
    ctx.PreloadWeights(ws[:3])
    with pytest.raises(hip.ERangeError):
        ctx.Int4Linear(yt, xt, ws[3], 1, K, N)  # only fits by evicting a preloaded weight
    ctx.Flush()  # releases the preload pins
    ctx.Int4Linear(yt, xt, ws[3], 1, K, N)
    ctx.Flush()
    ctx.Recycle(xt)
    ctx.Recycle(yt)


def test_retain_and_capacity(small, rng):
    from quicknn_amd import hip

    ctx = small
    ws = mats(rng, 3)
    limit = ctx.status().weight_limit
    assert limit == CACHE
    assert ctx.WeightBatchCapacity() == CACHE
    ctx.RetainWeight(ws[0], N, ws[0].shape[1])
    ctx.RetainWeight(ws[0], N, ws[0].shape[1])  # once
    per = ctx.status().weight_bytes
    assert ctx.WeightBatchCapacity() == CACHE - ws[0].data.size
    xt, yt = ctx.UploadRaw(rng.standard_normal(K).astype(np.float32)), ctx.NewTensor(N)
    for w in mats(rng, 6):  # stream more matrices than fit: the retained one stays
        run(ctx, w, xt, yt)
        assert ctx.IsWeightResident(ws[0], N, ws[0].shape[1])
    assert per >= ws[0].data.size
    big = hip.MemoryBlock.int4(rand_int4(rng, 4 * N, K))  # 10 MiB > the whole cache
    with pytest.raises(hip.ERangeError):
        ctx.Int4Linear(ctx.NewTensor(4 * N), xt, big, 1, K, 4 * N)
    ctx.Recycle(xt)
    ctx.Recycle(yt)
