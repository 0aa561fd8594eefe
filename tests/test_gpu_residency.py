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


def test_fp16_gemm_copy_is_an_unreported_cache_entry(small, rng):
    """The pre-expanded fp16 copy the Q8_0 GEMM makes from a resident weight (k_h16_gemm) is a
    cache entry of its own: LRU eviction may drop it while the Q8_0 weight stays resident, and
    that eviction is not reported through OnWeightEvicted (no weight left the cache); the next
    GEMM on the weight makes it again, with the same result.  Runs first: an empty 9 MiB cache
    holds one Q8_0 weight (2.2 MB) with its fp16 copy (4.3 MB) and a second Q8_0 weight, not
    a second fp16 copy."""
    from quicknn_amd import hip

    ctx = small
    m, k, n = 128, 1024, 2048
    ws = [hip.MemoryBlock.gguf(hip.gguf_quantize(hip.WE_Q8_0, (rng.standard_normal(n * k) * 0.02).astype(np.float32)),
                               n, k, hip.WE_Q8_0) for _ in range(2)]
    a = ctx.UploadRaw(rng.standard_normal((m, k)).astype(np.float32))
    y, y1, x1 = ctx.NewTensor(m * n), ctx.NewTensor(n), ctx.UploadRaw(rng.standard_normal(k).astype(np.float32))
    seen = []
    ctx.OnWeightEvicted = seen.append
    s0 = ctx.status()
    ctx.Linear(y, a, ws[0], None, None, m, k, n)  # the Q8_0 copy and its fp16 copy
    first = ctx.Download(y).copy()
    ctx.Linear(y1, x1, ws[0], None, None, 1, k, n)  # one row: the Q8_0 copy only, now the newer entry
    ctx.Download(y1)
    ctx.Linear(y, a, ws[1], None, None, m, k, n)  # room for its fp16 copy: the first fp16 copy goes
    ctx.Download(y)
    assert ctx.status().weight_evictions - s0.weight_evictions == 1
    assert seen == []
    assert ctx.IsWeightResident(ws[0], n, k)
    ctx.Linear(y, a, ws[0], None, None, m, k, n)  # makes the fp16 copy again
    assert np.array_equal(ctx.Download(y).view(np.uint32), first.view(np.uint32))
    assert ctx.status().gemm_h16 - s0.gemm_h16 == 3
    ctx.OnWeightEvicted = None
    for t in (a, y, y1, x1):
        ctx.Recycle(t)
    ctx.Flush()


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


def test_on_weight_evicted_reports_each_evicted_identity(small, rng):
    """OnWeightEvicted (Context.API.inc:164) hears the identity of every entry
    the cache evicts, in LRU order (QuickNN.Vulkan.pas:568-569); the MoE layer
    uses it to hand the native bytes back to its cache (LLM.MoE.pas:196-203).
    Streams six matrices through the three-matrix cache (less what earlier
    tests retained), so each new one evicts the oldest."""
    ctx = small
    ctx.Flush()
    ws = mats(rng, 6)
    ids = [w.identity for w in ws]
    xt, yt = ctx.UploadRaw(rng.standard_normal(K).astype(np.float32)), ctx.NewTensor(N)
    heard = []
    ctx.OnWeightEvicted = heard.append
    e0 = ctx.status().weight_evictions
    for w in ws:
        run(ctx, w, xt, yt)
    assert len(heard) == ctx.status().weight_evictions - e0 >= 3
    ours = [i for i in heard if i in ids]
    assert ours == ids[:len(ours)] and len(ours) >= 3  # ours leave oldest first
    for w in ws[:len(ours)]:
        assert not ctx.IsWeightResident(w, N, w.shape[1])
    ctx.OnWeightEvicted = None
    n = len(heard)
    run(ctx, ws[0], xt, yt)  # evicts again; nobody is told
    assert len(heard) == n
    ctx.Recycle(xt)
    ctx.Recycle(yt)


def test_upload_memory_block(small, rng):
    """Upload(TMemoryBlock) (Context.Implementation.inc:700-705): F32 storage only,
    Size floats from element Offset (Common.pas:1597-1605)."""
    from quicknn_amd import hip

    ctx = small
    v = rng.standard_normal(100).astype(np.float32)
    t = ctx.Upload(hip.MemoryBlock(v, (100,), hip.DT_F32, offset=10, size=60))
    assert t.count == 60 and np.array_equal(ctx.Download(t), v[10:70])
    with pytest.raises(hip.EArgumentException):
        ctx.Upload(hip.MemoryBlock(v.view(np.uint16)[:100], (100,), hip.DT_BF16))
    ctx.Recycle(t)
