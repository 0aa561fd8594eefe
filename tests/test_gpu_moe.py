"""GPU parity of the MoE path (native INT4 experts) against the CPU oracle.

* GO_MOE_ROUTE (moe.comp:25-50): expert ids and routing weights identical to
  the oracle bit for bit (both rank by fp32 probability with a correctly
  rounded exp and the reference's summation order).
* GO_MOE_GATHER / GO_MOE_SCATTER (moe.comp:124-126): exact.
* TLLMMoE.forward (LLM.MoE.pas:376-448) replayed op by op on this backend,
  and the device-routed qnn_moe_experts: within a normwise relative error of
  1e-3 of the composed CPU path (experts in ascending id, out += y*p).
"""
import numpy as np
import pytest

import oracle
from quicknn_amd import hip
from tests.conftest import normwise_rel_err, rand_int4

pytestmark = pytest.mark.gpu
TOL = 1e-3


def route_on_gpu(ctx, logits, k, normalize=True):
    rows, E = logits.shape
    lt = ctx.UploadRaw(logits)
    routes = ctx.NewTensor(2 * rows * k)
    ctx.Kernel(hip.GO_MOE_ROUTE, 2 * rows * k, routes, lt, None, None, [rows, E, k, int(normalize)])
    raw = ctx.Download(routes)
    return routes, raw[:rows * k].view(np.uint32).reshape(rows, k), raw[rows * k:].reshape(rows, k)


@pytest.mark.parametrize("rows,E,k", [(1, 128, 8), (16, 128, 8), (3, 512, 64), (2, 8, 8), (4, 1000, 4), (7, 60, 1),
                                      (2, 1024, 8), (2, 1025, 8), (1, 8192, 64), (1, 64, 64), (5, 65, 3)])
@pytest.mark.parametrize("normalize", [True, False])
def test_route_matches_oracle(ctx, rng, rows, E, k, normalize):
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    _, ids, probs = route_on_gpu(ctx, logits, k, normalize)
    want_ids, want_p = oracle.moe_route(logits, k, normalize)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(probs.view(np.uint32), want_p.view(np.uint32))


@pytest.mark.parametrize("E,k", [(128, 1), (128, 2), (2000, 2)])  # register and LDS selection
def test_route_equal_probabilities_of_distinct_logits_tie_to_lower_id(ctx, E, k):
    """moe.comp:36-46 ranks by probability: logits 0 (id 7) and -1e-8 (id 3)
    give exp values that both round to 1.0f, so their probabilities are equal
    and the lower id ranks first although its logit is smaller."""
    logits = np.full((1, E), -4.0, np.float32)
    logits[0, 7], logits[0, 3] = 0.0, -1e-8
    _, ids, probs = route_on_gpu(ctx, logits, k)
    want_ids, want_p = oracle.moe_route(logits, k)
    assert ids[0].tolist() == [3, 7][:k] == want_ids[0].tolist()
    assert np.array_equal(probs.view(np.uint32), want_p.view(np.uint32))
    by_logit, _ = oracle.moe_route(logits, k, select_on_logits=True)
    assert by_logit[0, 0] == 7  # the logit rule would rank id 7 first


@pytest.mark.parametrize("E", [6, 2000])  # register and LDS selection
def test_route_signed_zero_and_equal_logits_tie_to_lower_id(ctx, E):
    logits = np.full((1, E), -1.0, np.float32)
    logits[0, 3], logits[0, 1], logits[0, 5] = 0.0, -0.0, 0.0
    _, ids, probs = route_on_gpu(ctx, logits, 3)
    want_ids, want_p = oracle.moe_route(logits, 3)
    assert ids[0].tolist() == [1, 3, 5] == want_ids[0].tolist()
    assert np.array_equal(probs.view(np.uint32), want_p.view(np.uint32))


def test_route_ties_take_lower_id(ctx):
    logits = np.array([[0.5, 2.0, 2.0, -1.0, 2.0, 0.5], [1.0] * 6], np.float32)
    _, ids, probs = route_on_gpu(ctx, logits, 4)
    assert ids[0].tolist() == [1, 2, 4, 0]
    assert ids[1].tolist() == [0, 1, 2, 3]
    assert np.allclose(probs[1], 0.25, rtol=1e-6)


def test_gather_scatter_exact(ctx, rng):
    rows, k, hidden = 5, 3, 40
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    order = np.array([4, 0, 7, 13], np.uint32)  # route positions t*k + j of distinct tokens (one expert's rows)
    src, idx = ctx.UploadRaw(x), ctx.UploadRaw(order.view(np.float32))
    g = ctx.NewTensor(len(order) * hidden)
    ctx.Kernel(hip.GO_MOE_GATHER, len(order) * hidden, g, src, idx, None, [hidden, k, 0])
    assert np.array_equal(ctx.Download(g).reshape(-1, hidden), x[order // k])
    # scatter with probabilities at ProbBase + route
    y = rng.standard_normal((len(order), hidden)).astype(np.float32)
    probs = rng.uniform(0, 1, rows * k).astype(np.float32)
    plane = np.concatenate([np.zeros(rows * k, np.float32), probs])
    out0 = rng.standard_normal((rows, hidden)).astype(np.float32)
    yt, pt, out = ctx.UploadRaw(y), ctx.UploadRaw(plane), ctx.UploadRaw(out0)
    ctx.Kernel(hip.GO_MOE_SCATTER, y.size, out, yt, idx, pt, [hidden, k, 0, 0, 0, rows * k])
    want = out0.copy()
    for i, R in enumerate(order):
        want[R // k] = want[R // k] + y[i] * probs[R]
    assert np.array_equal(ctx.Download(out).reshape(rows, hidden), want)
    # single-row form: route index from the args
    one = ctx.UploadRaw(out0[:1].copy())
    y1 = ctx.UploadRaw(y[:1].copy())
    ctx.Kernel(hip.GO_MOE_SCATTER, hidden, one, y1, None, pt, [hidden, k, 0, 2, 1, rows * k])
    assert np.array_equal(ctx.Download(one), out0[0] + y[0] * probs[2])


def test_dispatch_index_out_of_range_is_reported(ctx, rng):
    x = ctx.UploadRaw(rng.standard_normal((2, 16)).astype(np.float32))
    idx = ctx.UploadRaw(np.array([1, 99], np.uint32).view(np.float32))
    g = ctx.NewTensor(32)
    ctx.Kernel(hip.GO_MOE_GATHER, 32, g, x, idx, None, [16, 1, 0])
    with pytest.raises(hip.EInvalidOp):
        ctx.Download(g)


class Experts:
    def __init__(self, rng, E, hidden, inter):
        self.E, self.hidden, self.inter = E, hidden, inter
        if hidden % 32 == 0 and inter % 32 == 0:
            mk = lambda n, k: rand_int4(rng, n, k)
        else:
            mk = lambda n, k: hip.quantize_int4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        self.g = [mk(inter, hidden) for _ in range(E)]
        self.u = [mk(inter, hidden) for _ in range(E)]
        self.d = [mk(hidden, inter) for _ in range(E)]
        self.bg = [hip.MemoryBlock.int4(p) for p in self.g]
        self.bu = [hip.MemoryBlock.int4(p) for p in self.u]
        self.bd = [hip.MemoryBlock.int4(p) for p in self.d]

    def oracle(self, x, ids, probs):
        return oracle.cpu_moe(self.g, self.u, self.d, x, ids, probs, self.hidden, self.inter)


def reference_forward(ctx, ex, src, routes, ids, rows, k):
    """TLLMMoE.forward's dispatch (LLM.MoE.pas:376-448) on this backend's ops."""
    hidden, inter, E = ex.hidden, ex.inter, ex.E
    host = ids.reshape(-1)
    counts = np.bincount(host, minlength=E)
    offsets = np.concatenate([[0], np.cumsum(counts)[:-1]])
    out = ctx.NewTensor(rows * hidden)
    ctx.Kernel(hip.GO_FILL, rows * hidden, out, None, None, None, [0])
    indices = None
    if rows > 1:
        order = np.argsort(host, kind="stable").astype(np.uint32)  # positions grouped by expert, ascending
        indices = ctx.UploadRaw(order.view(np.float32))
    for e in range(E):
        c = int(counts[e])
        if c == 0:
            continue
        if rows == 1:
            gathered, route_index = src, int(np.nonzero(host == e)[0][0])
        else:
            gathered = ctx.NewTensor(c * hidden)
            ctx.Kernel(hip.GO_MOE_GATHER, c * hidden, gathered, src, indices, None, [hidden, k, int(offsets[e])])
        g = ctx.NewTensor(c * inter)
        if c != 1 or not ctx.TrySwiGLUVector(g, gathered, ex.bg[e], ex.bu[e], hidden, inter):
            u = ctx.NewTensor(c * inter)
            ctx.Int4Linear(g, gathered, ex.bg[e], c, hidden, inter)
            ctx.Int4Linear(u, gathered, ex.bu[e], c, hidden, inter)
            ctx.Kernel(hip.GO_SWIGLU, c * inter, g, g, u, None, [inter, 0])
        if rows == 1:
            ctx.Int4LinearAccumulate(out, g, routes, ex.bd[e], inter, hidden, rows * k + route_index)
        else:
            y = ctx.NewTensor(c * hidden)
            ctx.Int4Linear(y, g, ex.bd[e], c, inter, hidden)
            ctx.Kernel(hip.GO_MOE_SCATTER, c * hidden, out, y, indices, routes,
                       [hidden, k, int(offsets[e]), 0, 0, rows * k])
    return ctx.Download(out).reshape(rows, hidden)


@pytest.fixture(scope="module")
def qwen3_moe(ctx):
    """Qwen3-30B-A3B expert shapes: 128 experts, hidden 2048, intermediate 768."""
    ex = Experts(np.random.default_rng(30), 128, 2048, 768)
    s = ctx.CreateExpertSet(ex.bg, ex.bu, ex.bd, ex.hidden, ex.inter)
    yield ex, s
    ctx.DestroyExpertSet(s)


@pytest.mark.parametrize("rows", [1, 2, 16])
def test_reference_dispatch_matches_cpu(ctx, rng, qwen3_moe, rows):
    ex, _ = qwen3_moe
    k = 8
    x = rng.standard_normal((rows, ex.hidden)).astype(np.float32)
    routes, ids, probs = route_on_gpu(ctx, rng.standard_normal((rows, ex.E)).astype(np.float32), k)
    got = reference_forward(ctx, ex, ctx.UploadRaw(x), routes, ids, rows, k)
    want = ex.oracle(x, ids, probs)
    for r in range(rows):
        assert normwise_rel_err(got[r], want[r]) <= TOL, r


@pytest.mark.parametrize("rows", [1, 2, 16, 128])
def test_moe_experts_matches_cpu(ctx, rng, qwen3_moe, rows):
    ex, s = qwen3_moe
    k = 8
    x = rng.standard_normal((rows, ex.hidden)).astype(np.float32)
    routes, ids, probs = route_on_gpu(ctx, rng.standard_normal((rows, ex.E)).astype(np.float32), k)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(rows * ex.hidden)
    ctx.MoEExperts(s, dst, src, routes, rows, k)
    got = ctx.Download(dst).reshape(rows, ex.hidden)
    want = ex.oracle(x, ids, probs)
    for r in range(rows):
        assert normwise_rel_err(got[r], want[r]) <= TOL, r


def test_moe_experts_deterministic_and_matches_reference_dispatch(ctx, rng, qwen3_moe):
    ex, s = qwen3_moe
    rows, k = 4, 8
    x = rng.standard_normal((rows, ex.hidden)).astype(np.float32)
    routes, ids, _ = route_on_gpu(ctx, rng.standard_normal((rows, ex.E)).astype(np.float32), k)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(rows * ex.hidden)
    outs = []
    for _ in range(3):
        ctx.MoEExperts(s, dst, src, routes, rows, k)
        outs.append(ctx.Download(dst).copy())
    assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs)
    ref = reference_forward(ctx, ex, src, routes, ids, rows, k)
    assert normwise_rel_err(outs[0].reshape(rows, -1), ref) <= TOL


@pytest.mark.parametrize("E,hidden,inter,k,rows", [
    (6, 100, 72, 2, 3),    # ragged groups and tiles
    (3, 64, 96, 3, 9),     # every expert takes every token (9 tokens > the 4-token chunk)
    (4, 256, 128, 2, 16),  # ~8 tokens per expert
    (1, 128, 64, 1, 1),
])
def test_moe_experts_small_shapes(ctx, rng, E, hidden, inter, k, rows):
    ex = Experts(rng, E, hidden, inter)
    s = ctx.CreateExpertSet(ex.bg, ex.bu, ex.bd, hidden, inter)
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    routes, ids, probs = route_on_gpu(ctx, rng.standard_normal((rows, E)).astype(np.float32), k)
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(rows * hidden)
    ctx.MoEExperts(s, dst, src, routes, rows, k)
    got = ctx.Download(dst).reshape(rows, hidden)
    want = ex.oracle(x, ids, probs)
    ctx.DestroyExpertSet(s)
    for r in range(rows):
        assert normwise_rel_err(got[r], want[r]) <= TOL, r


def test_moe_experts_invalid_route_id(ctx, rng):
    ex = Experts(rng, 4, 64, 64)
    s = ctx.CreateExpertSet(ex.bg, ex.bu, ex.bd, 64, 64)
    plane = np.concatenate([np.array([1, 9], np.uint32).view(np.float32), np.array([0.5, 0.5], np.float32)])
    routes, src, dst = ctx.UploadRaw(plane), ctx.UploadRaw(np.ones(64, np.float32)), ctx.NewTensor(64)
    ctx.MoEExperts(s, dst, src, routes, 1, 2)
    with pytest.raises(hip.EInvalidOp):
        ctx.Download(dst)
    ctx.DestroyExpertSet(s)


def test_moe_experts_argument_errors(ctx, rng):
    ex = Experts(rng, 4, 64, 64)
    s = ctx.CreateExpertSet(ex.bg, ex.bu, ex.bd, 64, 64)
    src, dst, routes = ctx.NewTensor(129 * 64), ctx.NewTensor(129 * 64), ctx.NewTensor(2 * 129 * 5)
    with pytest.raises(hip.EArgumentException):
        ctx.MoEExperts(s, dst, src, routes, 129, 1)  # rows > 128
    with pytest.raises(hip.EArgumentException):
        ctx.MoEExperts(s, dst, src, routes, 1, 5)  # topk > experts
    with pytest.raises(hip.EArgumentException):
        ctx.MoEExperts(s, src, src, routes, 1, 1)  # aliasing
    with pytest.raises(hip.EArgumentException):
        ctx.CreateExpertSet(ex.bg, ex.bu, ex.bd, 64, 96)  # shapes do not match
    ctx.DestroyExpertSet(s)


def _run_moe(ctx, s, x, routes, rows, k, hidden):
    src, dst = ctx.UploadRaw(x), ctx.NewTensor(rows * hidden)
    ctx.MoEExperts(s, dst, src, routes, rows, k)
    out = ctx.Download(dst).copy()
    ctx.Recycle(src)
    ctx.Recycle(dst)
    return out


@pytest.mark.parametrize("E,hidden,inter,k", [
    (6, 100, 72, 2),     # ragged groups and tiles (blocks not a multiple of 8)
    (1, 128, 64, 1),
    (16, 512, 320, 8),   # h blocks of 64 rows in 5 per expert
    (64, 1024, 256, 16),
    (40, 192, 4100, 3),  # many gate/up blocks, ragged
])
def test_moe_decode_single_launch_equals_two_launch(ctx, rng, tune, E, hidden, inter, k):
    """One token: the single-launch path and the two-launch path give the same bits."""
    ex = Experts(rng, E, hidden, inter)
    s = ctx.CreateExpertSet(ex.bg, ex.bu, ex.bd, hidden, inter)
    x = rng.standard_normal((1, hidden)).astype(np.float32)
    routes, ids, probs = route_on_gpu(ctx, rng.standard_normal((1, E)).astype(np.float32), k)
    f0 = ctx.status().moe_fused
    one = _run_moe(ctx, s, x, routes, 1, k, hidden)
    again = _run_moe(ctx, s, x, routes, 1, k, hidden)
    assert ctx.status().moe_fused - f0 == 2
    tune("QNN_FUSE_MOE", "0")
    two = _run_moe(ctx, s, x, routes, 1, k, hidden)
    assert ctx.status().moe_fused - f0 == 2
    ctx.DestroyExpertSet(s)
    assert np.array_equal(one.view(np.uint32), two.view(np.uint32))
    assert np.array_equal(again.view(np.uint32), one.view(np.uint32))
    assert normwise_rel_err(one.reshape(1, -1)[0], ex.oracle(x, ids, probs)[0]) <= TOL


def test_moe_decode_qwen3_equals_two_launch(ctx, rng, tune, qwen3_moe):
    ex, s = qwen3_moe
    k = 8
    for trial in range(3):  # fresh routes each time: other experts, other flags
        x = rng.standard_normal((1, ex.hidden)).astype(np.float32)
        routes, ids, probs = route_on_gpu(ctx, rng.standard_normal((1, ex.E)).astype(np.float32), k)
        tune("QNN_FUSE_MOE", "1")
        f0 = ctx.status().moe_fused
        one = _run_moe(ctx, s, x, routes, 1, k, ex.hidden)
        assert ctx.status().moe_fused - f0 == 1
        tune("QNN_FUSE_MOE", "0")
        two = _run_moe(ctx, s, x, routes, 1, k, ex.hidden)
        assert np.array_equal(one.view(np.uint32), two.view(np.uint32)), trial
        assert normwise_rel_err(one, ex.oracle(x, ids, probs)[0]) <= TOL


@pytest.mark.parametrize("fuse", ["1", "0"])
def test_moe_experts_duplicate_route_id(ctx, rng, tune, fuse):
    """An expert twice in one token's routes is reported (bit 8), on either path."""
    tune("QNN_FUSE_MOE", fuse)
    ex = Experts(rng, 4, 64, 64)
    s = ctx.CreateExpertSet(ex.bg, ex.bu, ex.bd, 64, 64)
    plane = np.concatenate([np.array([2, 2], np.uint32).view(np.float32), np.array([0.5, 0.5], np.float32)])
    routes, src, dst = ctx.UploadRaw(plane), ctx.UploadRaw(np.ones(64, np.float32)), ctx.NewTensor(64)
    ctx.MoEExperts(s, dst, src, routes, 1, 2)
    with pytest.raises(hip.EInvalidOp):
        ctx.Download(dst)
    ctx.DestroyExpertSet(s)


@pytest.mark.parametrize("E,hidden,inter,k", [(128, 512, 256, 8), (64, 256, 128, 4), (512, 128, 64, 8), (8, 128, 64, 8)])
def test_moe_route_then_experts_one_launch(ctx, rng, E, hidden, inter, k):
    """A one-token GO_MOE_ROUTE followed by qnn_moe_experts on its output runs
    as one launch that computes the routes itself: the output and the route
    tensor are bit-identical to the route op followed by the experts."""
    ex = Experts(rng, E, hidden, inter)
    s = ctx.CreateExpertSet(ex.bg, ex.bu, ex.bd, hidden, inter)
    x = rng.standard_normal((1, hidden)).astype(np.float32)
    logits = rng.standard_normal((1, E)).astype(np.float32)
    lt, src = ctx.UploadRaw(logits), ctx.UploadRaw(x)
    st0 = ctx.status()

    rt1, out1 = ctx.NewTensor(2 * k), ctx.NewTensor(hidden)
    ctx.Kernel(hip.GO_MOE_ROUTE, 2 * k, rt1, lt, None, None, [1, E, k, 1])
    ctx.MoEExperts(s, out1, src, rt1, 1, k)  # fused with the recorded route
    got, got_routes = ctx.Download(out1), ctx.Download(rt1)
    st1 = ctx.status()
    assert st1.moe_route_fused - st0.moe_route_fused == 1

    rt2, out2 = ctx.NewTensor(2 * k), ctx.NewTensor(hidden)
    ctx.Kernel(hip.GO_MOE_ROUTE, 2 * k, rt2, lt, None, None, [1, E, k, 1])
    want_routes = ctx.Download(rt2)  # settles the route op on its own
    ctx.MoEExperts(s, out2, src, rt2, 1, k)
    want = ctx.Download(out2)
    assert ctx.status().moe_route_fused == st1.moe_route_fused
    assert np.array_equal(got_routes.view(np.uint32), want_routes.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ids, probs = oracle.moe_route(logits, k, True)
    assert np.array_equal(got_routes[:k].view(np.uint32), ids[0])
    assert normwise_rel_err(got, ex.oracle(x, ids, probs)[0]) <= TOL
    for t in (lt, src, rt1, rt2, out1, out2):
        ctx.Recycle(t)
    ctx.DestroyExpertSet(s)


def test_recorded_route_settles_on_other_calls(ctx, rng):
    """A recorded route op runs before any call that could observe it, and a
    MoE call on other routes does not consume it."""
    E, k, hidden, inter = 32, 4, 128, 64
    ex = Experts(rng, E, hidden, inter)
    s = ctx.CreateExpertSet(ex.bg, ex.bu, ex.bd, hidden, inter)
    logits = rng.standard_normal((2, E)).astype(np.float32)
    l0, l1 = ctx.UploadRaw(logits[:1]), ctx.UploadRaw(logits[1:])
    r0, r1 = ctx.NewTensor(2 * k), ctx.NewTensor(2 * k)
    ctx.Kernel(hip.GO_MOE_ROUTE, 2 * k, r1, l1, None, None, [1, E, k, 1])
    want1 = ctx.Download(r1)
    f0 = ctx.status().moe_route_fused
    ctx.Kernel(hip.GO_MOE_ROUTE, 2 * k, r0, l0, None, None, [1, E, k, 0])  # recorded
    src, out = ctx.UploadRaw(rng.standard_normal(hidden).astype(np.float32)), ctx.NewTensor(hidden)
    ctx.MoEExperts(s, out, src, r1, 1, k)  # other routes: the recorded op runs first, unfused
    assert ctx.status().moe_route_fused == f0
    ids, p = oracle.moe_route(logits[:1], k, False)
    got0 = ctx.Download(r0)
    assert np.array_equal(got0[:k].view(np.uint32), ids[0])
    assert np.allclose(got0[k:], p[0], rtol=2e-6, atol=0)
    assert np.array_equal(ctx.Download(r1).view(np.uint32), want1.view(np.uint32))
    # recorded, then a different op: settled by it
    ctx.Kernel(hip.GO_MOE_ROUTE, 2 * k, r0, l1, None, None, [1, E, k, 1])
    ctx.Kernel(hip.GO_FILL, hidden, out, None, None, None, [0])
    assert np.array_equal(ctx.Download(r0).view(np.uint32), want1.view(np.uint32))
    for t in (l0, l1, r0, r1, src, out):
        ctx.Recycle(t)
    ctx.DestroyExpertSet(s)


def test_route_over_1024_experts_is_not_recorded(ctx, rng):
    E, k = 2000, 8
    logits = rng.standard_normal((1, E)).astype(np.float32)
    lt, rt = ctx.UploadRaw(logits), ctx.NewTensor(2 * k)
    ctx.Kernel(hip.GO_MOE_ROUTE, 2 * k, rt, lt, None, None, [1, E, k, 1])
    ids, p = oracle.moe_route(logits, k, True)
    got = ctx.Download(rt)
    assert np.array_equal(got[:k].view(np.uint32), ids[0])
    ctx.Recycle(lt)
    ctx.Recycle(rt)
