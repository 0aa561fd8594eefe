"""GPU tests of the context's small ops and plumbing.

* GO_FILL, GO_ADD (tensor.comp:219, :221): exact (alpha a power of two).
* GO_SWIGLU / GO_GEGLU (tensor.comp:228), plain and interleaved: SwiGLU within
  2e-6 relative of float64 silu elementwise; GEGLU within 4e-6 elementwise where
  |g| < 2 and 2e-6 normwise (1 + tanh cancels for negative g in fp32).
* GO_NORM through KernelWeights (tensor.comp:63-73): RMS form against the
  oracle's RMSNorm (QwenHybrid.CPU.pas:110-120), LayerNorm form (flags&1,
  beta) and the (1 + gamma) form against float64, bf16 and fp32 gamma.
* CheckFinite / GO_FINITE: Download raises on NaN/Inf and leaves the
  destination untouched (Context.Implementation.inc:745-756); clean data passes.
* Copy with offsets, partial Download, Scratch slots, Recycle, events.
* HIP graph capture of a decode MLP (fused gate/up, down, GO_ADD residual),
  and of GGUF projections of 1, 6 and 64 rows (one-token matvec, multi-token
  matvec, fp16-copy GEMM with K-slices) with a 4096-key cached attention
  (LDS-streamed kernel and chunk merge): every replay, with eager work and
  synchronisations between replays, equals the eager result bit for bit.
"""
import numpy as np
import pytest
from scipy.special import expit

import oracle
from tests.conftest import bf16_bits, bf16_to_f32, normwise_rel_err, rand_int4

pytestmark = pytest.mark.gpu


def f32_bits(v: float) -> int:
    return int(np.array([v], np.float32).view(np.int32)[0])


def test_fill_and_add(ctx, rng):
    from quicknn_amd import hip

    n = 1000
    t = ctx.NewTensor(n)
    ctx.Kernel(hip.GO_FILL, n, t, None, None, None, [f32_bits(1.5)])
    assert np.all(ctx.Download(t) == np.float32(1.5))
    # GO_ADD: rows of `cols` from a into a strided window of dst
    cols, stride, doff, soff = 7, 10, 3, 2
    rows = 9
    dst0 = rng.standard_normal(doff + rows * stride).astype(np.float32)
    a0 = rng.standard_normal(soff + rows * cols).astype(np.float32)
    d, a = ctx.UploadRaw(dst0), ctx.UploadRaw(a0)
    ctx.Kernel(hip.GO_ADD, rows * cols, d, a, None, None, [cols, stride, f32_bits(0.5), doff, soff])
    want = dst0.copy()
    for i in range(rows * cols):
        r, j = divmod(i, cols)
        want[doff + r * stride + j] += np.float32(0.5) * a0[soff + i]
    assert np.array_equal(ctx.Download(d), want)
    for x in (t, d, a):
        ctx.Recycle(x)


def silu64(g):
    g = np.asarray(g, np.float64)
    return np.where(g >= 20, g, np.where(g <= -20, 0.0, g * expit(g)))


def gelu64(g):
    g = np.asarray(g, np.float64)
    return 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3)))


@pytest.mark.parametrize("op", ["swiglu", "geglu", "swiglu_interleaved"])
def test_glu(ctx, rng, op):
    from quicknn_amd import hip

    rows, inter = 3, 777
    g = (rng.standard_normal((rows, inter)) * 6).astype(np.float32)
    g[0, :4] = [25.0, -25.0, 0.0, 19.9]
    u = rng.standard_normal((rows, inter)).astype(np.float32)
    out = ctx.NewTensor(rows * inter)
    if op == "swiglu_interleaved":
        a = ctx.UploadRaw(np.concatenate([g, u], axis=1))
        ctx.Kernel(hip.GO_SWIGLU, rows * inter, out, a, None, None, [inter, 1])
        tensors = [a]
    else:
        a, b = ctx.UploadRaw(g), ctx.UploadRaw(u)
        code = hip.GO_SWIGLU if op == "swiglu" else hip.GO_GEGLU
        ctx.Kernel(code, rows * inter, out, a, b, None, [inter, 0])
        tensors = [a, b]
    want = (gelu64(g) if op == "geglu" else silu64(g)) * u
    got = ctx.Download(out).reshape(rows, inter)
    if op == "geglu":
        # 1 + tanh(z) cancels for negative g in the fp32 shader formula (the same
        # formula evaluated in numpy fp32 is already 2e-5 off at g = -3):
        # elementwise where |g| < 2, normwise everywhere.
        near = np.abs(g) < 2
        rel = np.where(near, np.abs(got - want) / (np.abs(want) + 1e-30), 0)
        w = np.unravel_index(np.argmax(rel), rel.shape)
        assert rel[w] <= 4e-6, (rel[w], g[w], got[w], want[w])
        worst = np.unravel_index(np.argmax(np.abs(got - want)), got.shape)
        assert normwise_rel_err(got, want) < 2e-6, (normwise_rel_err(got, want), g[worst], got[worst], want[worst])
    else:
        assert np.all(np.abs(got - want) <= 2e-6 * np.abs(want) + 1e-30)
    for t in tensors + [out]:
        ctx.Recycle(t)


@pytest.mark.parametrize("gamma_kind", ["unit", "f32", "bf16", "add_one"])
def test_rms_norm(ctx, rng, gamma_kind):
    from quicknn_amd import hip

    rows, dim = 4, 2560
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    gf = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    flags, unit, gamma_block, gamma_ref = 0, 0, None, gf
    if gamma_kind == "unit":
        unit, gamma_ref = 1, np.ones(dim, np.float32)
    elif gamma_kind == "f32":
        gamma_block = hip.MemoryBlock(gf, (dim,), hip.DT_F32)
    elif gamma_kind == "bf16":
        gb = bf16_bits(gf)
        gamma_block = hip.MemoryBlock(gb, (dim,), hip.DT_BF16)
        gamma_ref = bf16_to_f32(gb)
    else:  # Gemma's (1 + gamma)
        flags = 4
        gamma_block = hip.MemoryBlock(gf, (dim,), hip.DT_F32)
    xt, out = ctx.UploadRaw(x), ctx.NewTensor(rows * dim)
    ctx.KernelWeights(hip.GO_NORM, rows * dim, out, xt, gamma_block, None,
                      [rows, dim, flags, 0, 0, 0, unit, f32_bits(1e-6)])
    got = ctx.Download(out).reshape(rows, dim)
    want = oracle.rmsnorm(x, gamma_ref, eps=1e-6, add_one=(flags == 4))
    assert normwise_rel_err(got, want) < 2e-6
    ctx.Recycle(xt)
    ctx.Recycle(out)


def test_layer_norm_with_beta(ctx, rng):
    from quicknn_amd import hip

    rows, dim = 3, 1000
    x = (rng.standard_normal((rows, dim)) + 3).astype(np.float32)
    gamma = rng.standard_normal(dim).astype(np.float32)
    beta = rng.standard_normal(dim).astype(np.float32)
    xt, out = ctx.UploadRaw(x), ctx.NewTensor(rows * dim)
    ctx.KernelWeights(hip.GO_NORM, rows * dim, out, xt, hip.MemoryBlock(gamma, (dim,), hip.DT_F32),
                      hip.MemoryBlock(beta, (dim,), hip.DT_F32), [rows, dim, 1, 0, 0, 0, 0, f32_bits(1e-5)])
    x64 = x.astype(np.float64)
    c = x64 - x64.mean(axis=1, keepdims=True)
    want = c / np.sqrt((c ** 2).mean(axis=1, keepdims=True) + 1e-5) * gamma + beta
    assert normwise_rel_err(ctx.Download(out).reshape(rows, dim), want) < 2e-6
    ctx.Recycle(xt)
    ctx.Recycle(out)


def test_check_finite(ctx):
    from quicknn_amd import hip

    clean = ctx.UploadRaw(np.arange(300, dtype=np.float32))
    ctx.CheckFinite(clean)
    assert np.array_equal(ctx.Download(clean), np.arange(300, dtype=np.float32))
    for bad in (np.nan, np.inf, -np.inf):
        v = np.ones(300, np.float32)
        v[123] = bad
        t = ctx.UploadRaw(v)
        ctx.Kernel(hip.GO_FINITE, 300, None, t, None, None, [])
        dst = np.full(300, 7.0, np.float32)
        with pytest.raises(hip.EInvalidOp):
            hip._raise(hip.lib().qnn_download(ctx.h, t.handle, dst.ctypes.data, 300))
        assert np.all(dst == 7.0)  # destination untouched on error
        assert np.array_equal(ctx.Download(t)[:123], v[:123])  # the flag was cleared
        ctx.Recycle(t)
    ctx.Recycle(clean)


def test_copy_download_scratch_and_errors(ctx, rng):
    from quicknn_amd import hip

    src = rng.standard_normal(100).astype(np.float32)
    a, b = ctx.UploadRaw(src), ctx.NewTensor(100)
    ctx.Kernel(hip.GO_FILL, 100, b, None, None, None, [0])
    ctx.Copy(b, a, 30, 50, 10)
    got = ctx.Download(b)
    assert np.array_equal(got[50:80], src[10:40]) and not got[:50].any() and not got[80:].any()
    assert np.array_equal(ctx.Download(a, 17), src[:17])
    with pytest.raises(hip.EArgumentException):
        ctx.Copy(b, a, 60, 50, 0)  # past the end of dst
    with pytest.raises(hip.EArgumentException):
        hip._raise(hip.lib().qnn_download(ctx.h, a.handle, np.empty(1, np.float32).ctypes.data, 0))
    s1 = ctx.Scratch(2, 64)
    s2 = ctx.Scratch(2, 32)  # an existing slot that is large enough is reused
    assert s1.handle == s2.handle
    s3 = ctx.Scratch(2, 4096)  # grown
    assert s3.count >= 4096
    with pytest.raises(hip.EArgumentException):
        ctx.Scratch(4, 8)
    ctx.Recycle(a)
    with pytest.raises(hip.EArgumentException):
        ctx.Download(a)  # recycled tensors are no longer live
    ctx.Recycle(b)


def test_events_time_forward(ctx):
    from quicknn_amd import hip

    t = ctx.NewTensor(1 << 20)
    ctx.EventRecord(10)
    for _ in range(20):
        ctx.Kernel(hip.GO_FILL, 1 << 20, t, None, None, None, [0])
    ctx.EventRecord(11)
    ms = ctx.EventElapsedMs(10, 11)
    assert 0.0 < ms < 1000.0
    with pytest.raises(hip.EArgumentException):
        ctx.EventRecord(64)
    ctx.Recycle(t)


def test_graph_replays_match_eager(ctx, rng):
    """Capture fused gate/up + down + residual GO_ADD; replay with eager work in between."""
    from quicknn_amd import hip

    hidden, inter = 1024, 3072
    g, u = hip.MemoryBlock.int4(rand_int4(rng, inter, hidden)), hip.MemoryBlock.int4(rand_int4(rng, inter, hidden))
    d = hip.MemoryBlock.int4(rand_int4(rng, hidden, inter))
    xs = [rng.standard_normal(hidden).astype(np.float32) for _ in range(4)]
    x, h, y = ctx.UploadRaw(xs[0]), ctx.NewTensor(inter), ctx.NewTensor(hidden)
    other = ctx.NewTensor(4096)

    def layer():
        ctx.TrySwiGLUVector(h, x, g, u, hidden, inter)
        ctx.Int4Linear(y, h, d, 1, inter, hidden)
        ctx.Kernel(hip.GO_ADD, hidden, y, x, None, None, [hidden, hidden, f32_bits(1.0), 0, 0])

    eager = []
    for xv in xs:  # eager results (also sizes every workspace before capture)
        xt = ctx.UploadRaw(xv)
        ctx.Copy(x, xt, hidden)
        layer()
        eager.append(ctx.Download(y))
        ctx.Recycle(xt)
    ctx.GraphBegin()
    layer()
    gid = ctx.GraphEnd()
    for rep in range(3):
        for i, xv in enumerate(xs):
            xt = ctx.UploadRaw(xv)
            ctx.Copy(x, xt, hidden)
            ctx.Kernel(hip.GO_FILL, 4096, other, None, None, None, [f32_bits(float(rep))])  # eager work
            ctx.GraphLaunch(gid)
            got = ctx.Download(y)
            assert np.array_equal(got, eager[i]), (rep, i)
            assert np.all(ctx.Download(other) == np.float32(rep))
            ctx.Recycle(xt)
    # parity of the captured layer with the CPU path (residual added)
    want = oracle.cpu_mlp(g.data, u.data, d.data, oracle.ENC_INT4, xs[0], hidden, inter)[0] + xs[0]
    assert normwise_rel_err(eager[0], want) < 1e-3
    for t in (x, h, y, other):
        ctx.Recycle(t)


def test_graph_replays_gguf_projections_and_attention_match_eager(ctx, rng):
    """Capture a Q4_K projection of one row, a Q6_K projection of six rows, a Q4_K projection of
    64 rows (its fp16 copy, made by the eager runs, split over two K-slices and summed by a second
    launch) and a cached attention over 4096 keys at head dim 128; replay with eager work between."""
    from quicknn_amd import hip

    k, n = 1024, 384
    w4 = hip.MemoryBlock.gguf(hip.gguf_quantize(hip.WE_Q4_K, (rng.standard_normal(n * k) * 0.02).astype(np.float32)),
                              n, k, hip.WE_Q4_K)
    w6 = hip.MemoryBlock.gguf(hip.gguf_quantize(hip.WE_Q6_K, (rng.standard_normal(n * k) * 0.02).astype(np.float32)),
                              n, k, hip.WE_Q6_K)
    heads, kvh, dim, cap = 32, 8, 128, 4096
    cache = ctx.UploadRaw(rng.standard_normal(2 * cap * kvh * dim).astype(np.float32))
    rows = (1, 6, 64)
    xs = [ctx.NewTensor(r * k) for r in rows]
    ys = [ctx.NewTensor(r * n) for r in rows]
    q, o, other = ctx.NewTensor(heads * dim), ctx.NewTensor(heads * dim), ctx.NewTensor(4096)
    h0 = ctx.status().gemm_h16

    def step():
        ctx.Linear(ys[0], xs[0], w4, None, None, 1, k, n)
        ctx.Linear(ys[1], xs[1], w6, None, None, 6, k, n)
        ctx.Linear(ys[2], xs[2], w4, None, None, 64, k, n)
        ctx.CachedAttention(o, q, cache, 1, cap, heads, kvh, dim, cap - 1)

    sets = [([rng.standard_normal(r * k).astype(np.float32) for r in rows],
             (rng.standard_normal(heads * dim) * 0.3).astype(np.float32)) for _ in range(3)]

    def load(i):
        tmp = [ctx.UploadRaw(v) for v in sets[i][0]] + [ctx.UploadRaw(sets[i][1])]
        for dst, src, cnt in zip(xs + [q], tmp, [r * k for r in rows] + [heads * dim]):
            ctx.Copy(dst, src, cnt)
        return tmp

    eager = []
    for i in range(len(sets)):  # eager results (also make the fp16 copy and size every workspace)
        tmp = load(i)
        step()
        eager.append([ctx.Download(t) for t in ys + [o]])
        for t in tmp:
            ctx.Recycle(t)
    assert ctx.status().gemm_h16 - h0 == len(sets)
    ctx.GraphBegin()
    step()
    gid = ctx.GraphEnd()
    for rep in range(3):
        for i in range(len(sets)):
            tmp = load(i)
            ctx.Kernel(hip.GO_FILL, 4096, other, None, None, None, [f32_bits(float(rep))])  # eager work
            ctx.GraphLaunch(gid)
            got = [ctx.Download(t) for t in ys + [o]]
            for j, (gv, ev) in enumerate(zip(got, eager[i])):
                assert np.array_equal(gv.view(np.uint32), ev.view(np.uint32)), (rep, i, j)
            assert np.all(ctx.Download(other) == np.float32(rep))
            for t in tmp:
                ctx.Recycle(t)
    # the eager runs against the CPU path
    w4b, w6b = w4.data, w6.data
    x0, q0 = sets[0]
    assert normwise_rel_err(eager[0][0], oracle.cpu_linear(w4b, oracle.ENC_Q4_K, x0[0], k, n)) <= 1e-3
    for r in (0, 5):
        assert normwise_rel_err(eager[0][1][r * n:(r + 1) * n],
                                oracle.cpu_linear(w6b, oracle.ENC_Q6_K, x0[1][r * k:(r + 1) * k], k, n)) <= 1e-3
    for r in (0, 63):
        assert normwise_rel_err(eager[0][2][r * n:(r + 1) * n],
                                oracle.cpu_linear(w4b, oracle.ENC_Q4_K, x0[2][r * k:(r + 1) * k], k, n)) <= 1e-3
    for t in xs + ys + [q, o, other, cache]:
        ctx.Recycle(t)
