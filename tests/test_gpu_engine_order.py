"""The engine's own call sequences, replayed op for op through the C ABI.

The reference models create each output right before the projection that
writes it (Work.New / NewTensor, QwenHybrid.pas:540-551, LLM.pas:588-598,
Gemma2.pas:142-148), run the GLU in place (Kernel(GO_SWIGLU, .., G, G, U)) and
reach the MoE layer through its router (LLM.MoE.pas:357-448).  These tests
issue exactly those sequences and check:

* the recorded-call fusions still happen (the tensor creation between the calls
  does not launch them), and their outputs equal the unfused path bit for bit;
* TLLMMoE.forward from the router VectorLinear / Linear (F32 and BF16 router
  weights) through CheckFinite, GO_MOE_ROUTE, the route readback, per-expert
  gather, SwiGLU, down and scatter/accumulate matches the CPU oracle;
* a multi-row Int4Linear recorded before qnn_moe_experts runs before the
  experts read its output.
"""
import numpy as np
import pytest

import oracle
from quicknn_amd import hip
from tests.conftest import bf16_bits, bf16_to_f32, normwise_rel_err, rand_int4

pytestmark = pytest.mark.gpu
TOL = 1e-3


def mlp_reference_order(ctx, x, rows, gate, up, down, hidden, inter):
    """LLM.pas:588-598: G := New; TrySwiGLUVector (one row); otherwise Release(G),
    G := Project(gate), U := Project(up), GO_SWIGLU in place; Y := Project(down)."""
    src = ctx.UploadRaw(x)
    g = ctx.NewTensor(rows * inter)
    if rows != 1 or not ctx.TrySwiGLUVector(g, src, gate, up, hidden, inter):
        ctx.Recycle(g)
        g = ctx.NewTensor(rows * inter)
        ctx.Int4Linear(g, src, gate, rows, hidden, inter)
        u = ctx.NewTensor(rows * inter)
        ctx.Int4Linear(u, src, up, rows, hidden, inter)
        ctx.Kernel(hip.GO_SWIGLU, rows * inter, g, g, u, None, [inter, 0])
    y = ctx.NewTensor(rows * hidden)
    ctx.Int4Linear(y, g, down, rows, inter, hidden)
    out = ctx.Download(y).reshape(rows, hidden)
    for t in (src, g, y):
        ctx.Recycle(t)
    return out


@pytest.mark.parametrize("rows", [1, 8])
def test_mlp_in_engine_order_fuses_and_matches(ctx, rng, tune, rows):
    hidden, inter = 2560, 9728
    pg, pu, pd = rand_int4(rng, inter, hidden), rand_int4(rng, inter, hidden), rand_int4(rng, hidden, inter)
    gate, up, down = (hip.MemoryBlock.int4(p) for p in (pg, pu, pd))
    x = rng.standard_normal((rows, hidden)).astype(np.float32)
    s0 = ctx.status()
    fused = mlp_reference_order(ctx, x, rows, gate, up, down, hidden, inter)
    s1 = ctx.status()
    if rows == 1:
        assert s1.mlp_fused - s0.mlp_fused == 1  # gate/up SwiGLU + down: one launch
    else:
        assert s1.glu_fused - s0.glu_fused == 1  # gate + up + in-place GO_SWIGLU: one launch
    tune("QNN_FUSE_MLP", "0")
    plain = mlp_reference_order(ctx, x, rows, gate, up, down, hidden, inter)
    s2 = ctx.status()
    assert s2.mlp_fused == s1.mlp_fused and s2.glu_fused == s1.glu_fused
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    for r in range(rows):
        want = oracle.cpu_mlp(pg, pu, pd, oracle.ENC_INT4, x[r], hidden, inter)[0]
        assert normwise_rel_err(fused[r], want) <= TOL, r


def test_gemma_layer_in_engine_order_groups(ctx, rng, tune):
    """Gemma2.pas:160-188 at batch 1: Project (New + Linear) for q, k, v, then
    gate and up, GO_GEGLU in place, down.  q+k+v share a launch, gate+up+GEGLU
    run as one, and every output equals the ungrouped path."""
    H, Q, KV, I = 1024, 1024, 512, 2816
    specs = {"q": (hip.WE_Q4_K, Q, H), "k": (hip.WE_Q3_K, KV, H), "v": (hip.WE_Q3_K, KV, H),
             "gate": (hip.WE_Q2_K, I, H), "up": (hip.WE_Q2_K, I, H), "down": (hip.WE_Q6_K, H, I)}
    data = {nm: hip.gguf_quantize(e, (rng.standard_normal(n * k) * 0.02).astype(np.float32))
            for nm, (e, n, k) in specs.items()}
    ws = {nm: hip.MemoryBlock.gguf(data[nm], n, k, e) for nm, (e, n, k) in specs.items()}
    x = rng.standard_normal(H).astype(np.float32)

    def layer():
        n_ = ctx.UploadRaw(x)
        outs = {}
        for nm in ("q", "k", "v"):
            e, n, k = specs[nm]
            outs[nm] = ctx.NewTensor(n)
            ctx.Linear(outs[nm], n_, ws[nm], None, None, 1, k, n)
        for nm in ("gate", "up"):
            e, n, k = specs[nm]
            outs[nm] = ctx.NewTensor(n)
            ctx.Linear(outs[nm], n_, ws[nm], None, None, 1, k, n)
        ctx.Kernel(hip.GO_GEGLU, I, outs["gate"], outs["gate"], outs["up"], None, [I, 0])
        y = ctx.NewTensor(H)
        ctx.Linear(y, outs["gate"], ws["down"], None, None, 1, I, H)
        res = {nm: ctx.Download(t) for nm, t in list(outs.items()) + [("down", y)]}
        for t in list(outs.values()) + [y, n_]:
            ctx.Recycle(t)
        return res

    s0 = ctx.status()
    grouped = layer()
    s1 = ctx.status()
    assert s1.linear_grouped - s0.linear_grouped == 3
    assert s1.glu_fused - s0.glu_fused == 1
    tune("QNN_GROUP_LINEAR", "0")
    plain = layer()
    for nm in grouped:
        assert np.array_equal(grouped[nm].view(np.uint32), plain[nm].view(np.uint32)), nm
    g = oracle.cpu_linear(data["gate"], hip.WE_Q2_K, x, H, I)
    c = np.float32(0.7978845608)
    u = oracle.cpu_linear(data["up"], hip.WE_Q2_K, x, H, I)
    h = (0.5 * g * (1 + np.tanh(c * (g + np.float32(0.044715) * g ** 3))) * u).astype(np.float32)
    assert normwise_rel_err(grouped["down"], oracle.cpu_linear(data["down"], hip.WE_Q6_K, h, I, H)) <= TOL


class MoELayer:
    """Qwen3-30B-A3B expert shapes (128 experts, hidden 2048, intermediate 768,
    top 8) with an F32 or BF16 router [128, 2048]."""

    def __init__(self, seed, bf16_router):
        rng = np.random.default_rng(seed)
        self.E, self.H, self.I, self.k = 128, 2048, 768, 8
        self.g = [rand_int4(rng, self.I, self.H) for _ in range(self.E)]
        self.u = [rand_int4(rng, self.I, self.H) for _ in range(self.E)]
        self.d = [rand_int4(rng, self.H, self.I) for _ in range(self.E)]
        self.bg, self.bu, self.bd = ([hip.MemoryBlock.int4(p) for p in ps] for ps in (self.g, self.u, self.d))
        r = (rng.standard_normal((self.E, self.H)) * 0.02).astype(np.float32)
        if bf16_router:
            self.router = hip.MemoryBlock.matrix(bf16_bits(r))
            self.r64 = bf16_to_f32(bf16_bits(r)).astype(np.float64)
        else:
            self.router = hip.MemoryBlock.matrix(r)
            self.r64 = r.astype(np.float64)

    def forward(self, ctx, src, rows):
        """TLLMMoE.forward (LLM.MoE.pas:357-448) in its call order."""
        E, H, I, k = self.E, self.H, self.I, self.k
        logits = ctx.NewTensor(rows * E)
        if rows == 1:
            ctx.VectorLinear(logits, src, self.router, H, E)
        else:
            ctx.Linear(logits, src, self.router, None, None, rows, H, E)
        ctx.CheckFinite(logits)
        routes = ctx.NewTensor(rows * k * 2)
        ctx.Kernel(hip.GO_MOE_ROUTE, routes.count, routes, logits, None, None, [rows, E, k, 1])
        host = ctx.Download(routes, rows * k).view(np.uint32).copy()
        counts = np.bincount(host, minlength=E)
        offsets = np.concatenate([[0], np.cumsum(counts)[:-1]])
        indices = None
        if rows > 1:
            order = np.argsort(host, kind="stable").astype(np.uint32)
            indices = ctx.UploadRaw(order.view(np.float32))
        out = ctx.NewTensor(rows * H)
        filled = False
        for e in range(E):
            c = int(counts[e])
            if c == 0:
                continue
            if not filled:
                ctx.Kernel(hip.GO_FILL, out.count, out, None, None, None, [0])
                filled = True
            if rows == 1:
                gathered, route_index = src, int(np.nonzero(host == e)[0][0])
            else:
                gathered, route_index = ctx.NewTensor(c * H), 0
                ctx.Kernel(hip.GO_MOE_GATHER, gathered.count, gathered, src, indices, None, [H, k, int(offsets[e])])
            g = ctx.NewTensor(c * I)
            if c != 1 or not ctx.TrySwiGLUVector(g, gathered, self.bg[e], self.bu[e], H, I):
                ctx.Recycle(g)
                g = ctx.NewTensor(c * I)
                ctx.Int4Linear(g, gathered, self.bg[e], c, H, I)
                u = ctx.NewTensor(c * I)
                ctx.Int4Linear(u, gathered, self.bu[e], c, H, I)
                ctx.Kernel(hip.GO_SWIGLU, c * I, g, g, u, None, [I, 0])
            if rows == 1:
                ctx.Int4LinearAccumulate(out, g, routes, self.bd[e], I, H, rows * k + route_index)
            else:
                y = ctx.NewTensor(c * H)
                ctx.Int4Linear(y, g, self.bd[e], c, I, H)
                ctx.Kernel(hip.GO_MOE_SCATTER, y.count, out, y, indices, routes,
                           [H, k, int(offsets[e]), route_index, int(rows == 1), rows * k])
        raw_logits = ctx.Download(logits).reshape(rows, E)
        raw_routes = ctx.Download(routes)
        return ctx.Download(out).reshape(rows, H), raw_logits, raw_routes


@pytest.mark.parametrize("bf16_router", [False, True], ids=["f32-router", "bf16-router"])
@pytest.mark.parametrize("rows", [1, 16])
def test_moe_forward_from_router_matches_cpu(ctx, rng, bf16_router, rows):
    lay = MoELayer(31 + rows, bf16_router)
    x = rng.standard_normal((rows, lay.H)).astype(np.float32)
    src = ctx.UploadRaw(x)
    got, logits, routes = lay.forward(ctx, src, rows)
    k = lay.k
    # router: fp32 sums of the same values, against float64
    want_logits = x.astype(np.float64) @ lay.r64.T
    for r in range(rows):
        assert normwise_rel_err(logits[r], want_logits[r]) <= 1e-5, r
    # route op on the device's logits: identical to the oracle's rule
    ids = routes[:rows * k].view(np.uint32).reshape(rows, k)
    probs = routes[rows * k:].reshape(rows, k)
    want_ids, want_p = oracle.moe_route(logits, k, True)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(probs.view(np.uint32), want_p.view(np.uint32))
    # the experts: composed CPU path over the same routes
    want = oracle.cpu_moe(lay.g, lay.u, lay.d, x, ids, probs, lay.H, lay.I)
    for r in range(rows):
        assert normwise_rel_err(got[r], want[r]) <= TOL, r
    # and the routes match the ones float64 logits give, where no two probabilities are close
    ref_ids, ref_p = oracle.moe_route(want_logits.astype(np.float32), k + 1, False)
    for r in range(rows):
        if ref_p[r, k - 1] > ref_p[r, k] * (1 + 1e-4):
            assert sorted(ids[r].tolist()) == sorted(ref_ids[r, :k].tolist()), r
    ctx.Recycle(src)


def test_recorded_multi_row_linear_runs_before_moe_experts(ctx, rng, tune):
    """A multi-row Int4Linear into T may be recorded (to meet a GO_SWIGLU); a
    following qnn_moe_experts(src=T) must see T written."""
    E, H, I, k, rows = 4, 256, 128, 2, 3
    gs = [rand_int4(rng, I, H) for _ in range(E)]
    us = [rand_int4(rng, I, H) for _ in range(E)]
    ds = [rand_int4(rng, H, I) for _ in range(E)]
    s = ctx.CreateExpertSet(*([hip.MemoryBlock.int4(p) for p in ps] for ps in (gs, us, ds)), H, I)
    pre = rand_int4(rng, H, H)
    x = rng.standard_normal((rows, H)).astype(np.float32)
    logits = rng.standard_normal((rows, E)).astype(np.float32)

    def run():
        xt, lt = ctx.UploadRaw(x), ctx.UploadRaw(logits)
        routes = ctx.NewTensor(2 * rows * k)
        ctx.Kernel(hip.GO_MOE_ROUTE, routes.count, routes, lt, None, None, [rows, E, k, 1])
        t = ctx.NewTensor(rows * H)
        ctx.Int4Linear(t, xt, hip.MemoryBlock.int4(pre, identity=991), rows, H, H)
        out = ctx.NewTensor(rows * H)
        ctx.MoEExperts(s, out, t, routes, rows, k)
        res = ctx.Download(out).reshape(rows, H), ctx.Download(t).reshape(rows, H), ctx.Download(routes)
        for tt in (xt, lt, routes, t, out):
            ctx.Recycle(tt)
        return res

    got, tvals, routes = run()
    tune("QNN_FUSE_MLP", "0")
    plain, _, _ = run()
    ctx.DestroyExpertSet(s)
    assert np.array_equal(got.view(np.uint32), plain.view(np.uint32))
    ids = routes[:rows * k].view(np.uint32).reshape(rows, k)
    probs = routes[rows * k:].reshape(rows, k)
    want = oracle.cpu_moe(gs, us, ds, tvals, ids, probs, H, I)
    for r in range(rows):
        assert normwise_rel_err(got[r], want[r]) <= TOL, r
