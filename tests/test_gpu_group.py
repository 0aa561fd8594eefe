"""GPU tests of grouped one-row GGUF Linear launches.

Consecutive one-row Linear calls on the same input with the same encoding (a
layer's k/v or gate/up projections) are recorded and run as one launch.  Each
output must be bit-identical to its own launch (QNN_GROUP_LINEAR=0) and within
1e-3 normwise of the reference CPU path; anything that is not such a call
(another input, a Download, another op) launches what was recorded first.
"""
import numpy as np
import pytest

import oracle
from tests.conftest import normwise_rel_err

pytestmark = pytest.mark.gpu


def mats(rng, hip, specs):
    out = {}
    for name, enc, n, k in specs:
        w = (rng.standard_normal(n * k) * 0.02).astype(np.float32)
        out[name] = (hip.MemoryBlock.gguf(hip.gguf_quantize(enc, w), n, k, enc), enc, n, k)
    return out


def gemma_like(ctx, hip, ws, x0):
    H = 1024
    x = ctx.UploadRaw(x0)
    outs = {name: ctx.NewTensor(n) for name, (_, _, n, _) in ws.items()}
    # q, k, v, gate, up on x (k+v and gate+up group), o on q (a different input)
    for name in ("q", "k", "v", "gate", "up"):
        w, enc, n, k = ws[name]
        ctx.Linear(outs[name], x, w, None, None, 1, k, n)
    w, enc, n, k = ws["o"]
    ctx.Linear(outs["o"], outs["q"], w, None, None, 1, k, n)
    res = {name: ctx.Download(t) for name, t in outs.items()}
    for t in list(outs.values()) + [x]:
        ctx.Recycle(t)
    return res


def recorded_groups(encs):
    """Calls that share a launch when one-row K-quant Linear calls on one input
    (one unit per wave) are recorded in this order: a group takes up to four
    members of at most two encodings."""
    groups, cur = [], []
    for e in encs:
        if cur and (len(cur) == 4 or (e not in cur and len(set(cur)) == 2)):
            groups.append(cur)
            cur = []
        cur.append(e)
    groups.append(cur)
    return sum(len(g) for g in groups if len(g) > 1)


# q's encoding and k/v's: two K-quant encodings share one launch (k_gguf_matvec_mixed).
@pytest.mark.parametrize("eq,ekv", [(2, 4), (2, 3), (3, 9), (4, 2), (9, 3), (3, 2)],
                         ids=["q4k+q3k", "q4k+q6k", "q6k+q2k", "q3k+q4k", "q2k+q6k", "q6k+q4k"])
def test_grouped_equals_single(ctx, rng, tune, eq, ekv):
    from quicknn_amd import hip

    H = 1024
    ws = mats(rng, hip, [("q", eq, 1024, H), ("k", ekv, 512, H), ("v", ekv, 512, H),
                         ("o", hip.WE_Q4_K, H, 1024), ("gate", hip.WE_Q2_K, 2816, H), ("up", hip.WE_Q2_K, 2816, H)])
    x0 = rng.standard_normal(H).astype(np.float32)
    g0 = ctx.status().linear_grouped
    grouped = gemma_like(ctx, hip, ws, x0)
    want = recorded_groups([eq, ekv, ekv, hip.WE_Q2_K, hip.WE_Q2_K])
    assert ctx.status().linear_grouped - g0 == want  # e.g. q+k+v (two encodings) and gate+up
    tune("QNN_GROUP_LINEAR", "0")
    single = gemma_like(ctx, hip, ws, x0)
    assert ctx.status().linear_grouped - g0 == want
    for name in grouped:
        assert np.array_equal(grouped[name], single[name]), name
    for name in ("k", "gate"):
        w, enc, n, k = ws[name]
        want = oracle.cpu_linear(w.data, enc, x0, k, n)
        assert normwise_rel_err(grouped[name], want) < 1e-3, name


def test_group_limits_and_interleaving(ctx, rng):
    """Five matvecs on one input run as a group of four plus one; a repeated
    output tensor and an interleaved op each launch the recorded group first."""
    from quicknn_amd import hip

    H, N = 512, 320
    ws = mats(rng, hip, [(f"m{i}", hip.WE_Q6_K, N, H) for i in range(5)])
    x0 = rng.standard_normal(H).astype(np.float32)
    x = ctx.UploadRaw(x0)
    ys = [ctx.NewTensor(N) for _ in range(5)]
    want = [oracle.cpu_linear(ws[f"m{i}"][0].data, hip.WE_Q6_K, x0, H, N) for i in range(5)]
    g0 = ctx.status().linear_grouped
    for i in range(5):
        ctx.Linear(ys[i], x, ws[f"m{i}"][0], None, None, 1, H, N)
    got = [ctx.Download(y) for y in ys]
    assert ctx.status().linear_grouped - g0 == 4
    for i in range(5):
        assert normwise_rel_err(got[i], want[i]) < 1e-3, i
    # the same output twice: the second call must see the first one's result overwritten in order
    ctx.Linear(ys[0], x, ws["m0"][0], None, None, 1, H, N)
    ctx.Linear(ys[0], x, ws["m1"][0], None, None, 1, H, N)
    assert np.array_equal(ctx.Download(ys[0]), got[1])
    # an interleaved op between two recorded calls
    ctx.Linear(ys[2], x, ws["m2"][0], None, None, 1, H, N)
    ctx.Kernel(hip.GO_FILL, N, ys[3], None, None, None, [0])
    ctx.Linear(ys[4], x, ws["m4"][0], None, None, 1, H, N)
    assert np.array_equal(ctx.Download(ys[2]), got[2])
    assert np.array_equal(ctx.Download(ys[4]), got[4])
    assert not ctx.Download(ys[3]).any()
    for t in ys + [x]:
        ctx.Recycle(t)


@pytest.mark.parametrize("op_name,enc_name,inter,hidden", [("GO_GEGLU", "WE_Q2_K", 14336, 3584),
                                                             ("GO_GEGLU", "WE_Q4_K", 2816, 1024),
                                                             ("GO_SWIGLU", "WE_Q6_K", 1536, 512),
                                                             ("GO_SWIGLU", "WE_Q8_0", 1000, 768)])
def test_gate_up_glu_one_launch(ctx, rng, tune, op_name, enc_name, inter, hidden):
    """One-row GGUF Linear gate + up on the same input followed by a GLU of their two outputs
    run as one gate/up pair launch (qnn_status.glu_fused) that still writes both outputs; all
    three outputs are bit-identical to the grouped launch followed by the GLU kernel, and the
    projections (and the SwiGLU) are within 1e-3 of the CPU path."""
    from quicknn_amd import hip

    enc, op = getattr(hip, enc_name), getattr(hip, op_name)
    ws = mats(rng, hip, [("gate", enc, inter, hidden), ("up", enc, inter, hidden)])
    x0 = rng.standard_normal(hidden).astype(np.float32)

    def run():
        x = ctx.UploadRaw(x0)
        g, u, hh = ctx.NewTensor(inter), ctx.NewTensor(inter), ctx.NewTensor(inter)
        ctx.Linear(g, x, ws["gate"][0], None, None, 1, hidden, inter)
        ctx.Linear(u, x, ws["up"][0], None, None, 1, hidden, inter)
        ctx.Kernel(op, inter, hh, g, u, None, [inter, 0] if op_name == "GO_SWIGLU" else [inter])
        out = [ctx.Download(t).view(np.uint32).copy() for t in (g, u, hh)]
        for t in (x, g, u, hh):
            ctx.Recycle(t)
        return out

    n0 = ctx.status().glu_fused
    fused = run()
    n1 = ctx.status().glu_fused
    tune("QNN_GROUP_LINEAR", "0")
    sep = run()
    assert ctx.status().glu_fused == n1
    for a, b, nm in zip(fused, sep, ("gate", "up", "glu")):
        assert np.array_equal(a, b), nm
    if (enc_name, inter) == ("WE_Q2_K", 14336):  # the Gemma-2 layer shape: plans agree
        assert n1 - n0 == 1
    gw = oracle.cpu_linear(ws["gate"][0].data, enc, x0, hidden, inter)
    uw = oracle.cpu_linear(ws["up"][0].data, enc, x0, hidden, inter)
    assert normwise_rel_err(fused[0].view(np.float32), gw) < 1e-3
    assert normwise_rel_err(fused[1].view(np.float32), uw) < 1e-3
    if op_name == "GO_SWIGLU":
        silu = np.vectorize(oracle.silu, otypes=[np.float32])
        assert normwise_rel_err(fused[2].view(np.float32), silu(gw) * uw) < 1e-3
