"""GPU regression against the committed golden vectors (tests/golden/*.json).

The device-resident dequant of every frozen block must reproduce the frozen
fp32 words bit for bit (the scalar GGUFValue / readGGUF4 words, sign of zero
included); each frozen 64-row matvec must match the frozen reference-CPU output
within a normwise relative error of 1e-3; the frozen route case must select the
same expert ids, with weights within 2e-6 relative (device expf vs the host's).
"""
import numpy as np
import pytest

from tests.test_golden import ELEMS, ENC, f32, load, same_bits, u8
from tests.conftest import normwise_rel_err

pytestmark = pytest.mark.gpu


def test_int4_blocks_dequant(ctx):
    from quicknn_amd import hip

    for case in load("blocks.json")["INT4"]:
        packed = u8(case["packed_hex"]).reshape(1, -1)
        out = ctx.NewTensor(case["cols"])
        ctx.Dequantize(out, hip.MemoryBlock.int4(packed), 1, case["cols"])
        assert same_bits(ctx.Download(out), f32(case["values_hex"])), case["name"]
        ctx.Recycle(out)


@pytest.mark.parametrize("fmt", list(ENC))
def test_gguf_blocks_dequant(ctx, fmt):
    from quicknn_amd import hip

    for case in load("blocks.json")[fmt]:
        b = u8(case["bytes_hex"])
        out = ctx.NewTensor(ELEMS[fmt])
        ctx.Dequantize(out, hip.MemoryBlock.gguf(b, 1, ELEMS[fmt], ENC[fmt]), 1, ELEMS[fmt])
        assert same_bits(ctx.Download(out), f32(case["values_hex"])), (fmt, case["name"])
        ctx.Recycle(out)


@pytest.mark.parametrize("fmt", ["INT4"] + list(ENC))
def test_matvec(ctx, fmt):
    from quicknn_amd import hip

    m = load("matvec.json")[fmt]
    rows, cols = m["rows"], m["cols"]
    w, x, y = u8(m["w_hex"]), f32(m["x_hex"]), f32(m["y_hex"])
    xt, yt = ctx.UploadRaw(x), ctx.NewTensor(rows)
    if fmt == "INT4":
        ctx.Int4Linear(yt, xt, hip.MemoryBlock.int4(w.reshape(rows, -1)), 1, cols, rows)
    else:
        ctx.Linear(yt, xt, hip.MemoryBlock.gguf(w, rows, cols, ENC[fmt]), None, None, 1, cols, rows)
    assert normwise_rel_err(ctx.Download(yt), y) < 1e-3
    ctx.Recycle(xt)
    ctx.Recycle(yt)


def test_moe_route(ctx):
    from quicknn_amd import hip

    r = load("moe_route.json")
    rows, E, k = r["rows"], r["experts"], r["topk"]
    lt = ctx.UploadRaw(f32(r["logits_hex"]))
    routes = ctx.NewTensor(2 * rows * k)
    ctx.Kernel(hip.GO_MOE_ROUTE, 2 * rows * k, routes, lt, None, None, [rows, E, k, r["normalize"]])
    raw = ctx.Download(routes)
    assert raw[:rows * k].view(np.uint32).reshape(rows, k).astype(int).tolist() == r["ids"]
    want = f32(r["probs_hex"])
    assert np.array_equal(raw[rows * k:].view(np.uint32), want.view(np.uint32))
    ctx.Recycle(lt)
    ctx.Recycle(routes)
