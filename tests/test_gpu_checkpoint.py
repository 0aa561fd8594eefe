"""Checkpoint files feed the kernels.

Weights read through the library's loaders -- an INT4 cache built from a BF16
safetensors checkpoint, an F32/BF16 router from safetensors, K-quant matrices
from a GGUF file -- give the same device results as the same bytes handed over
in memory, and match the CPU oracle on the oracle's own packing of the source
values (normwise relative error <= 1e-3, as every matvec test here).
"""
import os

import numpy as np
import pytest

import oracle
from quicknn_amd import hip
from tests.conftest import normwise_rel_err
from tests.gguf_writer import STRING, gguf_bytes

ck = pytest.importorskip("quicknn_amd.checkpoint")
pytestmark = pytest.mark.gpu
TOL = 1e-3


def torch_bf16_bits(v: np.ndarray) -> np.ndarray:
    import torch

    return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(
        np.uint16)


def run_int4(ctx, w: hip.MemoryBlock, x: np.ndarray, rows: int, k: int, n: int) -> np.ndarray:
    src = ctx.UploadRaw(x.reshape(-1))
    dst = ctx.NewTensor(rows * n)
    ctx.Int4Linear(dst, src, w, rows, k, n)
    out = ctx.Download(dst).reshape(rows, n)
    ctx.Recycle(src)
    ctx.Recycle(dst)
    return out


def test_int4_cache_feeds_int4_linear(ctx, tmp_path, rng):
    torch = pytest.importorskip("torch")
    import safetensors.torch as stt

    hidden, inter = 2048, 768  # Qwen3-30B-A3B expert shapes
    vals = {}
    for e in range(2):
        for proj, shape in (("gate_proj", (inter, hidden)), ("up_proj", (inter, hidden)),
                            ("down_proj", (hidden, inter))):
            vals[f"model.layers.0.mlp.experts.{e}.{proj}.weight"] = (rng.standard_normal(shape) * 0.02).astype(
                np.float32)
    p = os.path.join(tmp_path, "model.safetensors")
    stt.save_file({k: torch.from_numpy(v).to(torch.bfloat16) for k, v in vals.items()}, p)
    with ck.SafeTensorFiles.Open(p) as src, ck.LLMInt4Cache(src, os.path.join(tmp_path, "cache")) as cache:
        for name, v in vals.items():
            n, k = v.shape
            packed = oracle.quantize_int4(torch_bf16_bits(v))
            w = cache.Weight(name, n, k)
            assert np.array_equal(w.data.reshape(packed.shape), packed)
            for rows in (1, 4):
                x = rng.standard_normal((rows, k)).astype(np.float32)
                got = run_int4(ctx, w, x, rows, k, n)
                mem = run_int4(ctx, hip.MemoryBlock.int4(packed), x, rows, k, n)
                assert np.array_equal(got.view(np.uint32), mem.view(np.uint32)), (name, rows)
                for r in range(rows):
                    want = oracle.cpu_linear(packed, oracle.ENC_INT4, x[r], k, n)
                    assert normwise_rel_err(got[r], want) <= TOL, (name, rows, r)


@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
def test_router_weight_feeds_vector_linear(ctx, tmp_path, rng, bf16):
    torch = pytest.importorskip("torch")
    import safetensors.torch as stt

    e, hidden = 128, 2048
    v = rng.standard_normal((e, hidden)).astype(np.float32) * 0.05
    t = torch.from_numpy(v)
    p = os.path.join(tmp_path, "router.safetensors")
    stt.save_file({"model.layers.0.mlp.gate.weight": t.to(torch.bfloat16) if bf16 else t}, p)
    wv = (torch_bf16_bits(v).astype(np.uint32) << 16).view(np.float32) if bf16 else v
    with ck.SafeTensorFiles.Open(p) as f:
        w = f.GetLinearWeight("model.layers.0.mlp.gate.weight")
        assert w.dtype == (hip.DT_BF16 if bf16 else hip.DT_F32) and w.shape == (e, hidden)
        x = rng.standard_normal(hidden).astype(np.float32)
        src = ctx.UploadRaw(x)
        dst = ctx.NewTensor(e)
        ctx.VectorLinear(dst, src, w, hidden, e)
        got = ctx.Download(dst)
        want = wv.astype(np.float64) @ x.astype(np.float64)
        assert normwise_rel_err(got, want) <= TOL
        ctx.Recycle(src)
        ctx.Recycle(dst)


# GGML storage type of each encoding (GGUF.Quantization.pas:44-60).
GGML_TYPE = {oracle.ENC_Q8_0: 8, oracle.ENC_Q4_K: 12, oracle.ENC_Q6_K: 14, oracle.ENC_Q3_K: 11, oracle.ENC_Q2_K: 10,
             oracle.ENC_Q5_K: 13, oracle.ENC_IQ4_NL: 20, oracle.ENC_IQ4_XS: 23, oracle.ENC_Q2_0: 42,
             oracle.ENC_IQ2_XXS: 16, oracle.ENC_IQ2_S: 22, oracle.ENC_IQ3_XXS: 18, oracle.ENC_IQ3_S: 21}


def test_gguf_file_feeds_linear(ctx, tmp_path, rng):
    shapes = {oracle.ENC_Q4_K: (512, 3584), oracle.ENC_Q6_K: (300, 3584), oracle.ENC_Q8_0: (256, 3072),
              oracle.ENC_Q3_K: (128, 3584), oracle.ENC_Q2_K: (200, 14336), oracle.ENC_Q5_K: (96, 2048),
              oracle.ENC_IQ4_NL: (70, 1056), oracle.ENC_IQ4_XS: (64, 2048), oracle.ENC_Q2_0: (33, 1088),
              oracle.ENC_IQ2_XXS: (64, 1024), oracle.ENC_IQ2_S: (40, 768), oracle.ENC_IQ3_XXS: (80, 1024),
              oracle.ENC_IQ3_S: (50, 1280)}
    blocks, tensors = {}, []
    for enc, (n, k) in shapes.items():
        blocks[enc] = hip.gguf_quantize(enc, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        tensors.append((f"blk.0.w{enc}.weight", [k, n], GGML_TYPE[enc], blocks[enc].tobytes(), None))
    p = os.path.join(tmp_path, "m.gguf")
    with open(p, "wb") as f:
        f.write(gguf_bytes([("general.architecture", STRING, "gemma2")], tensors))
    with ck.SafeTensorFiles.Open(p) as files:
        for enc, (n, k) in shapes.items():
            w = files.GetLinearWeight(f"blk.0.w{enc}.weight")
            assert (w.encoding, w.shape, w.size) == (enc, (n, k), n * k)
            x = rng.standard_normal(k).astype(np.float32)
            src = ctx.UploadRaw(x)
            outs = []
            for blk in (w, hip.MemoryBlock.gguf(blocks[enc], n, k, enc)):
                dst = ctx.NewTensor(n)
                ctx.Linear(dst, src, blk, None, None, 1, k, n)
                outs.append(ctx.Download(dst))
                ctx.Recycle(dst)
            assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), enc
            want = oracle.cpu_linear(blocks[enc], enc, x, k, n)
            assert normwise_rel_err(outs[0], want) <= TOL, enc
            ctx.Recycle(src)
