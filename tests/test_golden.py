"""Regression tests against the committed golden vectors (tests/golden/*.json,
written by tests/golden/make_golden.py).

CPU side: the oracle's three GGUF decoders, its INT4 packer and dequant, its
CPU projection and its route op reproduce the frozen words bit for bit; the
backend's host encoders (qnn_quantize_int4, qnn_gguf_quantize) reproduce the
frozen bytes and SHA-256 digests; and each frozen matvec output stays within
one fp32 rounding chain of a float64 brute force over the frozen weights, so
the fixtures themselves are pinned by arithmetic, not only by the oracle that
wrote them.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from tests.conftest import normwise_rel_err

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ENC = {"Q8_0": oracle.ENC_Q8_0, "Q4_K": oracle.ENC_Q4_K, "Q6_K": oracle.ENC_Q6_K, "Q3_K": oracle.ENC_Q3_K,
       "Q2_K": oracle.ENC_Q2_K, "Q5_K": oracle.ENC_Q5_K, "IQ4_NL": oracle.ENC_IQ4_NL, "IQ4_XS": oracle.ENC_IQ4_XS,
       "Q2_0": oracle.ENC_Q2_0, "IQ2_XXS": oracle.ENC_IQ2_XXS, "IQ2_S": oracle.ENC_IQ2_S,
       "IQ3_XXS": oracle.ENC_IQ3_XXS, "IQ3_S": oracle.ENC_IQ3_S}
ELEMS = {"Q8_0": 32, "Q4_K": 256, "Q6_K": 256, "Q3_K": 256, "Q2_K": 256, "Q5_K": 256, "IQ4_NL": 32, "IQ4_XS": 256,
         "Q2_0": 64, "IQ2_XXS": 256, "IQ2_S": 256, "IQ3_XXS": 256, "IQ3_S": 256}


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def f32(h):
    return np.frombuffer(bytes.fromhex(h), np.float32).copy()


def u8(h):
    return np.frombuffer(bytes.fromhex(h), np.uint8).copy()


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_int4_blocks():
    from quicknn_amd import hip

    for case in load("blocks.json")["INT4"]:
        dt = np.uint16 if case["dtype"] == "bf16" else np.float32
        src = np.frombuffer(bytes.fromhex(case["input_hex"]), dt).reshape(1, case["cols"])
        packed = u8(case["packed_hex"]).reshape(1, -1)
        assert np.array_equal(oracle.quantize_int4(src), packed), case["name"]
        assert np.array_equal(hip.quantize_int4(src), packed), case["name"]
        assert same_bits(oracle.int4_dequant(packed, case["cols"])[0], f32(case["values_hex"])), case["name"]
    tie = load("blocks.json")["INT4"][1]
    nib = u8(tie["packed_hex"])[4:20]
    assert (int(nib[5 // 2]) >> 4) & 15 == 8 - 4  # element 5: -3.5 steps rounded half to even


@pytest.mark.parametrize("fmt", list(ENC))
def test_gguf_blocks_three_decoders(fmt):
    enc, n = ENC[fmt], ELEMS[fmt]
    for case in load("blocks.json")[fmt]:
        b, want = u8(case["bytes_hex"]), f32(case["values_hex"])
        assert same_bits(oracle.gguf_dequant_scalar(b, enc, n), want), (fmt, case["name"])
        assert same_bits(oracle.gguf_read4_all(b, enc, n), want), (fmt, case["name"])
        # The AVX2 block decode adds a +0 bias (GGUF.Quantization.pas:291, :335), so where
        # (d*sc)*(q-center) is -0 it writes +0: equal values, the sign of zero may differ.
        blk = oracle.gguf_dequantize(b, enc, n)
        assert np.array_equal(blk, want) and not np.isnan(blk).any(), (fmt, case["name"])


@pytest.mark.parametrize("fmt", ["INT4"] + list(ENC))
def test_matvec(fmt):
    m = load("matvec.json")[fmt]
    rows, cols = m["rows"], m["cols"]
    w, x, y = u8(m["w_hex"]), f32(m["x_hex"]), f32(m["y_hex"])
    enc = oracle.ENC_INT4 if fmt == "INT4" else ENC[fmt]
    got = oracle.cpu_linear(w.reshape(rows, -1) if fmt == "INT4" else w, enc, x, cols, rows)
    assert same_bits(got, y)
    wd = oracle.int4_dequant(w.reshape(rows, -1), cols) if fmt == "INT4" else \
        oracle.gguf_dequantize(w, enc, rows * cols).reshape(rows, cols)
    assert normwise_rel_err(y, wd.astype(np.float64) @ x.astype(np.float64)) < 1e-5


def test_moe_route():
    r = load("moe_route.json")
    logits = f32(r["logits_hex"]).reshape(r["rows"], r["experts"])
    ids, probs = oracle.moe_route(logits, r["topk"], bool(r["normalize"]))
    assert ids.astype(int).tolist() == r["ids"]
    assert same_bits(probs.ravel(), f32(r["probs_hex"]))
    for row in range(r["rows"]):  # ranking by logit, ties to the lower id
        assert r["ids"][row] == np.argsort(-logits[row].astype(np.float64), kind="stable")[:r["topk"]].tolist()


def test_sha256_of_seeded_weight_sets():
    from quicknn_amd import hip

    d = load("sha256.json")
    rng = np.random.default_rng(1000)
    shapes = d["int4_qwen3_4b_layer0_seed1000"]["shapes"]
    for (n, k), digest in zip(shapes, d["int4_qwen3_4b_layer0_seed1000"]["sha256"]):
        m = rng.standard_normal((n, k), dtype=np.float32)
        m *= np.float32(0.02)
        b = (m.view(np.uint32) >> 16).astype(np.uint16)
        assert hashlib.sha256(hip.quantize_int4(b).tobytes()).hexdigest() == digest
        if n == 2560:  # one oracle pass as well (the packers agree on the largest matrix)
            assert hashlib.sha256(oracle.quantize_int4(b).tobytes()).hexdigest() == digest
    for key, entry in d.items():
        if key.startswith("int4_"):
            continue
        fmt, seed = key.split("_")[0] + "_" + key.split("_")[1], int(key.rsplit("seed", 1)[1])
        n, k = entry["shape"]
        w = np.random.default_rng(seed).standard_normal(n * k, dtype=np.float32) * np.float32(0.02)
        assert hashlib.sha256(hip.gguf_quantize(ENC[fmt], w).tobytes()).hexdigest() == entry["sha256"], key
