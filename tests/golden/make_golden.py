#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ (run from the repository root).

The reference's own test vectors are not part of its source snapshot, so these
fixtures are produced by this repository's pinned CPU oracle (oracle/, checked
against known answers, invariants and brute force in tests/test_oracle_*.py)
and by the backend's host-side encoders (the reference ships no GGUF
quantizer).  They freeze, per format:

  blocks.json   - a few blocks (one drawn from N(0, 0.02) through the encoder,
                  one of random bytes with finite fp16 scale fields, and for
                  INT4 a hand-built tie case) with their dequantised fp32 words;
  matvec.json   - one 64-row matvec per format: packed weight, x, and the
                  reference CPU path's y (TCPUProjection.Linear restated);
  moe_route.json- GO_MOE_ROUTE over 2 tokens x 128 experts, top-8 renormalised;
  sha256.json   - SHA-256 of larger seeded weight sets (the benchmark's first
                  INT4 layer and one K-quant matrix per format).

Floats are stored as hex of their IEEE-754 little-endian bytes, so the files
compare bit for bit.  Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from quicknn_amd import hip  # noqa: E402  (host encoders only; no device use)

OUT = os.path.dirname(os.path.abspath(__file__))

# (encoding, name, block elements, block bytes, byte offsets of fp16 scale fields)
FORMATS = [
    (oracle.ENC_Q8_0, "Q8_0", 32, 34, (0,)),
    (oracle.ENC_Q4_K, "Q4_K", 256, 144, (0, 2)),
    (oracle.ENC_Q6_K, "Q6_K", 256, 210, (208,)),
    (oracle.ENC_Q3_K, "Q3_K", 256, 110, (108,)),
    (oracle.ENC_Q2_K, "Q2_K", 256, 84, (80, 82)),
]
# Formats added later draw from their own random stream, so the fixtures of
# the formats above stay as they were.
FORMATS_EXT = [
    (oracle.ENC_Q5_K, "Q5_K", 256, 176, (0, 2)),
    (oracle.ENC_IQ4_NL, "IQ4_NL", 32, 18, (0,)),
    (oracle.ENC_IQ4_XS, "IQ4_XS", 256, 136, (0,)),
]
FORMATS_EXT2 = [
    (oracle.ENC_Q2_0, "Q2_0", 64, 18, (0,)),
]
FORMATS_EXT3 = [
    (oracle.ENC_IQ2_XXS, "IQ2_XXS", 256, 66, (0,)),
    (oracle.ENC_IQ2_S, "IQ2_S", 256, 82, (0,)),
    (oracle.ENC_IQ3_XXS, "IQ3_XXS", 256, 98, (0,)),
    (oracle.ENC_IQ3_S, "IQ3_S", 256, 110, (0,)),
]


def hexf(a) -> str:
    return np.ascontiguousarray(a, np.float32).tobytes().hex()


def hexb(a) -> str:
    return np.ascontiguousarray(a, np.uint8).tobytes().hex()


def bf16(x: np.ndarray) -> np.ndarray:
    """SingleToBF16 truncation (src/core/QuickNN.Common.pas:1779-1797)."""
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def random_block(rng, nbytes: int, half_offsets) -> np.ndarray:
    b = rng.integers(0, 256, nbytes, dtype=np.uint8)
    for off in half_offsets:  # finite fp16 in [2^-14, 2^-2): exponent field 1..12
        h = (int(rng.integers(1, 13)) << 10) | int(rng.integers(0, 1024)) | (int(rng.integers(0, 2)) << 15)
        b[off:off + 2] = np.array([h], np.uint16).view(np.uint8)
    return b


def blocks(rng) -> dict:
    out = {}
    # INT4: two 32-groups from bf16 N(0, 0.02), and one group of multiples of
    # 1/64 (max 7/64, so the first scale is 1/64) with one element at exactly
    # -3.5 steps, which rounds half to even (to -4) before the refit.
    w = bf16(rng.standard_normal((1, 64)).astype(np.float32) * np.float32(0.02))
    tie = np.array([[(k % 15 - 7) / 64.0 for k in range(32)]], np.float32)
    tie[0, 5] = np.float32(-7.0 / 64 * 0.5)  # exactly half a step: rounds to even
    cases = []
    for name, src in (("bf16_normal", w), ("f32_grid_tie", tie)):
        packed = oracle.quantize_int4(src)
        cols = src.shape[1]
        cases.append({"name": name, "dtype": "bf16" if src.dtype == np.uint16 else "f32",
                      "cols": cols, "input_hex": src.tobytes().hex(), "packed_hex": hexb(packed),
                      "values_hex": hexf(oracle.int4_dequant(packed, cols)[0])})
    out["INT4"] = cases
    out.update(gguf_blocks(rng, FORMATS))
    return out


def gguf_blocks(rng, formats) -> dict:
    out = {}
    for enc, name, elems, nbytes, halves in formats:
        enc_block = hip.gguf_quantize(enc, (rng.standard_normal(elems) * 0.02).astype(np.float32))
        rnd = random_block(rng, nbytes, halves)
        cases = []
        for cname, b in (("encoded_normal", enc_block), ("random_bytes", rnd)):
            cases.append({"name": cname, "bytes_hex": hexb(b),
                          "values_hex": hexf(oracle.gguf_dequant_scalar(b, enc, elems))})
        out[name] = cases
    return out


def matvecs(rng) -> dict:
    out = {}
    k = 64
    w = bf16(rng.standard_normal((64, k)).astype(np.float32) * np.float32(0.02))
    packed = oracle.quantize_int4(w)
    x = rng.standard_normal(k).astype(np.float32)
    y = oracle.cpu_linear(packed, oracle.ENC_INT4, x, k, 64)
    out["INT4"] = {"rows": 64, "cols": k, "w_hex": hexb(packed), "x_hex": hexf(x), "y_hex": hexf(y)}
    out.update(gguf_matvecs(rng, FORMATS))
    return out


def gguf_matvecs(rng, formats) -> dict:
    out = {}
    for enc, name, elems, nbytes, _ in formats:
        kk = max(64, elems)
        wb = hip.gguf_quantize(enc, (rng.standard_normal(64 * kk) * 0.02).astype(np.float32))
        x = rng.standard_normal(kk).astype(np.float32)
        y = oracle.cpu_linear(wb, enc, x, kk, 64)
        out[name] = {"rows": 64, "cols": kk, "w_hex": hexb(wb), "x_hex": hexf(x), "y_hex": hexf(y)}
    return out


def moe_route(rng) -> dict:
    logits = rng.standard_normal((2, 128)).astype(np.float32)
    ids, probs = oracle.moe_route(logits, 8, True)
    return {"rows": 2, "experts": 128, "topk": 8, "normalize": 1, "logits_hex": hexf(logits),
            "ids": ids.astype(int).tolist(), "probs_hex": hexf(probs)}


def bench_layer0() -> list:
    """The benchmark's layer 0 (seed 1000): gate, up [9728, 2560], down [2560, 9728]."""
    r = np.random.default_rng(1000)

    def mat(n, kk):
        m = r.standard_normal((n, kk), dtype=np.float32)
        m *= np.float32(0.02)
        return oracle.quantize_int4(bf16(m))

    return [mat(9728, 2560), mat(9728, 2560), mat(2560, 9728)]


def sha256s() -> dict:
    out = {"int4_qwen3_4b_layer0_seed1000": {
        "shapes": [[9728, 2560], [9728, 2560], [2560, 9728]],
        "sha256": [hashlib.sha256(m.tobytes()).hexdigest() for m in bench_layer0()]}}
    for enc, name, elems, nbytes, _ in FORMATS + FORMATS_EXT + FORMATS_EXT2 + FORMATS_EXT3:
        r = np.random.default_rng(2000 + enc)
        n, kk = 512, 3584 if elems == 256 else 3072
        w = (r.standard_normal(n * kk, dtype=np.float32) * np.float32(0.02))
        out[f"{name}_{n}x{kk}_seed{2000 + enc}"] = {
            "shape": [n, kk], "sha256": hashlib.sha256(hip.gguf_quantize(enc, w).tobytes()).hexdigest()}
    return out


def main() -> None:
    rng = np.random.default_rng(20240601)
    files = {"blocks.json": blocks(rng), "matvec.json": matvecs(rng), "moe_route.json": moe_route(rng),
             "sha256.json": sha256s()}
    rng_ext = np.random.default_rng(20261202)
    files["blocks.json"].update(gguf_blocks(rng_ext, FORMATS_EXT))
    files["matvec.json"].update(gguf_matvecs(rng_ext, FORMATS_EXT))
    rng_ext2 = np.random.default_rng(20261215)
    files["blocks.json"].update(gguf_blocks(rng_ext2, FORMATS_EXT2))
    files["matvec.json"].update(gguf_matvecs(rng_ext2, FORMATS_EXT2))
    rng_ext3 = np.random.default_rng(20261216)
    files["blocks.json"].update(gguf_blocks(rng_ext3, FORMATS_EXT3))
    files["matvec.json"].update(gguf_matvecs(rng_ext3, FORMATS_EXT3))
    for fname, data in files.items():
        with open(os.path.join(OUT, fname), "w") as f:
            json.dump(data, f, indent=1)
            f.write("\n")
        print("wrote", fname)


if __name__ == "__main__":
    main()
