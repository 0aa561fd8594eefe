"""Pins the GGUF part of the oracle (src/io/QuickNN.GGUF.Quantization.pas):
the three independent reference decoders (scalar GGUFValue :136-253, the AVX2
block decoders :274-368, the shader's readGGUF4 gguf.glsl:591-655) must agree
on random valid blocks; hand-built blocks give known answers from the format
definitions; the IQ2/IQ3 tables match digests of the reference's own tables
(tests/golden/iq_grids.json); the packed AVX2 dots agree with a
double-precision dot over the decoded weights; the product's block encoders
round-trip."""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

import oracle
from oracle import (ENC_IQ2_S, ENC_IQ2_XXS, ENC_IQ3_S, ENC_IQ3_XXS, ENC_IQ4_NL, ENC_IQ4_XS, ENC_Q2_0, ENC_Q2_K, ENC_Q3_K,
                    ENC_Q4_K, ENC_Q5_K, ENC_Q6_K, ENC_Q8_0, BLOCK_BYTES, BLOCK_ELEMENTS)

FMTS = [ENC_Q8_0, ENC_Q4_K, ENC_Q6_K, ENC_Q3_K, ENC_Q2_K, ENC_Q5_K, ENC_IQ4_NL, ENC_IQ4_XS, ENC_Q2_0, ENC_IQ2_XXS, ENC_IQ2_S,
        ENC_IQ3_XXS, ENC_IQ3_S]
# fp16 fields (byte offsets within a block)
HALF_FIELDS = {ENC_Q8_0: [0], ENC_Q4_K: [0, 2], ENC_Q6_K: [208], ENC_Q3_K: [108], ENC_Q2_K: [80, 82],
               ENC_Q5_K: [0, 2], ENC_IQ4_NL: [0], ENC_IQ4_XS: [0], ENC_Q2_0: [0], ENC_IQ2_XXS: [0], ENC_IQ2_S: [0],
               ENC_IQ3_XXS: [0], ENC_IQ3_S: [0]}
# IQ4_NL_VALUES (src/io/QuickNN.GGUF.Quantization.pas:34), typed in from the format definition
IQ4 = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def f16(v: float) -> int:
    return int(np.array([v], np.float16).view(np.uint16)[0])


def random_blocks(rng, enc: int, nblocks: int) -> np.ndarray:
    """Random bytes with every fp16 field replaced by a finite value (incl. negatives and subnormals)."""
    bb = BLOCK_BYTES[enc]
    b = rng.integers(0, 256, (nblocks, bb), dtype=np.uint8)
    for off in HALF_FIELDS[enc]:
        vals = rng.standard_normal(nblocks) * 0.01
        vals[::7] = 3.0e-6  # fp16 subnormal
        vals[1::11] = -vals[1::11]
        h = np.array(vals, np.float16).view(np.uint16)
        b[:, off] = h & 255
        b[:, off + 1] = h >> 8
    return b.reshape(-1)


def same_values(a: np.ndarray, b: np.ndarray) -> bool:
    """Equal as floats (+0 == -0; the reference's decoders differ only in the sign of zero)."""
    return bool(np.all(a == b)) and not np.any(np.isnan(a)) and not np.any(np.isnan(b))


def test_half_to_float_known_answers():
    assert oracle.half_to_float(0x3C00) == 1.0
    assert oracle.half_to_float(0xC000) == -2.0
    assert oracle.half_to_float(0x0001) == 2.0 ** -24
    assert oracle.half_to_float(0x03FF) == 1023 * 2.0 ** -24
    assert oracle.half_to_float(0x7BFF) == 65504.0
    assert np.isinf(oracle.half_to_float(0x7C00))
    for v in [0.5, -3.25, 1e-3, 6.1e-5, 1e-7]:
        h = f16(v)
        assert oracle.half_to_float(h) == float(np.array([h], np.uint16).view(np.float16)[0])


@pytest.mark.parametrize("enc", FMTS)
def test_three_decoders_agree(rng, enc):
    n = 12 * BLOCK_ELEMENTS[enc]
    data = random_blocks(rng, enc, 12)
    scalar = oracle.gguf_dequant_scalar(data, enc, n)
    block = oracle.gguf_dequantize(data, enc, n)
    shader = oracle.gguf_read4_all(data, enc, n)
    assert same_values(scalar, block)
    assert same_values(scalar, shader)


def test_q8_0_known_answer():
    b = np.zeros(34, np.uint8)
    b[0:2] = np.frombuffer(struct.pack("<H", f16(0.5)), np.uint8)
    q = np.arange(-16, 16, dtype=np.int8)
    b[2:] = q.view(np.uint8)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_Q8_0, 32), q.astype(np.float32) * 0.5)


def test_q4_k_known_answer():
    # d = 1, dmin = 0.25; sub-block j: scale 2j+1, min j; quants ramp i % 16.
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(struct.pack("<H", f16(1.0)), np.uint8)
    b[2:4] = np.frombuffer(struct.pack("<H", f16(0.25)), np.uint8)
    sc = [2 * j + 1 for j in range(8)]
    mn = [j for j in range(8)]
    for j in range(4):
        b[4 + j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[8 + j] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        b[12 + j] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    q = np.array([i % 16 for i in range(256)])
    for i in range(256):
        j = i // 32
        b[16 + (i // 64) * 32 + i % 32] |= q[i] << ((j & 1) * 4)
    want = np.array([sc[i // 32] * q[i] - 0.25 * mn[i // 32] for i in range(256)], np.float32)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_Q4_K, 256), want)


def test_q6_k_known_answer():
    # d = 0.5; sub-block scales alternate +-(j+1); q = (i * 7) % 64.
    b = np.zeros(210, np.uint8)
    b[208:210] = np.frombuffer(struct.pack("<H", f16(0.5)), np.uint8)
    scales = [(j + 1) * (1 if j % 2 == 0 else -1) for j in range(16)]
    b[192:208] = np.array(scales, np.int8).view(np.uint8)
    q = np.array([(i * 7) % 64 for i in range(256)])
    for i in range(256):
        part, quarter, lane = i // 128, (i % 128) // 32, i % 32
        b[part * 64 + (quarter & 1) * 32 + lane] |= (q[i] & 15) << ((quarter // 2) * 4)
        b[128 + part * 32 + lane] |= ((q[i] >> 4) & 3) << (quarter * 2)
    want = np.array([0.5 * scales[i // 16] * (q[i] - 32) for i in range(256)], np.float32)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_Q6_K, 256), want)


def test_q3_k_known_answer():
    # d = 2; 6-bit scales sc = 20 + g (value sc - 32); q in [-4, 3] = (i % 8) - 4.
    b = np.zeros(110, np.uint8)
    b[108:110] = np.frombuffer(struct.pack("<H", f16(2.0)), np.uint8)
    sc6 = [20 + g for g in range(16)]
    for g in range(16):
        b[96 + g % 8] |= (sc6[g] & 15) << ((g // 8) * 4)
        b[104 + g % 4] |= ((sc6[g] >> 4) & 3) << ((g // 4) * 2)
    q = np.array([(i % 8) - 4 for i in range(256)])
    for i in range(256):
        low = q[i] + 4 if q[i] < 0 else q[i]
        b[32 + (i // 128) * 32 + i % 32] |= low << (((i % 128) // 32) * 2)
        if q[i] >= 0:
            b[i % 32] |= 1 << (i // 32)
    want = np.array([2.0 * (sc6[i // 16] - 32) * q[i] for i in range(256)], np.float32)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_Q3_K, 256), want)


def test_q2_k_known_answer():
    # d = 1, dmin = 0.5; scale nibble = j % 16, min nibble = 15 - j; q = i % 4.
    b = np.zeros(84, np.uint8)
    b[80:82] = np.frombuffer(struct.pack("<H", f16(1.0)), np.uint8)
    b[82:84] = np.frombuffer(struct.pack("<H", f16(0.5)), np.uint8)
    for j in range(16):
        b[j] = (j % 16) | ((15 - j) << 4)
    q = np.array([i % 4 for i in range(256)])
    for i in range(256):
        b[16 + (i // 128) * 32 + i % 32] |= q[i] << (((i % 128) // 32) * 2)
    want = np.array([(i // 16 % 16) * q[i] - 0.5 * (15 - i // 16) for i in range(256)], np.float32)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_Q2_K, 256), want)


def test_q5_k_known_answer():
    # Q4_K's fields (d = 1, dmin = 0.25, scale 2j+1, min j) with 5-bit quants q = (3i) % 32: the low
    # nibble at 48 + (i/64)*32 + i%32, the fifth bit in byte 16 + i%32 at bit i/32.
    b = np.zeros(176, np.uint8)
    b[0:2] = np.frombuffer(struct.pack("<H", f16(1.0)), np.uint8)
    b[2:4] = np.frombuffer(struct.pack("<H", f16(0.25)), np.uint8)
    sc = [2 * j + 1 for j in range(8)]
    mn = [j for j in range(8)]
    for j in range(4):
        b[4 + j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        b[8 + j] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        b[12 + j] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    q = np.array([(3 * i) % 32 for i in range(256)])
    for i in range(256):
        j = i // 32
        b[48 + (i // 64) * 32 + i % 32] |= (q[i] & 15) << ((j & 1) * 4)
        b[16 + i % 32] |= ((q[i] >> 4) & 1) << j
    want = np.array([sc[i // 32] * q[i] - 0.25 * mn[i // 32] for i in range(256)], np.float32)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_Q5_K, 256), want)
    # a Q4_K block reads the same quants' low nibbles at 16, so the fifth bit is the only difference
    assert np.any(q >= 16)


def test_iq4_nl_known_answer():
    # d = 0.5; element i: nibble of byte 2 + i % 16 (high half for i >= 16), q = (5i + 3) % 16.
    b = np.zeros(18 * 2, np.uint8)
    for blk, d in enumerate((0.5, -2.0)):
        b[18 * blk:18 * blk + 2] = np.frombuffer(struct.pack("<H", f16(d)), np.uint8)
    q = np.array([(5 * i + 3) % 16 for i in range(64)])
    for i in range(64):
        blk, j = i // 32, i % 32
        b[18 * blk + 2 + j % 16] |= q[i] << ((j // 16) * 4)
    want = np.array([(0.5 if i < 32 else -2.0) * IQ4[q[i]] for i in range(64)], np.float32)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_IQ4_NL, 64), want)


def test_q2_0_known_answer():
    # Two blocks, d = 0.5 and -2.0; element i: 2-bit q at bits 2(i % 4) of byte 2 + i / 4, q = (3i + 1) % 4;
    # value d * (q - 1).  Every q occurs in every bit position of a byte.
    b = np.zeros(18 * 2, np.uint8)
    for blk, d in enumerate((0.5, -2.0)):
        b[18 * blk:18 * blk + 2] = np.frombuffer(struct.pack("<H", f16(d)), np.uint8)
    q = np.array([(3 * i + 1) % 4 for i in range(128)])
    for i in range(128):
        blk, j = i // 64, i % 64
        b[18 * blk + 2 + j // 4] |= q[i] << ((j % 4) * 2)
    want = np.array([(0.5 if i < 64 else -2.0) * (q[i] - 1) for i in range(128)], np.float32)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_Q2_0, 128), want)
    assert np.array_equal(oracle.gguf_read4_all(b, ENC_Q2_0, 128), want)
    # the CPU Linear decodes the row and runs VectorDot (no packed dot for Q2_0); these sums are exact
    assert oracle.cpu_linear(b, ENC_Q2_0, np.ones(128, np.float32), 128, 1)[0] == want.sum()


def iq_grid(name):
    width = 4 if name.startswith("IQ3") else 8
    return np.frombuffer(oracle.iq_table(name), np.uint32 if width == 4 else np.uint64)


def test_iq_tables_match_reference_digests():
    """The codebooks and the sign table, as the oracle and the kernels build them, hash to the
    digests of the reference's own tables (Tables.inc:20-309, gguf.glsl:20-460)."""
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "iq_grids.json")) as f:
        want = json.load(f)
    for name, entry in want.items():
        data = oracle.iq_table(name)
        assert len(data) == entry["entries"] * (1 if name == "IQ2_SIGNS" else 4 if name.startswith("IQ3") else 8)
        assert hashlib.sha256(data).hexdigest() == entry["sha256"], name


def test_iq_table_invariants():
    """What the format definitions fix without the tables: IQ2_SIGNS[i] is i with an eighth bit for even
    parity; every grid is strictly increasing; IQ2 entries take the levels 8, 25, 43, IQ3_XXS 4..52 by 8
    and 62, IQ3_S the odd numbers 1..15."""
    signs = np.frombuffer(oracle.iq_table("IQ2_SIGNS"), np.uint8)
    assert [int(v) for v in signs] == [i | ((bin(i).count("1") & 1) << 7) for i in range(128)]
    for name, levels in (("IQ2_XXS_GRID", {8, 25, 43}), ("IQ2_S_GRID", {8, 25, 43}),
                         ("IQ3_XXS_GRID", {4, 12, 20, 28, 36, 44, 52, 62}), ("IQ3_S_GRID", set(range(1, 16, 2)))):
        g = iq_grid(name)
        assert np.all(g[1:] > g[:-1]), name
        assert set(np.unique(g.view(np.uint8)).tolist()) <= levels, name


def _put_half(b, off, v):
    b[off:off + 2] = np.frombuffer(struct.pack("<H", f16(v)), np.uint8)


def _grid_bytes(entry, width):
    return [(int(entry) >> (8 * i)) & 255 for i in range(width)]


def test_iq2_xxs_known_answer():
    # d = 0.5; group g: scale n = g (delta = 0.5 (0.5 + g) / 4); lane L: grid index 37g + 11L + 5 (mod 256),
    # 7 stored sign bits 5g + 3L (mod 128), the eighth from parity.
    grid, b = iq_grid("IQ2_XXS_GRID"), np.zeros(66, np.uint8)
    _put_half(b, 0, 0.5)
    want = np.zeros(256, np.float32)
    for g in range(8):
        bits = g << 28
        for L in range(4):
            idx, s7 = (37 * g + 11 * L + 5) % 256, (5 * g + 3 * L) % 128
            b[2 + 8 * g + L] = idx
            bits |= s7 << (7 * L)
            s8 = s7 | ((bin(s7).count("1") & 1) << 7)
            for e, v in enumerate(_grid_bytes(grid[idx], 8)):
                want[32 * g + 8 * L + e] = np.float32(0.5 * (0.5 + g) * 0.25) * (-v if s8 >> e & 1 else v)
        b[6 + 8 * g:10 + 8 * g] = np.frombuffer(struct.pack("<I", bits), np.uint8)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_IQ2_XXS, 256), want)


def test_iq2_s_known_answer():
    # d = -0.25; lane L of group g: 10-bit index (97g + 29L + 3) mod 1024 (low byte, 2 high bits in the
    # group's qh byte), sign byte 17g + 61L (mod 256), scale nibbles g (elements 0-15) and 15 - g (16-31).
    grid, b = iq_grid("IQ2_S_GRID"), np.zeros(82, np.uint8)
    _put_half(b, 0, -0.25)
    want = np.zeros(256, np.float32)
    for g in range(8):
        b[74 + g] = g | ((15 - g) << 4)
        for L in range(4):
            idx, sg = (97 * g + 29 * L + 3) % 1024, (17 * g + 61 * L) % 256
            b[2 + 4 * g + L] = idx & 255
            b[66 + g] |= (idx >> 8) << (2 * L)
            b[34 + 4 * g + L] = sg
            n = g if L < 2 else 15 - g
            for e, v in enumerate(_grid_bytes(grid[idx], 8)):
                want[32 * g + 8 * L + e] = np.float32(-0.25 * (0.5 + n) * 0.25) * (-v if sg >> e & 1 else v)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_IQ2_S, 256), want)


def test_iq3_xxs_known_answer():
    # d = 2; 4-element piece j (0-63): grid index 53j + 7 (mod 256); group g: scale n = 15 - g
    # (delta = 2 (0.5 + n) / 2), 7 stored sign bits per 8 elements (9g + 5L) mod 128, the eighth from parity.
    grid, b = iq_grid("IQ3_XXS_GRID"), np.zeros(98, np.uint8)
    _put_half(b, 0, 2.0)
    want = np.zeros(256, np.float32)
    for j in range(64):
        b[2 + j] = (53 * j + 7) % 256
    for g in range(8):
        bits = (15 - g) << 28
        for L in range(4):
            s7 = (9 * g + 5 * L) % 128
            bits |= s7 << (7 * L)
            s8 = s7 | ((bin(s7).count("1") & 1) << 7)
            for e in range(8):
                i = 32 * g + 8 * L + e
                v = _grid_bytes(grid[b[2 + i // 4]], 4)[i % 4]
                want[i] = np.float32(2.0 * (0.5 + 15 - g) * 0.5) * (-v if s8 >> e & 1 else v)
        b[66 + 4 * g:70 + 4 * g] = np.frombuffer(struct.pack("<I", bits), np.uint8)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_IQ3_XXS, 256), want)


def test_iq3_s_known_answer():
    # d = 0.125; piece j: 9-bit index (41j + 13) mod 512 (low byte; high bit j % 8 of byte 66 + j / 8);
    # sign byte per 8 elements 23k + 1 (mod 256); group g: scale 1 + 2 (3g mod 16).
    grid, b = iq_grid("IQ3_S_GRID"), np.zeros(110, np.uint8)
    _put_half(b, 0, 0.125)
    for j in range(64):
        idx = (41 * j + 13) % 512
        b[2 + j] = idx & 255
        b[66 + j // 8] |= (idx >> 8) << (j % 8)
    for k in range(32):
        b[74 + k] = (23 * k + 1) % 256
    for g in range(8):
        b[106 + g // 2] |= ((3 * g) % 16) << (4 * (g % 2))
    want = np.zeros(256, np.float32)
    for i in range(256):
        j, g = i // 4, i // 32
        v = _grid_bytes(grid[(41 * j + 13) % 512], 4)[i % 4]
        sign = ((23 * (i // 8) + 1) % 256) >> (i % 8) & 1
        want[i] = np.float32(0.125 * (1 + 2 * ((3 * g) % 16))) * (-v if sign else v)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_IQ3_S, 256), want)


def test_iq4_xs_known_answer():
    # d = 0.25; 6-bit sub-block scales ls (value ls - 32) with every high-bit pattern; q = (7i) % 16.
    b = np.zeros(136, np.uint8)
    b[0:2] = np.frombuffer(struct.pack("<H", f16(0.25)), np.uint8)
    ls = [0, 5, 31, 32, 33, 47, 63, 16]
    high = 0
    for j in range(8):
        b[4 + j // 2] |= (ls[j] & 15) << ((j % 2) * 4)
        high |= ((ls[j] >> 4) & 3) << (2 * j)
    b[2], b[3] = high & 255, high >> 8
    q = np.array([(7 * i) % 16 for i in range(256)])
    for i in range(256):
        j = i // 32
        b[8 + j * 16 + i % 16] |= q[i] << (((i % 32) // 16) * 4)
    want = np.array([0.25 * (ls[i // 32] - 32) * IQ4[q[i]] for i in range(256)], np.float32)
    assert np.array_equal(oracle.gguf_dequant_scalar(b, ENC_IQ4_XS, 256), want)


@pytest.mark.parametrize("enc", FMTS)
def test_packed_dot_and_linear_brute_force(rng, enc):
    k = 1024
    rows = 8
    data = random_blocks(rng, enc, rows * k // BLOCK_ELEMENTS[enc])
    x = rng.standard_normal(k).astype(np.float32)
    y = oracle.cpu_linear(data, enc, x, k, rows)
    rb = k // BLOCK_ELEMENTS[enc] * BLOCK_BYTES[enc]
    for r in range(rows):
        w = oracle.gguf_dequant_scalar(np.ascontiguousarray(data[r * rb:(r + 1) * rb]), enc, k).astype(np.float64)
        want = float(w @ x.astype(np.float64))
        assert abs(y[r] - want) <= 4e-6 * float(np.abs(w) @ np.abs(x)) + 1e-30, (enc, r)


@pytest.mark.parametrize("enc", FMTS)
def test_product_encoder_round_trip(rng, enc):
    """qnn_gguf_quantize writes valid blocks whose decode tracks the input."""
    from quicknn_amd import hip

    w = (rng.standard_normal(4096) * 0.02).astype(np.float32)
    blocks = hip.gguf_quantize(enc, w)
    assert blocks.size == 4096 // BLOCK_ELEMENTS[enc] * BLOCK_BYTES[enc]
    dec = oracle.gguf_dequant_scalar(blocks, enc, 4096)
    assert np.all(np.isfinite(dec))
    rel = np.linalg.norm(dec - w) / np.linalg.norm(w)
    bound = {ENC_Q8_0: 0.01, ENC_Q6_K: 0.03, ENC_Q4_K: 0.12, ENC_Q3_K: 0.25, ENC_Q2_K: 0.45, ENC_Q5_K: 0.06,
             ENC_IQ4_NL: 0.12, ENC_IQ4_XS: 0.12, ENC_Q2_0: 0.45, ENC_IQ2_XXS: 0.4, ENC_IQ2_S: 0.3, ENC_IQ3_XXS: 0.25,
             ENC_IQ3_S: 0.2}[enc]
    assert rel < bound, rel
