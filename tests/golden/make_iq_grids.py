#!/usr/bin/env python3
"""Writes tests/golden/iq_grids.json: SHA-256 digests of the reference's IQ2/IQ3
tables (run from the repository root, where /root/reference is present).

The reference holds each table twice, as Pascal constants
(src/io/QuickNN.GGUF.Tables.inc:20-309) and as GLSL constants
(src/backends/vulkan/shaders/gguf.glsl:20-460, 64-bit entries split into two
32-bit words, low word first).  Both are read as text; the script checks that
the two copies agree and records, per table, the entry count and the digest of
its entries as little-endian bytes (4 per entry for the IQ3 grids, 8 for the
IQ2 grids, 1 for IQ2_SIGNS).  tests/test_oracle_gguf.py compares these digests
with the tables this repository builds from its own storage of them.

Usage: python tests/golden/make_iq_grids.py [reference root]
"""
from __future__ import annotations

import hashlib
import json
import os
import re
import sys

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "iq_grids.json")
WIDTH = {"IQ3_S_GRID": 4, "IQ2_XXS_GRID": 8, "IQ2_S_GRID": 8, "IQ2_SIGNS": 1, "IQ3_XXS_GRID": 4}


def pascal_tables(text: str) -> dict:
    out = {}
    for name in WIDTH:
        m = re.search(name + r"\s*:\s*array\[0\.\.(\d+)\] of \w+ = \((.*?)\);", text, re.S)
        vals = [int(v, 16) for v in re.findall(r"\$([0-9A-Fa-f]+)", m.group(2))]
        assert len(vals) == int(m.group(1)) + 1, name
        out[name] = vals
    return out


def glsl_tables(text: str) -> dict:
    out = {}
    for name in WIDTH:
        m = re.search(r"const uint " + name + r"\[(\d+)\]\s*=\s*uint\[\d+\]\((.*?)\);", text, re.S)
        words = [int(v, 16) for v in re.findall(r"0x([0-9A-Fa-f]+)", m.group(2))]
        if not words:
            words = [int(v) for v in re.findall(r"\b(\d+)u?\b", m.group(2))]
        assert len(words) == int(m.group(1)), name
        if WIDTH[name] == 8:
            words = [words[2 * i] | (words[2 * i + 1] << 32) for i in range(len(words) // 2)]
        out[name] = words
    return out


def main() -> None:
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    with open(os.path.join(root, "src/io/QuickNN.GGUF.Tables.inc"), encoding="utf-8-sig") as f:
        pas = pascal_tables(f.read())
    with open(os.path.join(root, "src/backends/vulkan/shaders/gguf.glsl"), encoding="utf-8-sig") as f:
        glsl = glsl_tables(f.read())
    res = {}
    for name, w in WIDTH.items():
        assert pas[name] == glsl[name], f"{name}: the Pascal and GLSL copies differ"
        data = b"".join(v.to_bytes(w, "little") for v in pas[name])
        res[name] = {"entries": len(pas[name]), "sha256": hashlib.sha256(data).hexdigest()}
    with open(OUT, "w") as f:
        json.dump(res, f, indent=1)
        f.write("\n")
    print("wrote", OUT)


if __name__ == "__main__":
    main()
