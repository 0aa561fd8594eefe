"""Shared pytest configuration.

`gpu` tests need an MI355X (libqnn_hip.so + a visible HIP device); everything
else runs on the CPU.  One resident context per process is allowed (as in the
reference), so the GPU tests of a module share the module-scoped `ctx` fixture.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and the built HIP library")


@pytest.fixture(scope="module")
def ctx():
    """One resident context per test module (closed before the next module
    opens its own, so modules may also create contexts with other settings)."""
    from quicknn_amd import hip

    c = hip.GPUContext(0)
    yield c
    c.close()


@pytest.fixture
def tune(monkeypatch):
    """tune(name, value): set a QNN_* tuning switch for this test.  The library reads the
    switches once per context (qnn_reload_tuning re-reads them), so each change is followed
    by a reload, and the test's end restores the environment and reloads again."""
    from quicknn_amd import hip

    def set_switch(name: str, value: str) -> None:
        monkeypatch.setenv(name, value)
        hip.reload_tuning()

    yield set_switch
    monkeypatch.undo()
    hip.reload_tuning()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits by truncation, as SingleToBF16 (src/core/QuickNN.Common.pas:1779-1797)."""
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def normwise_rel_err(y: np.ndarray, r: np.ndarray) -> float:
    """max_i |y - r| / max_i |r|: the tolerance metric for matvec/MLP/GEMM outputs."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    den = np.max(np.abs(r))
    return float(np.max(np.abs(y - r)) / den) if den > 0 else float(np.max(np.abs(y - r)))


def rand_int4(rng, n: int, k: int) -> np.ndarray:
    """Valid packed INT4 rows [n, Int4RowBytes(k)] drawn directly: positive fp32 group
    scales in [0.001, 0.004) and uniform nibbles, the shape of QuantizeInt4's output for
    N(0, 0.02) weights, without the packing cost.  Elements past k in the last group hold
    nibble 8 (value 0), as QuantizeInt4 writes them."""
    g = (k + 31) // 32
    p = rng.integers(0, 256, (n, g, 20), dtype=np.uint8)
    p[:, :, :4] = rng.uniform(0.001, 0.004, (n, g)).astype(np.float32)[..., None].view(np.uint8).reshape(n, g, 4)
    tail = k - 32 * (g - 1)
    for j in range(tail, 32):  # element j: byte 4 + j // 2, low nibble for even j
        b = p[:, g - 1, 4 + j // 2]
        p[:, g - 1, 4 + j // 2] = (b & 0xF0) | 8 if j % 2 == 0 else (b & 0x0F) | 0x80
    return p.reshape(n, g * 20)
