"""A process that exits with its context still open ends cleanly.

`quicknn_amd.hip` closes contexts left open at interpreter exit (an atexit
hook), before the HIP runtime's own teardown; without it the context's
stream, events, graphs and pinned readback buffer were released by a runtime
already shutting down, which ended one such process with a segmentation fault
inside exit().  The child below runs real work (a weight upload, an INT4
matvec with split-K, a recorded SwiGLU fused with its down projection) and
returns without calling close().
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from quicknn_amd import hip
rng = np.random.default_rng(3)
H, I = 256, 512
def mat(n, k):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return hip.MemoryBlock.int4(hip.quantize_int4((w.view(np.uint32) >> 16).astype(np.uint16)))
g, u, d = mat(I, H), mat(I, H), mat(H, I)
ctx = hip.GPUContext(0)
x = ctx.UploadRaw(rng.standard_normal(H).astype(np.float32))
h, y = ctx.NewTensor(I), ctx.NewTensor(H)
ctx.TrySwiGLUVector(h, x, g, u, H, I)
ctx.Int4Linear(y, h, d, 1, I, H)
out = ctx.Download(y)
assert np.isfinite(out).all()
print("child done", flush=True)
# no ctx.close(): the interpreter exits with the context open
"""


@pytest.mark.gpu
def test_exit_with_open_context():
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT], capture_output=True, text=True, timeout=300)
    assert "child done" in r.stdout, r.stdout + r.stderr
    assert r.returncode == 0, f"exit status {r.returncode}\n{r.stderr[-2000:]}"
