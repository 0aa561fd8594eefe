"""Split-K results do not depend on where the device places workgroups.

A K-split tile's combine reads the partial sums through one XCD's L2 only when
every workgroup of the tile ran on the XCD the tile map intended, and with
device-coherent loads otherwise (quicknn_amd/csrc/qnn_exchange.h).  Other GPU
work in the process, such as PyTorch kernels on PyTorch's own stream, changes
the order in which the device deals workgroups to XCDs; every entry point must
give bit-identical results before and after it, and raise nothing.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from tests.conftest import rand_int4

pytestmark = pytest.mark.gpu


def run_all(ctx, hip, w):
    out = {}
    x = ctx.UploadRaw(w["x"])
    y = ctx.NewTensor(4096)
    ctx.Int4Linear(y, x, w["i4"], 1, 4096, 4096)  # split-K INT4 matvec
    out["int4"] = ctx.Download(y)
    h = ctx.NewTensor(3072)
    assert ctx.TrySwiGLUVector(h, x, w["g"], w["u"], 4096, 3072)
    out["swiglu"] = ctx.Download(h)  # the SwiGLU on its own
    assert ctx.TrySwiGLUVector(h, x, w["g"], w["u"], 4096, 3072)
    ctx.Int4Linear(y, h, w["d"], 1, 3072, 4096)  # fused MLP
    out["mlp"] = ctx.Download(y)
    q = ctx.NewTensor(1024)
    ctx.Linear(q, x, w["q4k"], None, None, 1, 4096, 1024)  # GGUF Q4_K matvec
    out["gguf"] = ctx.Download(q)
    xm = ctx.UploadRaw(w["xm"])
    for rows in (1, 4):
        m = ctx.NewTensor(rows * 512)
        ctx.MoEExperts(w["set"], m, xm, w["routes"][rows], rows, 4)
        out[f"moe{rows}"] = ctx.Download(m)
        ctx.Recycle(m)
    for t in (x, y, h, q, xm):
        ctx.Recycle(t)
    return out


def scenario(rng):
    import torch

    from quicknn_amd import hip

    E = 16
    w = {"x": rng.standard_normal(4096).astype(np.float32),
         "xm": rng.standard_normal((4, 512)).astype(np.float32),
         "i4": hip.MemoryBlock.int4(rand_int4(rng, 4096, 4096)),
         "g": hip.MemoryBlock.int4(rand_int4(rng, 3072, 4096)),
         "u": hip.MemoryBlock.int4(rand_int4(rng, 3072, 4096)),
         "d": hip.MemoryBlock.int4(rand_int4(rng, 4096, 3072))}
    wq = (rng.standard_normal(1024 * 4096) * 0.02).astype(np.float32)
    w["q4k"] = hip.MemoryBlock.gguf(hip.gguf_quantize(hip.WE_Q4_K, wq), 1024, 4096, hip.WE_Q4_K)
    with hip.GPUContext(0) as ctx:
        ex = [[hip.MemoryBlock.int4(rand_int4(rng, n, k)) for _ in range(E)] for n, k in ((320, 512), (320, 512), (512, 320))]
        w["set"] = ctx.CreateExpertSet(ex[0], ex[1], ex[2], 512, 320)
        w["routes"] = {}
        for rows in (1, 4):
            lt = ctx.UploadRaw(rng.standard_normal((rows, E)).astype(np.float32))
            rt = ctx.NewTensor(2 * rows * 4)
            ctx.Kernel(hip.GO_MOE_ROUTE, 2 * rows * 4, rt, lt, None, None, [rows, E, 4, 1])
            w["routes"][rows] = rt
        before = run_all(ctx, hip, w)
        # PyTorch work on its own stream: allocation, odd-sized grids, a reduction, a copy back
        dev = torch.device("cuda:0")
        a = torch.ones(7 * 256 + 3, device=dev)
        a.mul_(3.0)
        s = torch.ones(1 << 20, device=dev).sum()
        _ = (a.cpu(), float(s))
        torch.cuda.synchronize()
        for trial in range(2):
            after = run_all(ctx, hip, w)
            for k, v in before.items():
                assert np.array_equal(v.view(np.uint32), after[k].view(np.uint32)), (trial, k)
            torch.ones(5 * 256 + 1, device=dev).add_(1.0)
            torch.cuda.synchronize()
        ctx.DestroyExpertSet(w["set"])
        print("placement scenario: all results bit-identical", flush=True)


def test_results_survive_foreign_gpu_work():
    # In a process of its own: the scenario needs PyTorch to initialise the GPU
    # after this library has, as an application would, independent of what the
    # test session did before.
    r = subprocess.run([sys.executable, os.path.abspath(__file__)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "all results bit-identical" in r.stdout


if __name__ == "__main__":
    scenario(np.random.default_rng(1234))
