"""Build recipe for libqnn_hip.so (gfx950).

Compiles every HIP source under quicknn_amd/csrc with hipcc for gfx950 and the
host-only C++ with g++, then links one shared library in-tree
(quicknn_amd/libqnn_hip.so) so it travels with the source tree.  A second
library, libqnn_hip_trace.so, is the same objects with the fused decode-MLP
kernels built with per-workgroup phase timestamps (QNN_PHASE_TRACE), for
quicknn_amd/phase_trace.py; nothing else loads it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libqnn_hip.so")
TRACE_LIB = os.path.join(HERE, "libqnn_hip_trace.so")  # diagnostic build (phase timestamps)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Packed fp32 VALU forms are disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-parameter",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall"]
# Per-file device flags.  The int8 GEMM starts every block's MFMA from zero and
# converts its int32 results at once: with the results in VGPRs (not AGPRs)
# it saves 16 accumulator reads per MFMA on the VALU, its bound.
FILE_FLAGS = {"qnn_gemm_i8.hip": ["-Xarch_device", "-mllvm=-amdgpu-mfma-vgpr-form"]}


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def build(jobs: int | None = None) -> str:
    """Compile and link libqnn_hip.so; always rebuilds.  Returns the library path."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    cmds = []
    for src in sources():
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        objs.append(obj)
        if src.endswith(".hip"):
            cmds.append([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj])
        else:
            cmds.append(["g++", *HOST_FLAGS, "-c", src, "-o", obj])
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp, "-lpthread"])
    os.replace(tmp, LIB)
    # The phase-trace variant: the fused decode-MLP, one-token MoE and
    # LDS-streamed attention kernels with per-workgroup timestamps
    # (QNN_PHASE_TRACE), everything else the same objects.
    traced = {}
    for name in ("qnn_mlp.hip", "qnn_moe.hip", "qnn_decode.hip"):
        tobj = os.path.join(BUILD, name + ".trace.o")
        _run([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(name, []), "-DQNN_PHASE_TRACE", "-c", os.path.join(CSRC, name),
              "-o", tobj])
        traced[os.path.join(BUILD, name + ".o")] = tobj
    tobjs = [traced.get(o, o) for o in objs]
    tmp = TRACE_LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *tobjs, "-o", tmp, "-lpthread"])
    os.replace(tmp, TRACE_LIB)
    return LIB


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)
    for f in (LIB, TRACE_LIB):
        if os.path.exists(f):
            os.remove(f)


if __name__ == "__main__":
    print(build())
