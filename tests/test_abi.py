"""The C-ABI libraries load and export every symbol their headers declare
(no compute calls: runs without a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header: str, prefix: str) -> set[str]:
    text = open(os.path.join(ROOT, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text))


def test_hip_library_exports_header():
    from quicknn_amd import hip

    lib = ctypes.CDLL(hip.LIB_PATH)
    names = declared("include/qnn_hip.h", "qnn_")
    assert len(names) >= 35
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(hip.EXPORTED) == names


def test_oracle_library_exports_header():
    import oracle

    lib = ctypes.CDLL(oracle.LIB_PATH)
    names = declared("oracle/qnn_oracle.h", "qo_")
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


def test_error_codes_map_to_reference_exceptions():
    from quicknn_amd import hip

    assert issubclass(hip.EArgumentException, ValueError)
    assert hip._ERRORS[-1] is hip.EArgumentException
    assert hip._ERRORS[-2] is hip.ERangeError
    assert hip._ERRORS[-3] is hip.ENotSupportedException
    assert hip._ERRORS[-4] is hip.EInvalidOp


def test_no_device_is_reported_not_faked():
    """Without a visible GPU the context reports ENotSupportedException; there is no CPU fallback."""
    from quicknn_amd import hip

    try:
        import torch  # noqa: F401  (only to learn whether a GPU is present)
        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is visible")
    with pytest.raises(hip.ENotSupportedException):
        hip.GPUContext(0)


def pascal_externals() -> dict[str, int]:
    """Name -> parameter count of every `external QNN_LIB` routine in the Pascal unit."""
    text = open(os.path.join(ROOT, "src/backends/hip/QuickNN.HIP.pas")).read()
    out = {}
    for m in re.finditer(r"(?:function|procedure)\s+(qnn_\w+)\s*(\((.*?)\))?[^;]*;\s*cdecl;\s*external QNN_LIB;",
                         text, flags=re.S):
        params = m.group(3) or ""
        names = 0
        for group in params.split(";"):
            if ":" in group:
                names += len(group.split(":")[0].replace("out ", "").replace("var ", "").replace("const ", "")
                             .split(","))
        out[m.group(1)] = names
    return out


def c_param_counts() -> dict[str, int]:
    text = open(os.path.join(ROOT, "include/qnn_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^(?:int|void \*|const char \*|uint64_t)\s*(qnn_\w+)\(([^;]*)\);", text, flags=re.M):
        args = " ".join(m.group(2).split())
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_pascal_unit_binds_every_entry_point():
    """src/backends/hip/QuickNN.HIP.pas declares each C entry point with the same parameter count."""
    pas, c = pascal_externals(), c_param_counts()
    assert set(c) == declared("include/qnn_hip.h", "qnn_")
    missing = sorted(set(c) - set(pas))
    assert not missing, missing
    wrong = {n: (pas[n], c[n]) for n in c if pas[n] != c[n]}
    assert not wrong, wrong
