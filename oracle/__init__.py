"""ctypes binding of the CPU oracle (libqnn_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP backend and the CPU baseline
timed beside it.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py may import this package; the product package
``quicknn_amd`` never does.

Each wrapper names the reference file:line its C++ function restates
(paths relative to the QuickNN source tree).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqnn_oracle.so")

ENC_INT4 = -1
ENC_Q8_0 = 1
ENC_Q4_K = 2
ENC_Q6_K = 3
ENC_Q3_K = 4
ENC_Q2_K = 9
ENC_Q5_K, ENC_IQ4_NL, ENC_IQ4_XS = 5, 6, 8
ENC_Q2_0 = 12
ENC_IQ3_S, ENC_IQ2_XXS, ENC_IQ2_S, ENC_IQ3_XXS = 7, 10, 11, 13
GGUF_ENCODINGS = (ENC_Q8_0, ENC_Q4_K, ENC_Q6_K, ENC_Q3_K, ENC_Q2_K, ENC_Q5_K, ENC_IQ4_NL, ENC_IQ4_XS, ENC_Q2_0,
                  ENC_IQ2_XXS, ENC_IQ2_S, ENC_IQ3_XXS, ENC_IQ3_S)
BLOCK_ELEMENTS = {ENC_Q8_0: 32, ENC_Q4_K: 256, ENC_Q6_K: 256, ENC_Q3_K: 256, ENC_Q2_K: 256, ENC_Q5_K: 256,
                  ENC_IQ4_NL: 32, ENC_IQ4_XS: 256, ENC_Q2_0: 64, ENC_IQ2_XXS: 256, ENC_IQ2_S: 256, ENC_IQ3_XXS: 256,
                  ENC_IQ3_S: 256}
BLOCK_BYTES = {ENC_Q8_0: 34, ENC_Q4_K: 144, ENC_Q6_K: 210, ENC_Q3_K: 110, ENC_Q2_K: 84, ENC_Q5_K: 176,
               ENC_IQ4_NL: 18, ENC_IQ4_XS: 136, ENC_Q2_0: 18, ENC_IQ2_XXS: 66, ENC_IQ2_S: 82, ENC_IQ3_XXS: 98,
               ENC_IQ3_S: 110}
IQ_TABLES = {"IQ2_XXS_GRID": 0, "IQ2_S_GRID": 1, "IQ3_XXS_GRID": 2, "IQ3_S_GRID": 3, "IQ2_SIGNS": 4}

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i8p = ctypes.POINTER(ctypes.c_int8)
_vp = ctypes.c_void_p


def build() -> None:
    """Compile libqnn_oracle.so from oracle/qnn_oracle.cpp (always rebuilds)."""
    import subprocess

    subprocess.run(["make", "-B", "-C", _HERE], check=True, stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library not built: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "qo_int4_row_bytes": (ctypes.c_int, [ctypes.c_int]),
            "qo_quantize_int4": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _u8p]),
            "qo_int4_value": (ctypes.c_float, [_u8p, ctypes.c_int]),
            "qo_int4_dequant_row": (None, [_u8p, ctypes.c_int, _f32p]),
            "qo_gguf_value": (ctypes.c_float, [_u8p, ctypes.c_int, ctypes.c_int64]),
            "qo_gguf_decode_block": (ctypes.c_int, [_u8p, ctypes.c_int, _f32p]),
            "qo_gguf_dequantize": (ctypes.c_int, [_u8p, ctypes.c_int, ctypes.c_int64, _f32p]),
            "qo_gguf_read4": (ctypes.c_int, [_u8p, ctypes.c_int, ctypes.c_int64, _f32p]),
            "qo_vector_dot": (ctypes.c_float, [ctypes.c_int, _f32p, _f32p]),
            "qo_int4_vector_dot": (ctypes.c_float, [ctypes.c_int, _f32p, _u8p]),
            "qo_packed_dot": (ctypes.c_float, [_u8p, ctypes.c_int, _f32p, ctypes.c_int]),
            "qo_iq_table": (ctypes.c_int, [ctypes.c_int, _vp]),
            "qo_pool_create": (_vp, [ctypes.c_int]),
            "qo_pool_destroy": (None, [_vp]),
            "qo_pool_threads": (ctypes.c_int, [_vp]),
            "qo_cpu_linear": (ctypes.c_int, [_vp, _u8p, ctypes.c_int, _f32p, _f32p, ctypes.c_int, ctypes.c_int]),
            "qo_rmsnorm": (ctypes.c_int, [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, _f32p]),
            "qo_silu": (ctypes.c_float, [ctypes.c_float]),
            "qo_cpu_mlp": (ctypes.c_int, [_vp, _u8p, _u8p, _u8p, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, _f32p]),
            "qo_moe_route": (ctypes.c_int, [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, _u32p, _f32p]),
            "qo_cpu_moe": (ctypes.c_int, [_vp, ctypes.POINTER(_u8p), ctypes.POINTER(_u8p), ctypes.POINTER(_u8p),
                                          _f32p, _u32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, _f32p]),
            "qo_q8_act_quant": (ctypes.c_int, [_f32p, ctypes.c_int, ctypes.c_int, _i8p, _f32p]),
            "qo_q8_gemm_i8": (ctypes.c_int, [_u8p, _i8p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]),
            "qo_gguf_gemm_scalar": (ctypes.c_int, [_u8p, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int,
                                                   ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int]),
            "qo_rope": (ctypes.c_int, [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float]),
            "qo_cache_write": (ctypes.c_int, [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_int]),
            "qo_cached_attention": (ctypes.c_int, [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                   ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                   ctypes.c_float, ctypes.c_float, ctypes.c_int, _f32p]),
            "qo_sample_topk": (ctypes.c_int, [_f32p, _u32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, _f32p,
                                              _u32p]),
            "qo_sample_token": (ctypes.c_uint32, [_f32p, _u32p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                                  ctypes.c_float, ctypes.c_float, ctypes.c_float]),
            "qo_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
            "qo_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data_as(t)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} failed (rc={rc})")


# ---- INT4: src/core/QuickNN.Quantization.Int4.pas ----
def int4_row_bytes(cols: int) -> int:
    """Int4RowBytes (Int4.pas:25-33)."""
    return lib().qo_int4_row_bytes(cols)


def quantize_int4(w: np.ndarray) -> np.ndarray:
    """QuantizeInt4 (Int4.pas:96-144) of an fp32 or bf16 (uint16 bits) [rows, cols] matrix."""
    w = np.ascontiguousarray(w)
    rows, cols = w.shape
    out = np.zeros((rows, int4_row_bytes(cols)), np.uint8)
    is_bf16 = 1 if w.dtype == np.uint16 else 0
    if not is_bf16:
        w = w.astype(np.float32, copy=False)
    _check(lib().qo_quantize_int4(w.ctypes.data, is_bf16, rows, cols, _p(out, _u8p)), "quantize_int4")
    return out


def int4_dequant(packed: np.ndarray, cols: int) -> np.ndarray:
    """Row-wise scalar dequant (CPU.Inference.pas:413-420): fl32((n-8)*s)."""
    packed = np.ascontiguousarray(packed, np.uint8)
    out = np.zeros((packed.shape[0], cols), np.float32)
    for r in range(packed.shape[0]):
        row = np.ascontiguousarray(packed[r])
        lib().qo_int4_dequant_row(_p(row, _u8p), cols, _p(out[r], _f32p))
    return out


# ---- GGUF: src/io/QuickNN.GGUF.Quantization.pas ----
def gguf_value(data: np.ndarray, enc: int, index: int) -> float:
    """GGUFValue (GGUF.Quantization.pas:136-253)."""
    return lib().qo_gguf_value(_p(data, _u8p), enc, index)


def gguf_dequant_scalar(data: np.ndarray, enc: int, count: int) -> np.ndarray:
    """Element-by-element GGUFValue."""
    data = np.ascontiguousarray(data, np.uint8)
    L = lib()
    ptr = _p(data, _u8p)
    return np.array([L.qo_gguf_value(ptr, enc, i) for i in range(count)], np.float32)


def gguf_dequantize(data: np.ndarray, enc: int, count: int) -> np.ndarray:
    """GGUFDequantize (GGUF.Quantization.pas:370-383): AVX2 block decoders."""
    data = np.ascontiguousarray(data, np.uint8)
    out = np.zeros(count, np.float32)
    _check(lib().qo_gguf_dequantize(_p(data, _u8p), enc, count, _p(out, _f32p)), "gguf_dequantize")
    return out


def gguf_read4_all(data: np.ndarray, enc: int, count: int) -> np.ndarray:
    """readGGUF4 (gguf.glsl:591-655) over count elements, 4 at a time."""
    data = np.ascontiguousarray(data, np.uint8)
    out = np.zeros(count, np.float32)
    L = lib()
    ptr = _p(data, _u8p)
    for i in range(0, count, 4):
        _check(L.qo_gguf_read4(ptr, enc, i, _p(out[i:i + 4], _f32p)), "gguf_read4")
    return out


# ---- dots and the CPU projection ----
def iq_table(name: str) -> bytes:
    """The oracle's copy of an IQ2/IQ3 table (IQ_TABLES) as little-endian bytes."""
    which = IQ_TABLES[name]
    n = lib().qo_iq_table(which, None)
    buf = ctypes.create_string_buffer(n)
    lib().qo_iq_table(which, buf)
    return buf.raw


def vector_dot(a: np.ndarray, b: np.ndarray) -> float:
    """VectorDot (CPU.Inference.AVX2.inc:7-67)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().qo_vector_dot(a.size, _p(a, _f32p), _p(b, _f32p))


def int4_vector_dot(x: np.ndarray, row: np.ndarray) -> float:
    """Int4VectorDot (CPU.Inference.AVX2.inc:210-285)."""
    x = np.ascontiguousarray(x, np.float32)
    row = np.ascontiguousarray(row, np.uint8)
    return lib().qo_int4_vector_dot(x.size, _p(x, _f32p), _p(row, _u8p))


class Pool:
    """TInferencePool (CPU.Inference.pas:109-158); threads=0 -> min(8, nproc)."""

    def __init__(self, threads: int = 0):
        self.handle = lib().qo_pool_create(threads)
        if not self.handle:
            raise RuntimeError("oracle pool creation failed (needs AVX2/F16C, threads in [0,64])")
        self.threads = lib().qo_pool_threads(self.handle)

    def close(self):
        if self.handle:
            lib().qo_pool_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_default_pool = None


def default_pool() -> Pool:
    global _default_pool
    if _default_pool is None:
        _default_pool = Pool(0)
    return _default_pool


def cpu_linear(w: np.ndarray, enc: int, x: np.ndarray, in_dim: int, out_dim: int, pool: Pool | None = None) -> np.ndarray:
    """TCPUProjection.Linear (CPU.Inference.pas:316-428) for one activation row."""
    pool = pool or default_pool()
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(out_dim, np.float32)
    _check(lib().qo_cpu_linear(pool.handle, _p(w, _u8p), enc, _p(x, _f32p), _p(y, _f32p), in_dim, out_dim),
           "cpu_linear")
    return y


def rmsnorm(x: np.ndarray, gamma: np.ndarray | None, eps: float = 1e-6, add_one: bool = False) -> np.ndarray:
    """TQwenCPULayer.Normalize (QwenHybrid.CPU.pas:110-120)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, dim = x.reshape(-1, x.shape[-1]).shape
    out = np.zeros_like(x)
    g = None if gamma is None else np.ascontiguousarray(gamma, np.float32)
    _check(lib().qo_rmsnorm(_p(x, _f32p), None if g is None else _p(g, _f32p), rows, dim, eps, int(add_one),
                            _p(out, _f32p)), "rmsnorm")
    return out


def silu(g: float) -> float:
    return lib().qo_silu(g)


def cpu_mlp(gate, up, down, enc, x, hidden, inter, pool: Pool | None = None) -> np.ndarray:
    """TQwenCPULayer.Step MLP (QwenHybrid.CPU.pas:238-248) for each row of x."""
    pool = pool or default_pool()
    x = np.ascontiguousarray(x, np.float32).reshape(-1, hidden)
    out = np.zeros_like(x)
    _check(lib().qo_cpu_mlp(pool.handle, _p(gate, _u8p), _p(up, _u8p), _p(down, _u8p), enc, _p(x, _f32p),
                            x.shape[0], hidden, inter, _p(out, _f32p)), "cpu_mlp")
    return out


def moe_route(logits: np.ndarray, k: int, normalize: bool = True, select_on_logits: bool = False):
    """GO_MOE_ROUTE (moe.comp:25-50): ranked by fp32 probability, ties to the lower id.
    Returns (ids uint32 [rows,k], probs f32 [rows,k])."""
    logits = np.ascontiguousarray(logits, np.float32)
    rows, experts = logits.shape
    ids = np.zeros((rows, k), np.uint32)
    probs = np.zeros((rows, k), np.float32)
    _check(lib().qo_moe_route(_p(logits, _f32p), rows, experts, k, int(normalize), int(select_on_logits),
                              _p(ids, _u32p), _p(probs, _f32p)), "moe_route")
    return ids, probs


def cpu_moe(gates, ups, downs, x, ids, probs, hidden, inter, pool: Pool | None = None) -> np.ndarray:
    """Composed MoE layer (LLM.MoE.pas:230-449 orchestration, experts in ascending id)."""
    pool = pool or default_pool()
    x = np.ascontiguousarray(x, np.float32).reshape(-1, hidden)
    ids = np.ascontiguousarray(ids, np.uint32)
    probs = np.ascontiguousarray(probs, np.float32)
    E = len(gates)
    arr = lambda ws: (_u8p * E)(*[_p(np.ascontiguousarray(w, np.uint8), _u8p) for w in ws])
    out = np.zeros_like(x)
    _check(lib().qo_cpu_moe(pool.handle, arr(gates), arr(ups), arr(downs), _p(x, _f32p), _p(ids, _u32p),
                            _p(probs, _f32p), x.shape[0], ids.shape[1], hidden, inter, _p(out, _f32p)), "cpu_moe")
    return out


def gguf_gemm_scalar(w, enc, a, n, row_begin=0, row_end=None) -> np.ndarray:
    """Scalar double-accumulated GGUF GEMM (QuickNN.Quantization.pas:247-258)."""
    a = np.ascontiguousarray(a, np.float32)
    m, k = a.shape
    row_end = m if row_end is None else row_end
    c = np.zeros((m, n), np.float32)
    _check(lib().qo_gguf_gemm_scalar(_p(w, _u8p), enc, _p(a, _f32p), m, k, n, _p(c, _f32p), row_begin, row_end),
           "gguf_gemm_scalar")
    return c


def q8_act_quant(a):
    """Activations [m, k] -> (int8 q [m, k], fp32 d [m, k/32]): per 32-element block, GGML's Q8_0 rule."""
    a = np.ascontiguousarray(a, np.float32)
    m, k = a.shape
    q = np.zeros((m, k), np.int8)
    d = np.zeros((m, k // 32), np.float32)
    _check(lib().qo_q8_act_quant(_p(a, _f32p), m, k, _p(q, _i8p), _p(d, _f32p)), "q8_act_quant")
    return q, d


def q8_gemm_i8(w, q, d, n) -> np.ndarray:
    """The int8-activation Q8_0 GEMM: acc = fma(float(S_b), dx * dw, acc) over blocks in order."""
    q = np.ascontiguousarray(q, np.int8)
    d = np.ascontiguousarray(d, np.float32)
    m, k = q.shape
    c = np.zeros((m, n), np.float32)
    _check(lib().qo_q8_gemm_i8(_p(np.ascontiguousarray(w, np.uint8), _u8p), _p(q, _i8p), _p(d, _f32p), m, k, n,
                               _p(c, _f32p)), "q8_gemm_i8")
    return c


def half_to_float(h: int) -> float:
    return lib().qo_half_to_float(h)


def float_to_half(f: float) -> int:
    return lib().qo_float_to_half(f)


# ---------------------------------------------------------------------------
# The rest of a decode layer
# ---------------------------------------------------------------------------
def rope(x: np.ndarray, rows: int, heads: int, dim: int, position: int, theta: float) -> np.ndarray:
    """QwenCPUApplyRoPE (QwenHybrid.CPU.pas:51-67), rows at position + row; returns a rotated copy."""
    y = np.array(x, np.float32, copy=True).reshape(-1)
    _check(lib().qo_rope(_p(y, _f32p), rows, heads, dim, position, theta), "rope")
    return y


def cache_write(cache: np.ndarray, k: np.ndarray, v: np.ndarray, rows: int, kv_heads: int, dim: int, cap: int,
                position: int) -> None:
    """KV-cache append (QwenHybrid.CPU.pas:198-204, tensor.comp:313-317), in place."""
    k = np.ascontiguousarray(k, np.float32).reshape(-1)
    v = np.ascontiguousarray(v, np.float32).reshape(-1)
    _check(lib().qo_cache_write(_p(cache, _f32p), _p(k, _f32p), _p(v, _f32p), rows, kv_heads, dim, cap, position),
           "cache_write")


def cached_attention(q, cache, rows, cap, heads, kv_heads, dim, position, window=0, softcap=0.0, scale=0.0,
                     masked=False) -> np.ndarray:
    """CachedAttention (attention.comp mask modes 2 and 4) in double."""
    q = np.ascontiguousarray(q, np.float32).reshape(-1)
    cache = np.ascontiguousarray(cache, np.float32).reshape(-1)
    out = np.empty(rows * heads * dim, np.float32)
    _check(lib().qo_cached_attention(_p(q, _f32p), _p(cache, _f32p), rows, cap, heads, kv_heads, dim, position, window,
                                     softcap, scale, int(masked), _p(out, _f32p)), "cached_attention")
    return out


def sample_topk(logits, seen, k: int, penalty: float = 1.0):
    """SampleToken's ranked top-k: (scores, ids)."""
    logits = np.ascontiguousarray(logits, np.float32)
    seen = np.ascontiguousarray(seen, np.uint32)
    s = np.empty(k, np.float32)
    i = np.empty(k, np.uint32)
    _check(lib().qo_sample_topk(_p(logits, _f32p), _p(seen, _u32p), logits.size, k, penalty, _p(s, _f32p),
                                _p(i, _u32p)), "sample_topk")
    return s, i


def sample_token(logits, seen, top_k: int, temperature: float, top_p: float, penalty: float, uniform: float) -> int:
    """SampleToken (Context.Implementation.inc:1137-1187, tensor.comp:177-197)."""
    logits = np.ascontiguousarray(logits, np.float32)
    seen = np.ascontiguousarray(seen, np.uint32)
    return int(lib().qo_sample_token(_p(logits, _f32p), _p(seen, _u32p), logits.size, top_k, temperature, top_p,
                                     penalty, uniform))
