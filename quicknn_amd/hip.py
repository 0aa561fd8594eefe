"""Python mirror of the HIP backend's C ABI (include/qnn_hip.h).

``GPUContext`` follows the resident context QuickNN's LLM engine calls,
TQNNGPUContext (src/backends/vulkan/QuickNN.Vulkan.Context.API.inc:14-165):
same method names, argument meaning and exception classes, so tests read like
the engine's own call sites.  ``MemoryBlock`` mirrors the TMemoryBlock weight
descriptor (src/core/QuickNN.Common.pas:135-155).

The library is loaded from the package directory; if it is missing the import
of this module raises -- there is no CPU fallback.
"""
from __future__ import annotations

import atexit
import ctypes
import itertools
import os
import struct

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqnn_hip.so")

# ---- status codes -> the reference's exception classes ----
QNN_OK = 0
QNN_NOT_HANDLED = 1
QNN_NOT_FOUND = 2
QNN_E_ARGUMENT = -1
QNN_E_RANGE = -2
QNN_E_NOT_SUPPORTED = -3
QNN_E_INVALID_OP = -4
QNN_E_FORMAT = -5
QNN_E_IO = -6


class QNNError(RuntimeError):
    code = 0


class EArgumentException(QNNError, ValueError):
    code = QNN_E_ARGUMENT


class ERangeError(QNNError):
    code = QNN_E_RANGE


class ENotSupportedException(QNNError):
    code = QNN_E_NOT_SUPPORTED


class EInvalidOp(QNNError):
    code = QNN_E_INVALID_OP


class ESafeTensorError(QNNError):
    """ESafeTensorError / EGGUFError: a malformed, stale or missing checkpoint entry."""
    code = QNN_E_FORMAT


class EInOutError(QNNError, OSError):
    """EFOpenError / EFCreateError / EInOutError: a file that cannot be opened or written."""
    code = QNN_E_IO


_ERRORS = {c.code: c for c in (EArgumentException, ERangeError, ENotSupportedException, EInvalidOp,
                               ESafeTensorError, EInOutError)}

# ---- TQNNDataType / TQNNWeightEncoding ordinals ----
DT_F16, DT_BF16, DT_F32, DT_S8, DT_U8 = 1, 2, 3, 5, 6
WE_NATIVE, WE_Q8_0, WE_Q4_K, WE_Q6_K, WE_Q3_K, WE_Q2_K = 0, 1, 2, 3, 4, 9
WE_Q5_K, WE_IQ4_NL, WE_IQ4_XS, WE_Q2_0 = 5, 6, 8, 12
WE_IQ3_S, WE_IQ2_XXS, WE_IQ2_S, WE_IQ3_XXS = 7, 10, 11, 13
GGUF_BLOCK = {WE_Q8_0: (32, 34), WE_Q4_K: (256, 144), WE_Q6_K: (256, 210), WE_Q3_K: (256, 110),
              WE_Q2_K: (256, 84), WE_Q5_K: (256, 176), WE_IQ4_NL: (32, 18), WE_IQ4_XS: (256, 136),
              WE_Q2_0: (64, 18), WE_IQ2_XXS: (256, 66), WE_IQ2_S: (256, 82), WE_IQ3_XXS: (256, 98),
              WE_IQ3_S: (256, 110)}

# ---- op codes (Context.API.inc:167-258) ----
GO_FILL, GO_NORM, GO_ADD, GO_SWIGLU, GO_FINITE = 0, 2, 4, 9, 13
GO_SCALE, GO_LLM_CACHE_WRITE, GO_LLM_ROPE, GO_LLM_SEEN = 43, 44, 45, 48
GO_MOE_ROUTE, GO_MOE_GATHER, GO_MOE_SCATTER, GO_GEGLU, GO_SOFTCAP = 52, 53, 54, 75, 76


class _Weight(ctypes.Structure):
    _fields_ = [("identity", ctypes.c_uint64), ("data", ctypes.c_void_p), ("offset", ctypes.c_int64),
                ("size", ctypes.c_int64), ("shape0", ctypes.c_int64), ("shape1", ctypes.c_int64),
                ("dtype", ctypes.c_int32), ("encoding", ctypes.c_int32)]


class Status(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "gemm_calls", "gguf_calls", "int4_calls", "moe_calls", "weight_uploads", "weight_upload_bytes",
        "weight_cache_hits", "weight_cache_misses", "weight_evictions", "readbacks", "submissions",
        "weight_bytes", "weight_limit", "activation_bytes", "activation_peak_bytes", "mlp_fused", "linear_grouped", "moe_fused", "moe_route_fused",
        "glu_fused", "async_weight_batches", "async_weight_bytes", "gemm_h16")]


_lib = None
_vp = ctypes.c_void_p
_ip = ctypes.POINTER(ctypes.c_int)
_EVICTED = ctypes.CFUNCTYPE(None, ctypes.c_uint64, ctypes.c_void_p)  # qnn_weight_evicted_fn
_PROGRESS = ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_int, ctypes.c_void_p)  # qnn_progress_fn


def lib():
    """Loads libqnn_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libqnn_hip.so not built at {LIB_PATH}: run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        W = ctypes.POINTER(_Weight)
        sig = {
            "qnn_last_error": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int]),
            "qnn_ctx_create": (ctypes.c_int, [ctypes.c_int, ctypes.c_uint64, ctypes.POINTER(_vp)]),
            "qnn_ctx_destroy": (ctypes.c_int, [_vp]),
            "qnn_get_status": (ctypes.c_int, [_vp, ctypes.POINTER(Status)]),
            "qnn_reload_tuning": (ctypes.c_int, []),
            "qnn_phase_trace": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]),
            "qnn_stream_read": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _vp]),
            "qnn_tensor_new": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.POINTER(_vp)]),
            "qnn_recycle": (ctypes.c_int, [_vp, ctypes.POINTER(_vp)]),
            "qnn_scratch": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_vp)]),
            "qnn_upload_raw": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.POINTER(_vp)]),
            "qnn_download": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int]),
            "qnn_copy": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "qnn_flush": (ctypes.c_int, [_vp]),
            "qnn_tensor_count": (ctypes.c_int, [_vp]),
            "qnn_tensor_device_ptr": (_vp, [_vp]),
            "qnn_retain_weight": (ctypes.c_int, [_vp, W, ctypes.c_int, ctypes.c_int]),
            "qnn_preload_weights": (ctypes.c_int, [_vp, W, ctypes.c_int, ctypes.c_uint64]),
            "qnn_is_weight_resident": (ctypes.c_int, [_vp, W, ctypes.c_int, ctypes.c_int, _ip]),
            "qnn_weight_batch_capacity": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_uint64)]),
            "qnn_set_weight_evicted": (ctypes.c_int, [_vp, _EVICTED, _vp]),
            "qnn_enable_weight_prefetch": (ctypes.c_int, [_vp, ctypes.c_uint64, _ip]),
            "qnn_begin_weight_prefetch": (ctypes.c_int, [_vp]),
            "qnn_prefetch_weights": (ctypes.c_int, [_vp, W, ctypes.c_int, ctypes.c_int]),
            "qnn_stage_weight_prefetch": (ctypes.c_int, [_vp, W, ctypes.c_int]),
            "qnn_complete_weight_prefetch": (ctypes.c_int, [_vp]),
            "qnn_activate_prefetched_weights": (ctypes.c_int, [_vp, W, ctypes.c_int, _ip]),
            "qnn_seal_weight_prefetch": (ctypes.c_int, [_vp]),
            "qnn_end_weight_prefetch": (ctypes.c_int, [_vp]),
            "qnn_upload": (ctypes.c_int, [_vp, W, ctypes.POINTER(_vp)]),
            "qnn_vector_linear": (ctypes.c_int, [_vp, _vp, _vp, W, ctypes.c_int, ctypes.c_int]),
            "qnn_linear": (ctypes.c_int, [_vp, _vp, _vp, W, W, W, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "qnn_int4_linear": (ctypes.c_int, [_vp, _vp, _vp, W, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "qnn_q8_gemm_int8": (ctypes.c_int, [_vp, _vp, _vp, W, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "qnn_int4_linear_noalloc": (ctypes.c_int, [_vp, _vp, _vp, W, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "qnn_swiglu_vector": (ctypes.c_int, [_vp, _vp, _vp, W, W, ctypes.c_int, ctypes.c_int]),
            "qnn_int4_linear_accumulate": (ctypes.c_int, [_vp, _vp, _vp, _vp, W, ctypes.c_int, ctypes.c_int,
                                                          ctypes.c_int]),
            "qnn_kernel": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp, _vp, _ip, ctypes.c_int]),
            "qnn_kernel_weights": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _vp, _vp, W, W, _ip,
                                                  ctypes.c_int]),
            "qnn_check_finite": (ctypes.c_int, [_vp, _vp, ctypes.c_int]),
            "qnn_cached_attention": (ctypes.c_int, [_vp, _vp, _vp, _vp] + [ctypes.c_int] * 7 +
                                     [ctypes.c_float, ctypes.c_float, ctypes.c_int]),
            "qnn_gather": (ctypes.c_int, [_vp, _vp, _vp, W, W, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "qnn_sample_token": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int, ctypes.c_int] +
                                 [ctypes.c_float] * 4),
            "qnn_expert_set_create": (ctypes.c_int, [_vp, W, W, W, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                     ctypes.POINTER(_vp)]),
            "qnn_expert_set_destroy": (ctypes.c_int, [_vp, _vp]),
            "qnn_moe_experts": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int, ctypes.c_int]),
            "qnn_dequantize": (ctypes.c_int, [_vp, _vp, W, ctypes.c_int, ctypes.c_int]),
            "qnn_event_record": (ctypes.c_int, [_vp, ctypes.c_int]),
            "qnn_event_elapsed_ms": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int,
                                                    ctypes.POINTER(ctypes.c_float)]),
            "qnn_graph_begin": (ctypes.c_int, [_vp]),
            "qnn_graph_end": (ctypes.c_int, [_vp, _ip]),
            "qnn_graph_launch": (ctypes.c_int, [_vp, ctypes.c_int]),
            "qnn_stream": (_vp, [_vp]),
            "qnn_int4_row_bytes": (ctypes.c_int, [ctypes.c_int]),
            "qnn_quantize_int4": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp]),
            "qnn_gguf_quantize": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.c_int64, _vp]),
            "qnn_tensor_files_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
            "qnn_tensor_files_open_shards": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                                                            ctypes.POINTER(_vp)]),
            "qnn_tensor_files_close": (ctypes.c_int, [_vp]),
            "qnn_tensor_files_count": (ctypes.c_int, [_vp, _ip]),
            "qnn_tensor_files_file": (ctypes.c_int, [_vp, ctypes.c_int, _vp]),
            "qnn_tensor_files_tensor": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _vp]),
            "qnn_tensor_files_find": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp]),
            "qnn_tensor_files_linear_weight": (ctypes.c_int, [_vp, ctypes.c_char_p, W]),
            "qnn_gguf_read_file": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_vp)]),
            "qnn_gguf_header_free": (ctypes.c_int, [_vp]),
            "qnn_gguf_header_get": (ctypes.c_int, [_vp, _vp]),
            "qnn_gguf_header_tensor": (ctypes.c_int, [_vp, ctypes.c_int, _vp]),
            "qnn_int4_cache_create": (ctypes.c_int, [_vp, ctypes.c_char_p, _PROGRESS, _vp, ctypes.c_int,
                                                     ctypes.POINTER(_vp)]),
            "qnn_int4_cache_destroy": (ctypes.c_int, [_vp]),
            "qnn_int4_cache_weight": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int, ctypes.c_int, W]),
            "qnn_int4_cache_mapped_bytes": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_uint64)]),
            "qnn_int4_cache_directory": (ctypes.c_char_p, [_vp]),
            "qnn_int4_source_fingerprint": (ctypes.c_int, [_vp, ctypes.c_char_p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


EXPORTED = (
    "qnn_last_error", "qnn_ctx_create", "qnn_ctx_destroy", "qnn_get_status", "qnn_reload_tuning", "qnn_phase_trace", "qnn_stream_read",
    "qnn_tensor_new",
    "qnn_recycle",
    "qnn_scratch", "qnn_upload_raw", "qnn_download", "qnn_copy", "qnn_flush", "qnn_tensor_count",
    "qnn_tensor_device_ptr", "qnn_retain_weight", "qnn_preload_weights", "qnn_is_weight_resident",
    "qnn_weight_batch_capacity", "qnn_set_weight_evicted", "qnn_enable_weight_prefetch", "qnn_begin_weight_prefetch",
    "qnn_prefetch_weights", "qnn_stage_weight_prefetch", "qnn_complete_weight_prefetch",
    "qnn_activate_prefetched_weights", "qnn_seal_weight_prefetch", "qnn_end_weight_prefetch", "qnn_upload", "qnn_vector_linear", "qnn_linear", "qnn_q8_gemm_int8", "qnn_int4_linear", "qnn_int4_linear_noalloc", "qnn_swiglu_vector",
    "qnn_int4_linear_accumulate", "qnn_kernel", "qnn_kernel_weights", "qnn_check_finite",
    "qnn_cached_attention", "qnn_sample_token", "qnn_gather",
    "qnn_expert_set_create", "qnn_expert_set_destroy", "qnn_moe_experts", "qnn_dequantize",
    "qnn_event_record", "qnn_event_elapsed_ms", "qnn_graph_begin", "qnn_graph_end", "qnn_graph_launch",
    "qnn_stream", "qnn_int4_row_bytes", "qnn_quantize_int4", "qnn_gguf_quantize",
    "qnn_tensor_files_open", "qnn_tensor_files_open_shards", "qnn_tensor_files_close", "qnn_tensor_files_count",
    "qnn_tensor_files_file", "qnn_tensor_files_tensor", "qnn_tensor_files_find", "qnn_tensor_files_linear_weight",
    "qnn_gguf_read_file", "qnn_gguf_header_free", "qnn_gguf_header_get", "qnn_gguf_header_tensor",
    "qnn_int4_cache_create", "qnn_int4_cache_destroy", "qnn_int4_cache_weight", "qnn_int4_cache_mapped_bytes",
    "qnn_int4_cache_directory", "qnn_int4_source_fingerprint",
)


def _raise(rc: int) -> int:
    if rc < 0:
        buf = ctypes.create_string_buffer(1024)
        lib().qnn_last_error(buf, 1024)
        raise _ERRORS.get(rc, QNNError)(buf.value.decode(errors="replace"))
    return rc


def float_bits(v: float) -> int:
    """QNNGPUFloatBits (Context.API.inc:166): reinterpret a float as an Integer argument."""
    return struct.unpack("<i", struct.pack("<f", v))[0]


# ---------------------------------------------------------------------------
# Weight descriptors
# ---------------------------------------------------------------------------
_identity = itertools.count(1)


class MemoryBlock:
    """TMemoryBlock view of host weight storage (Common.pas:135-155).

    ``identity`` plays the role of WeightIdentity: blocks with the same identity
    must hold the same immutable bytes.  Keep the array alive while the block
    may be uploaded.
    """

    def __init__(self, data: np.ndarray, shape, dtype: int, encoding: int = WE_NATIVE, offset: int = 0,
                 size: int | None = None, identity: int | None = None):
        self.data = np.ascontiguousarray(data)
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.encoding = encoding
        self.offset = offset
        self.size = int(size if size is not None else int(np.prod(self.shape)))
        self.identity = identity if identity is not None else next(_identity)

    def desc(self) -> _Weight:
        return _Weight(self.identity, self.data.ctypes.data, self.offset, self.size, self.shape[0],
                       self.shape[1] if len(self.shape) > 1 else 1, self.dtype, self.encoding)

    @staticmethod
    def mapped(ptr: int, nbytes: int, shape, dtype: int, encoding: int, size: int, identity: int,
               owner) -> "MemoryBlock":
        """A view of ``nbytes`` at ``ptr`` inside a mapping that ``owner`` keeps open (DataPtr of a
        TMemoryBlock returned with UseMMAP = True)."""
        view = np.ctypeslib.as_array((ctypes.c_uint8 * max(int(nbytes), 1)).from_address(ptr))
        b = MemoryBlock(view, shape, dtype, encoding, 0, size, identity)
        b.owner = owner
        return b

    @staticmethod
    def int4(packed: np.ndarray, **kw) -> "MemoryBlock":
        """Native INT4 cache matrix: dtU8 [N, Int4RowBytes(K)] (LLM.Quantization.pas:299-317)."""
        packed = np.ascontiguousarray(packed, np.uint8)
        return MemoryBlock(packed, packed.shape, DT_U8, WE_NATIVE, 0, packed.size, **kw)

    @staticmethod
    def gguf(blocks: np.ndarray, rows: int, cols: int, encoding: int, **kw) -> "MemoryBlock":
        """GGUF tensor: dtU8 with element shape [N, K] (SafeTensors.pas:874-890)."""
        blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
        return MemoryBlock(blocks, (rows, cols), DT_U8, encoding, 0, rows * cols, **kw)

    @staticmethod
    def matrix(values: np.ndarray, **kw) -> "MemoryBlock":
        """F32 [N, K] (float32) or BF16 [N, K] (uint16 bits) weight, e.g. the MoE router."""
        v = np.ascontiguousarray(values)
        dt = DT_BF16 if v.dtype == np.uint16 else DT_F32
        if dt == DT_F32:
            v = v.astype(np.float32, copy=False)
        return MemoryBlock(v, v.shape, dt, WE_NATIVE, 0, v.size, **kw)

    @staticmethod
    def vector(values: np.ndarray, **kw) -> "MemoryBlock":
        v = np.ascontiguousarray(values)
        dt = DT_BF16 if v.dtype == np.uint16 else DT_F32
        if dt == DT_F32:
            v = v.astype(np.float32, copy=False)
        return MemoryBlock(v, (v.size,), dt, WE_NATIVE, 0, v.size, **kw)


def _wd(w: MemoryBlock | None):
    return None if w is None else ctypes.byref(w.desc())


# ---------------------------------------------------------------------------
# Host utilities
# ---------------------------------------------------------------------------
def int4_row_bytes(cols: int) -> int:
    """Int4RowBytes (Quantization.Int4.pas:25-33)."""
    r = lib().qnn_int4_row_bytes(cols)
    if r < 0:
        raise EArgumentException("INT4 matrix width")
    return r


def quantize_int4(w: np.ndarray) -> np.ndarray:
    """QuantizeInt4 (Quantization.Int4.pas:96-144): fp32 or bf16 bits (uint16) [N, K] -> U8 [N, RowBytes]."""
    w = np.ascontiguousarray(w)
    dt = DT_BF16 if w.dtype == np.uint16 else DT_F32
    if dt == DT_F32:
        w = w.astype(np.float32, copy=False)
    rows, cols = w.shape
    out = np.empty((rows, int4_row_bytes(cols)), np.uint8)
    _raise(lib().qnn_quantize_int4(w.ctypes.data, dt, rows, cols, out.ctypes.data))
    return out


def gguf_quantize(encoding: int, w: np.ndarray) -> np.ndarray:
    """Synthetic GGML blocks of fp32 values (row-major, rows are whole blocks)."""
    w = np.ascontiguousarray(w, np.float32)
    elems, nbytes = GGUF_BLOCK[encoding]
    out = np.empty(w.size // elems * nbytes, np.uint8)
    _raise(lib().qnn_gguf_quantize(encoding, w.ctypes.data, w.size, out.ctypes.data))
    return out


# ---------------------------------------------------------------------------
# Resident context
# ---------------------------------------------------------------------------
class Tensor:
    """TQNNGPUTensor: context-owned fp32 device buffer of ``count`` floats."""

    __slots__ = ("handle", "count", "ctx")

    def __init__(self, ctx: "GPUContext", handle: int):
        self.ctx = ctx
        self.handle = handle
        self.count = lib().qnn_tensor_count(handle)

    @property
    def device_ptr(self) -> int:
        return lib().qnn_tensor_device_ptr(self.handle)


def _th(t: Tensor | None):
    return None if t is None else t.handle


# Contexts still open when the interpreter exits are destroyed by an atexit
# hook, before the HIP runtime's own teardown (a context left alive into
# process exit races that teardown: its stream, events, graphs and pinned
# readback buffer would be released by a runtime that is shutting down).
_open_contexts: set = set()


@atexit.register
def _close_open_contexts() -> None:
    for c in list(_open_contexts):
        try:
            c.close()
        except Exception:  # created on another thread, or the runtime already failed
            _open_contexts.discard(c)


def reload_tuning() -> None:
    """qnn_reload_tuning: re-read the QNN_* tuning switches from the environment (the
    library reads them once when a context is created)."""
    _raise(lib().qnn_reload_tuning())


class GPUContext:
    """TQNNGPUContext over libqnn_hip.so (one per process, bound to its creating thread)."""

    def __init__(self, device: int = 0, weight_cache_bytes: int = 0):
        h = _vp()
        _raise(lib().qnn_ctx_create(device, weight_cache_bytes, ctypes.byref(h)))
        self.h = h.value
        self._evicted_cb = self._evicted_fn = None
        _open_contexts.add(self)

    # -- lifetime
    def close(self) -> None:
        if self.h:
            _raise(lib().qnn_ctx_destroy(self.h))
            self.h = None
        _open_contexts.discard(self)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def status(self) -> Status:
        s = Status()
        _raise(lib().qnn_get_status(self.h, ctypes.byref(s)))
        return s

    def StreamRead(self, src: Tensor, count: int, dst: Tensor) -> None:
        """qnn_stream_read: one plain streaming read of count floats of src (diagnostic)."""
        _raise(lib().qnn_stream_read(self.h, src.handle, count, dst.handle))

    def PhaseTrace(self, kernel: str = "mlp"):
        """qnn_phase_trace: [2048, 16] uint64 phase timestamps of the fused MLP kernel ("mlp"), the
        one-token MoE kernel ("moe") or the LDS-streamed attention kernel ("attn") (trace builds
        only); all three are cleared afterwards."""
        import numpy as np

        buf = np.zeros((3, 2048, 16), np.uint64)
        n = ctypes.c_uint64()
        _raise(lib().qnn_phase_trace(self.h, ctypes.c_void_p(buf.ctypes.data), buf.size, ctypes.byref(n)))
        return buf[{"mlp": 0, "moe": 1, "attn": 2}[kernel]]

    # -- tensors
    def NewTensor(self, count: int) -> Tensor:
        h = _vp()
        _raise(lib().qnn_tensor_new(self.h, count, ctypes.byref(h)))
        return Tensor(self, h.value)

    def Recycle(self, t: Tensor) -> None:
        h = _vp(t.handle)
        _raise(lib().qnn_recycle(self.h, ctypes.byref(h)))

    def Scratch(self, slot: int, count: int) -> Tensor:
        h = _vp()
        _raise(lib().qnn_scratch(self.h, slot, count, ctypes.byref(h)))
        return Tensor(self, h.value)

    def UploadRaw(self, data: np.ndarray) -> Tensor:
        a = np.ascontiguousarray(data)
        if a.dtype.itemsize != 4:
            a = a.astype(np.float32)
        h = _vp()
        _raise(lib().qnn_upload_raw(self.h, a.ctypes.data, a.size, ctypes.byref(h)))
        return Tensor(self, h.value)

    def Upload(self, data: MemoryBlock) -> Tensor:
        """Upload(TMemoryBlock) (Context.Implementation.inc:700-705): F32 storage only."""
        h = _vp()
        _raise(lib().qnn_upload(self.h, _wd(data), ctypes.byref(h)))
        return Tensor(self, h.value)

    def Download(self, t: Tensor, count: int = -1, dtype=np.float32) -> np.ndarray:
        n = t.count if count < 0 else count
        out = np.empty(n, dtype)
        _raise(lib().qnn_download(self.h, t.handle, out.ctypes.data, n))
        return out

    def Copy(self, dst: Tensor, src: Tensor, count: int, dst_offset: int = 0, src_offset: int = 0) -> None:
        _raise(lib().qnn_copy(self.h, dst.handle, src.handle, count, dst_offset, src_offset))

    def Flush(self) -> None:
        _raise(lib().qnn_flush(self.h))

    # -- weights
    def RetainWeight(self, w: MemoryBlock, rows: int, cols: int) -> None:
        _raise(lib().qnn_retain_weight(self.h, _wd(w), rows, cols))

    def PreloadWeights(self, ws, staging_limit: int = 134217728) -> None:
        arr = (_Weight * len(ws))(*[w.desc() for w in ws])
        _raise(lib().qnn_preload_weights(self.h, arr, len(ws), staging_limit))

    def IsWeightResident(self, w: MemoryBlock, rows: int, cols: int) -> bool:
        r = ctypes.c_int()
        _raise(lib().qnn_is_weight_resident(self.h, _wd(w), rows, cols, ctypes.byref(r)))
        return bool(r.value)

    @property
    def OnWeightEvicted(self):
        """OnWeightEvicted (Context.API.inc:164): fn(identity) per evicted cache entry, or None."""
        return self._evicted_fn

    @OnWeightEvicted.setter
    def OnWeightEvicted(self, fn) -> None:
        cb = None if fn is None else _EVICTED(lambda ident, _user: fn(int(ident)))
        _raise(lib().qnn_set_weight_evicted(self.h, cb if cb is not None else _EVICTED(), None))
        self._evicted_cb, self._evicted_fn = cb, fn  # the C side keeps the pointer: hold the thunk

    # -- asynchronous layer prefetch (Context.API.inc:88-95)
    @staticmethod
    def _wlist(ws):
        return (_Weight * len(ws))(*[w.desc() for w in ws]), len(ws)

    def EnableWeightPrefetch(self, max_layer_bytes: int) -> bool:
        r = ctypes.c_int()
        _raise(lib().qnn_enable_weight_prefetch(self.h, max_layer_bytes, ctypes.byref(r)))
        return bool(r.value)

    def BeginWeightPrefetch(self) -> None:
        _raise(lib().qnn_begin_weight_prefetch(self.h))

    def PrefetchWeights(self, ws, defer_join: bool = False) -> None:
        arr, n = self._wlist(ws)
        _raise(lib().qnn_prefetch_weights(self.h, arr, n, int(defer_join)))

    def StageWeightPrefetch(self, ws) -> None:
        arr, n = self._wlist(ws)
        _raise(lib().qnn_stage_weight_prefetch(self.h, arr, n))

    def CompleteWeightPrefetch(self) -> None:
        _raise(lib().qnn_complete_weight_prefetch(self.h))

    def ActivatePrefetchedWeights(self, ws) -> bool:
        arr, n = self._wlist(ws)
        r = ctypes.c_int()
        _raise(lib().qnn_activate_prefetched_weights(self.h, arr, n, ctypes.byref(r)))
        return bool(r.value)

    def SealWeightPrefetch(self) -> None:
        _raise(lib().qnn_seal_weight_prefetch(self.h))

    def EndWeightPrefetch(self) -> None:
        _raise(lib().qnn_end_weight_prefetch(self.h))

    def WeightBatchCapacity(self) -> int:
        v = ctypes.c_uint64()
        _raise(lib().qnn_weight_batch_capacity(self.h, ctypes.byref(v)))
        return v.value

    # -- hot-path ops
    def Linear(self, dst: Tensor, src: Tensor, weight: MemoryBlock, scales: MemoryBlock | None,
               bias: MemoryBlock | None, rows: int, input_dim: int, output_dim: int) -> None:
        _raise(lib().qnn_linear(self.h, dst.handle, src.handle, _wd(weight), _wd(scales), _wd(bias), rows,
                                input_dim, output_dim))

    def Q8GemmInt8(self, dst: Tensor, src: Tensor, weight: MemoryBlock, rows: int, input_dim: int,
                   output_dim: int) -> None:
        """qnn_q8_gemm_int8: Q8_0 projection with per-32 int8 activations on the int8 matrix cores."""
        _raise(lib().qnn_q8_gemm_int8(self.h, dst.handle, src.handle, _wd(weight), rows, input_dim, output_dim))

    def VectorLinear(self, dst: Tensor, src: Tensor, weight: MemoryBlock, input_dim: int, output_dim: int) -> None:
        _raise(lib().qnn_vector_linear(self.h, dst.handle, src.handle, _wd(weight), input_dim, output_dim))

    def Int4Linear(self, dst: Tensor, src: Tensor, weight: MemoryBlock, rows: int, input_dim: int,
                   output_dim: int) -> None:
        _raise(lib().qnn_int4_linear(self.h, dst.handle, src.handle, _wd(weight), rows, input_dim, output_dim))

    def TrySwiGLUVector(self, dst: Tensor, src: Tensor, gate: MemoryBlock, up: MemoryBlock, input_dim: int,
                        output_dim: int) -> bool:
        rc = _raise(lib().qnn_swiglu_vector(self.h, dst.handle, src.handle, _wd(gate), _wd(up), input_dim,
                                            output_dim))
        return rc == QNN_OK

    def Int4LinearNoAlloc(self, dst: Tensor, src: Tensor, weight: MemoryBlock, rows: int, input_dim: int,
                          output_dim: int) -> None:
        """qnn_int4_linear_noalloc: Int4Linear without device allocation (resident weight, fixed scratch)."""
        _raise(lib().qnn_int4_linear_noalloc(self.h, dst.handle, src.handle, _wd(weight), rows, input_dim,
                                             output_dim))

    def Int4LinearAccumulate(self, dst: Tensor, src: Tensor, probabilities: Tensor, weight: MemoryBlock,
                             input_dim: int, output_dim: int, probability_index: int) -> None:
        _raise(lib().qnn_int4_linear_accumulate(self.h, dst.handle, src.handle, probabilities.handle, _wd(weight),
                                                input_dim, output_dim, probability_index))

    def Kernel(self, op: int, n: int, dst: Tensor | None, a: Tensor | None, b: Tensor | None, c: Tensor | None,
               args) -> None:
        arr = (ctypes.c_int * max(1, len(args)))(*args)
        _raise(lib().qnn_kernel(self.h, op, n, _th(dst), _th(a), _th(b), _th(c), arr, len(args)))

    def KernelWeights(self, op: int, n: int, dst: Tensor, a: Tensor, b: MemoryBlock | None,
                      c: MemoryBlock | None, args) -> None:
        arr = (ctypes.c_int * max(1, len(args)))(*args)
        _raise(lib().qnn_kernel_weights(self.h, op, n, dst.handle, a.handle, _wd(b), _wd(c), arr, len(args)))

    def CachedAttention(self, dst: Tensor, q: Tensor, cache: Tensor, query_rows: int, capacity: int, heads: int,
                        kv_heads: int, dim: int, position: int, window: int = 0, softcap: float = 0.0,
                        scale: float = 0.0, masked: bool = False) -> None:
        """CachedAttention (Context.API.inc:142-146)."""
        _raise(lib().qnn_cached_attention(self.h, dst.handle, q.handle, cache.handle, query_rows, capacity, heads,
                                          kv_heads, dim, position, window, softcap, scale, int(masked)))

    def Gather(self, dst: Tensor, ids: Tensor, weight: MemoryBlock, scales: MemoryBlock | None, rows: int, dim: int,
               vocab: int, rotation: int = 0) -> None:
        """Gather (Context.API.inc:147-151): embedding rows by token id."""
        _raise(lib().qnn_gather(self.h, dst.handle, ids.handle, _wd(weight), _wd(scales), rows, dim, vocab, rotation))

    def SampleToken(self, dst: Tensor, logits: Tensor, seen: Tensor, vocab: int, top_k: int, temperature: float,
                    top_p: float, penalty: float, uniform: float) -> None:
        """SampleToken (Context.API.inc:136-140): dst[0] receives the token id as raw bits."""
        _raise(lib().qnn_sample_token(self.h, dst.handle, logits.handle, seen.handle, vocab, top_k, temperature, top_p,
                                      penalty, uniform))

    def CheckFinite(self, t: Tensor, count: int = -1) -> None:
        _raise(lib().qnn_check_finite(self.h, t.handle, count))

    # -- routed experts on the device
    def CreateExpertSet(self, gates, ups, downs, hidden: int, inter: int) -> int:
        E = len(gates)
        mk = lambda ws: (_Weight * E)(*[w.desc() for w in ws])
        h = _vp()
        _raise(lib().qnn_expert_set_create(self.h, mk(gates), mk(ups), mk(downs), E, hidden, inter,
                                           ctypes.byref(h)))
        return h.value

    def DestroyExpertSet(self, s: int) -> None:
        _raise(lib().qnn_expert_set_destroy(self.h, s))

    def MoEExperts(self, expert_set: int, dst: Tensor, src: Tensor, routes: Tensor, rows: int, topk: int) -> None:
        _raise(lib().qnn_moe_experts(self.h, expert_set, dst.handle, src.handle, routes.handle, rows, topk))

    # -- diagnostics
    def Dequantize(self, dst: Tensor, w: MemoryBlock, rows: int, cols: int) -> None:
        _raise(lib().qnn_dequantize(self.h, dst.handle, _wd(w), rows, cols))

    def EventRecord(self, slot: int) -> None:
        _raise(lib().qnn_event_record(self.h, slot))

    def EventElapsedMs(self, a: int, b: int) -> float:
        v = ctypes.c_float()
        _raise(lib().qnn_event_elapsed_ms(self.h, a, b, ctypes.byref(v)))
        return v.value

    def GraphBegin(self) -> None:
        _raise(lib().qnn_graph_begin(self.h))

    def GraphEnd(self) -> int:
        g = ctypes.c_int()
        _raise(lib().qnn_graph_end(self.h, ctypes.byref(g)))
        return g.value

    def GraphLaunch(self, graph_id: int) -> None:
        _raise(lib().qnn_graph_launch(self.h, graph_id))
