"""Checkpoint files: safetensors and GGUF tables and the INT4 weight cache.

Python mirror of the library's checkpoint entry points (include/qnn_hip.h),
which restate the reference's readers:

* ``SafeTensorFiles.Open`` / ``LoadSafeTensorShards`` -- TSafeTensorFile.Open
  and LoadSafeTensorShards (src/io/QuickNN.SafeTensors.pas:522-690, :777-837);
  ``GetTensor`` / ``GetLinearWeight`` (:874-912);
* ``GGUFHeader.ReadFile`` -- TGGUFHeader (src/io/QuickNN.GGUF.pas:206-337);
* ``LLMInt4Cache`` -- TLLMInt4Cache (src/models/QuickNN.Models.LLM.Quantization.pas).

Weights come back as ``MemoryBlock`` views of the mapped files, ready for the
``GPUContext`` entry points; they are valid while their files stay open.
"""
from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass

import numpy as np

from . import hip
from .hip import _raise, _Weight, lib

# TSafeTensorType ordinals (SafeTensors.pas:34-77)
(ST_BOOL, ST_F4, ST_F6_E2M3, ST_F6_E3M2, ST_U8, ST_I8, ST_F8_E5M2, ST_F8_E4M3, ST_F8_E8M0, ST_I16, ST_U16,
 ST_F16, ST_BF16, ST_I32, ST_U32, ST_F32, ST_C64, ST_F64, ST_I64, ST_U64, ST_I4) = range(21)
ST_UNKNOWN = -1
IQ_EXPERTS, IQ_DENSE = 0, 1

_vp = ctypes.c_void_p


class _TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("data", _vp), ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("identity", ctypes.c_uint64), ("data_offset", ctypes.c_int64), ("data_size", ctypes.c_int64),
                ("ndim", ctypes.c_int32), ("st_dtype", ctypes.c_int32), ("dtype", ctypes.c_int32),
                ("encoding", ctypes.c_int32), ("file", ctypes.c_int32), ("storage_type", ctypes.c_uint32)]


class _FileInfo(ctypes.Structure):
    _fields_ = [("path", ctypes.c_char_p), ("architecture", ctypes.c_char_p), ("header_json", ctypes.c_char_p),
                ("data", _vp), ("file_size", ctypes.c_int64), ("header_size", ctypes.c_int64),
                ("data_size", ctypes.c_int64), ("offset", ctypes.c_int64), ("is_gguf", ctypes.c_int32),
                ("tensor_count", ctypes.c_int32)]


class _GGUFInfo(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("alignment", ctypes.c_uint32), ("data_offset", ctypes.c_int64),
                ("vocabulary_size", ctypes.c_int32), ("tensor_count", ctypes.c_int32),
                ("architecture", ctypes.c_char_p), ("metadata_json", ctypes.c_char_p)]


class _GGUFTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("shape", ctypes.POINTER(ctypes.c_int64)), ("offset", ctypes.c_int64),
                ("byte_size", ctypes.c_int64), ("ndim", ctypes.c_int32), ("storage_type", ctypes.c_uint32),
                ("encoding", ctypes.c_int32)]


@dataclass(frozen=True)
class SafeTensor:
    """TSafeTensor (SafeTensors.pas:149-180): one descriptor of an open file."""
    name: str
    shape: tuple
    st_dtype: int
    dtype: int
    encoding: int
    data_offset: int
    data_size: int
    identity: int
    file: int
    storage_type: int
    data: int  # address of the mapped bytes


@dataclass(frozen=True)
class SafeTensorFile:
    """TSafeTensorFile fields (SafeTensors.pas:184-197)."""
    path: str
    architecture: str
    header_json: bytes
    is_gguf: bool
    file_size: int
    header_size: int
    data_size: int
    offset: int
    tensor_count: int


def _tensor(info: _TensorInfo) -> SafeTensor:
    return SafeTensor(info.name.decode(), tuple(info.shape[i] for i in range(info.ndim)), info.st_dtype, info.dtype,
                      info.encoding, info.data_offset, info.data_size, info.identity, info.file, info.storage_type,
                      info.data or 0)


_NP = {ST_F32: np.float32, ST_F16: np.float16, ST_BF16: np.uint16, ST_U8: np.uint8, ST_I8: np.int8,
       ST_I16: np.int16, ST_U16: np.uint16, ST_I32: np.int32, ST_U32: np.uint32, ST_F64: np.float64,
       ST_I64: np.int64, ST_U64: np.uint64, ST_BOOL: np.uint8}


class SafeTensorFiles:
    """TSafeTensorFiles: the open files of one checkpoint, searched in order (GetTensor)."""

    def __init__(self, handle: int):
        self._h = handle

    @staticmethod
    def Open(path: str) -> "SafeTensorFiles":
        """TSafeTensorFile.Open: one safetensors or GGUF file."""
        h = _vp()
        _raise(lib().qnn_tensor_files_open(str(path).encode(), ctypes.byref(h)))
        return SafeTensorFiles(h.value)

    def close(self) -> None:
        if self._h:
            lib().qnn_tensor_files_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> int:
        if not self._h:
            raise hip.EInvalidOp("checkpoint files are closed")
        return self._h

    @property
    def files(self) -> list[SafeTensorFile]:
        n = ctypes.c_int()
        _raise(lib().qnn_tensor_files_count(self.handle, ctypes.byref(n)))
        out = []
        for i in range(n.value):
            fi = _FileInfo()
            _raise(lib().qnn_tensor_files_file(self.handle, i, ctypes.byref(fi)))
            out.append(SafeTensorFile(fi.path.decode(), fi.architecture.decode(), fi.header_json or b"",
                                      bool(fi.is_gguf), fi.file_size, fi.header_size, fi.data_size, fi.offset,
                                      fi.tensor_count))
        return out

    def Tensors(self, file: int = 0) -> list[SafeTensor]:
        """Tensors of one file in descriptor order."""
        out = []
        for i in range(self.files[file].tensor_count):
            info = _TensorInfo()
            _raise(lib().qnn_tensor_files_tensor(self.handle, file, i, ctypes.byref(info)))
            out.append(_tensor(info))
        return out

    def GetTensor(self, name: str) -> SafeTensor | None:
        info = _TensorInfo()
        rc = _raise(lib().qnn_tensor_files_find(self.handle, name.encode(), ctypes.byref(info)))
        return None if rc == hip.QNN_NOT_FOUND else _tensor(info)

    def GetLinearWeight(self, name: str) -> hip.MemoryBlock:
        """GetLinearWeight(Name, UseMMAP = True): the weight as the context takes it."""
        w = _Weight()
        _raise(lib().qnn_tensor_files_linear_weight(self.handle, name.encode(), ctypes.byref(w)))
        t = self.GetTensor(name)
        if w.encoding != hip.WE_NATIVE:
            nbytes = t.data_size
        else:
            nbytes = w.size * (2 if w.dtype == hip.DT_BF16 else 4)
        return hip.MemoryBlock.mapped(w.data, nbytes, (w.shape0, w.shape1), w.dtype, w.encoding, w.size, w.identity,
                                      self)

    def array(self, name: str) -> np.ndarray:
        """The mapped bytes of a tensor as a read-only numpy view (packed GGUF and 4/6-bit types as uint8)."""
        t = self.GetTensor(name)
        if t is None:
            raise hip.ESafeTensorError(f'Cannot find tensor "{name}"')
        raw = np.ctypeslib.as_array((ctypes.c_uint8 * max(t.data_size, 1)).from_address(t.data))[:t.data_size]
        raw.flags.writeable = False
        dt = _NP.get(t.st_dtype)
        if t.encoding != hip.WE_NATIVE or dt is None:
            return raw
        return raw.view(dt).reshape(t.shape)


def LoadSafeTensorShards(directory: str, index_file: str, single_file: str) -> SafeTensorFiles:
    """LoadSafeTensorShards (SafeTensors.pas:777-837)."""
    h = _vp()
    _raise(lib().qnn_tensor_files_open_shards(str(directory).encode(), index_file.encode(), single_file.encode(),
                                              ctypes.byref(h)))
    return SafeTensorFiles(h.value)


@dataclass(frozen=True)
class GGUFTensor:
    """TGGUFTensor (GGUF.pas:18-23)."""
    name: str
    shape: tuple
    storage_type: int
    offset: int
    byte_size: int
    encoding: int


@dataclass(frozen=True)
class GGUFHeader:
    """TGGUFHeader (GGUF.pas:26-34); ``metadata`` is None unless requested."""
    version: int
    alignment: int
    architecture: str
    data_offset: int
    vocabulary_size: int
    tensors: tuple
    metadata: dict | None

    @staticmethod
    def ReadFile(path: str, metadata: bool = False, include_vocabulary: bool = True) -> "GGUFHeader":
        h = _vp()
        _raise(lib().qnn_gguf_read_file(str(path).encode(), int(metadata), int(include_vocabulary), ctypes.byref(h)))
        try:
            info = _GGUFInfo()
            _raise(lib().qnn_gguf_header_get(h, ctypes.byref(info)))
            tensors = []
            for i in range(info.tensor_count):
                t = _GGUFTensor()
                _raise(lib().qnn_gguf_header_tensor(h, i, ctypes.byref(t)))
                tensors.append(GGUFTensor(t.name.decode(), tuple(t.shape[j] for j in range(t.ndim)),
                                          t.storage_type, t.offset, t.byte_size, t.encoding))
            meta = json.loads(info.metadata_json.decode()) if metadata else None
            return GGUFHeader(info.version, info.alignment, info.architecture.decode(), info.data_offset,
                              info.vocabulary_size, tuple(tensors), meta)
        finally:
            lib().qnn_gguf_header_free(h)


class LLMInt4Cache:
    """TLLMInt4Cache (LLM.Quantization.pas:13-28): packed INT4 matrices of a checkpoint, built on first use."""

    def __init__(self, sources: SafeTensorFiles, directory: str, progress=None, scope: int = IQ_EXPERTS):
        h = _vp()
        cb = hip._PROGRESS(lambda done, total, _u: progress(done, total)) if progress else hip._PROGRESS()
        _raise(lib().qnn_int4_cache_create(sources.handle, str(directory).encode(), cb, None, scope, ctypes.byref(h)))
        self._h = h.value

    def close(self) -> None:
        if self._h:
            lib().qnn_int4_cache_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def Directory(self) -> str:
        return lib().qnn_int4_cache_directory(self._h).decode()

    def Weight(self, name: str, rows: int, columns: int) -> hip.MemoryBlock:
        w = _Weight()
        _raise(lib().qnn_int4_cache_weight(self._h, name.encode(), rows, columns, ctypes.byref(w)))
        return hip.MemoryBlock.mapped(w.data, w.size, (w.shape0, w.shape1), w.dtype, w.encoding, w.size, w.identity,
                                      self)

    def MappedBytes(self) -> int:
        n = ctypes.c_uint64()
        _raise(lib().qnn_int4_cache_mapped_bytes(self._h, ctypes.byref(n)))
        return n.value

    @staticmethod
    def SourceFingerprint(sources: SafeTensorFiles) -> str:
        buf = ctypes.create_string_buffer(65)
        _raise(lib().qnn_int4_source_fingerprint(sources.handle, buf))
        return buf.value.decode()


# The reference keeps the old name for MoE callers (LLM.Quantization.pas:30-31).
MoEInt4Cache = LLMInt4Cache
