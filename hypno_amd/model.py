"""Python mirror of hypno's `.hypno` reader (loader.rs:20-169, format.rs).

    HypnoModel.open(path)              HypnoModel::open (loader.rs:39)
    model.manifest                     HypnoManifest (format.rs:100-105)
    model.get_tensor_data(name)        loader.rs:139  -> (memoryview, DType) | None
    model.find_tensor(name)            loader.rs:151  -> TensorMeta | None
    model.get_metadata(key)            loader.rs:158  -> str | None
    model.is_col_major()               loader.rs:166

Parsing, the read-only mapping and the upload of every payload to HBM all
happen in libhypno_hip (hypno_hip_model_*).  `device_tensor(name)` returns
the device copy as (pointer, length, DType), ready for the matmul entry
points; pass `device=False` to parse and map only.  A malformed file raises
FormatError with the reference's message for that FormatError variant; a
missing file raises FileNotFoundError.
"""
from __future__ import annotations

import ctypes
import dataclasses
from typing import List, Optional, Tuple

from ._lib import (EFILE, EFORMAT, ENOENT, MODEL_HOST_ONLY, HypnoHipError, TensorInfo, check,
                   load)
from .kernels import DType

__all__ = ["FormatError", "HypnoHeader", "MetaKV", "TensorMeta", "HypnoManifest", "HypnoModel"]


class FormatError(HypnoHipError):
    """format::FormatError (format.rs:109-131)."""


@dataclasses.dataclass(frozen=True)
class HypnoHeader:
    """format.rs:13-24 (the magic is validated on open)."""
    magic: bytes
    version: int
    metadata_kv_count: int
    tensor_count: int


@dataclasses.dataclass(frozen=True)
class MetaKV:
    key: str
    value: str


@dataclasses.dataclass(frozen=True)
class TensorMeta:
    """format.rs:60-73."""
    name: str
    ndim: int
    shape: Tuple[int, ...]
    dtype: DType
    offset: int
    data_len: int

    def num_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


@dataclasses.dataclass(frozen=True)
class HypnoManifest:
    header: HypnoHeader
    metadata: List[MetaKV]
    tensors: List[TensorMeta]


def _meta(info: TensorInfo) -> TensorMeta:
    shape = tuple(int(info.shape[i]) for i in range(info.ndim))
    return TensorMeta(info.name.decode(), int(info.ndim), shape, DType(info.dtype),
                      int(info.offset), int(info.data_len))


class HypnoModel:
    """A mapped `.hypno` file whose payloads are resident on the current device."""

    def __init__(self, handle: int, path: str, device: bool):
        self._h = ctypes.c_void_p(handle)
        self.path = path
        self.on_device = device
        lib = load()
        ver, kvs, nt = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        check(lib.hypno_hip_model_header(self._h, ctypes.byref(ver), ctypes.byref(kvs),
                                         ctypes.byref(nt)), "model_header")
        metadata = []
        for i in range(kvs.value):
            k, v = ctypes.c_char_p(), ctypes.c_char_p()
            check(lib.hypno_hip_model_metadata_at(self._h, i, ctypes.byref(k), ctypes.byref(v)),
                  "metadata_at")
            metadata.append(MetaKV(k.value.decode(), v.value.decode()))
        self._infos = []
        for i in range(nt.value):
            info = TensorInfo()
            check(lib.hypno_hip_model_tensor_at(self._h, i, ctypes.byref(info)), "tensor_at")
            self._infos.append(info)
        self.manifest = HypnoManifest(HypnoHeader(b"HYPN", ver.value, kvs.value, nt.value),
                                      metadata, [_meta(i) for i in self._infos])

    @classmethod
    def open(cls, path, device: bool = True) -> "HypnoModel":
        lib = load()
        h = ctypes.c_void_p()
        st = lib.hypno_hip_model_open(str(path).encode(), 0 if device else MODEL_HOST_ONLY,
                                      ctypes.byref(h))
        if st == ENOENT:
            raise FileNotFoundError(lib.hypno_hip_last_error().decode())
        if st == EFORMAT:
            raise FormatError(st, "HypnoModel.open")
        if st == EFILE:
            raise OSError(lib.hypno_hip_last_error().decode())
        check(st, "HypnoModel.open")
        return cls(h.value, str(path), device)

    def close(self) -> None:
        if self._h:
            check(load().hypno_hip_model_close(self._h), "model_close")
            self._h = None
            self._infos = []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _find(self, name: str) -> Optional[TensorInfo]:
        for info in self._infos:  # first match, like Iterator::find
            if info.name.decode() == name:
                return info
        return None

    def get_tensor_data(self, name: str) -> Optional[Tuple[memoryview, DType]]:
        """Zero-copy view of the tensor's bytes in the mapping (read-only)."""
        info = self._find(name)
        if info is None:
            return None
        n = int(info.data_len)
        buf = (ctypes.c_uint8 * n).from_address(info.host) if n else (ctypes.c_uint8 * 0)()
        return memoryview(buf).cast("B").toreadonly(), DType(info.dtype)

    def device_tensor(self, name: str) -> Optional[Tuple[int, int, DType]]:
        """(device pointer, byte length, dtype) of the tensor's HBM copy."""
        if not self.on_device:
            raise ValueError("model was opened with device=False")
        info = self._find(name)
        if info is None:
            return None
        return int(info.device or 0), int(info.data_len), DType(info.dtype)

    def find_tensor(self, name: str) -> Optional[TensorMeta]:
        info = self._find(name)
        return None if info is None else _meta(info)

    def get_metadata(self, key: str) -> Optional[str]:
        v = ctypes.c_char_p()
        st = load().hypno_hip_model_metadata(self._h, key.encode(), ctypes.byref(v))
        if st == ENOENT:
            return None
        check(st, "get_metadata")
        return v.value.decode()

    def is_col_major(self) -> bool:
        return bool(load().hypno_hip_model_is_col_major(self._h))
