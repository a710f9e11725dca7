"""Loads libhypno_hip.so (built in-tree by hypno_amd.build) through ctypes.

There is no fallback: if the library is missing or does not export a symbol
of include/hypno_hip.h, importing the matmul API raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhypno_hip.so")

# Every entry point of include/hypno_hip.h: name -> (restype, argtypes).
_vp, _sz, _i, _u32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint32
SIGNATURES = {
    "hypno_hip_abi_version": (_i, []),
    "hypno_hip_strerror": (ctypes.c_char_p, [_i]),
    "hypno_hip_last_error": (ctypes.c_char_p, []),
    "hypno_hip_device_count": (_i, []),
    "hypno_hip_matmul_q4_0": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz]),
    "hypno_hip_matmul_f16": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz]),
    "hypno_hip_matmul_q8_0": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz]),
    "hypno_hip_matmul_vec_auto": (_i, [_vp, _vp, _sz, _u32, _vp, _vp, _sz, _sz]),
    "hypno_hip_batch_matmul": (_i, [_vp, _vp, _sz, _u32, _vp, _sz, _sz, _sz]),
    "hypno_hip_matmul_q4_0_col": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz]),
    "hypno_hip_matmul_vec_col": (_i, [_vp, _vp, _sz, _u32, _vp, _vp, _sz, _sz]),
    "hypno_hip_batch_matmul_col": (_i, [_vp, _vp, _sz, _u32, _vp, _sz, _sz, _sz]),
    "hypno_hip_matmul_q4_0_col_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _vp]),
    "hypno_hip_weight_register": (_i, [_vp, _sz]),
    "hypno_hip_weight_unregister": (_i, [_vp]),
    "hypno_hip_matmul_q4_0_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _vp]),
    "hypno_hip_matmul_q4_0_dev_noalloc": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _vp]),
    "hypno_hip_matmul_f16_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _vp]),
    "hypno_hip_matmul_q8_0_dev": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _vp]),
    "hypno_hip_quantize_q8_0_dev": (_i, [_vp, _vp, _sz, _vp]),
    "hypno_hip_dequantize_q8_0_dev": (_i, [_vp, _vp, _sz, _vp]),
    "hypno_hip_quantize_q4_0_dev": (_i, [_vp, _vp, _sz, _vp]),
    "hypno_hip_dequantize_q4_0_dev": (_i, [_vp, _vp, _sz, _vp]),
    "hypno_hip_q4_0_gemv_plan_create": (_i, [_vp, _sz, _vp]),
    "hypno_hip_q4_0_gemv_plan_run": (_i, [_vp, _vp]),
    "hypno_hip_q4_0_gemv_plan_launches": (_i, [_vp]),
    "hypno_hip_q4_0_gemv_plan_destroy": (_i, [_vp]),
    "hypno_hip_q4_0_gemv_plan_create_ex": (_i, [_vp, _vp, _sz, _vp]),
    "hypno_hip_rms_norm_dev": (_i, [_vp, _vp, _vp, _sz, _sz, ctypes.c_float, _vp]),
    "hypno_hip_silu_mul_dev": (_i, [_vp, _vp, _vp, _sz, _vp]),
    "hypno_hip_stream_synchronize": (_i, [_vp]),
    "hypno_hip_set_gemm_numerics": (_i, [_u32]),
    "hypno_hip_q4_0_extract_row_dev": (_i, [_vp, _vp, _sz, _sz, _sz, _vp]),
    "hypno_hip_q8_0_extract_row_dev": (_i, [_vp, _vp, _sz, _sz, _sz, _vp]),
    "hypno_hip_embed_tokens_dev": (_i, [_vp, _vp, _sz, _u32, _vp, _sz, _sz, _vp]),
    "hypno_hip_argmax_dev": (_i, [_vp, _vp, _sz, _vp]),
    "hypno_hip_sample_token_dev": (_i, [_vp, _vp, _vp, _sz, ctypes.c_float, ctypes.c_float,
                                        _sz, _vp]),
    "hypno_hip_model_open": (_i, [ctypes.c_char_p, _u32, ctypes.POINTER(_vp)]),
    "hypno_hip_model_close": (_i, [_vp]),
    "hypno_hip_model_header": (_i, [_vp, ctypes.POINTER(_u32), ctypes.POINTER(_u32),
                                    ctypes.POINTER(_u32)]),
    "hypno_hip_model_metadata_at": (_i, [_vp, _sz, ctypes.POINTER(ctypes.c_char_p),
                                         ctypes.POINTER(ctypes.c_char_p)]),
    "hypno_hip_model_metadata": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]),
    "hypno_hip_model_tensor_at": (_i, [_vp, _sz, _vp]),
    "hypno_hip_model_find_tensor": (_i, [_vp, ctypes.c_char_p, _vp]),
    "hypno_hip_model_is_col_major": (_i, [_vp]),
}


class GemvDesc(ctypes.Structure):
    """struct hypno_hip_gemv_desc of include/hypno_hip.h."""
    _fields_ = [("y", ctypes.c_void_p), ("w_q", ctypes.c_void_p), ("w_len", ctypes.c_size_t),
                ("x", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("n", ctypes.c_size_t),
                ("m", ctypes.c_size_t)]

class GemvPrologue(ctypes.Structure):
    """struct hypno_hip_gemv_prologue of include/hypno_hip.h."""
    _fields_ = [("kind", ctypes.c_uint32), ("aux", ctypes.c_void_p), ("eps", ctypes.c_float)]


PROLOGUE_NONE, PROLOGUE_RMS_NORM, PROLOGUE_SILU_MUL = 0, 1, 2


class TensorInfo(ctypes.Structure):
    """struct hypno_hip_tensor_info of include/hypno_hip.h."""
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_uint32), ("ndim", ctypes.c_uint32),
                ("shape", ctypes.POINTER(ctypes.c_uint64)), ("offset", ctypes.c_uint64),
                ("data_len", ctypes.c_uint64), ("host", ctypes.c_void_p),
                ("device", ctypes.c_void_p)]


MODEL_HOST_ONLY = 1  # HYPNO_HIP_MODEL_HOST_ONLY
ENOENT, EFILE, EFORMAT = 2, 9, 74  # HYPNO_HIP_ENOENT / _EFILE / _EFORMAT

_lib = None


class HypnoHipError(RuntimeError):
    """A non-zero status from libhypno_hip (the reference panics instead)."""

    def __init__(self, status: int, where: str):
        lib = _lib
        detail = lib.hypno_hip_last_error().decode() if lib else ""
        name = lib.hypno_hip_strerror(status).decode() if lib else str(status)
        super().__init__(f"{where}: {name} (status {status}): {detail}")
        self.status = status


def load():
    """Return the loaded library; raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m hypno_amd.build` "
            "(hypno_amd has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the export is missing
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int, where: str) -> None:
    if status != 0:
        raise HypnoHipError(status, where)
