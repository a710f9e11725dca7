"""ctypes view of the CPU oracle (oracle/q4_0_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline.  Only
tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg import
this module; the product package ``hypno_amd`` never does.

Each wrapper names the hypno function it restates (crates/hypno/src/...).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle_q4.so")

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc only; seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, fp = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f16_to_f32.restype = fp
    L.orc_f32_to_f16.argtypes = [fp]
    L.orc_f32_to_f16.restype = ctypes.c_uint16
    L.orc_f16_to_f32_array.argtypes = [vp, vp, sz]
    L.orc_f32_to_f16_array.argtypes = [vp, vp, sz]
    L.orc_quantize_q4_0.argtypes = [vp, sz, vp]
    L.orc_quantize_q4_0.restype = sz
    L.orc_dequantize_q4_0.argtypes = [vp, sz, vp]
    L.orc_dequantize_q4_0.restype = sz
    for name in ("orc_rms_norm_avx2", "orc_rms_norm_scalar"):
        getattr(L, name).argtypes = [vp, vp, sz, fp]
        getattr(L, name).restype = None
    L.orc_rms_norm.argtypes = [vp, vp, sz, sz, fp]
    L.orc_rms_norm.restype = None
    L.orc_batch_rms_norm.argtypes = [vp, vp, vp, sz, sz, fp]
    L.orc_batch_rms_norm.restype = None
    L.orc_silu_mul.argtypes = [vp, vp, vp, sz]
    L.orc_silu_mul.restype = None
    L.orc_quantize_q8_0.argtypes = [vp, sz, vp]
    L.orc_quantize_q8_0.restype = sz
    L.orc_dequantize_q8_0.argtypes = [vp, sz, vp]
    L.orc_dequantize_q8_0.restype = sz
    L.orc_matmul_q8_0.argtypes = [vp, vp, sz, vp, vp, sz, sz]
    L.orc_matmul_q8_0.restype = ctypes.c_int
    L.orc_matmul_q8_0_f64.argtypes = [vp, vp, sz, vp, vp, sz, sz]
    L.orc_matmul_q8_0_f64.restype = None
    L.orc_matmul_q4_0_col.argtypes = [vp, vp, sz, vp, vp, sz, sz]
    L.orc_matmul_q4_0_col.restype = None
    L.orc_matmul_q4_0_col_f64.argtypes = [vp, vp, sz, vp, vp, sz, sz]
    L.orc_matmul_q4_0_col_f64.restype = None
    for name in ("orc_matmul_q4_0", "orc_matmul_q4_0_scalar", "orc_matmul_q4_0_avx2",
                 "orc_matmul_f16", "orc_matmul_f16_scalar", "orc_matmul_f16_avx2"):
        getattr(L, name).argtypes = [vp, vp, sz, vp, vp, sz, sz]
        getattr(L, name).restype = None
    L.orc_batch_matmul.argtypes = [vp, vp, sz, ctypes.c_int, vp, sz, sz, sz]
    L.orc_batch_matmul.restype = ctypes.c_int
    L.orc_matmul_q4_0_f64.argtypes = [vp, vp, sz, vp, vp, sz, sz]
    L.orc_matmul_f16_f64.argtypes = [vp, vp, vp, vp, sz, sz]
    L.orc_matmul_q4_0_absdot_f64.argtypes = [vp, vp, sz, vp, sz, sz]
    L.orc_f32_to_f16_f16c.argtypes = [vp, vp, sz]
    L.orc_f16_to_f32_f16c.argtypes = [vp, vp, sz]
    L.orc_xorshift64_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    L.orc_xorshift64_next.restype = ctypes.c_uint64
    L.orc_xorshift64_next_f32.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    L.orc_xorshift64_next_f32.restype = fp
    L.orc_argmax.argtypes = [vp, sz]
    L.orc_argmax.restype = ctypes.c_uint32
    L.orc_sample_token.argtypes = [vp, sz, fp, fp, sz, ctypes.POINTER(ctypes.c_uint64)]
    L.orc_sample_token.restype = ctypes.c_uint32
    L.orc_set_threads.argtypes = [ctypes.c_int]
    L.orc_have_avx2_fma.restype = ctypes.c_int
    L.orc_have_f16c.restype = ctypes.c_int
    _lib = L
    return L


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def have_avx2_fma() -> bool:
    return bool(lib().orc_have_avx2_fma())


# --- half 2.7.1 conversions (kernels.rs:297, quant.rs:26,57) ----------------

def f16_bits_to_f32(bits) -> np.ndarray:
    b = _c(bits, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(b), _p(out), b.size)
    return out


def f32_to_f16_bits(x) -> np.ndarray:
    a = _c(x, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(a), _p(out), a.size)
    return out


def f32_to_f16_bits_f16c(x) -> np.ndarray:
    """F16C hardware conversion (RNE), an independent cross-check."""
    a = _c(x, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f32_to_f16_f16c(_p(a), _p(out), a.size)
    return out


def f16_bits_to_f32_f16c(bits) -> np.ndarray:
    b = _c(bits, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_f16_to_f32_f16c(_p(b), _p(out), b.size)
    return out


# --- Q4_0 codec (quant.rs) ---------------------------------------------------

def quantize_q4_0(w) -> np.ndarray:
    """quantize_f32_to_q4_0 (quant.rs:108-117) over the flattened array."""
    a = _c(w, np.float32).ravel()
    out = np.empty((a.size // 32) * 18, np.uint8)
    lib().orc_quantize_q4_0(_p(a), a.size, _p(out))
    return out


def dequantize_q4_0(q) -> np.ndarray:
    """dequantize_q4_0 (quant.rs:120-132)."""
    b = _c(q, np.uint8).ravel()
    out = np.empty((b.size // 18) * 32, np.float32)
    lib().orc_dequantize_q4_0(_p(b), b.size, _p(out))
    return out


# --- matmul kernels (kernels.rs) -----------------------------------------------

def _gemv(fn, w, x, bias, n, m):
    w = _c(w, np.uint8).ravel()
    x = _c(x, np.float32).ravel()
    if x.size < m:
        raise ValueError("x shorter than m")
    b = None
    if bias is not None:
        b = _c(bias, np.float32).ravel()
        if b.size < n:
            raise ValueError("bias shorter than n")
    y = np.empty(n, np.float32)
    fn(_p(y), _p(w), w.size, _p(x), _p(b), n, m)
    return y


def matmul_q4_0(w_q, x, bias, n, m) -> np.ndarray:
    """matmul_q4_0 dispatch (kernels.rs:256-265): AVX2+FMA or scalar."""
    return _gemv(lib().orc_matmul_q4_0, w_q, x, bias, n, m)


def matmul_q4_0_scalar(w_q, x, bias, n, m) -> np.ndarray:
    """matmul_q4_0_scalar (kernels.rs:362-400)."""
    return _gemv(lib().orc_matmul_q4_0_scalar, w_q, x, bias, n, m)


def matmul_q4_0_avx2(w_q, x, bias, n, m) -> np.ndarray:
    """matmul_q4_0_avx2 (kernels.rs:270-359, hsum256 :169-178)."""
    return _gemv(lib().orc_matmul_q4_0_avx2, w_q, x, bias, n, m)


def matmul_f16(w, x, bias, n, m) -> np.ndarray:
    """matmul_f16 dispatch (kernels.rs:571-586)."""
    if np.asarray(w).nbytes < 2 * n * m:
        raise ValueError("w shorter than 2*n*m bytes")
    return _gemv(lib().orc_matmul_f16, w, x, bias, n, m)


def matmul_f16_scalar(w, x, bias, n, m) -> np.ndarray:
    return _gemv(lib().orc_matmul_f16_scalar, w, x, bias, n, m)


def batch_matmul(w, dtype: int, x, n, m, batch) -> np.ndarray:
    """turbo::batch_matmul Q4_0/FP16 arms (turbo.rs:306-333): one GEMV per token."""
    w = _c(w, np.uint8).ravel()
    x = _c(x, np.float32).ravel()
    if x.size < batch * m:
        raise ValueError("x shorter than batch*m")
    y = np.empty(batch * n, np.float32)
    rc = lib().orc_batch_matmul(_p(y), _p(w), w.size, int(dtype), _p(x), n, m, batch)
    if rc != 0:
        raise ValueError("unsupported dtype %r" % dtype)
    return y.reshape(batch, n)


def matmul_q4_0_f64(w_q, x, bias, n, m) -> np.ndarray:
    """fp64 brute force over the dequantised matrix (quant.rs:120-132)."""
    w = _c(w_q, np.uint8).ravel()
    x = _c(x, np.float32).ravel()
    b = _c(bias, np.float32).ravel() if bias is not None else None
    y = np.empty(n, np.float64)
    lib().orc_matmul_q4_0_f64(_p(y), _p(w), w.size, _p(x), _p(b), n, m)
    return y


def matmul_q4_0_absdot_f64(w_q, x, n, m) -> np.ndarray:
    w = _c(w_q, np.uint8).ravel()
    x = _c(x, np.float32).ravel()
    y = np.empty(n, np.float64)
    lib().orc_matmul_q4_0_absdot_f64(_p(y), _p(w), w.size, _p(x), n, m)
    return y


def matmul_f16_f64(w, x, bias, n, m) -> np.ndarray:
    w = _c(w, np.uint8).ravel()
    x = _c(x, np.float32).ravel()
    b = _c(bias, np.float32).ravel() if bias is not None else None
    y = np.empty(n, np.float64)
    lib().orc_matmul_f16_f64(_p(y), _p(w), _p(x), _p(b), n, m)
    return y


# --- seeded synthetic inputs ---------------------------------------------------

def normal_f32(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """N(0, std^2) fp32 from numpy's PCG64 with the given seed."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def normwise_err(y, ref) -> float:
    """max_i |y_i - r_i| / max_i |r_i| (the GEMV tolerance metric)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref)) if ref.size else 0.0
    if den == 0.0:
        return float(np.max(np.abs(y - ref))) if ref.size else 0.0
    return float(np.max(np.abs(y - ref)) / den)


def rel_l2(y, ref) -> float:
    """||Y - R||_2 / ||R||_2 (the GEMM tolerance metric)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(y - ref) / den) if den > 0 else float(np.linalg.norm(y - ref))


def rms_norm(x, weight, eps, rows=1) -> np.ndarray:
    """ops::rms_norm (ops.rs:52-55 -> kernels.rs:592-625) on `rows` rows; returns a copy."""
    y = _c(x, np.float32).ravel().copy()
    w = _c(weight, np.float32)
    n = y.size // rows
    lib().orc_rms_norm(_p(y), _p(w), n, rows, eps)
    return y


def rms_norm_variant(x, weight, eps, kind) -> np.ndarray:
    """One branch of rms_norm_fused: kind "avx2" (kernels.rs:599-619) or
    "scalar" (kernels.rs:621-624); one row."""
    y = _c(x, np.float32).ravel().copy()
    w = _c(weight, np.float32)
    fn = lib().orc_rms_norm_avx2 if kind == "avx2" else lib().orc_rms_norm_scalar
    fn(_p(y), _p(w), y.size, eps)
    return y


def batch_rms_norm(x, weight, dim, batch, eps) -> np.ndarray:
    """turbo::batch_rms_norm (turbo.rs:288-303), the f64-accumulating form."""
    a = _c(x, np.float32).ravel()
    w = _c(weight, np.float32)
    out = np.empty(dim * batch, np.float32)
    lib().orc_batch_rms_norm(_p(out), _p(a), _p(w), dim, batch, eps)
    return out


def silu_mul(gate, up) -> np.ndarray:
    """silu_in_place(gate); gate *= up (ops.rs:81-83, transformer.rs:446-449)."""
    g = _c(gate, np.float32).ravel()
    u = _c(up, np.float32).ravel()
    out = np.empty(g.size, np.float32)
    lib().orc_silu_mul(_p(out), _p(g), _p(u), g.size)
    return out


def quantize_q8_0(w) -> np.ndarray:
    """quantize_f32_to_q8_0 (quant.rs:177-191) over the flattened array."""
    a = _c(w, np.float32).ravel()
    out = np.empty((a.size // 32) * 34, np.uint8)
    lib().orc_quantize_q8_0(_p(a), a.size, _p(out))
    return out


def dequantize_q8_0(q) -> np.ndarray:
    """dequantize_q8_0 (quant.rs:194-206)."""
    b = _c(q, np.uint8).ravel()
    out = np.empty((b.size // 34) * 32, np.float32)
    lib().orc_dequantize_q8_0(_p(b), b.size, _p(out))
    return out


def matmul_q8_0(w_q, x, bias, n, m) -> np.ndarray:
    """ops::matmul_vec_auto's Q8_0 arm (ops.rs:33-36): dequantize, matmul_f32."""
    w = _c(w_q, np.uint8).ravel()
    xx = _c(x, np.float32).ravel()
    b = _c(bias, np.float32) if bias is not None else None
    y = np.empty(n, np.float32)
    rc = lib().orc_matmul_q8_0(_p(y), _p(w), w.size, _p(xx), _p(b), n, m)
    if rc != 0:
        raise ValueError("Q8_0 weights shorter than n*m elements (the reference panics)")
    return y


def matmul_q8_0_f64(w_q, x, bias, n, m) -> np.ndarray:
    w = _c(w_q, np.uint8).ravel()
    xx = _c(x, np.float32).ravel()
    b = _c(bias, np.float32) if bias is not None else None
    y = np.empty(n, np.float64)
    lib().orc_matmul_q8_0_f64(_p(y), _p(w), w.size, _p(xx), _p(b), n, m)
    return y


def matmul_q4_0_col(w_q, x, bias, n, m) -> np.ndarray:
    """matmul_q4_0_col_scalar (kernels.rs:506-535): W_col[m][n], y[n]."""
    w = _c(w_q, np.uint8).ravel()
    xx = _c(x, np.float32).ravel()
    b = _c(bias, np.float32) if bias is not None else None
    y = np.empty(n, np.float32)
    lib().orc_matmul_q4_0_col(_p(y), _p(w), w.size, _p(xx), _p(b), n, m)
    return y


def matmul_q4_0_col_f64(w_q, x, bias, n, m) -> np.ndarray:
    w = _c(w_q, np.uint8).ravel()
    xx = _c(x, np.float32).ravel()
    b = _c(bias, np.float32) if bias is not None else None
    y = np.empty(n, np.float64)
    lib().orc_matmul_q4_0_col_f64(_p(y), _p(w), w.size, _p(xx), _p(b), n, m)
    return y


# --- next-token choice (run.rs:203-278) -------------------------------------------

def xorshift64_seed(seed: int) -> int:
    """XorShift64::new (run.rs:270): max(seed, 1)."""
    return max(int(seed) & ((1 << 64) - 1), 1)


def xorshift64_next(state: int):
    """(value, new state) of XorShift64::next (run.rs:271-276)."""
    st = ctypes.c_uint64(state)
    v = lib().orc_xorshift64_next(ctypes.byref(st))
    return int(v), int(st.value)


def xorshift64_next_f32(state: int):
    st = ctypes.c_uint64(state)
    v = lib().orc_xorshift64_next_f32(ctypes.byref(st))
    return float(v), int(st.value)


def argmax(v) -> int:
    """Iterator::max_by(partial_cmp) index (run.rs:232-234)."""
    v = _c(v, np.float32).ravel()
    return int(lib().orc_argmax(_p(v), v.size))


def sample_token(logits, temperature: float, top_p: float, top_k: int, state: int):
    """(token, new state) of sample_token (run.rs:203-251)."""
    lg = _c(logits, np.float32).ravel()
    st = ctypes.c_uint64(state)
    tok = lib().orc_sample_token(_p(lg), lg.size, ctypes.c_float(temperature),
                                 ctypes.c_float(top_p), int(top_k), ctypes.byref(st))
    return int(tok), int(st.value)
