"""Python mirror of hypno's matmul interface for the Q4_0 / FP16 path.

Same names, argument order and meaning as the reference (paths relative to
crates/hypno/src/):

    matmul_q4_0(y, w_q, x, bias, n, m)           kernels.rs:256
    matmul_f16(y, w, x, bias, n, m)              kernels.rs:571
    matmul_vec_q4_0 / matmul_vec_f16             ops.rs:15, ops.rs:20
    matmul_vec_auto(y, w, dtype, x, bias, n, m)  ops.rs:25
    batch_matmul(y, w, dtype, x, n, dim, batch, col_major)   turbo.rs:306
    quantize_f32_to_q4_0(data) / dequantize_q4_0(q)          quant.rs:108 / :120

`y` is written in place.  Arguments are either all torch tensors on the GPU
(the device path: asynchronous on torch's current stream, no host copies) or
all numpy arrays (the host-slice path of the C ABI: staged to the GPU and
copied back).  Every computation runs in libhypno_hip on the GPU; there is
no CPU implementation here.  Where the reference would panic (an
out-of-bounds slice) these functions raise ValueError; a library failure
raises HypnoHipError.
"""
from __future__ import annotations

import ctypes
import enum

import numpy as np

from ._lib import HypnoHipError, check, load

__all__ = [
    "DType", "HypnoHipError", "matmul_q4_0", "matmul_f16", "matmul_vec_q4_0",
    "matmul_vec_f16", "matmul_vec_auto", "batch_matmul", "quantize_f32_to_q4_0",
    "dequantize_q4_0", "register_weight", "unregister_weight", "device_count", "GemvPlan",
    "rms_norm", "rms_norm_in_place", "silu_mul", "matmul_q8_0", "quantize_f32_to_q8_0",
    "dequantize_q8_0", "matmul_q4_0_col", "matmul_vec_col", "set_gemm_numerics",
    "GEMM_AUTO", "GEMM_EXACT", "GEMM_FOLDED", "q4_0_extract_row", "q8_0_extract_row", "embed_tokens",
    "argmax", "sample_token",
]

GEMM_AUTO, GEMM_EXACT, GEMM_FOLDED = 0, 1, 2  # HYPNO_HIP_GEMM_AUTO / _EXACT / _FOLDED


def set_gemm_numerics(mode: int) -> int:
    """Q4_0 prefill GEMM arithmetic: GEMM_AUTO (the default) and GEMM_EXACT
    feed the matrix cores the integer nibbles and apply each block's scale in
    fp32; GEMM_FOLDED opts into fp16 weights with the scale folded in (from
    128-256 tokens).  Process-wide; returns the previous mode."""
    prev = int(load().hypno_hip_set_gemm_numerics(int(mode)))
    if prev < 0:
        check(-prev, "set_gemm_numerics")
    return prev


class DType(enum.IntEnum):
    """Tensor element types (dtype.rs:4-15), with the size rules of dtype.rs:40-70."""
    FP32 = 0
    FP16 = 1
    Q8_0 = 2
    Q4_0 = 3

    def block_size(self) -> int:
        return 32 if self in (DType.Q8_0, DType.Q4_0) else 1

    def block_bytes(self) -> int:
        return {DType.Q8_0: 34, DType.Q4_0: 18}.get(self, 0)

    def data_bytes(self, n_elems: int) -> int:
        if self == DType.FP32:
            return n_elems * 4
        if self == DType.FP16:
            return n_elems * 2
        return -(-n_elems // 32) * self.block_bytes()


def device_count() -> int:
    return int(load().hypno_hip_device_count())


# --- argument handling ---------------------------------------------------------

def _is_torch(a) -> bool:
    return type(a).__module__.startswith("torch")


def _torch():
    import torch
    return torch


def _dev_ptr(t, dtype_name: str, what: str):
    torch = _torch()
    want = {"f32": torch.float32, "u8": torch.uint8}[dtype_name]
    if not t.is_cuda:
        raise ValueError(f"{what} must be a GPU tensor")
    if t.dtype != want:
        raise ValueError(f"{what} must be {want}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def _host_ptr(a, dtype, what: str):
    if not isinstance(a, np.ndarray):
        raise ValueError(f"{what} must be a numpy array or a GPU torch tensor")
    if a.dtype != dtype:
        raise ValueError(f"{what} must be {np.dtype(dtype)}, got {a.dtype}")
    if not a.flags.c_contiguous:
        raise ValueError(f"{what} must be C-contiguous")
    return a.ctypes.data_as(ctypes.c_void_p)


def _numel(a) -> int:
    return int(a.numel()) if _is_torch(a) else int(a.size)


def _nbytes(a) -> int:
    return int(a.numel() * a.element_size()) if _is_torch(a) else int(a.nbytes)


def _stream(device) -> ctypes.c_void_p:
    torch = _torch()
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _check_lengths(y, x, bias, n, m, batch):
    # The reference indexes y by row, x[..m] and bias[row]; a short slice panics.
    if n < 0 or m < 0 or batch < 0:
        raise ValueError("n, m and batch must be non-negative")
    if _numel(y) != n * batch:
        raise ValueError(f"y has {_numel(y)} elements, expected n*batch = {n * batch}")
    if _numel(x) < m * batch:
        raise ValueError(f"x has {_numel(x)} elements, expected at least {m * batch}")
    if bias is not None and _numel(bias) < n:
        raise ValueError(f"bias has {_numel(bias)} elements, expected at least {n}")


def _matmul(y, w, dtype: DType, x, bias, n: int, m: int, batch: int, col: bool = False) -> None:
    _check_lengths(y, x, bias, n, m, batch)
    lib = load()
    tensors = [a for a in (y, w, x, bias) if a is not None]
    on_gpu = [_is_torch(a) for a in tensors]
    if all(on_gpu):
        yp = _dev_ptr(y, "f32", "y")
        wp = _dev_ptr(w, "u8", "w")
        xp = _dev_ptr(x, "f32", "x")
        bp = _dev_ptr(bias, "f32", "bias") if bias is not None else None
        fn = {DType.Q4_0: (lib.hypno_hip_matmul_q4_0_col_dev if col
                           else lib.hypno_hip_matmul_q4_0_dev),
              DType.Q8_0: lib.hypno_hip_matmul_q8_0_dev,
              DType.FP16: lib.hypno_hip_matmul_f16_dev}.get(dtype)
        if fn is None:
            raise HypnoHipError(95, f"matmul dtype {dtype.name}")
        check(fn(yp, wp, _nbytes(w), xp, bp, n, m, batch, _stream(y.device)),
              f"matmul {dtype.name}")
        return
    if any(on_gpu):
        raise ValueError("mixing GPU tensors and host arrays is not supported")
    yp = _host_ptr(y, np.float32, "y")
    wp = _host_ptr(w, np.uint8, "w")
    xp = _host_ptr(x, np.float32, "x")
    bp = _host_ptr(bias, np.float32, "bias") if bias is not None else None
    if batch == 1:
        fn = lib.hypno_hip_matmul_vec_col if col else lib.hypno_hip_matmul_vec_auto
        check(fn(yp, wp, w.nbytes, int(dtype), xp, bp, n, m), f"matmul {dtype.name}")
    else:
        if bias is not None:
            raise ValueError("batch_matmul takes no bias (turbo.rs:306-333)")
        fn = lib.hypno_hip_batch_matmul_col if col else lib.hypno_hip_batch_matmul
        check(fn(yp, wp, w.nbytes, int(dtype), xp, n, m, batch), f"batch_matmul {dtype.name}")


# --- the reference's entry points --------------------------------------------------

def matmul_q4_0(y, w_q, x, bias, n: int, m: int) -> None:
    """y[n] = W_q[n][m] . x[m] (+ bias), Q4_0 weights (kernels.rs:256-265)."""
    _matmul(y, w_q, DType.Q4_0, x, bias, n, m, 1)


def matmul_f16(y, w, x, bias, n: int, m: int) -> None:
    """y[n] = W[n][m] . x[m] (+ bias), fp16 weights as bytes (kernels.rs:571-586)."""
    _matmul(y, w, DType.FP16, x, bias, n, m, 1)


def matmul_q8_0(y, w_q, x, bias, n: int, m: int) -> None:
    """y[n] = dequantize_q8_0(W_q)[n][m] . x[m] (+ bias): the Q8_0 arm of
    matmul_vec_auto (ops.rs:33-36), streamed instead of dequantised."""
    _matmul(y, w_q, DType.Q8_0, x, bias, n, m, 1)


def matmul_q4_0_col(y, w_q, x, bias, n: int, m: int) -> None:
    """Column-major Q4_0 (kernels.rs:414-535): w_q holds W_col[m][n] — for each
    input index k, n outputs quantised in blocks along n — and
    y[j] = sum_k W_col[k][j] * x[k] (+ bias)."""
    _matmul(y, w_q, DType.Q4_0, x, bias, n, m, 1, col=True)


def matmul_vec_col(y, w, dtype, x, bias, n: int, m: int) -> None:
    """ops::matmul_vec_col (ops.rs:41-51): Q4_0 column-major, other dtypes as
    matmul_vec_auto."""
    dtype = DType(int(dtype))
    if dtype not in (DType.Q4_0, DType.Q8_0, DType.FP16):
        raise HypnoHipError(95, f"matmul_vec_col dtype {dtype.name}")
    _matmul(y, w, dtype, x, bias, n, m, 1, col=True)


def matmul_vec_q4_0(y, w_q, x, bias, n: int, m: int) -> None:
    """ops.rs:15-17."""
    matmul_q4_0(y, w_q, x, bias, n, m)


def matmul_vec_f16(y, w, x, bias, n: int, m: int) -> None:
    """ops.rs:20-22."""
    matmul_f16(y, w, x, bias, n, m)


def matmul_vec_auto(y, w, dtype, x, bias, n: int, m: int) -> None:
    """Dtype switch of ops.rs:25-38: FP16, Q4_0 and Q8_0.  FP32 weights are
    outside this path and raise HypnoHipError (ENOTSUP)."""
    dtype = DType(int(dtype))
    if dtype not in (DType.Q4_0, DType.Q8_0, DType.FP16):
        raise HypnoHipError(95, f"matmul_vec_auto dtype {dtype.name}")
    _matmul(y, w, dtype, x, bias, n, m, 1)


def batch_matmul(y, w, dtype, x, n: int, dim: int, batch: int, col_major: bool = False) -> None:
    """turbo::batch_matmul (turbo.rs:306-343) for FP16 / Q4_0 / Q8_0 weights:
    X[batch][dim] -> Y[batch][n] in one call; col_major selects the
    column-major Q4_0 kernel (turbo.rs:322-326; other dtypes ignore it)."""
    dtype = DType(int(dtype))
    if dtype not in (DType.Q4_0, DType.Q8_0, DType.FP16):
        raise HypnoHipError(95, f"batch_matmul dtype {dtype.name}")
    _matmul(y, w, dtype, x, None, n, dim, batch, col=bool(col_major))


# --- codec (device) ---------------------------------------------------------------

def quantize_f32_to_q4_0(data):
    """quant.rs:108-117 on the GPU: floor(len/32) blocks, bit-exact.  `data` is
    a float32 GPU tensor; returns a uint8 GPU tensor of blocks*18 bytes."""
    torch = _torch()
    src = data.reshape(-1)
    nb = src.numel() // 32
    out = torch.empty(nb * 18, dtype=torch.uint8, device=src.device)
    check(load().hypno_hip_quantize_q4_0_dev(_dev_ptr(out, "u8", "out"),
                                              _dev_ptr(src, "f32", "data"), src.numel(),
                                              _stream(src.device)), "quantize_q4_0")
    return out


def dequantize_q4_0(q):
    """quant.rs:120-132 on the GPU: floor(len/18) blocks -> fp32, bit-exact."""
    torch = _torch()
    nb = q.numel() // 18
    out = torch.empty(nb * 32, dtype=torch.float32, device=q.device)
    check(load().hypno_hip_dequantize_q4_0_dev(_dev_ptr(out, "f32", "out"),
                                                _dev_ptr(q, "u8", "q"), q.numel(),
                                                _stream(q.device)), "dequantize_q4_0")
    return out


def quantize_f32_to_q8_0(data):
    """quant.rs:177-191 on the GPU: floor(len/32) blocks of 34 bytes, bit-exact."""
    torch = _torch()
    src = data.reshape(-1)
    nb = src.numel() // 32
    out = torch.empty(nb * 34, dtype=torch.uint8, device=src.device)
    check(load().hypno_hip_quantize_q8_0_dev(_dev_ptr(out, "u8", "out"),
                                              _dev_ptr(src, "f32", "data"), src.numel(),
                                              _stream(src.device)), "quantize_q8_0")
    return out


def dequantize_q8_0(q):
    """quant.rs:194-206 on the GPU: floor(len/34) blocks -> fp32, bit-exact."""
    torch = _torch()
    nb = q.numel() // 34
    out = torch.empty(nb * 32, dtype=torch.float32, device=q.device)
    check(load().hypno_hip_dequantize_q8_0_dev(_dev_ptr(out, "f32", "out"),
                                                _dev_ptr(q, "u8", "q"), q.numel(),
                                                _stream(q.device)), "dequantize_q8_0")
    return out


# --- multi-GEMV plans ---------------------------------------------------------------

class GemvPlan:
    """Several independent Q4_0 GEMVs (one token each) run as one launch.

    `jobs` is a sequence of (y, w_q, x, bias, n, m) with GPU tensors, each with
    the meaning of matmul_q4_0's arguments, optionally followed by a prologue
    applied to x as the GEMV stages it: ("rms_norm", norm_weight, eps)
    (ops::rms_norm, kernels.rs:592-625) or ("silu_mul", up) (silu(x) * up,
    transformer.rs:446-449); x itself is left unchanged.  The plan keeps the
    tensors' addresses: refill the x tensors in place and call run() again."""

    def __init__(self, jobs):
        from ._lib import (PROLOGUE_NONE, PROLOGUE_RMS_NORM, PROLOGUE_SILU_MUL, GemvDesc,
                           GemvPrologue)
        lib = load()
        self._keep = []
        descs = (GemvDesc * len(jobs))()
        pros = (GemvPrologue * len(jobs))()
        any_pro = False
        for i, job in enumerate(jobs):
            y, w, x, bias, n, m = job[:6]
            pro = job[6] if len(job) > 6 else None
            _check_lengths(y, x, bias, n, m, 1)
            pros[i].kind = PROLOGUE_NONE
            if pro is not None:
                kind, aux = pro[0], pro[1]
                if _numel(aux) < m:
                    raise ValueError(f"prologue operand has {_numel(aux)} elements, expected {m}")
                pros[i].aux = _dev_ptr(aux, "f32", "prologue operand").value
                if kind == "rms_norm":
                    pros[i].kind, pros[i].eps = PROLOGUE_RMS_NORM, float(pro[2])
                elif kind == "silu_mul":
                    pros[i].kind = PROLOGUE_SILU_MUL
                else:
                    raise ValueError(f"unknown prologue {kind!r}")
                self._keep.append(aux)
                any_pro = True
            descs[i].y = _dev_ptr(y, "f32", "y").value
            descs[i].w_q = _dev_ptr(w, "u8", "w_q").value
            descs[i].w_len = _nbytes(w)
            descs[i].x = _dev_ptr(x, "f32", "x").value
            descs[i].bias = _dev_ptr(bias, "f32", "bias").value if bias is not None else None
            descs[i].n = n
            descs[i].m = m
            self._keep.append((y, w, x, bias))
        self._plan = ctypes.c_void_p()
        check(lib.hypno_hip_q4_0_gemv_plan_create_ex(descs, pros if any_pro else None, len(jobs),
                                                     ctypes.byref(self._plan)),
              "gemv_plan_create")
        self.device = self._keep[0][0].device if self._keep else None

    @property
    def launches(self) -> int:
        return int(load().hypno_hip_q4_0_gemv_plan_launches(self._plan))

    def run(self, stream=None) -> None:
        st = ctypes.c_void_p(stream) if stream is not None else (
            _stream(self.device) if self.device is not None else None)
        check(load().hypno_hip_q4_0_gemv_plan_run(self._plan, st), "gemv_plan_run")

    def close(self) -> None:
        if self._plan:
            load().hypno_hip_q4_0_gemv_plan_destroy(self._plan)
            self._plan = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# --- the decode step's neighbours of the GEMV (device tensors) -----------------------

def rms_norm(x, weight, eps: float, rows: int = 1, out=None):
    """ops::rms_norm (ops.rs:52-55 -> kernels.rs:592-625) over `rows` rows of
    x (GPU float32), into `out` (a new tensor by default)."""
    if out is None:
        out = _torch().empty_like(x)
    elif _numel(out) != _numel(x):
        raise ValueError("out and x differ in size")
    _rms_norm(out, x, weight, eps, rows)
    return out


def rms_norm_in_place(x, weight, eps: float, rows: int = 1) -> None:
    """ops::rms_norm_in_place (ops.rs:59-61)."""
    _rms_norm(x, x, weight, eps, rows)


def _rms_norm(out, x, weight, eps, rows):
    n = _numel(x) // rows if rows else 0
    if rows and n * rows != _numel(x):
        raise ValueError("x does not split into `rows` equal rows")
    if _numel(weight) < n:
        raise ValueError(f"weight has {_numel(weight)} elements, expected {n}")
    check(load().hypno_hip_rms_norm_dev(_dev_ptr(out, "f32", "out"), _dev_ptr(x, "f32", "x"),
                                        _dev_ptr(weight, "f32", "weight"), n, rows,
                                        ctypes.c_float(eps), _stream(x.device)), "rms_norm")


def silu_mul(gate, up, out=None):
    """silu_in_place(gate); gate *= up (ops.rs:81-83, transformer.rs:446-449)
    as out = silu(gate) * up (out=gate for the in-place form)."""
    if _numel(up) < _numel(gate):
        raise ValueError("up is shorter than gate")
    if out is None:
        out = _torch().empty_like(gate)
    check(load().hypno_hip_silu_mul_dev(_dev_ptr(out, "f32", "out"), _dev_ptr(gate, "f32", "gate"),
                                        _dev_ptr(up, "f32", "up"), _numel(gate),
                                        _stream(gate.device)), "silu_mul")
    return out


# --- weight residency for the host-slice path -------------------------------------

def register_weight(w: np.ndarray) -> None:
    """Upload a host weight buffer once (the mmap'd slice of loader.rs:139-148);
    later host-slice calls with the same array reuse the device copy."""
    check(load().hypno_hip_weight_register(_host_ptr(w, np.uint8, "w"), w.nbytes),
          "weight_register")


def unregister_weight(w: np.ndarray) -> None:
    check(load().hypno_hip_weight_unregister(_host_ptr(w, np.uint8, "w")), "weight_unregister")


# --- the embedding gather and the next-token choice (device tensors) ---------------

def _extract_row(fn, q, row_idx: int, row_width: int):
    torch = _torch()
    out = torch.empty(row_width, dtype=torch.float32, device=q.device)
    check(fn(_dev_ptr(out, "f32", "out"), _dev_ptr(q, "u8", "q"), _nbytes(q), int(row_idx),
             int(row_width), _stream(q.device)), "extract_row")
    return out


def q4_0_extract_row(q4_data, row_idx: int, row_width: int):
    """quant.rs:139-153: row row_idx of a Q4_0 matrix, dequantised (new tensor)."""
    return _extract_row(load().hypno_hip_q4_0_extract_row_dev, q4_data, row_idx, row_width)


def q8_0_extract_row(q8_data, row_idx: int, row_width: int):
    """quant.rs:158-175: the same for Q8_0."""
    return _extract_row(load().hypno_hip_q8_0_extract_row_dev, q8_data, row_idx, row_width)


def embed_tokens(table, dtype, token_ids, hd: int, out=None):
    """Token embedding (transformer.rs:476-497, turbo.rs:38-66): rows
    token_ids (int32/uint32 GPU tensor) of the table -> [len(ids), hd] fp32."""
    torch = _torch()
    ids = token_ids.to(torch.int32) if token_ids.dtype != torch.int32 else token_ids
    if not ids.is_contiguous():
        ids = ids.contiguous()
    count = ids.numel()
    if out is None:
        out = torch.empty(count, hd, dtype=torch.float32, device=table.device)
    check(load().hypno_hip_embed_tokens_dev(_dev_ptr(out, "f32", "out"),
                                            _dev_ptr(table, "u8", "table"), _nbytes(table),
                                            int(DType(dtype)), ctypes.c_void_p(ids.data_ptr()),
                                            count, int(hd), _stream(table.device)),
          "embed_tokens")
    return out


def argmax(logits):
    """Index of the largest logit as Iterator::max_by picks it (run.rs:232-234),
    as a one-element int32 GPU tensor."""
    torch = _torch()
    out = torch.empty(1, dtype=torch.int32, device=logits.device)
    check(load().hypno_hip_argmax_dev(ctypes.c_void_p(out.data_ptr()),
                                      _dev_ptr(logits, "f32", "logits"), logits.numel(),
                                      _stream(logits.device)), "argmax")
    return out


def sample_token(logits, temperature: float, top_p: float, top_k: int, rng_state):
    """sample_token (run.rs:203-251) on the GPU.  rng_state is a one-element
    int64 GPU tensor holding the XorShift64 state (advanced in place); returns
    a one-element int32 GPU tensor with the token."""
    torch = _torch()
    if rng_state.dtype != torch.int64 or rng_state.numel() != 1 or not rng_state.is_cuda:
        raise ValueError("rng_state must be a one-element int64 GPU tensor")
    out = torch.empty(1, dtype=torch.int32, device=logits.device)
    check(load().hypno_hip_sample_token_dev(ctypes.c_void_p(out.data_ptr()),
                                            ctypes.c_void_p(rng_state.data_ptr()),
                                            _dev_ptr(logits, "f32", "logits"), logits.numel(),
                                            float(temperature), float(top_p), int(top_k),
                                            _stream(logits.device)), "sample_token")
    return out
