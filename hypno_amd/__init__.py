"""hypno_amd: hypno's Q4_0 / FP16 quantized matmul path, native on MI355X (gfx950).

The computation lives in libhypno_hip.so (hand-written HIP kernels behind the
C ABI of include/hypno_hip.h); this package is its Python face and mirrors
the reference's function names (see hypno_amd.kernels).
"""
from .kernels import (  # noqa: F401
    GEMM_AUTO,
    GEMM_EXACT,
    GEMM_FOLDED,
    DType,
    GemvPlan,
    HypnoHipError,
    argmax,
    batch_matmul,
    dequantize_q4_0,
    dequantize_q8_0,
    device_count,
    embed_tokens,
    matmul_f16,
    matmul_q4_0,
    matmul_q4_0_col,
    matmul_q8_0,
    matmul_vec_auto,
    matmul_vec_col,
    matmul_vec_f16,
    matmul_vec_q4_0,
    q4_0_extract_row,
    q8_0_extract_row,
    quantize_f32_to_q4_0,
    quantize_f32_to_q8_0,
    register_weight,
    rms_norm,
    rms_norm_in_place,
    sample_token,
    set_gemm_numerics,
    silu_mul,
    unregister_weight,
)

from .model import FormatError, HypnoModel  # noqa: F401

__version__ = "0.1.0"
