#!/usr/bin/env python3
"""Writes tests/golden/q4_0_fixtures.npz: small input/output vectors of the
Q4_0 / FP16 matmul path, computed by the CPU restatement in oracle/ (which the
CPU tests pin against hypno's known-answer tests and IEEE/fp64 checks).

Inputs come from numpy's PCG64 with fixed seeds (oracle.normal_f32).  The
expected outputs are the restatement's scalar kernel (kernels.rs:362-400,
exact reference summation order) and an fp64 brute-force sum.  Regenerate
with `python3 tests/golden/make_fixtures.py` after `make -C oracle`.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402

# (name, n, m): 64x256 plain; 37x100 has blocks straddling rows (K % 32 != 0)
# and a short last row (quantize_f32_to_q4_0 keeps floor(len/32) blocks);
# 33x512 an odd row count; 5x3072 a long row.
GEMV_CASES = [("g64x256", 64, 256), ("g37x100", 37, 100), ("g33x512", 33, 512),
              ("g5x3072", 5, 3072)]


def quant_input():
    """Eight 32-element blocks covering the quantizer's cases (quant.rs:49-71)."""
    blocks = [orc.normal_f32(101, 32, 0.02),          # typical weights
              np.zeros(32, np.float32),               # amax = 0 -> d = 1.0
              orc.normal_f32(102, 32, 1000.0),        # large scale
              orc.normal_f32(103, 32, 1e-6),          # subnormal f16 scale
              np.full(32, -3.5, np.float32),          # all equal, negative
              np.arange(32, dtype=np.float32) - 16.0, # integer ramp, ties
              orc.normal_f32(104, 32, 0.02),
              orc.normal_f32(105, 32, 3.0)]
    blocks[6][7] = 0.5                                # one outlier
    return np.concatenate(blocks).astype(np.float32)


def main():
    out = {}
    q_in = quant_input()
    out["quant_in"] = q_in
    out["quant_out"] = orc.quantize_q4_0(q_in)
    out["dequant_out"] = orc.dequantize_q4_0(out["quant_out"])
    for i, (name, n, m) in enumerate(GEMV_CASES):
        w = orc.quantize_q4_0(orc.normal_f32(200 + i, n * m, 0.02))
        x = orc.normal_f32(300 + i, m)
        bias = orc.normal_f32(400 + i, n)
        out[f"{name}_w"] = w
        out[f"{name}_x"] = x
        out[f"{name}_bias"] = bias
        out[f"{name}_y"] = orc.matmul_q4_0_scalar(w, x, None, n, m)
        out[f"{name}_ybias"] = orc.matmul_q4_0_scalar(w, x, bias, n, m)
        out[f"{name}_y64"] = orc.matmul_q4_0_f64(w, x, None, n, m)
    # FP16 weights, 17 x 100 (kernels.rs:571-586)
    wf = orc.f32_to_f16_bits(orc.normal_f32(500, 17 * 100, 0.02)).view(np.uint8)
    xf = orc.normal_f32(501, 100)
    out["f16_w"] = wf
    out["f16_x"] = xf
    out["f16_y"] = orc.matmul_f16_scalar(wf, xf, None, 17, 100)
    out["f16_y64"] = orc.matmul_f16_f64(wf, xf, None, 17, 100)
    # batch_matmul, Q4_0, 3 tokens x 64x256 (turbo.rs:306-333)
    wb = orc.quantize_q4_0(orc.normal_f32(600, 64 * 256, 0.02))
    xb = orc.normal_f32(601, (3, 256))
    out["batch_w"] = wb
    out["batch_x"] = xb
    out["batch_y"] = np.stack([orc.matmul_q4_0_scalar(wb, xb[t], None, 64, 256)
                               for t in range(3)])
    np.savez_compressed(os.path.join(HERE, "q4_0_fixtures.npz"), **out)
    print("wrote", len(out), "arrays")


if __name__ == "__main__":
    main()
