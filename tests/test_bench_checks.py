"""The fp64 references bench.py checks its timed outputs with are pinned to
the oracle's bit-exact dequantizers (CPU only)."""
import numpy as np

import bench


def test_bench_q4_rows_match_oracle(orc):
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, size=(7, 5 * 18), dtype=np.uint8)
    raw[:, 1::18] &= 0x7B   # keep the scales finite
    got = bench.q4_rows_f64(raw)
    ref = orc.dequantize_q4_0(raw.ravel()).reshape(7, 160).astype(np.float64)
    assert np.array_equal(got, ref)


def test_bench_q8_rows_match_oracle(orc):
    rng = np.random.default_rng(4)
    raw = rng.integers(0, 256, size=(3, 4 * 34), dtype=np.uint8)
    raw[:, 1::34] &= 0x7B
    got = bench.q8_rows_f64(raw)
    ref = orc.dequantize_q8_0(raw.ravel()).reshape(3, 128).astype(np.float64)
    assert np.array_equal(got, ref)


def test_bench_error_metrics():
    ref = np.array([1.0, -4.0, 2.0])
    assert bench.normwise(np.array([1.0, -4.0, 2.5]), ref) == 0.125
    assert abs(bench.rel_l2(ref * 1.01, ref) - 0.01) < 1e-12
    assert bench.sample_idx(10, 3, 1)[0] == 0 and bench.sample_idx(10, 3, 1)[-1] == 9
