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


def _fake_result(us, M, n, m, checked=True):
    r = bench.result(us, M, n, m, bench.q4_bytes(n, m))
    r["check"] = {"checked": checked, "max_err": 1e-6, "bar": "normwise 1e-4",
                  "sampled_cols": 66}
    return r


def test_bench_compact_record():
    """The final stdout line carries one flat {us, frac, ok} entry per timed
    result; frac is the binding roofline (the larger fraction)."""
    sweep = {}
    for name, n, m in bench.MISTRAL_SHAPES:
        for M in (1, 2, 4, 8, 64, 512, 2048):
            r = _fake_result(10.0 + M / 10, M, n, m)
            if M >= 512:
                r["folded_scales"] = _fake_result(20.0 + M / 10, M, n, m, checked=False)
            sweep[f"{name}_M{M}"] = r
    sec = {"c3_m_sweep": {"workload": "x" * 300, "results": sweep},
           "model_load": {"open_upload_ms": 900.0, "check": {"checked": True}}}
    flat = bench.compact(sec)
    assert len(flat) == 4 * 7 + 4 * 2 + 1
    e = flat["c3.gate_up_M512"]
    r = sweep["gate_up_M512"]
    assert e["us"] == r["us"] and e["ok"] is True
    assert e["frac"] == max(r["frac_hbm_peak"], r["frac_fp16_peak"])
    assert flat["c3.gate_up_M512.folded"]["ok"] is False
    assert flat["load"]["us"] == 900000.0
    # 61 entries of this form stay far below the ~8 KB a driver log tail keeps.
    import json
    assert len(json.dumps(flat)) < 3000


def test_bench_compact_decode_step():
    """The Mistral decode step (one dict with ms_per_step and gbs) appears in
    the flat map under its short name, with its HBM fraction."""
    step = {"workload": "x", "launches": 128, "ms_per_step": 1.25, "gbs": 3140.7,
            "frac_hbm_peak": 0.3926, "check": {"checked": True}}
    flat = bench.compact({"c3_decode_step": step})
    assert flat == {"c3.decode_step_grouped": {"us": 1250.0, "frac": 0.3926, "ok": True}}
