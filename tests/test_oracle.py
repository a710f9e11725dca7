"""Pins the CPU oracle (oracle/q4_0_oracle.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the restatement fails:
banker's rounding instead of half-away, dividing by the rounded f16 scale,
swapped nibble order, a dropped -8 offset, a wrong straddle index, ignoring the
short-buffer rule, or a transposed batch layout.  Expected values come from
the reference's own tests (file:line cited), from IEEE definitions checked
against numpy and the F16C hardware converter, and from exact integer
arithmetic that no fp32 summation order can change.
"""
import numpy as np
import pytest


# --- f16 <-> f32 (half 2.7.1 at kernels.rs:297, quant.rs:26,57) ---------------

def test_f16_to_f32_all_patterns(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    hw = orc.f16_bits_to_f32_f16c(bits)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.array_equal(got.view(np.uint32), hw.view(np.uint32))  # NaN payloads too


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(7)
    # every exponent from f32 subnormals to overflow, random mantissas
    raw = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = raw.view(np.float32)
    x = x[np.isfinite(x)]
    # halfway and boundary cases
    special = np.array([
        65504.0, 65519.99, 65520.0, 1e9, -65520.0,       # overflow edge: 65520 rounds to inf
        2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001, 3 * 2.0**-26, 2.0**-14,
        1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 1.0 / 7.0, -0.0, 0.0,
        2049.0, 2051.0, 4097.0,                           # ties to even above 2048
    ], dtype=np.float32)
    x = np.concatenate([x, special, -special])
    got = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    hw = orc.f32_to_f16_bits_f16c(x)
    assert np.array_equal(got, ref)
    assert np.array_equal(got, hw)
    assert orc.f32_to_f16_bits(np.float32(65520.0)) == 0x7C00
    assert orc.f32_to_f16_bits(np.float32(2049.0)) == 0x6800  # 2049 -> 2048 (even)
    assert orc.f32_to_f16_bits(np.float32(2051.0)) == 0x6802  # 2051 -> 2052 (even)


# --- quantizer (quant.rs:49-71, 108-117) ----------------------------------------

def test_quantize_roundtrip_kat(orc):
    # quant.rs:213-225: src = (i - 15.5) * 0.1, |src - deq| < 0.5
    src = ((np.arange(32, dtype=np.float32) - np.float32(15.5)) * np.float32(0.1)).astype(np.float32)
    q = orc.quantize_q4_0(src)
    assert q.size == 18
    dst = orc.dequantize_q4_0(q)
    assert np.all(np.abs(src - dst) < 0.5)


def test_quantize_zero_block_kat(orc):
    # quant.rs:228-237 (zeros -> zeros) and quant.rs:52-56 (scale 1.0 when amax == 0)
    q = orc.quantize_q4_0(np.zeros(32, np.float32))
    assert q[0] == 0x00 and q[1] == 0x3C  # f16 1.0, little-endian
    assert np.all(q[2:] == 0x88)          # q = 0 -> nibble 8 in both halves
    assert np.all(orc.dequantize_q4_0(q) == 0.0)


def test_quantize_sizes_kat(orc):
    # loader.rs:297-319: 32 elements -> 18 bytes; sft_convert.rs:430-457: 128x64 -> 4608
    assert orc.quantize_q4_0(np.ones(32, np.float32)).size == 18
    assert orc.quantize_q4_0(np.ones(128 * 64, np.float32)).size == 4608
    # quant.rs:109: floor(len/32) blocks; a partial trailing block is dropped
    assert orc.quantize_q4_0(np.ones(100, np.float32)).size == 3 * 18


def test_quantize_hand_block(orc):
    # amax = 7 -> s = 1.0 exactly -> d = 0x3C00; q = round_half_away(v)
    src = np.zeros(32, np.float32)
    src[:12] = [7.0, -7.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 3.49, -3.51, 6.5, 0.49]
    q = orc.quantize_q4_0(src)
    assert (q[0], q[1]) == (0x00, 0x3C)
    # element 2i -> low nibble, 2i+1 -> high nibble (quant.rs:16, :66-69)
    want_q = [7, -7, 3, -3, 1, -1, 2, -2, 3, -4, 7, 0] + [0] * 20
    nib = [v + 8 for v in want_q]
    want_bytes = [nib[2 * i] | (nib[2 * i + 1] << 4) for i in range(16)]
    assert list(q[2:]) == want_bytes
    # bankers' rounding would give 2.5->2, 0.5->0, 6.5->6: those bytes must differ
    assert want_bytes[1] == (11 | (5 << 4))


def test_quantize_negative_amax_and_clamp(orc):
    # amax comes from |v|: the largest magnitude is negative here
    src = np.zeros(32, np.float32)
    src[5] = -14.0
    src[6] = 2.0
    q = orc.quantize_q4_0(src)
    d = orc.f16_bits_to_f32(np.array([int(q[0]) | (int(q[1]) << 8)], np.uint16))[0]
    assert d == np.float32(2.0)           # 14/7 = 2 exactly
    deq = orc.dequantize_q4_0(q)
    assert deq[5] == -14.0 and deq[6] == 2.0
    assert np.all(deq[[i for i in range(32) if i not in (5, 6)]] == 0.0)


def test_quantize_divides_by_unrounded_scale(orc):
    # quant.rs:63 divides by the f32 scale s, not by d = f16(s).  Search blocks
    # where the two choices give different nibbles and check the oracle takes s.
    rng = np.random.default_rng(11)
    hits = 0
    for _ in range(400):
        blk = (rng.standard_normal(32).astype(np.float32) * np.float32(0.02)).astype(np.float32)
        amax = np.max(np.abs(blk))
        s = np.float32(amax / np.float32(7.0))
        d = np.float32(np.float16(s))
        qs = np.clip(np.trunc(blk / s + np.copysign(np.float32(0.5), blk / s)), -8, 7)
        qd = np.clip(np.trunc(blk / d + np.copysign(np.float32(0.5), blk / d)), -8, 7)
        if np.array_equal(qs, qd):
            continue
        hits += 1
        q = orc.quantize_q4_0(blk)
        nib = np.empty(32, np.int64)
        nib[0::2] = q[2:] & 0x0F
        nib[1::2] = q[2:] >> 4
        assert np.array_equal(nib - 8, qs.astype(np.int64))
    assert hits > 0


def test_quantize_special_values(orc):
    # NaN is ignored by the f32::max fold and maps to q = 0 via the saturating cast
    src = np.zeros(32, np.float32)
    src[0] = np.nan
    src[1] = 3.5
    q = orc.quantize_q4_0(src)
    assert (q[2] & 0x0F) == 8                 # NaN -> q = 0
    assert (q[2] >> 4) == 15                  # 3.5 / 0.5 = 7
    # amax/7 above f16 max -> d = +inf, nibbles from v/s with s finite
    big = np.full(32, 1e6, np.float32)
    q = orc.quantize_q4_0(big)
    assert (int(q[0]) | (int(q[1]) << 8)) == 0x7C00
    assert np.all(q[2:] == 0xFF)


# --- dequantizer (quant.rs:25-34, 120-132) -------------------------------------

def _block(d_bits, qs):
    return np.array([d_bits & 0xFF, d_bits >> 8] + list(qs), np.uint8)


def test_dequantize_hand_blocks(orc):
    qs = [0x10, 0xF8, 0x00, 0xFF] + [0x88] * 12
    out = orc.dequantize_q4_0(_block(0x3C00, qs))     # d = 1
    assert list(out[:8]) == [-8, -7, 0, 7, -8, -8, 7, 7]
    assert np.all(out[8:] == 0)
    out = orc.dequantize_q4_0(_block(0xC000, qs))     # d = -2
    assert list(out[:8]) == [16, 14, 0, -14, 16, 16, -14, -14]
    out = orc.dequantize_q4_0(_block(0x0001, qs))     # d = 2^-24 (f16 subnormal)
    assert out[0] == np.float32(-8 * 2.0**-24) and out[3] == np.float32(7 * 2.0**-24)
    out = orc.dequantize_q4_0(_block(0x7C00, [0x98] + [0x88] * 15))  # d = inf
    assert np.isnan(out[0]) and out[1] == np.inf
    # a trailing partial block is ignored (floor(len/18))
    two = np.concatenate([_block(0x3C00, [0x99] * 16), np.zeros(10, np.uint8)])
    assert orc.dequantize_q4_0(two).size == 32


# --- Q4_0 GEMV (kernels.rs:256-400) --------------------------------------------

def _int_q4(rng, n_elems, d_bits=0x3C00):
    """Packed Q4_0 with d = 1.0 and random nibbles; returns (bytes, ints)."""
    nb = (n_elems + 31) // 32
    nib = rng.integers(0, 16, size=(nb, 32))
    q = np.empty((nb, 18), np.uint8)
    q[:, 0] = d_bits & 0xFF
    q[:, 1] = d_bits >> 8
    q[:, 2:] = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return q.ravel(), (nib - 8).ravel()


@pytest.mark.parametrize("n,m", [(3, 32), (4, 64), (5, 48), (7, 40), (3, 13), (9, 100)])
@pytest.mark.parametrize("kind", ["dispatch", "scalar", "avx2"])
def test_gemv_exact_integer(orc, n, m, kind):
    # d = 1, integer x: every partial sum is an exact small integer, so any
    # summation order gives the same fp32 result.  Rows are the flattened
    # ranges [r*m, (r+1)*m), so blocks straddle rows when m % 32 != 0.
    rng = np.random.default_rng(n * 100 + m)
    q, ints = _int_q4(rng, n * m)
    x = rng.integers(-5, 6, size=m).astype(np.float32)
    bias = rng.integers(-3, 4, size=n).astype(np.float32)
    want = ints[: n * m].reshape(n, m).astype(np.int64) @ x.astype(np.int64) + bias.astype(np.int64)
    fn = {"dispatch": orc.matmul_q4_0, "scalar": orc.matmul_q4_0_scalar,
          "avx2": orc.matmul_q4_0_avx2}[kind]
    y = fn(q, x, bias, n, m)
    assert np.array_equal(y, want.astype(np.float32))


def test_gemv_short_buffer_semantics(orc):
    # kernels.rs:275-277 + :374: a short w_q falls back to the scalar loop, and
    # a block whose 18 bytes do not fit ends the row; later rows see nothing.
    rng = np.random.default_rng(5)
    n, m = 6, 64
    q, ints = _int_q4(rng, n * m)
    x = rng.integers(-4, 5, size=m).astype(np.float32)
    keep_blocks = 7                                   # 3.5 rows' worth
    w_short = q[: keep_blocks * 18 + 11]              # plus a partial block
    full = ints.reshape(n, m).astype(np.int64).copy()
    flat = full.ravel()
    flat[keep_blocks * 32:] = 0
    want = flat.reshape(n, m) @ x.astype(np.int64)
    for fn in (orc.matmul_q4_0, orc.matmul_q4_0_avx2, orc.matmul_q4_0_scalar):
        assert np.array_equal(fn(w_short, x, None, n, m), want.astype(np.float32))


def test_gemv_q4_0_rs_kat(orc):
    # q4_0.rs:222-255: n=64, x = i*0.1, y = ((i%7)-3)*0.5, Q4_0 dot vs fp32 rel < 0.15
    x = (np.arange(64, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    w = (((np.arange(64) % 7) - 3) * 0.5).astype(np.float32)
    q = orc.quantize_q4_0(w)
    dot = orc.matmul_q4_0(q, x, None, 1, 64)[0]
    fp32 = np.float32(np.dot(x.astype(np.float64), w.astype(np.float64)))
    assert abs(fp32 - dot) / max(abs(fp32), 1e-6) < 0.15
    # q4_0.rs:258-278: all-ones against all-ones quantised -> positive
    q1 = orc.quantize_q4_0(np.ones(32, np.float32))
    assert orc.matmul_q4_0(q1, np.ones(32, np.float32), None, 1, 32)[0] > 0


@pytest.mark.parametrize("n,m", [(64, 256), (37, 96), (33, 512), (16, 4096), (5, 200)])
def test_gemv_random_vs_f64(orc, n, m):
    rng_w = orc.normal_f32(1000 + n, n * m, 0.02)
    x = orc.normal_f32(2000 + m, m)
    q = orc.quantize_q4_0(np.concatenate([rng_w, np.zeros((-n * m) % 32, np.float32)]))
    ref = orc.matmul_q4_0_f64(q, x, None, n, m)
    for fn in (orc.matmul_q4_0, orc.matmul_q4_0_scalar, orc.matmul_q4_0_avx2):
        assert orc.normwise_err(fn(q, x, None, n, m), ref) < 1e-5
    # the brute-force reference itself equals dequantise-then-matmul in fp64
    deq = orc.dequantize_q4_0(q)[: n * m].astype(np.float64).reshape(n, m)
    assert np.allclose(ref, deq @ x.astype(np.float64), rtol=1e-12, atol=1e-12)


def test_gemv_threads_deterministic(orc):
    q = orc.quantize_q4_0(orc.normal_f32(3, 128 * 512, 0.02))
    x = orc.normal_f32(4, 512)
    orc.set_threads(1)
    a = orc.matmul_q4_0(q, x, None, 128, 512)
    orc.set_threads(4)
    b = orc.matmul_q4_0(q, x, None, 128, 512)
    orc.set_threads(1)
    assert np.array_equal(a, b)   # row-parallel: each row summed by one thread


# --- FP16 GEMV (kernels.rs:543-586) and batch_matmul (turbo.rs:306-333) ---------

def _f16_bytes(a):
    return np.asarray(a, np.float16).view(np.uint8).ravel()


def test_f16_kat_ops_rs(orc):
    # ops.rs:114-121 ([[1,2],[3,4]] . [5,6] = [17,39]) with FP16 weights (exact)
    y = orc.matmul_f16(_f16_bytes([[1, 2], [3, 4]]), np.array([5, 6], np.float32), None, 2, 2)
    assert list(y) == [17.0, 39.0]


@pytest.mark.parametrize("n,m", [(7, 13), (16, 64), (3, 1000)])
def test_f16_random_vs_f64(orc, n, m):
    w = orc.normal_f32(5, (n, m), 0.02).astype(np.float16)
    x = orc.normal_f32(6, m)
    b = orc.normal_f32(7, n)
    ref = orc.matmul_f16_f64(_f16_bytes(w), x, b, n, m)
    direct = w.astype(np.float64) @ x.astype(np.float64) + b
    assert np.allclose(ref, direct, rtol=1e-12, atol=1e-12)
    for fn in (orc.matmul_f16, orc.matmul_f16_scalar):
        assert orc.normwise_err(fn(_f16_bytes(w), x, b, n, m), ref) < 1e-5


def test_batch_matmul_kats(orc):
    # turbo.rs:956-977 (W = [1 0; 0 2], three tokens) and turbo.rs:991-1004
    # (W = [1 2 3], four tokens), with FP16 weights holding the same exact values
    y = orc.batch_matmul(_f16_bytes([[1, 0], [0, 2]]), 1,
                         np.array([1, 0, 0, 1, 3, 4], np.float32), 2, 2, 3)
    assert y.ravel().tolist() == [1, 0, 0, 2, 3, 8]
    y = orc.batch_matmul(_f16_bytes([1, 2, 3]), 1,
                         np.array([1, 0, 0, 0, 1, 0, 0, 0, 1, 5, 5, 5], np.float32), 1, 3, 4)
    assert y.ravel().tolist() == [1, 2, 3, 30]


def test_batch_matmul_q4_0_per_token(orc):
    n, m, t = 24, 96, 5
    q = orc.quantize_q4_0(orc.normal_f32(8, n * m, 0.02))
    x = orc.normal_f32(9, (t, m))
    y = orc.batch_matmul(q, 3, x, n, m, t)
    for i in range(t):
        assert np.array_equal(y[i], orc.matmul_q4_0(q, x[i], None, n, m))
    with pytest.raises(ValueError):
        orc.batch_matmul(q, 2, x, n, m, t)   # Q8_0 is not on this path
