"""Q8_0 weights (quant.rs:74-103, 176-206; ops.rs:33-36; turbo.rs:334-341).

The reference has no Q8_0 test of its own, so the oracle's codec is pinned
here by hand-built blocks whose bytes follow from the definition — chosen so
that dividing by the unrounded scale (what Q4_0 does), half-even rounding, a
missing clamp or a non-saturating cast each give a different byte — and by
the round-trip bound; its GEMV by exact integer cases and fp64.  GPU tests
check the device codec bit for bit and the GEMVs against the oracle."""
import numpy as np
import pytest

GEMV_TOL = 1e-4  # max|y - ref| / max|ref| (fp32 accumulation)


def _f16(v) -> np.float32:
    return np.float32(np.float16(np.float32(v)))


# --- oracle pins (CPU) ----------------------------------------------------------------

def test_quantizer_divides_by_the_rounded_scale(orc):
    """amax = 1: d = f16(1/127) = 0.00787353515625 < 1/127.  For v = 100.4995
    unrounded steps, v/d lands above 100.5 (q = 101) while v*127 stays below
    (q = 100): the byte tells the two apart."""
    s_unrounded = np.float32(1.0) / np.float32(127.0)
    d = _f16(s_unrounded)
    assert d < s_unrounded
    v = np.float32(100.4995) * s_unrounded
    assert np.floor(np.float32(v / d) + 0.5) == 101 and np.floor(np.float32(v / s_unrounded) + 0.5) == 100
    block = np.zeros(32, np.float32)
    block[0], block[1] = 1.0, v
    q = orc.quantize_q8_0(block)
    assert int(q[0]) | (int(q[1]) << 8) == int(np.float16(d).view(np.uint16))
    assert q[2] == 127 + 128 and q[3] == 101 + 128


def test_quantizer_rounds_half_away_and_zero_block(orc):
    """amax = 127 gives d = 1.0 exactly, so v / d = v: ties go away from zero
    (2.5 -> 3, -2.5 -> -3, 0.5 -> 1, -0.5 -> -1, 126.5 -> 127)."""
    block = np.zeros(32, np.float32)
    block[:7] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -127.0]
    q = orc.quantize_q8_0(block)
    assert (q[0], q[1]) == (0x00, 0x3C)
    assert list(q[2:9]) == [255, 131, 125, 129, 127, 255, 1]
    assert np.all(q[9:] == 128)
    z = orc.quantize_q8_0(np.zeros(32, np.float32))   # amax = 0 -> d = 1.0
    assert (z[0], z[1]) == (0x00, 0x3C) and np.all(z[2:] == 128)


def test_quantizer_special_scales(orc):
    # inf: amax = inf -> d = inf; finite/inf = 0 and inf/inf = NaN -> 0: all 128
    b = np.full(32, 1.0, np.float32)
    b[3] = np.inf
    q = orc.quantize_q8_0(b)
    assert (q[0], q[1]) == (0x00, 0x7C) and np.all(q[2:] == 128)
    # NaN is skipped by the max fold and quantises to 0 (saturating cast)
    b = np.linspace(-1, 1, 32).astype(np.float32)
    b[5] = np.nan
    q = orc.quantize_q8_0(b)
    assert q[2 + 5] == 128 and q[2] == 1 and q[2 + 31] == 255
    # amax / 127 below the smallest f16 subnormal: d = 0, v / 0 = +-inf -> +-127
    b = np.zeros(32, np.float32)
    b[0], b[1] = 1e-30, -1e-30
    q = orc.quantize_q8_0(b)
    assert (q[0], q[1]) == (0, 0) and (q[2], q[3]) == (255, 1) and np.all(q[4:] == 128)


def test_round_trip_bound_and_dequant_closed_form(orc):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal(32 * 500) * 0.02).astype(np.float32)
    q = orc.quantize_q8_0(w)
    deq = orc.dequantize_q8_0(q).reshape(-1, 32)
    d = q.reshape(-1, 34)[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.all(np.abs(deq - w.reshape(-1, 32)) <= d * 0.5 * (1 + 1e-6))
    blk = np.zeros(34, np.uint8)
    blk[0], blk[1] = 0x00, 0x40   # d = 2.0
    blk[2:] = np.arange(32) * 8
    assert np.array_equal(orc.dequantize_q8_0(blk), (np.arange(32) * 8 - 128) * 2.0)
    assert orc.dequantize_q8_0(np.zeros(33, np.uint8)).size == 0   # floor(len/34)


def test_matmul_q8_0_oracle(orc):
    """Exact integer case (d = 1, integer x: every order gives the same sum),
    flattened rows straddling blocks (m = 40), fp64 agreement, short buffer."""
    rng = np.random.default_rng(6)
    n, m = 7, 40
    u = rng.integers(0, 256, n * m // 32 * 34 + 34, dtype=np.uint8).reshape(-1, 34)
    u[:, 0], u[:, 1] = 0x00, 0x3C
    w = u.ravel()
    x = rng.integers(-3, 4, m).astype(np.float32)
    ints = (u[:, 2:].astype(np.int64) - 128).ravel()[:n * m].reshape(n, m)
    want = (ints @ x.astype(np.int64)).astype(np.float32)
    assert np.array_equal(orc.matmul_q8_0(w, x, None, n, m), want)
    wq = orc.quantize_q8_0(orc.normal_f32(7, 64 * 4096, 0.02))
    xf = orc.normal_f32(8, 4096, 1.0)
    bias = orc.normal_f32(9, 64, 1.0)
    y = orc.matmul_q8_0(wq, xf, bias, 64, 4096)
    ref = orc.matmul_q8_0_f64(wq, xf, bias, 64, 4096)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-5  # sequential fp32 sum
    with pytest.raises(ValueError):
        orc.matmul_q8_0(wq[:-1], xf, None, 64, 4096)


# --- device (GPU) ---------------------------------------------------------------------

@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


@pytest.fixture(scope="module")
def hk():
    import hypno_amd
    return hypno_amd


@pytest.mark.gpu
def test_q8_0_codec_bit_exact(torch, hk, orc):
    rng = np.random.default_rng(10)
    blocks = [np.zeros(32, np.float32), (rng.standard_normal(32) * 1000).astype(np.float32),
              (rng.standard_normal(32) * 1e-6).astype(np.float32),
              np.full(32, -3.5, np.float32), (np.arange(32) - 16).astype(np.float32),
              (rng.standard_normal(32 * 4096) * 0.02).astype(np.float32)]
    b = np.full(32, 1.0, np.float32)
    b[3] = np.inf
    blocks.append(b)
    b = np.linspace(-1, 1, 32).astype(np.float32)
    b[5] = np.nan
    blocks.append(b)
    t = np.zeros(32, np.float32)
    t[:7] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -127.0]
    blocks.append(t)
    w = np.concatenate(blocks + [np.ones(17, np.float32)])  # trailing partial block dropped
    want = orc.quantize_q8_0(w)
    got = hk.quantize_f32_to_q8_0(torch.from_numpy(w).cuda()).cpu().numpy()
    assert np.array_equal(got, want)
    deq = hk.dequantize_q8_0(torch.from_numpy(want).cuda()).cpu().numpy()
    assert np.array_equal(deq.view(np.uint32), orc.dequantize_q8_0(want).view(np.uint32))


def _q8(orc, seed, n, m):
    # whole blocks covering all n*m elements (rows straddle blocks when
    # m % 32 != 0; the quantizer drops a partial last block)
    return orc.quantize_q8_0(orc.normal_f32(seed, -(-n * m // 32) * 32, 0.02))


@pytest.mark.gpu
@pytest.mark.parametrize("n,m", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336),
                                 (2048, 2048), (256, 2048), (5632, 2048), (2048, 5632),
                                 (37, 100), (33, 512), (5, 3072), (1, 256),
                                 # K = 32768: the streaming kernel's LDS (activation
                                 # staging + rings) does not fit, the generic kernel runs
                                 (40, 32768)])
def test_q8_0_gemv(torch, hk, orc, n, m):
    print(f"q8_0 gemv n={n} m={m}", flush=True)
    wq = _q8(orc, n + m, n, m)
    x = orc.normal_f32(n * 3 + m, m, 1.0)
    bias = orc.normal_f32(n + 1, n, 1.0) if n % 2 else None
    ref = orc.matmul_q8_0(wq, x, bias, n, m)
    y = torch.empty(n, device="cuda")
    hk.matmul_q8_0(y, torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda(),
                   torch.from_numpy(bias).cuda() if bias is not None else None, n, m)
    got = y.cpu().numpy()
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= GEMV_TOL
    f64 = orc.matmul_q8_0_f64(wq, x, bias, n, m)
    assert np.max(np.abs(got - f64)) / np.max(np.abs(f64)) <= GEMV_TOL


@pytest.mark.gpu
def test_q8_0_unaligned_repeat_and_extremes(torch, hk, orc):
    """x not 16-byte aligned (the generic kernel), repeat bit-exact on the
    streaming kernel, and activations spanning 1e-30..1e30 (per-block
    exponents of the digit planes)."""
    n, m = 512, 4096
    wq = _q8(orc, 3, n, m)
    dw = torch.from_numpy(wq).cuda()
    x = orc.normal_f32(4, m + 1, 1.0)
    exps = np.arange(-30, 34, 2)[np.arange((m + 32) // 32) % 32]   # one decade per block
    x = (x * np.repeat(np.float32(10.0) ** exps, 32)[: m + 1]).astype(np.float32)
    dx = torch.from_numpy(x).cuda()
    ys = []
    for xs in (dx[1:], dx[:m], dx[:m]):
        y = torch.empty(n, device="cuda")
        hk.matmul_q8_0(y, dw, xs, None, n, m)
        ys.append(y.cpu().numpy())
    assert np.array_equal(ys[1], ys[2])
    for got, xin in ((ys[0], x[1:]), (ys[1], x[:m])):
        ref = orc.matmul_q8_0_f64(wq, xin, None, n, m)
        assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= GEMV_TOL


@pytest.mark.gpu
def test_q8_0_batch_and_host_paths(torch, hk, orc):
    n, m, batch = 300, 1024, 3
    wq = _q8(orc, 11, n, m)
    x = orc.normal_f32(12, batch * m, 1.0)
    ref = np.concatenate([orc.matmul_q8_0(wq, x[t * m:(t + 1) * m], None, n, m)
                          for t in range(batch)])
    y = np.empty(batch * n, np.float32)
    hk.batch_matmul(y, wq, hk.DType.Q8_0, x, n, m, batch)          # host slices
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) <= GEMV_TOL
    y1 = np.empty(n, np.float32)
    hk.matmul_vec_auto(y1, wq, hk.DType.Q8_0, x[:m], None, n, m)   # ops.rs:33-36
    assert np.max(np.abs(y1 - ref[:n])) / np.max(np.abs(ref)) <= GEMV_TOL
    yd = torch.empty(batch * n, device="cuda")
    hk.batch_matmul(yd, torch.from_numpy(wq).cuda(), hk.DType.Q8_0, torch.from_numpy(x).cuda(),
                    n, m, batch)
    assert np.max(np.abs(yd.cpu().numpy() - ref)) / np.max(np.abs(ref)) <= GEMV_TOL
    with pytest.raises(hk.HypnoHipError) as e:
        hk.matmul_q8_0(torch.empty(n, device="cuda"), torch.from_numpy(wq[:-34]).cuda(),
                       torch.from_numpy(x[:m]).cuda(), None, n, m)
    assert e.value.status == 22


GEMM_TOL = 2e-3  # rel-L2 over all M x N (north_star: MFMA prefill, fp16 activations)


@pytest.mark.gpu
@pytest.mark.parametrize("batch,n,m", [(16, 512, 256), (64, 1000, 1024), (128, 4096, 4096),
                                       (512, 2048, 2048), (20, 3, 64)])
def test_q8_0_gemm(torch, hk, orc, batch, n, m):
    """M >= 16 runs the fp16 GEMM on weights expanded to fp16 (per-row
    normalised): against the per-token fp32 reference on the unrounded x
    (turbo.rs:334-341 semantics; the fp16 rounding of x and of the weights
    both count against the tolerance), and the bias on the device path."""
    print(f"q8_0 gemm batch={batch} n={n} m={m}", flush=True)
    wq = _q8(orc, batch + n + m, n, m)
    x = orc.normal_f32(batch * 7 + m, batch * m, 1.0).reshape(batch, m)
    bias = orc.normal_f32(n + 5, n, 1.0)
    w64 = orc.dequantize_q8_0(wq)[: n * m].reshape(n, m).astype(np.float64)
    ref = x.astype(np.float64) @ w64.T + bias           # fp64 of the reference's product
    for t in (0, batch - 1):                             # and its own per-token form
        assert orc.rel_l2(orc.matmul_q8_0(wq, x[t], bias, n, m), ref[t]) <= 1e-5
    y = torch.empty(batch * n, device="cuda")
    import ctypes
    from hypno_amd import _lib
    dw, dx, db = (torch.from_numpy(a).cuda() for a in (wq, np.ascontiguousarray(x), bias))
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.load().hypno_hip_matmul_q8_0_dev(
        ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(dw.data_ptr()), wq.size,
        ctypes.c_void_p(dx.data_ptr()), ctypes.c_void_p(db.data_ptr()), n, m, batch, st),
        "matmul_q8_0_dev")
    got = y.cpu().numpy().reshape(batch, n)
    err = orc.rel_l2(got, ref)
    assert err <= GEMM_TOL, f"rel L2 {err:.3e}"
    # a weight row with one huge block scale: per-row normalisation keeps the
    # fp16 expansion finite (|w| up to 127 * 60000 > fp16 max)
    if (batch, n, m) == (16, 512, 256):
        big = wq.copy().reshape(-1, 34)
        big[0, 0:2] = np.frombuffer(np.float16(60000.0).tobytes(), np.uint8)
        big = big.ravel()
        refb = x.astype(np.float64) @ orc.dequantize_q8_0(big)[: n * m].reshape(n, m).astype(
            np.float64).T
        yb = torch.empty(batch * n, device="cuda")
        hk.batch_matmul(yb, torch.from_numpy(big).cuda(), hk.DType.Q8_0, dx.reshape(-1), n, m,
                        batch)
        gb = yb.cpu().numpy().reshape(batch, n)
        assert np.all(np.isfinite(gb))
        assert orc.rel_l2(gb, refb) <= GEMM_TOL


@pytest.mark.gpu
@pytest.mark.parametrize("batch,n,m", [(2, 1000, 4096), (3, 37, 256), (4, 4096, 4096),
                                       (5, 4096, 14336), (8, 14336, 4096), (13, 300, 2048),
                                       (15, 2000, 1024), (6, 100, 512)])
def test_q8_0_few_tokens(torch, hk, orc, batch, n, m):
    """2 to 15 tokens: the few-row GEMV, in launches of 2 to 8 rows (the
    tokens split evenly).  Each token's row is bit-identical to its own
    one-token call (same digits, block partials and fixed-order sums), within
    the GEMV bar of the oracle; a NaN in one token stays in that token's row;
    the bias reaches every row."""
    print(f"q8_0 few tokens batch={batch} n={n} m={m}", flush=True)
    import ctypes
    from hypno_amd import _lib
    lib = _lib.load()
    wq = _q8(orc, batch + n, n, m)
    x = orc.normal_f32(batch + 31, (batch, m), 1.0)
    nan_row = batch // 2
    x[nan_row, m // 3] = np.float32("nan")
    bias = orc.normal_f32(n + 9, n, 1.0)
    dw, dx, db = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (wq, x, bias))

    def call(xp, rows):
        y = torch.full((rows * n,), float("nan"), device="cuda")
        _lib.check(lib.hypno_hip_matmul_q8_0_dev(
            ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(dw.data_ptr()), wq.size,
            ctypes.c_void_p(xp), ctypes.c_void_p(db.data_ptr()), n, m, rows, None),
            "matmul_q8_0_dev")
        torch.cuda.synchronize()
        return y.cpu().numpy().reshape(rows, n)

    got = call(dx.data_ptr(), batch)
    for t in range(batch):
        one = call(dx.data_ptr() + 4 * t * m, 1)[0]
        assert np.array_equal(got[t], one, equal_nan=True), t
        ref = orc.matmul_q8_0(wq, x[t], bias, n, m)
        if t == nan_row:
            assert np.array_equal(np.isnan(got[t]), np.isnan(ref))
        else:
            assert orc.normwise_err(got[t], ref) <= GEMV_TOL, t
    assert np.array_equal(got, call(dx.data_ptr(), batch), equal_nan=True)
