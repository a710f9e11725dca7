"""Column-major Q4_0 (kernels.rs:403-535; ops.rs:41-51; turbo.rs:322-326).

W_col[k][j]: for each input index k, n outputs quantised in Q4_0 blocks
along n (the layout hypno's bench builds by transposing W, bench.rs:135-148).
No reference test checks this path numerically, so the oracle's scalar
restatement is pinned by exact integer cases (d = 1, integer x: every
summation order gives the same bits), fp64, n % 32 != 0 and short buffers;
GPU tests compare the device kernel with both."""
import numpy as np
import pytest

GEMV_TOL = 1e-4


def _col_weights(orc, seed, n, m):
    """Transpose-then-quantise, as bench.rs:137-148 does."""
    w_row = orc.normal_f32(seed, n * m, 0.02).reshape(n, m)
    w_col = np.ascontiguousarray(w_row.T)           # [m][n]
    nb = n // 32
    flat = w_col[:, :nb * 32].reshape(-1)           # floor(n/32) blocks per column
    return orc.quantize_q4_0(flat)


def _int_weights(rng, n, m):
    """d = 1.0 in every block, random nibbles: values are small integers."""
    nb = n // 32
    blk = rng.integers(0, 256, (m * nb, 18), dtype=np.uint8)
    blk[:, 0], blk[:, 1] = 0x00, 0x3C
    return blk.ravel()


def _ints(wq, n, m):
    nb = n // 32
    b = wq.reshape(m * nb, 18)[:, 2:]
    q = np.empty((m * nb, 32), np.int64)
    q[:, 0::2] = (b & 15).astype(np.int64) - 8
    q[:, 1::2] = (b >> 4).astype(np.int64) - 8
    return q.reshape(m, nb * 32)                     # W_col[k][j] for j < 32 nb


# --- oracle pins (CPU) ----------------------------------------------------------------

def test_col_oracle_exact_integers_tail_and_short(orc):
    rng = np.random.default_rng(1)
    n, m = 100, 37                                   # 3 blocks per column, 4 tail outputs
    wq = _int_weights(rng, n, m)
    x = rng.integers(-4, 5, m).astype(np.float32)
    bias = rng.integers(-9, 10, n).astype(np.float32)
    want = np.zeros(n, np.float64)
    want[:96] = x.astype(np.int64) @ _ints(wq, n, m)
    want += bias
    assert np.array_equal(orc.matmul_q4_0_col(wq, x, bias, n, m), want.astype(np.float32))
    # short buffer: whole columns k >= 20, and the last block of column 19, missing
    cut = (19 * 3 + 2) * 18 + 5
    short = np.zeros(n, np.float64)
    full = _ints(wq, n, m)
    short[:96] = x[:19].astype(np.int64) @ full[:19]
    short[:64] += x[19] * full[19, :64]
    assert np.array_equal(orc.matmul_q4_0_col(wq[:cut], x, None, n, m), short.astype(np.float32))


def test_col_oracle_against_f64(orc):
    n, m = 4096, 512
    wq = _col_weights(orc, 2, n, m)
    x = orc.normal_f32(3, m, 1.0)
    y = orc.matmul_q4_0_col(wq, x, None, n, m)
    ref = orc.matmul_q4_0_col_f64(wq, x, None, n, m)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-5


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
@pytest.mark.parametrize("n,m", [(4096, 4096), (14336, 4096), (4096, 14336), (2048, 2048),
                                 (256, 2048), (96, 64), (100, 50), (4096, 1), (31, 8),
                                 (100, 10)])
def test_col_gemv(torch, hk, orc, n, m):
    """Shapes from the Mistral projections down to a single block column; a
    tail of n % 32 outputs (bias only); one k range written straight to y
    (m = 10, with bias)."""
    print(f"col n={n} m={m}", flush=True)
    wq = _col_weights(orc, n + m, n, m)
    x = orc.normal_f32(n + 2 * m, m, 1.0)
    bias = orc.normal_f32(n, n, 1.0) if m % 2 == 0 else None
    ref = orc.matmul_q4_0_col(wq, x, bias, n, m)
    f64 = orc.matmul_q4_0_col_f64(wq, x, bias, n, m)
    y = torch.empty(n, device="cuda")
    hk.matmul_q4_0_col(y, torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda(),
                       torch.from_numpy(bias).cuda() if bias is not None else None, n, m)
    got = y.cpu().numpy()
    scale = max(np.max(np.abs(ref)), 1e-30)
    assert np.max(np.abs(got - ref)) / scale <= GEMV_TOL
    assert np.max(np.abs(got - f64)) / scale <= GEMV_TOL


@pytest.mark.gpu
def test_col_exact_short_unaligned_and_batch(torch, hk, orc):
    rng = np.random.default_rng(4)
    n, m = 4096, 300
    wq = _int_weights(rng, n, m)
    x = rng.integers(-4, 5, m).astype(np.float32)
    exact = (x.astype(np.int64) @ _ints(wq, n, m)).astype(np.float32)
    dw = torch.from_numpy(wq).cuda()
    y = torch.empty(n, device="cuda")
    hk.matmul_q4_0_col(y, dw, torch.from_numpy(x).cuda(), None, n, m)
    assert np.array_equal(y.cpu().numpy(), exact)            # integer sums: exact
    # short buffer (odd block count: byte-load path at the end) and a w
    # offset by 2 bytes (byte-load path throughout)
    for cut, off in (((100 * 128 + 7) * 18 + 3, 0), (len(wq), 2)):
        buf = np.zeros(cut + off, np.uint8)
        buf[off:] = wq[:cut]
        dbuf = torch.from_numpy(buf).cuda()[off:]
        hk.matmul_q4_0_col(y, dbuf, torch.from_numpy(x).cuda(), None, n, m)
        want = orc.matmul_q4_0_col(wq[:cut], x, None, n, m)
        assert np.array_equal(y.cpu().numpy(), want), (cut, off)
    # batch (turbo.rs:322-326) on the host-slice path, and vec_col on FP16
    xb = orc.normal_f32(5, 3 * m, 1.0)
    yb = np.empty(3 * n, np.float32)
    wf = _col_weights(orc, 6, n, m)
    hk.batch_matmul(yb, wf, hk.DType.Q4_0, xb, n, m, 3, col_major=True)
    for t in range(3):
        ref = orc.matmul_q4_0_col(wf, xb[t * m:(t + 1) * m], None, n, m)
        assert np.max(np.abs(yb[t * n:(t + 1) * n] - ref)) / np.max(np.abs(ref)) <= GEMV_TOL
    w16 = (orc.normal_f32(7, 64 * 128, 0.02)).astype(np.float16).view(np.uint8)
    y16 = np.empty(64, np.float32)
    xf = orc.normal_f32(8, 128, 1.0)
    hk.matmul_vec_col(y16, w16, hk.DType.FP16, xf, None, 64, 128)   # ops.rs:47: not Q4_0
    ref16 = orc.matmul_f16(w16, xf, None, 64, 128)
    assert np.max(np.abs(y16 - ref16)) / np.max(np.abs(ref16)) <= GEMV_TOL


@pytest.mark.gpu
def test_col_nonfinite_x_and_missing_blocks(torch, hk, orc):
    """An inf and a NaN in x at rows whose blocks lie past a short buffer add
    nothing (kernels.rs:522: the column ends there), as in the scalar form;
    an inf at a row that is present spreads as the oracle's does."""
    n, m = 256, 64
    wq = _col_weights(orc, 11, n, m)
    cut = 40 * (n // 32) * 18 + 3 * 18 + 7             # rows >= 41 and most of row 40 missing
    x = orc.normal_f32(12, m, 1.0)
    x[50], x[45] = np.float32("inf"), np.float32("nan")
    y = torch.empty(n, device="cuda")
    dw = torch.from_numpy(wq[:cut].copy()).cuda()
    hk.matmul_q4_0_col(y, dw, torch.from_numpy(x).cuda(), None, n, m)
    want = orc.matmul_q4_0_col(wq[:cut], x, None, n, m)
    got = y.cpu().numpy()
    assert np.all(np.isfinite(want)) and np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) <= GEMV_TOL
    x[3] = np.float32("inf")
    hk.matmul_q4_0_col(y, dw, torch.from_numpy(x).cuda(), None, n, m)
    want = orc.matmul_q4_0_col(wq[:cut], x, None, n, m)
    got = y.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = np.isfinite(want)
    assert np.array_equal(got[~fin & ~np.isnan(want)], want[~fin & ~np.isnan(want)])


@pytest.mark.gpu
def test_col_long_k_exact(torch, hk, orc):
    """m past 65535 ranges of 128 rows (each work-group then loops over three
    ranges): d = 1 and x in {-1, 1}, so every partial sum is a small integer
    and the result is exact whatever the order."""
    rng = np.random.default_rng(13)
    n, m = 32, 65535 * 128 + 1000
    print(f"col long k n={n} m={m}", flush=True)
    wq = _int_weights(rng, n, m)
    x = rng.choice(np.array([-1.0, 1.0], np.float32), m)
    want = orc.matmul_q4_0_col(wq, x, None, n, m)
    y = torch.empty(n, device="cuda")
    hk.matmul_q4_0_col(y, torch.from_numpy(wq).cuda(), torch.from_numpy(x).cuda(), None, n, m)
    assert np.array_equal(y.cpu().numpy(), want)


@pytest.mark.gpu
@pytest.mark.parametrize("batch,n,m", [(5, 4096, 4096), (3, 100, 10), (300, 96, 512)])
def test_col_batch_groups(torch, hk, orc, batch, n, m):
    """Several tokens on the device path run as groups (one main launch over
    all the group's tokens, one reduction launch; 300 tokens make two
    groups): every token's row bit-identical to its own one-token call, and
    within the GEMV bar of the scalar restatement, bias included."""
    import ctypes
    from hypno_amd import _lib
    lib = _lib.load()
    print(f"col batch={batch} n={n} m={m}", flush=True)
    wq = _col_weights(orc, batch + n, n, m)
    x = orc.normal_f32(batch + 3 * n, (batch, m), 1.0)
    bias = orc.normal_f32(n + 4, n, 1.0)
    dw, dx, db = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (wq, x, bias))

    def call(xp, rows):
        y = torch.full((rows * n,), float("nan"), device="cuda")
        _lib.check(lib.hypno_hip_matmul_q4_0_col_dev(
            ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(dw.data_ptr()), wq.size,
            ctypes.c_void_p(xp), ctypes.c_void_p(db.data_ptr()), n, m, rows, None),
            "matmul_q4_0_col_dev")
        torch.cuda.synchronize()
        return y.cpu().numpy().reshape(rows, n)

    got = call(dx.data_ptr(), batch)
    for t in sorted({0, 1, batch // 2, batch - 1}):
        assert np.array_equal(got[t], call(dx.data_ptr() + 4 * t * m, 1)[0]), t
    for t in range(batch):
        ref = orc.matmul_q4_0_col(wq, x[t], bias, n, m)
        assert np.max(np.abs(got[t] - ref)) / np.max(np.abs(ref)) <= GEMV_TOL, t
