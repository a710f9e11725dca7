"""GPU parity: libhypno_hip (through its C ABI) against the CPU oracle.

Bars (from the north star):
  * dequantize / quantize: bit-exact;
  * GEMV (1..15 tokens, fp32 accumulation): max|y - r| / max|r| <= 1e-4 against
    the oracle's restatement of matmul_q4_0 (kernels.rs:256), with r in fp32;
  * MFMA GEMM (>= 16 tokens, activations rounded to fp16):
    ||Y - R||_2 / ||R||_2 <= 2e-3 against the fp32 CPU reference on fp32 X.
Inputs: seeded N(0, 0.02) weights quantised by the oracle's quantizer
(quant.rs:108), N(0, 1) activations.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-4
GEMM_TOL = 2e-3


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    assert _t.cuda.is_available(), "GPU tests need a visible MI355X"
    return _t


@pytest.fixture(scope="module")
def hk(torch):
    import hypno_amd
    from hypno_amd import _lib
    _lib.load()
    return hypno_amd


@pytest.fixture(scope="module", autouse=True)
def cpu_threads(orc):
    orc.set_threads(min(16, os.cpu_count() or 1))
    yield
    orc.set_threads(1)


def _q4(orc, n, m, seed):
    """Q4_0 bytes of an n x m N(0, 0.02) matrix (zero-padded to a whole block)."""
    w = orc.normal_f32(seed, n * m, 0.02)
    pad = (-n * m) % 32
    if pad:
        w = np.concatenate([w, np.zeros(pad, np.float32)])
    return orc.quantize_q4_0(w)


def _gpu(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _run_q4(torch, hk, q, x, bias, n, m, batch=1):
    y = torch.empty(batch * n, dtype=torch.float32, device="cuda")
    if batch == 1:
        hk.matmul_q4_0(y, q, x, bias, n, m)
    else:
        hk.batch_matmul(y, q, hk.DType.Q4_0, x, n, m, batch)
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(batch, n) if batch > 1 else y.cpu().numpy()


# --- codec ------------------------------------------------------------------------

def test_dequantize_bit_exact(torch, hk, orc):
    rng = np.random.default_rng(1)
    nb = 50_000
    q = rng.integers(0, 256, size=nb * 18, dtype=np.uint8)
    # include special scales: zero, subnormal, inf, NaN, negative
    blocks = q.reshape(nb, 18)
    for i, d in enumerate([0x0000, 0x0001, 0x03FF, 0x7C00, 0x7E00, 0xFC00, 0xBC00, 0x7BFF]):
        blocks[i, 0], blocks[i, 1] = d & 0xFF, d >> 8
    ref = orc.dequantize_q4_0(q)
    got = hk.dequantize_q4_0(_gpu(torch, q)).cpu().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # trailing partial block ignored
    assert hk.dequantize_q4_0(_gpu(torch, q[: 18 * 3 + 7])).numel() == 96


def test_quantize_bit_exact(torch, hk, orc):
    rng = np.random.default_rng(2)
    w = (rng.standard_normal(32 * 40_000).astype(np.float32) * np.float32(0.02))
    specials = w[: 32 * 8].reshape(8, 32)
    specials[0] = 0.0                                 # all zero -> d = 1.0
    specials[1, 3] = np.nan                           # NaN ignored by the max
    specials[2] = np.float32(1e6)                     # d overflows to inf
    specials[3] = np.float32(1e-40)                   # fp32 subnormals
    specials[4, 0] = np.inf
    specials[5] *= np.float32(1e-5)                   # f16-subnormal scales
    specials[6] = np.arange(32, dtype=np.float32) - 15.5
    specials[7] = np.float32(-7.0)
    w[: 32 * 8] = specials.ravel()
    ref = orc.quantize_q4_0(w)
    got = hk.quantize_f32_to_q4_0(_gpu(torch, w)).cpu().numpy()
    assert np.array_equal(got, ref)


# --- decode GEMV ---------------------------------------------------------------------

GEMV_SHAPES = [
    (2048, 2048),    # TinyLlama q/o, config 1
    (256, 2048),     # TinyLlama k/v
    (5632, 2048),    # TinyLlama gate/up
    (2048, 5632),    # TinyLlama down (m/64 = 88 pairs: rows span waves)
    (1024, 4096),    # Mistral k/v
    (3072, 8192),    # Llama-3.2-3B down
    (4096, 14336),   # Mistral down (224 pairs)
    (64, 256), (33, 512), (5, 3072), (1, 768),
]


@pytest.mark.parametrize("n,m", GEMV_SHAPES)
def test_gemv_q4_0(torch, hk, orc, n, m):
    q = _q4(orc, n, m, seed=n * 7 + m)
    x = orc.normal_f32(m + 1, m)
    bias = orc.normal_f32(n + 2, n) if n % 2 else None
    ref = orc.matmul_q4_0(q, x, bias, n, m)
    got = _run_q4(torch, hk, _gpu(torch, q), _gpu(torch, x),
                  None if bias is None else _gpu(torch, bias), n, m)
    err = orc.normwise_err(got, ref)
    assert err <= GEMV_TOL, f"normwise error {err:.3e}"
    ref64 = orc.matmul_q4_0_f64(q, x, bias, n, m)
    assert orc.normwise_err(got, ref64) <= GEMV_TOL


@pytest.mark.parametrize("n,m", [(5, 48), (7, 40), (9, 100), (3, 13), (37, 96), (16, 4160),
                                 (11, 320)])
def test_gemv_generic_shapes(torch, hk, orc, n, m):
    # m % 32 != 0 (blocks straddle rows), m % 256 != 0 (generic kernel)
    q = _q4(orc, n, m, seed=m)
    x = orc.normal_f32(5, m)
    bias = orc.normal_f32(6, n)
    ref = orc.matmul_q4_0(q, x, bias, n, m)
    got = _run_q4(torch, hk, _gpu(torch, q), _gpu(torch, x), _gpu(torch, bias), n, m)
    assert orc.normwise_err(got, ref) <= GEMV_TOL


def test_gemv_exact_integers(torch, hk, orc):
    # d = 1 and integer activations: exact in any order, so bit-equal
    rng = np.random.default_rng(3)
    for n, m in [(64, 256), (2048, 2048), (7, 48), (300, 5632)]:
        nb = (n * m + 31) // 32
        nib = rng.integers(0, 16, size=(nb, 32))
        q = np.empty((nb, 18), np.uint8)
        q[:, 0], q[:, 1] = 0x00, 0x3C
        q[:, 2:] = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
        q = q.ravel()
        x = rng.integers(-4, 5, size=m).astype(np.float32)
        want = (nib - 8).ravel()[: n * m].reshape(n, m).astype(np.int64) @ x.astype(np.int64)
        got = _run_q4(torch, hk, _gpu(torch, q), _gpu(torch, x), None, n, m)
        assert np.array_equal(got, want.astype(np.float32)), (n, m)


def test_gemv_unaligned_and_short(torch, hk, orc):
    n, m = 64, 512
    q = _q4(orc, n, m, seed=9)
    x = orc.normal_f32(10, m)
    # weights at an odd device address (generic kernel)
    buf = torch.zeros(q.size + 1, dtype=torch.uint8, device="cuda")
    buf[1:] = _gpu(torch, q)
    got = _run_q4(torch, hk, buf[1:], _gpu(torch, x), None, n, m)
    assert orc.normwise_err(got, orc.matmul_q4_0(q, x, None, n, m)) <= GEMV_TOL
    # short buffer: blocks past the end contribute nothing (kernels.rs:275-277, :374)
    short = q[: 18 * 500 + 5]
    ref = orc.matmul_q4_0(short, x, None, n, m)
    got = _run_q4(torch, hk, _gpu(torch, short), _gpu(torch, x), None, n, m)
    assert np.allclose(got[32:], 0.0) and np.allclose(ref[32:], 0.0)
    assert orc.normwise_err(got, ref) <= GEMV_TOL
    # m = 0: y = bias (kernels.rs: empty row sums to 0)
    y = torch.empty(4, dtype=torch.float32, device="cuda")
    b = torch.arange(4, dtype=torch.float32, device="cuda")
    hk.matmul_q4_0(y, _gpu(torch, q), _gpu(torch, x), b, 4, 0)
    assert y.cpu().tolist() == [0.0, 1.0, 2.0, 3.0]


@pytest.mark.parametrize("batch", [2, 8, 15])
def test_small_batch_matches_per_token(torch, hk, orc, batch):
    n, m = 1024, 4096
    q = _q4(orc, n, m, seed=batch)
    x = orc.normal_f32(20 + batch, (batch, m))
    ref = orc.batch_matmul(q, 3, x, n, m, batch)
    got = _run_q4(torch, hk, _gpu(torch, q), _gpu(torch, x), None, n, m, batch)
    for t in range(batch):
        assert orc.normwise_err(got[t], ref[t]) <= GEMV_TOL


# --- a few tokens (weight-streaming MFMA kernel) -------------------------------------

@pytest.mark.parametrize("batch,n,m", [
    (2, 37, 512), (7, 1000, 1024), (8, 4096, 4096), (9, 130, 2048), (15, 4097, 256),
    (16, 64, 768), (17, 300, 4096), (32, 1024, 3072), (33, 2048, 1024), (64, 4096, 4096),
    (6, 3000, 1536), (8, 12288, 512), (12, 12289, 256), (40, 12300, 256),
    (5, 12300, 8192), (4, 12289, 256), (7, 14336, 4096),
])
def test_skinny_q4_0(torch, hk, orc, batch, n, m):
    """2..64 tokens: against the oracle's per-token GEMVs (turbo.rs:329-331).
    Up to 15 tokens the bar is the GEMV's (fp32 activations, 1e-4 normwise
    per token); from 16 the prefill GEMM's (fp16 activations, 2e-3 rel L2).
    N >= 12288, or 16-row tiles that would re-read more than 64 MiB of
    activations (64 tokens at 4096 x 4096), takes 64-row work-groups; the
    other shapes here 16-row ones (one stage of K, 32 stages, a last tile of
    one row or of 12 rows)."""
    q = _q4(orc, n, m, seed=batch * 7 + n)
    x = orc.normal_f32(batch + 100, (batch, m))
    bias = orc.normal_f32(batch + 200, n)
    y = torch.empty(batch * n, dtype=torch.float32, device="cuda")
    from hypno_amd import _lib
    import ctypes
    lib = _lib.load()
    qg, xg, bg = _gpu(torch, q), _gpu(torch, x), _gpu(torch, bias)
    st = lib.hypno_hip_matmul_q4_0_dev(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(qg.data_ptr()),
                                       q.size, ctypes.c_void_p(xg.data_ptr()),
                                       ctypes.c_void_p(bg.data_ptr()), n, m, batch, None)
    assert st == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(batch, n)
    ref = orc.batch_matmul(q, 3, x, n, m, batch) + bias
    if batch < 16:
        for t in range(batch):
            assert orc.normwise_err(got[t], ref[t]) <= GEMV_TOL, t
    else:
        assert orc.rel_l2(got, ref) <= GEMM_TOL


@pytest.mark.parametrize("batch,n,m", [(8, 1000, 4096), (40, 1100, 4096), (16, 4096, 14336)])
def test_skinny_split_k_repeat(torch, hk, orc, batch, n, m):
    """Split-K (few row tiles): each split writes its own partial plane and a
    second launch adds the planes in split order (+ bias), so the workspace
    reused by back-to-back calls with other inputs in between leaves the
    results bit-identical and correct."""
    import ctypes
    from hypno_amd import _lib
    lib = _lib.load()
    qh = _q4(orc, n, m, seed=batch + n)
    q = _gpu(torch, qh)
    x1 = orc.normal_f32(batch + 1, (batch, m))
    x2 = orc.normal_f32(batch + 2, (batch, m))
    bias = orc.normal_f32(batch + 3, n)
    bg = _gpu(torch, bias)

    def run(x):
        y = torch.empty(batch * n, dtype=torch.float32, device="cuda")
        xg = _gpu(torch, x)
        st = lib.hypno_hip_matmul_q4_0_dev(ctypes.c_void_p(y.data_ptr()),
                                           ctypes.c_void_p(q.data_ptr()), qh.size,
                                           ctypes.c_void_p(xg.data_ptr()),
                                           ctypes.c_void_p(bg.data_ptr()), n, m, batch, None)
        assert st == 0
        torch.cuda.synchronize()
        return y.cpu().numpy().reshape(batch, n)

    y1, y2, y1b = run(x1), run(x2), run(x1)
    assert np.array_equal(y1, y1b)
    for x, got in ((x1, y1), (x2, y2)):
        ref = orc.batch_matmul(qh, 3, x, n, m, batch) + bias
        if batch < 16:
            for t in range(batch):
                assert orc.normwise_err(got[t], ref[t]) <= GEMV_TOL, t
        else:
            assert orc.rel_l2(got, ref) <= GEMM_TOL



@pytest.mark.parametrize("batch,n,m", [
    (2, 4096, 14336), (2, 4097, 256), (3, 1000, 4096), (3, 1024, 4096), (3, 300, 2048),
    (3, 4096, 4096), (3, 257, 2048),
])
def test_gemv_few_rows(torch, hk, orc, batch, n, m):
    """Two rows (three on a matrix of at most 16M weights) take one pass of
    the streaming GEMV with every block multiplied by each row: each row's result
    is bit-identical to that row alone through the one-row GEMV (the same
    integer digit products, block partials and fixed-order sums), and within
    the GEMV bar of the oracle's per-token GEMVs (turbo.rs:329-331).  Wide
    activation ranges, an outlier, a zero row and a NaN row included."""
    import ctypes
    from hypno_amd import _lib
    lib = _lib.load()
    q = _q4(orc, n, m, seed=batch * 13 + n)
    x = orc.normal_f32(batch + 300, (batch, m))
    x[0, 5] = np.float32(1e4)
    x[1] *= np.float32(1e-5)
    nan_row = 2 if batch > 2 and n % 2 == 1 else -1
    if batch > 2:
        if nan_row == 2:
            x[2, 77] = np.float32("nan")
        else:
            x[2] = 0.0
    bias = orc.normal_f32(batch + 400, n)
    qg, xg, bg = _gpu(torch, q), _gpu(torch, x), _gpu(torch, bias)

    def call(xp, rows):
        y = torch.empty(rows * n, dtype=torch.float32, device="cuda")
        st = lib.hypno_hip_matmul_q4_0_dev(ctypes.c_void_p(y.data_ptr()),
                                           ctypes.c_void_p(qg.data_ptr()), q.size,
                                           ctypes.c_void_p(xp), ctypes.c_void_p(bg.data_ptr()),
                                           n, m, rows, None)
        assert st == 0
        torch.cuda.synchronize()
        return y.cpu().numpy().reshape(rows, n)

    got = call(xg.data_ptr(), batch)
    ref = orc.batch_matmul(q, 3, x, n, m, batch) + bias
    for t in range(batch):
        one = call(xg.data_ptr() + 4 * t * m, 1)[0]
        assert np.array_equal(got[t], one, equal_nan=True), t
        if t == nan_row:
            assert np.isnan(got[t]).all() == np.isnan(ref[t]).all()
        else:
            assert orc.normwise_err(got[t], ref[t]) <= GEMV_TOL, t
    assert np.array_equal(got, call(xg.data_ptr(), batch), equal_nan=True)


@pytest.mark.parametrize("batch,n,m", [(4, 1024, 4096), (8, 1024, 4096), (5, 256, 2048),
                                        (8, 2000, 2048), (6, 4096, 14336), (8, 14336, 4096),
                                        (4, 14336, 4096), (7, 4096, 4096), (8, 300, 8192)])
def test_skinny_own_activation_stages(torch, hk, orc, batch, n, m):
    """Up to 8 tokens, activations as hi/lo rows with 1/s per stage: converted
    by the work-groups themselves (16-row tiles whose K is split into short
    ranges) or by the pre-pass launch (64-row tiles: gate/up, down; 16-row
    tiles without such a split: q/o).  Wide ranges, a 1e4 outlier, a zero token
    and a NaN in the last token's last stage; bit-identical repeats;
    every token within the GEMV bar of the oracle (the NaN token: NaN where
    the oracle's is)."""
    q = _q4(orc, n, m, seed=batch * 7 + n)
    x = orc.normal_f32(batch + 900, (batch, m))
    x[0] *= np.float32(3e3)
    x[1, 3] = np.float32(1e4)
    if batch > 3:
        x[2] = 0.0
    x[batch - 1, m - 5] = np.float32("nan")
    qg, xg = _gpu(torch, q), _gpu(torch, x)
    got = _run_q4(torch, hk, qg, xg, None, n, m, batch)
    again = _run_q4(torch, hk, qg, xg, None, n, m, batch)
    assert np.array_equal(got, again, equal_nan=True)
    ref = orc.batch_matmul(q, 3, x, n, m, batch)
    for t in range(batch - 1):
        if t == 2 and batch > 3:
            assert np.all(got[t] == 0.0)
        else:
            assert orc.normwise_err(got[t], ref[t]) <= GEMV_TOL, t
    assert np.array_equal(np.isnan(got[batch - 1]), np.isnan(ref[batch - 1]))


def test_skinny_wide_range_activations(torch, hk, orc):
    """Per-token power-of-two scaling: tokens of very different magnitude,
    a 1e4 outlier channel, tiny values and an all-zero token stay within the
    GEMV bar."""
    batch, n, m = 6, 512, 2048
    q = _q4(orc, n, m, seed=77)
    x = orc.normal_f32(78, (batch, m))
    x[0] *= np.float32(1e-6)
    x[1] *= np.float32(3e3)
    x[2, 17] = np.float32(1e4)
    x[3] = 0.0
    x[4, ::2] *= np.float32(1e-3)
    got = _run_q4(torch, hk, _gpu(torch, q), _gpu(torch, x), None, n, m, batch)
    ref = orc.batch_matmul(q, 3, x, n, m, batch)
    for t in range(batch):
        if t == 3:
            assert np.all(got[t] == 0.0)
        else:
            assert orc.normwise_err(got[t], ref[t]) <= GEMV_TOL, t


def test_gemv_linearity_and_determinism_full_size(torch, hk, orc):
    # Mistral gate/up at full size: size-independent properties
    n, m = 14336, 4096
    q = _gpu(torch, _q4(orc, n, m, seed=11))
    x1 = orc.normal_f32(12, m)
    x2 = orc.normal_f32(13, m)
    y1 = _run_q4(torch, hk, q, _gpu(torch, x1), None, n, m)
    y1b = _run_q4(torch, hk, q, _gpu(torch, x1), None, n, m)
    y2 = _run_q4(torch, hk, q, _gpu(torch, x2), None, n, m)
    y12 = _run_q4(torch, hk, q, _gpu(torch, x1 + x2), None, n, m)
    assert np.array_equal(y1, y1b)  # row-major: deterministic
    assert orc.normwise_err(y12, y1.astype(np.float64) + y2) <= 1e-5
    ref = orc.matmul_q4_0(q.cpu().numpy(), x1, None, n, m)
    assert orc.normwise_err(y1, ref) <= GEMV_TOL


def test_gemv_plan_mixed_jobs(torch, hk, orc):
    # one TinyLlama layer (m = 2048 and 5632 share one launch), plus a bias job
    # and a job the streaming kernel cannot take (m = 320 -> generic kernel)
    shapes = [(2048, 2048), (256, 2048), (256, 2048), (2048, 2048), (5632, 2048),
              (5632, 2048), (2048, 5632), (300, 2048), (40, 320)]
    jobs, refs = [], []
    for i, (n, m) in enumerate(shapes):
        q = _q4(orc, n, m, seed=500 + i)
        x = orc.normal_f32(600 + i, m)
        bias = orc.normal_f32(700 + i, n) if i == 7 else None
        y = torch.full((n,), float("nan"), device="cuda")
        jobs.append((y, _gpu(torch, q), _gpu(torch, x), None if bias is None else _gpu(torch, bias),
                     n, m))
        refs.append(orc.matmul_q4_0(q, x, bias, n, m))
    plan = hk.GemvPlan(jobs)
    assert plan.launches == 2          # one streaming launch + one generic launch
    for rep in range(3):               # plans are re-runnable
        for j in jobs:
            j[0].fill_(float("nan"))
        plan.run()
        torch.cuda.synchronize()
        for (y, *_), ref in zip(jobs, refs):
            assert orc.normwise_err(y.cpu().numpy(), ref) <= GEMV_TOL
    plan.close()


def test_gemv_plan_many_small_jobs(torch, hk, orc):
    """The streaming kernel's per-wave LDS rings run two or three steps ahead
    across job boundaries: 40 jobs of 1-100 rows (one or two steps each,
    most with a partial last step) so that a ring slot often belongs to a
    later job than the step being computed, and work-groups whose range is
    shorter than the ring (the run-out reads nothing)."""
    rng = np.random.default_rng(71)
    jobs, refs = [], []
    for i in range(40):
        m = int(rng.choice([256, 512]))
        n = int(rng.choice([1, 3, 17, 64, 100]))
        q = _q4(orc, n, m, seed=1000 + i)
        x = orc.normal_f32(1100 + i, m)
        bias = orc.normal_f32(1200 + i, n) if i % 5 == 0 else None
        y = torch.full((n,), float("nan"), device="cuda")
        jobs.append((y, _gpu(torch, q), _gpu(torch, x),
                     None if bias is None else _gpu(torch, bias), n, m))
        refs.append(orc.matmul_q4_0(q, x, bias, n, m))
    plan = hk.GemvPlan(jobs)
    assert plan.launches == 1
    for rep in range(2):
        for j in jobs:
            j[0].fill_(float("nan"))
        plan.run()
        torch.cuda.synchronize()
        for i, ((y, *_), ref) in enumerate(zip(jobs, refs)):
            assert orc.normwise_err(y.cpu().numpy(), ref) <= GEMV_TOL, (rep, i)
    plan.close()


@pytest.mark.parametrize("n,m", [(40, 32768), (300, 16384)])
def test_gemv_longest_rows(torch, hk, orc, n, m):
    """K = 32768 (1024-thread work-groups, 16 per-wave rings beside 86 KB of
    activation staging) and K = 16384, with partial last steps."""
    q = _q4(orc, n, m, seed=n + m)
    x = orc.normal_f32(m + 3, m)
    got = _run_q4(torch, hk, _gpu(torch, q), _gpu(torch, x), None, n, m)
    assert orc.normwise_err(got, orc.matmul_q4_0(q, x, None, n, m)) <= GEMV_TOL
    assert orc.normwise_err(got, orc.matmul_q4_0_f64(q, x, None, n, m)) <= GEMV_TOL


def test_gemv_plan_mistral_layer_in_graph(torch, hk, orc):
    # Mistral-7B layer shapes (m = 4096 and 14336 share T = 448), captured in a
    # HIP graph and replayed with fresh activations written in place
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096),
              (14336, 4096), (4096, 14336)]
    qs = [_q4(orc, n, m, seed=800 + i) for i, (n, m) in enumerate(shapes)]
    xs = [torch.empty(m, device="cuda") for _, m in shapes]
    ys = [torch.empty(n, device="cuda") for n, _ in shapes]
    plan = hk.GemvPlan([(y, _gpu(torch, q), x, None, n, m)
                        for y, q, x, (n, m) in zip(ys, qs, xs, shapes)])
    assert plan.launches == 1
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    for x in xs:
        x.zero_()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        plan.run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        plan.run()
    for rep in range(2):
        xh = [orc.normal_f32(900 + 10 * rep + i, m) for i, (_, m) in enumerate(shapes)]
        for x, h in zip(xs, xh):
            x.copy_(torch.from_numpy(h))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for y, q, h, (n, m) in zip(ys, qs, xh, shapes):
            assert orc.normwise_err(y.cpu().numpy(), orc.matmul_q4_0(q, h, None, n, m)) <= GEMV_TOL
    plan.close()


# --- prefill GEMM (MFMA) -------------------------------------------------------------

def _gemm_ref(orc, q, x, n, m):
    """fp64 brute force of X . W^T over the dequantised weights."""
    w = orc.dequantize_q4_0(q)[: n * m].reshape(n, m).astype(np.float64)
    return x.astype(np.float64) @ w.T


@pytest.mark.parametrize("batch,n,m", [
    (16, 1024, 4096), (64, 4096, 4096), (100, 200, 512), (130, 4097, 256),
    (512, 8192, 3072),   # Llama-3.2-3B gate/up, config 3
    (512, 3072, 8192),   # Llama-3.2-3B down
])
def test_gemm_q4_0(torch, hk, orc, batch, n, m):
    q = _q4(orc, n, m, seed=batch + n)
    x = orc.normal_f32(batch * 3 + 1, (batch, m))
    if batch == 512:  # config 3: 1% of channels scaled x20 as outliers
        rng = np.random.default_rng(99)
        ch = rng.permutation(m)[: round(0.01 * m)]
        x[:, ch] *= np.float32(20.0)
    got = _run_q4(torch, hk, _gpu(torch, q), _gpu(torch, x), None, n, m, batch)
    ref = _gemm_ref(orc, q, x, n, m)
    err = orc.rel_l2(got, ref)
    assert err <= GEMM_TOL, f"rel L2 {err:.3e}"
    # spot-check a few tokens against the oracle's per-token GEMV (turbo.rs:329-331)
    for t in (0, batch - 1):
        r32 = orc.matmul_q4_0(q, x[t], None, n, m)
        assert orc.rel_l2(got[t], r32) <= GEMM_TOL


@pytest.mark.parametrize("batch", [96, 300])
def test_gemm_q4_0_scale_range(torch, hk, orc, batch, gemm_mode):
    """The default GEMM scales each block's partial sum by its d in fp32;
    the folded mode, from 128 tokens (this W is small), rounds each weight to
    fp16 after dividing its row by a power of two above the row's largest
    block scale.  Either way rows of huge scales (whose weights overflow fp16
    unnormalised), tiny scales, mixed scales and zero scales each stay within
    the GEMM bar column by column."""
    n, m = 300, 512
    q = _q4(orc, n, m, seed=41)
    blk = q.reshape(n, m // 32, 18)
    def set_d(rows, vals):
        bits = np.asarray(vals, np.float16).view(np.uint8).reshape(-1, 2)
        blk[rows, :, 0] = bits[:, 0]
        blk[rows, :, 1] = bits[:, 1]
    set_d(0, np.full(m // 32, 60000.0))                         # |w| up to 480000
    set_d(1, np.full(m // 32, 1e-6))                            # fp16 subnormal scales
    set_d(2, np.where(np.arange(m // 32) % 2 == 0, 1e3, 1e-3))  # 1e6 apart in one row
    set_d(3, np.zeros(m // 32))
    set_d(299, np.full(m // 32, 65504.0))                       # largest fp16, tail tile
    x = orc.normal_f32(42, (batch, m))
    got = _run_q4(torch, hk, _gpu(torch, q), _gpu(torch, x), None, n, m, batch)
    ref = _gemm_ref(orc, q, x, n, m)
    assert np.all(got[:, 3] == 0.0)
    for j in [c for c in range(n) if c != 3]:
        err = orc.rel_l2(got[:, j], ref[:, j])
        assert err <= GEMM_TOL, (j, err)


@pytest.mark.parametrize("batch,n,m", [(500, 12289, 1024), (512, 12300, 512)])
def test_gemm_q4_0_256_row_tiles(torch, hk, orc, batch, n, m, gemm_mode):
    """Grids of 256-row tiles that fill the GPU take the 256-row tile
    kernels (the exact kernel's 16 M-tiles per wave; the folded mode's
    256 x 128 tiles): an M tail inside the last tile (500 of 512 rows), an N tail (one
    column past 96 tiles, or 12 past), a bias, and rows of extreme block
    scales (as test_gemm_q4_0_scale_range); checked on a seeded sample of
    columns plus the special ones against fp64."""
    q = _q4(orc, n, m, seed=batch + 3 * n)
    blk = q.reshape(n, m // 32, 18)

    def set_d(rows, vals):
        bits = np.asarray(vals, np.float16).view(np.uint8).reshape(-1, 2)
        blk[rows, :, 0] = bits[:, 0]
        blk[rows, :, 1] = bits[:, 1]
    set_d(0, np.full(m // 32, 60000.0))
    set_d(1, np.full(m // 32, 1e-6))
    set_d(2, np.where(np.arange(m // 32) % 2 == 0, 1e3, 1e-3))
    set_d(n - 1, np.full(m // 32, 65504.0))
    x = orc.normal_f32(batch + 17, (batch, m))
    bias = orc.normal_f32(batch + 18, n)
    import ctypes
    from hypno_amd import _lib
    lib = _lib.load()
    y = torch.empty(batch * n, dtype=torch.float32, device="cuda")
    qg, xg, bg = _gpu(torch, q), _gpu(torch, x), _gpu(torch, bias)
    st = lib.hypno_hip_matmul_q4_0_dev(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(qg.data_ptr()),
                                       q.size, ctypes.c_void_p(xg.data_ptr()),
                                       ctypes.c_void_p(bg.data_ptr()), n, m, batch, None)
    assert st == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(batch, n)
    rng = np.random.default_rng(n)
    cols = np.unique(np.concatenate([[0, 1, 2, n - 1, n - 2], rng.choice(n, 300, replace=False)]))
    w = orc.dequantize_q4_0(q).reshape(n, m)[cols].astype(np.float64)
    ref = x.astype(np.float64) @ w.T + bias[cols].astype(np.float64)
    assert orc.rel_l2(got[:, cols], ref) <= GEMM_TOL
    for k, c in enumerate(cols):
        if c < 3 or c >= n - 2:
            assert orc.rel_l2(got[:, c], ref[:, k]) <= GEMM_TOL, c


@pytest.mark.parametrize("m", [320, 384])
def test_gemm_bias_and_tails(torch, hk, orc, m):
    # M and N tails with a bias; m = 320 takes the 64-column kernel, m = 384
    # the 128-column-stage kernel
    batch, n = 33, 130
    q = _q4(orc, n, m, seed=5)
    x = orc.normal_f32(6, (batch, m))
    bias = orc.normal_f32(7, n)
    y = torch.empty(batch * n, dtype=torch.float32, device="cuda")
    from hypno_amd import _lib
    lib = _lib.load()
    import ctypes
    qg, xg, bg = _gpu(torch, q), _gpu(torch, x), _gpu(torch, bias)
    st = lib.hypno_hip_matmul_q4_0_dev(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(qg.data_ptr()),
                                       q.size, ctypes.c_void_p(xg.data_ptr()),
                                       ctypes.c_void_p(bg.data_ptr()), n, m, batch, None)
    assert st == 0
    torch.cuda.synchronize()
    ref = _gemm_ref(orc, q, x, n, m) + bias.astype(np.float64)
    assert orc.rel_l2(y.cpu().numpy().reshape(batch, n), ref) <= GEMM_TOL


@pytest.mark.parametrize("batch,n,m", [(128, 1024, 4096), (200, 300, 2048), (512, 1024, 4096)])
def test_gemm_split_k_deterministic(torch, hk, orc, batch, n, m, gemm_mode):
    """Small tile grids split K over work-groups and add the partial planes in
    a fixed order: within the GEMM bar, bias included, and bitwise equal from
    run to run."""
    q = _q4(orc, n, m, seed=n + m)
    x = orc.normal_f32(batch + 9, (batch, m))
    bias = orc.normal_f32(batch + 10, n)
    from hypno_amd import _lib
    import ctypes
    lib = _lib.load()
    qg, xg, bg = _gpu(torch, q), _gpu(torch, x), _gpu(torch, bias)
    outs = []
    for _ in range(2):
        y = torch.empty(batch * n, dtype=torch.float32, device="cuda")
        st = lib.hypno_hip_matmul_q4_0_dev(ctypes.c_void_p(y.data_ptr()),
                                           ctypes.c_void_p(qg.data_ptr()), q.size,
                                           ctypes.c_void_p(xg.data_ptr()),
                                           ctypes.c_void_p(bg.data_ptr()), n, m, batch, None)
        assert st == 0
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy().reshape(batch, n))
    assert np.array_equal(outs[0], outs[1])
    ref = _gemm_ref(orc, q, x, n, m) + bias.astype(np.float64)
    assert orc.rel_l2(outs[0], ref) <= GEMM_TOL


SPLIT_CASES = [(8, 4096, 14336), (40, 1024, 4096), (512, 3072, 8192), (128, 1024, 4096)]


def test_split_pieces_repeat_and_graph(torch, hk, orc):
    """Shapes whose K is split over work-groups (partial planes in the
    stream's workspace, added in split order by a second kernel): few tokens
    with hi/lo rows (8 x 4096 x 14336) and fp16 rows (40 x 1024 x 4096), the
    prefill GEMM (512 x 3072 x 8192, 128 x 1024 x 4096).  Three eager calls
    each, then all four captured in one HIP graph (consecutive kernels reuse
    one workspace) and replayed three times: every result bit-identical to
    the first, and the first within its bar against fp64 on sampled
    columns."""
    side = torch.cuda.Stream()
    cases = []
    for batch, n, m in SPLIT_CASES:
        print(f"[case] split pieces batch={batch} n={n} m={m}", flush=True)
        q = _q4(orc, n, m, seed=batch + n + m)
        x = orc.normal_f32(batch + 5, (batch, m))
        cases.append((batch, n, m, q, _gpu(torch, q), _gpu(torch, x), x))
    side.wait_stream(torch.cuda.current_stream())
    first = []
    with torch.cuda.stream(side):
        for batch, n, m, q, qg, xg, x in cases:
            outs = []
            for _ in range(3):
                y = torch.full((batch * n,), float("nan"), device="cuda")
                hk.batch_matmul(y, qg, hk.DType.Q4_0, xg, n, m, batch)
                outs.append(y)
            torch.cuda.synchronize()
            got = [o.cpu().numpy().reshape(batch, n) for o in outs]
            assert np.array_equal(got[0], got[1]) and np.array_equal(got[0], got[2])
            cols = np.random.default_rng(n).choice(n, min(n, 256), replace=False)
            w = orc.dequantize_q4_0(q).reshape(n, m)[cols].astype(np.float64)
            ref = x.astype(np.float64) @ w.T
            if batch < 16:
                for t in range(batch):
                    assert orc.normwise_err(got[0][t, cols], ref[t]) <= GEMV_TOL, t
            else:
                assert orc.rel_l2(got[0][:, cols], ref) <= GEMM_TOL
            first.append(got[0])
    torch.cuda.synchronize()
    ys = [torch.full((batch * n,), float("nan"), device="cuda") for batch, n, *_ in cases]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for (batch, n, m, q, qg, xg, x), y in zip(cases, ys):
            hk.batch_matmul(y, qg, hk.DType.Q4_0, xg, n, m, batch)
    for rep in range(3):
        for y in ys:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for (batch, n, *_), y, ref in zip(cases, ys, first):
            assert np.array_equal(y.cpu().numpy().reshape(batch, n), ref), (rep, batch, n)


# --- FP16 weights (lm_head variant) --------------------------------------------------

def _f16w(orc, n, m, seed):
    return orc.normal_f32(seed, (n, m), 0.02).astype(np.float16)


@pytest.mark.parametrize("n,m", [(4097, 4096), (1000, 4096), (7, 13), (64, 200), (333, 4104)])
def test_gemv_f16(torch, hk, orc, n, m):
    w = _f16w(orc, n, m, seed=n)
    wb = w.view(np.uint8).ravel()
    x = orc.normal_f32(3, m)
    bias = orc.normal_f32(4, n)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    hk.matmul_f16(y, _gpu(torch, wb), _gpu(torch, x), _gpu(torch, bias), n, m)
    torch.cuda.synchronize()
    ref = orc.matmul_f16(wb, x, bias, n, m)
    assert orc.normwise_err(y.cpu().numpy(), ref) <= GEMV_TOL


@pytest.mark.parametrize("batch,n,m", [(128, 4097, 4096), (16, 256, 512)])
def test_gemm_f16(torch, hk, orc, batch, n, m):
    w = _f16w(orc, n, m, seed=n + 1)
    wb = w.view(np.uint8).ravel()
    x = orc.normal_f32(8, (batch, m))
    y = torch.empty(batch * n, dtype=torch.float32, device="cuda")
    hk.batch_matmul(y, _gpu(torch, wb), hk.DType.FP16, _gpu(torch, x), n, m, batch)
    torch.cuda.synchronize()
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert orc.rel_l2(y.cpu().numpy().reshape(batch, n), ref) <= GEMM_TOL


@pytest.mark.parametrize("batch,n,m", [(200, 1000, 1024), (130, 3000, 2048), (40, 513, 320)])
def test_gemm_f16_bias_tails_and_repeat(torch, hk, orc, batch, n, m):
    """FP16 GEMM with bias through the C ABI: M and N tails, K split across
    work-groups (partials added in split order), and bit-identical repeats."""
    import ctypes
    from hypno_amd import _lib
    lib = _lib.load()
    w = _f16w(orc, n, m, seed=n + 3)
    wb = _gpu(torch, w.view(np.uint8).ravel())
    x = _gpu(torch, orc.normal_f32(9, (batch, m)))
    bias = orc.normal_f32(10, n)
    bg = _gpu(torch, bias)

    def run():
        y = torch.empty(batch * n, dtype=torch.float32, device="cuda")
        st = lib.hypno_hip_matmul_f16_dev(ctypes.c_void_p(y.data_ptr()),
                                          ctypes.c_void_p(wb.data_ptr()), wb.numel(),
                                          ctypes.c_void_p(x.data_ptr()),
                                          ctypes.c_void_p(bg.data_ptr()), n, m, batch, None)
        assert st == 0
        torch.cuda.synchronize()
        return y.cpu().numpy().reshape(batch, n)

    y1, y2 = run(), run()
    assert np.array_equal(y1, y2)
    ref = x.cpu().numpy().astype(np.float64) @ w.astype(np.float64).T + bias
    assert orc.rel_l2(y1, ref) <= GEMM_TOL


def _f16_dev(torch, wb, x, bias, n, m, batch):
    import ctypes
    from hypno_amd import _lib
    lib = _lib.load()
    y = torch.full((batch * n,), float("nan"), dtype=torch.float32, device="cuda")
    st = lib.hypno_hip_matmul_f16_dev(ctypes.c_void_p(y.data_ptr()),
                                      ctypes.c_void_p(wb.data_ptr()), wb.numel(),
                                      ctypes.c_void_p(x.data_ptr()),
                                      None if bias is None else ctypes.c_void_p(bias.data_ptr()),
                                      n, m, batch, None)
    assert st == 0
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(batch, n)


@pytest.mark.parametrize("batch,n,m", [(2, 4097, 4096), (5, 1000, 4160), (15, 513, 2048),
                                        (3, 300, 8192), (8, 98305, 512)])
def test_f16_few_tokens_hilo(torch, hk, orc, batch, n, m):
    """FP16 weights at 2..15 tokens: one pass of the streaming FP16 GEMM over
    hi/lo fp16 rows (x 2^s = hi + lo per token), held to the GEMV bar of
    each token's fp32 matmul_f16 (kernels.rs:543-586).  A 1e4 outlier, a
    tiny token, a zero token, a NaN token; N tails, a K split (n = 300),
    16-wave work-groups (n = 98305: 512-column tiles fill the GPU), bias;
    bit-identical repeats."""
    w = _f16w(orc, n, m, seed=n + 5)
    wb = _gpu(torch, w.view(np.uint8).ravel())
    x = orc.normal_f32(40 + batch, (batch, m))
    x[0, 7] = np.float32(1e4)
    x[1] *= np.float32(1e-6)
    if batch > 2:
        x[2] = 0.0
    if batch > 3:
        x[3, m - 1] = np.float32("nan")
    bias = orc.normal_f32(41, n)
    xg, bg = _gpu(torch, x), _gpu(torch, bias)
    got = _f16_dev(torch, wb, xg, bg, n, m, batch)
    assert np.array_equal(got, _f16_dev(torch, wb, xg, bg, n, m, batch), equal_nan=True)
    wbytes = w.view(np.uint8).ravel()
    for t in range(batch):
        ref = orc.matmul_f16(wbytes, x[t], bias, n, m)
        if t == 3:
            assert np.isnan(got[t]).all() and np.isnan(ref).all()
        else:
            assert orc.normwise_err(got[t], ref) <= GEMV_TOL, t


def test_f16_few_tokens_unaligned_x(torch, hk, orc):
    """Below 16 tokens with activations not 16-byte aligned: the FP16 arm
    runs the fp32 GEMV token by token (the hi/lo pre-pass reads float4);
    each token within the GEMV bar."""
    batch, n, m = 5, 600, 1024
    w = _f16w(orc, n, m, seed=21)
    x = orc.normal_f32(22, (batch, m))
    buf = torch.zeros(batch * m + 1, dtype=torch.float32, device="cuda")
    buf[1:] = _gpu(torch, x.ravel())
    got = _f16_dev(torch, _gpu(torch, w.view(np.uint8).ravel()), buf[1:], None, n, m, batch)
    wbytes = w.view(np.uint8).ravel()
    for t in range(batch):
        assert orc.normwise_err(got[t], orc.matmul_f16(wbytes, x[t], None, n, m)) <= GEMV_TOL, t


def test_f16_few_tokens_inf(torch, hk, orc):
    """An inf activation: every output of its token is the inf (or NaN for a
    zero weight) the fp32 reference gives, with its sign; other tokens are
    unaffected."""
    batch, n, m = 4, 700, 1024
    w = _f16w(orc, n, m, seed=9)
    w[5, 100] = 0.0
    x = orc.normal_f32(10, (batch, m))
    x[1, 100] = np.float32("inf")
    got = _f16_dev(torch, _gpu(torch, w.view(np.uint8).ravel()), _gpu(torch, x), None, n, m, batch)
    wbytes = w.view(np.uint8).ravel()
    ref = orc.matmul_f16(wbytes, x[1], None, n, m)
    assert np.array_equal(np.isnan(got[1]), np.isnan(ref))
    assert np.array_equal(got[1][np.isinf(ref)], ref[np.isinf(ref)])
    for t in (0, 2, 3):
        assert orc.normwise_err(got[t], orc.matmul_f16(wbytes, x[t], None, n, m)) <= GEMV_TOL


@pytest.mark.parametrize("batch,n,m", [(16, 4097, 4096), (17, 1000, 2048), (33, 2000, 4160),
                                        (24, 98305, 1024), (16, 98305, 512), (48, 98305, 512),
                                        (64, 300, 8192), (100, 4097, 1024), (128, 256, 4096)])
def test_f16_stream_gemm(torch, hk, orc, batch, n, m):
    """FP16 weights at 16..128 tokens (the streaming FP16 GEMM, all four tile
    heights, 8-, 12- and 16-wave work-groups): N tails, K % 256 != 0, a K split
    with the split-order reduction (n = 300), bias; GEMM bar against fp64;
    bit-identical repeats."""
    w = _f16w(orc, n, m, seed=n + 7)
    wb = _gpu(torch, w.view(np.uint8).ravel())
    x = orc.normal_f32(50 + batch, (batch, m))
    bias = orc.normal_f32(51, n)
    xg, bg = _gpu(torch, x), _gpu(torch, bias)
    got = _f16_dev(torch, wb, xg, bg, n, m, batch)
    assert np.array_equal(got, _f16_dev(torch, wb, xg, bg, n, m, batch))
    ref = x.astype(np.float64) @ w.astype(np.float64).T + bias
    assert orc.rel_l2(got, ref) <= GEMM_TOL


# --- host-slice ABI (drop-in for the &[f32]/&[u8] signature) --------------------------

def test_host_slice_entry_points(hk, orc):
    n, m = 300, 1024
    q = _q4(orc, n, m, seed=77)
    x = orc.normal_f32(78, m)
    bias = orc.normal_f32(79, n)
    y = np.empty(n, np.float32)
    hk.matmul_q4_0(y, q, x, bias, n, m)
    assert orc.normwise_err(y, orc.matmul_q4_0(q, x, bias, n, m)) <= GEMV_TOL
    # registered (resident) weights give identical results
    hk.register_weight(q)
    y2 = np.empty(n, np.float32)
    hk.matmul_vec_auto(y2, q, hk.DType.Q4_0, x, bias, n, m)
    hk.unregister_weight(q)
    assert np.array_equal(y, y2)
    # batch_matmul on host arrays, fp16 and q4_0
    xb = orc.normal_f32(80, (3, m))
    yb = np.empty(3 * n, np.float32)
    hk.batch_matmul(yb, q, hk.DType.Q4_0, xb, n, m, 3)
    ref = orc.batch_matmul(q, 3, xb, n, m, 3)
    for t in range(3):
        assert orc.normwise_err(yb.reshape(3, n)[t], ref[t]) <= GEMV_TOL
    w16 = _f16w(orc, n, m, 81).view(np.uint8).ravel()
    yf = np.empty(n, np.float32)
    hk.matmul_f16(yf, w16, x, None, n, m)
    assert orc.normwise_err(yf, orc.matmul_f16(w16, x, None, n, m)) <= GEMV_TOL


def test_error_paths(torch, hk, orc):
    n, m = 8, 64
    q = _gpu(torch, _q4(orc, n, m, 1))
    x = torch.zeros(m, device="cuda")
    y = torch.empty(n, device="cuda")
    with pytest.raises(ValueError):
        hk.matmul_q4_0(torch.empty(n + 1, device="cuda"), q, x, None, n, m)
    with pytest.raises(ValueError):
        hk.matmul_q4_0(y, q, torch.zeros(m - 1, device="cuda"), None, n, m)
    with pytest.raises(hk.HypnoHipError) as e:   # FP32 weights are not on this path
        hk.matmul_vec_auto(y, q, hk.DType.FP32, x, None, n, m)
    assert e.value.status == 95
    with pytest.raises(hk.HypnoHipError) as e:   # Q4_0-sized bytes are short for Q8_0
        hk.matmul_vec_auto(y, q, hk.DType.Q8_0, x, None, n, m)
    assert e.value.status == 22
    with pytest.raises(hk.HypnoHipError) as e:   # fp16 buffer too short
        hk.matmul_f16(y, torch.zeros(2 * n * m - 2, dtype=torch.uint8, device="cuda"), x, None,
                      n, m)
    assert e.value.status == 22
