"""GPU parity at BASELINE.json's full sizes, and numerics edge cases.

Full-size cases whose CPU reference over every output would take minutes
are checked on a seeded sample of output columns (every token, fp64 over the
dequantised weights), plus the oracle's own per-token GEMV
(matmul_q4_0, kernels.rs:256) for a few whole tokens:
  * configs[3] Mistral-7B projections at M = 2048 (turbo.rs:306-333);
  * configs[4] lm_head K = 4096, N = 128256 (not a multiple of 512), Q4_0 and
    FP16 (kernels.rs:256, :571), M = 1 and 128; Q4_0 at M = 128 runs the GEMM
    variant that scales each block's partial sum in fp32 (W > 64 MB);
  * tokens of extreme magnitude on every activation path: the decode GEMV
    (one vector mixing 1e-6 blocks, 1e3 blocks and a 1e4 outlier), the
    few-token plain rows (17 tokens), the prefill GEMMs (100 and 300 tokens)
    and the FP16 / Q8_0 GEMMs, each token held to its bar separately.
Weights are N(0, 0.02) from a seeded torch generator, quantised on the GPU by
the quantizer that test_gpu_parity.py pins bit-exact to the oracle; the
packed bytes are copied back, so the oracle sees identical bytes.
"""
import ctypes
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


@pytest.fixture(scope="module")
def lib(hk):
    from hypno_amd import _lib
    return _lib.load()


@pytest.fixture(scope="module", autouse=True)
def cpu_threads(orc):
    orc.set_threads(min(16, os.cpu_count() or 1))
    yield
    orc.set_threads(1)


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


def _q4_dev(torch, hk, n, m, seed):
    """(device Q4_0 bytes, host copy) of an n x m N(0, 0.02) matrix."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(n * m, generator=gen, device="cuda").mul_(0.02)
    q = hk.quantize_f32_to_q4_0(w)
    del w
    return q, q.cpu().numpy()


def _sample_cols(n, count, seed):
    """`count` distinct output columns: seeded random ones plus both ends."""
    rng = np.random.default_rng(seed)
    cols = set(rng.choice(n, size=min(n, count), replace=False).tolist())
    cols.update([0, 1, n - 2, n - 1])
    return np.array(sorted(cols))


def _q4_rows_f64(orc, qh, rows, m):
    """Dequantised weight rows (K % 32 == 0: row r is bytes [r B 18, (r+1) B 18))."""
    rb = m // 32 * 18
    sub = np.concatenate([qh[r * rb:(r + 1) * rb] for r in rows])
    return orc.dequantize_q4_0(sub).reshape(len(rows), m).astype(np.float64)


def _q4_dev_call(lib, y, q, x, n, m, batch, bias=None):
    st = lib.hypno_hip_matmul_q4_0_dev(_vp(y), _vp(q), q.numel(), _vp(x),
                                       None if bias is None else _vp(bias), n, m, batch, None)
    assert st == 0, lib.hypno_hip_last_error()


# --- configs[3] at 2048 tokens -----------------------------------------------------

@pytest.mark.parametrize("name,n,m", [("q_o", 4096, 4096), ("k_v", 1024, 4096),
                                      ("gate_up", 14336, 4096), ("down", 4096, 14336)])
def test_mistral_m2048(torch, hk, lib, orc, name, n, m, gemm_mode):
    batch = 2048
    print(f"[case] mistral {name} n={n} m={m} batch={batch} {gemm_mode}", flush=True)
    q, qh = _q4_dev(torch, hk, n, m, seed=n + m)
    gen = torch.Generator(device="cuda").manual_seed(n * 3 + 1)
    x = torch.randn(batch, m, generator=gen, device="cuda")
    y = torch.empty(batch, n, device="cuda")
    _q4_dev_call(lib, y, q, x, n, m, batch)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    xh = x.cpu().numpy()
    cols = _sample_cols(n, 256, seed=n)
    ref = xh.astype(np.float64) @ _q4_rows_f64(orc, qh, cols, m).T
    err = orc.rel_l2(got[:, cols], ref)
    assert err <= GEMM_TOL, f"rel L2 {err:.3e} over {len(cols)} sampled columns"
    for t in (0, 1023, batch - 1):   # whole tokens against the oracle's GEMV
        r32 = orc.matmul_q4_0(qh, xh[t], None, n, m)
        assert orc.rel_l2(got[t], r32) <= GEMM_TOL, t


def _check_sampled(orc, got, xh, qh, n, m, cols_seed, tol, norm, tokens):
    """Sampled columns over every token (fp64 over the dequantised rows),
    then whole tokens against the oracle's per-token GEMV."""
    cols = _sample_cols(n, 256, seed=cols_seed)
    ref = xh.astype(np.float64) @ _q4_rows_f64(orc, qh, cols, m).T
    metric = orc.normwise_err if norm else orc.rel_l2
    for t in range(xh.shape[0]):
        err = metric(got[t, cols], ref[t])
        assert err <= tol, f"token {t}: {err:.3e} over {len(cols)} sampled columns"
    for t in tokens:
        r32 = orc.matmul_q4_0(qh, xh[t], None, n, m)
        assert metric(got[t], r32) <= tol, t


MISTRAL_MLP = [("gate_up", 14336, 4096), ("down", 4096, 14336)]


@pytest.mark.parametrize("batch", [8, 64, 512])
@pytest.mark.parametrize("name,n,m", MISTRAL_MLP)
def test_mistral_mlp_batches(torch, hk, lib, orc, name, n, m, batch):
    """configs[3] gate/up and down at 8, 64 and 512 tokens in the default
    arithmetic: the few-token kernel's 64-row grids (8: hi/lo activation rows,
    held to the GEMV bar per token; 64: plain fp16 rows) and the 256-row
    prefill tiles (512), turbo.rs:306-333 semantics."""
    print(f"[case] mistral {name} n={n} m={m} batch={batch}", flush=True)
    q, qh = _q4_dev(torch, hk, n, m, seed=n + m + batch)
    gen = torch.Generator(device="cuda").manual_seed(n * 5 + batch)
    x = torch.randn(batch, m, generator=gen, device="cuda")
    y = torch.full((batch, n), float("nan"), device="cuda")
    _q4_dev_call(lib, y, q, x, n, m, batch)
    torch.cuda.synchronize()
    few = batch <= 16
    _check_sampled(orc, y.cpu().numpy(), x.cpu().numpy(), qh, n, m, cols_seed=n + batch,
                   tol=GEMV_TOL if few else GEMM_TOL, norm=few,
                   tokens=(0, batch // 2, batch - 1))


EXACT_CASES = [("c2_gate_up", 8192, 3072, 512), ("c2_down", 3072, 8192, 512),
               ("q_o", 4096, 4096, 512), ("gate_up", 14336, 4096, 512),
               ("down", 4096, 14336, 512), ("k_v", 1024, 4096, 512),
               ("q_o", 4096, 4096, 2048), ("gate_up", 14336, 4096, 2048),
               ("down", 4096, 14336, 2048)]


@pytest.mark.parametrize("name,n,m,batch", EXACT_CASES)
def test_gemm_exact_nibbles(torch, hk, lib, orc, name, n, m, batch):
    """The north-star prefill arithmetic (exact integer nibbles into the
    MFMAs, each block's scale applied in fp32; hypno_hip_set_gemm_numerics
    GEMM_EXACT) at configs[2] and the Mistral-7B shapes at 512 and 2048
    tokens (the default arithmetic, set explicitly here).
    configs[2]'s activations carry its 1% x20 outlier channels."""
    print(f"[case] exact {name} n={n} m={m} batch={batch}", flush=True)
    q, qh = _q4_dev(torch, hk, n, m, seed=n + m + batch + 1)
    gen = torch.Generator(device="cuda").manual_seed(n * 7 + batch)
    x = torch.randn(batch, m, generator=gen, device="cuda")
    if name.startswith("c2"):
        ch = torch.randperm(m, generator=torch.Generator().manual_seed(m))[: m // 100]
        x[:, ch.cuda()] *= 20.0
    y = torch.full((batch, n), float("nan"), device="cuda")
    prev = hk.set_gemm_numerics(hk.GEMM_EXACT)
    try:
        _q4_dev_call(lib, y, q, x, n, m, batch)
        torch.cuda.synchronize()
    finally:
        hk.set_gemm_numerics(prev)
    _check_sampled(orc, y.cpu().numpy(), x.cpu().numpy(), qh, n, m, cols_seed=n + batch + 3,
                   tol=GEMM_TOL, norm=False, tokens=(0, batch - 1))


# --- the lm_head --------------------------------------------------------

LM_N, LM_M = 128256, 4096


@pytest.fixture(scope="module")
def lm_q4(torch, hk):
    return _q4_dev(torch, hk, LM_N, LM_M, seed=17)


@pytest.fixture(scope="module")
def lm_f16(torch):
    gen = torch.Generator(device="cuda").manual_seed(18)
    w = torch.randn(LM_N * LM_M, generator=gen, device="cuda").mul_(0.02).half()
    return w.view(torch.uint8), w.cpu().numpy().view(np.uint8)


def test_lm_head_q4_0_m1(torch, lib, orc, lm_q4):
    q, qh = lm_q4
    print("[case] lm_head q4_0 M=1", flush=True)
    xh = orc.normal_f32(19, LM_M)
    x = torch.from_numpy(xh).cuda()
    y = torch.empty(LM_N, device="cuda")
    _q4_dev_call(lib, y, q, x, LM_N, LM_M, 1)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = orc.matmul_q4_0(qh, xh, None, LM_N, LM_M)
    assert orc.normwise_err(got, ref) <= GEMV_TOL
    assert orc.normwise_err(got, orc.matmul_q4_0_f64(qh, xh, None, LM_N, LM_M)) <= GEMV_TOL


def test_lm_head_q4_0_m128(torch, lib, orc, lm_q4):
    """128 tokens, W = 295 MB: the GEMM variant with the block scale applied
    to each block's partial in fp32, tiles over N = 128256 (a tail at 512)."""
    q, qh = lm_q4
    batch = 128
    print("[case] lm_head q4_0 M=128", flush=True)
    xh = orc.normal_f32(20, (batch, LM_M))
    x = torch.from_numpy(xh).cuda()
    y = torch.empty(batch, LM_N, device="cuda")
    _q4_dev_call(lib, y, q, x, LM_N, LM_M, batch)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    cols = _sample_cols(LM_N, 512, seed=21)
    cols = np.union1d(cols, np.arange(LM_N - 300, LM_N))   # the last (partial) tiles
    ref = xh.astype(np.float64) @ _q4_rows_f64(orc, qh, cols, LM_M).T
    assert orc.rel_l2(got[:, cols], ref) <= GEMM_TOL
    for t in (0, batch - 1):
        assert orc.rel_l2(got[t], orc.matmul_q4_0(qh, xh[t], None, LM_N, LM_M)) <= GEMM_TOL


def test_lm_head_f16_m1(torch, lib, orc, lm_f16):
    w, wh = lm_f16
    print("[case] lm_head f16 M=1", flush=True)
    xh = orc.normal_f32(22, LM_M)
    x = torch.from_numpy(xh).cuda()
    y = torch.empty(LM_N, device="cuda")
    st = lib.hypno_hip_matmul_f16_dev(_vp(y), _vp(w), w.numel(), _vp(x), None, LM_N, LM_M, 1, None)
    assert st == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert orc.normwise_err(got, orc.matmul_f16(wh, xh, None, LM_N, LM_M)) <= GEMV_TOL
    assert orc.normwise_err(got, orc.matmul_f16_f64(wh, xh, None, LM_N, LM_M)) <= GEMV_TOL


def test_lm_head_f16_m128(torch, lib, orc, lm_f16):
    w, wh = lm_f16
    batch = 128
    print("[case] lm_head f16 M=128", flush=True)
    xh = orc.normal_f32(23, (batch, LM_M))
    x = torch.from_numpy(xh).cuda()
    y = torch.empty(batch, LM_N, device="cuda")
    st = lib.hypno_hip_matmul_f16_dev(_vp(y), _vp(w), w.numel(), _vp(x), None, LM_N, LM_M, batch,
                                      None)
    assert st == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    cols = np.union1d(_sample_cols(LM_N, 512, seed=24), np.arange(LM_N - 300, LM_N))
    w16 = wh.view(np.float16).reshape(LM_N, LM_M)
    ref = xh.astype(np.float64) @ w16[cols].astype(np.float64).T
    assert orc.rel_l2(got[:, cols], ref) <= GEMM_TOL
    for t in (0, batch - 1):
        assert orc.rel_l2(got[t], orc.matmul_f16(wh, xh[t], None, LM_N, LM_M)) <= GEMM_TOL


def test_gemm_exact_variant_multi_tile(torch, lib, orc, hk):
    """W just over 64 MB at 200 tokens: the fp32-scale GEMM variant with two
    M tiles (the class the Q4_0 lm_head at 128 tokens belongs to)."""
    n, m, batch = 32768, 4096, 200
    assert n * m // 32 * 18 > 64 << 20
    print(f"[case] exact variant n={n} m={m} batch={batch}", flush=True)
    q, qh = _q4_dev(torch, hk, n, m, seed=25)
    xh = orc.normal_f32(26, (batch, m))
    x = torch.from_numpy(xh).cuda()
    bias_h = orc.normal_f32(27, n)
    bias = torch.from_numpy(bias_h).cuda()
    y = torch.empty(batch, n, device="cuda")
    _q4_dev_call(lib, y, q, x, n, m, batch, bias)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    cols = _sample_cols(n, 512, seed=28)
    ref = xh.astype(np.float64) @ _q4_rows_f64(orc, qh, cols, m).T + bias_h[cols]
    assert orc.rel_l2(got[:, cols], ref) <= GEMM_TOL


# --- extreme activation magnitudes ---------------------------------------------------

def test_gemv_wide_range_activations(torch, lib, orc, hk):
    """M = 1 streaming kernel: one activation vector mixing blocks scaled by
    1e-6 and 1e3, an isolated 1e4 outlier, an all-zero block and 1e-30
    values; normwise against the oracle and fp64, plus the 1e-6 blocks alone
    (their own magnitude, so a GEMV that lost them would fail)."""
    n, m = 4096, 4096
    print("[case] gemv wide-range activations", flush=True)
    q, qh = _q4_dev(torch, hk, n, m, seed=29)
    x = orc.normal_f32(30, m)
    x[0:512] *= np.float32(1e-6)
    x[512:1024] *= np.float32(1e3)
    x[1500] = np.float32(1e4)
    x[2048:2080] = 0.0
    x[3000:3032] *= np.float32(1e-30)
    y = torch.empty(n, device="cuda")
    _q4_dev_call(lib, y, q, torch.from_numpy(x).cuda(), n, m, 1)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert orc.normwise_err(got, orc.matmul_q4_0(qh, x, None, n, m)) <= GEMV_TOL
    assert orc.normwise_err(got, orc.matmul_q4_0_f64(qh, x, None, n, m)) <= GEMV_TOL
    small = np.zeros(m, np.float32)
    small[0:512] = x[0:512]
    y2 = torch.empty(n, device="cuda")
    _q4_dev_call(lib, y2, q, torch.from_numpy(small).cuda(), n, m, 1)
    torch.cuda.synchronize()
    assert orc.normwise_err(y2.cpu().numpy(),
                            orc.matmul_q4_0_f64(qh, small, None, n, m)) <= GEMV_TOL


def _extreme_tokens(orc, batch, m, seed):
    x = orc.normal_f32(seed, (batch, m))
    x[1] *= np.float32(1e5)      # |x| past fp16's 65504
    x[2] *= np.float32(1e-6)     # below fp16's normal range
    x[3] = 0.0
    x[4, 7] = np.float32(3e4)    # one large channel in an ordinary token
    return x


@pytest.mark.parametrize("batch", [17, 40, 100, 300])
def test_q4_0_batched_extreme_tokens(torch, lib, orc, hk, batch, gemm_mode):
    """17 and 40 tokens (few-token plain rows), 100 and 300 (GEMM, fp32
    block scale; 300 under the folded mode: folded scale): each token is scaled by its own power of two
    before the fp16 rounding, so every token meets the GEMM bar on its own."""
    n, m = 1024, 2048
    print(f"[case] q4_0 extreme tokens batch={batch}", flush=True)
    q, qh = _q4_dev(torch, hk, n, m, seed=31 + batch)
    x = _extreme_tokens(orc, batch, m, seed=32 + batch)
    y = torch.empty(batch, n, device="cuda")
    _q4_dev_call(lib, y, q, torch.from_numpy(x).cuda(), n, m, batch)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = x.astype(np.float64) @ _q4_rows_f64(orc, qh, np.arange(n), m).T
    assert np.all(np.isfinite(got))
    assert np.all(got[3] == 0.0)
    for t in range(batch):
        if t != 3:
            assert orc.rel_l2(got[t], ref[t]) <= GEMM_TOL, t


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
def test_f16_q8_0_gemm_extreme_tokens(torch, lib, orc, hk, dtype):
    n, m, batch = 512, 1024, 40
    print(f"[case] {dtype} extreme tokens", flush=True)
    w = orc.normal_f32(33, (n, m), 0.02)
    x = _extreme_tokens(orc, batch, m, seed=34)
    y = torch.empty(batch, n, device="cuda")
    xg = torch.from_numpy(x).cuda()
    if dtype == "f16":
        wb = w.astype(np.float16)
        wd = wb.astype(np.float64)
        wg = torch.from_numpy(wb.view(np.uint8).ravel()).cuda()
        st = lib.hypno_hip_matmul_f16_dev(_vp(y), _vp(wg), wg.numel(), _vp(xg), None, n, m, batch,
                                          None)
    else:
        qb = orc.quantize_q8_0(w.ravel())
        wd = orc.dequantize_q8_0(qb).reshape(n, m).astype(np.float64)
        wg = torch.from_numpy(qb).cuda()
        st = lib.hypno_hip_matmul_q8_0_dev(_vp(y), _vp(wg), wg.numel(), _vp(xg), None, n, m,
                                           batch, None)
    assert st == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = x.astype(np.float64) @ wd.T
    assert np.all(np.isfinite(got))
    for t in range(batch):
        if t != 3:
            assert orc.rel_l2(got[t], ref[t]) <= GEMM_TOL, t
