"""Seeded sweep over the batched device entry points (turbo.rs:306-341:
the Q4_0, FP16 and Q8_0 arms of batch_matmul) at random shapes, so that the
dispatch between the one-row GEMV, the few-row GEMV, the few-token MFMA
kernels, the FP16 streaming GEMM and the prefill GEMMs is crossed at many
(tokens, N, K) points, including K that is not a multiple of 32 (blocks
straddling rows), 0 or 1 output rows per tile and biases.  Each case is
checked against the oracle's per-token GEMVs on every output: below 16
tokens to the GEMV bar (normwise 1e-4 per token), from 16 to the prefill
GEMM's (rel-L2 2e-3); outputs start as NaN, so a row never written fails."""
import ctypes

import numpy as np
import pytest

GEMV_TOL, GEMM_TOL = 1e-4, 2e-3
MAX_MACS = 150_000_000  # keeps the oracle side of a case well under a second


def _cases():
    rng = np.random.default_rng(20261202)
    batches = [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 15, 16, 17, 24, 31, 32, 33, 48, 63, 64, 65,
               96, 127, 128, 129, 200, 256]
    ks = [32, 64, 96, 160, 256, 512, 768, 1024, 1280, 2048, 3072, 4096, 5632]
    out = []
    while len(out) < 120:
        i = len(out)
        dt = ("q4_0", "q8_0", "f16")[i % 3]
        batch = int(rng.choice(batches))
        m = int(rng.choice(ks))
        if rng.random() < 0.15:
            m += int(rng.integers(1, 31))  # K % 32 != 0
        n = int(rng.choice([int(rng.integers(1, 200)), int(rng.integers(200, 4200))]))
        if n * m * batch > MAX_MACS:
            continue
        out.append((dt, batch, n, m, bool(rng.integers(0, 2)), 1000 + i))
    return out


CASES = _cases()


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


@pytest.fixture(scope="module")
def lib():
    from hypno_amd import _lib
    return _lib.load()


def _weights(orc, dt, n, m, seed):
    w = orc.normal_f32(seed, n * m, 0.02)
    if dt == "f16":
        return w.astype(np.float16).view(np.uint8)
    pad = (-n * m) % 32
    if pad:
        w = np.concatenate([w, np.zeros(pad, np.float32)])
    return orc.quantize_q4_0(w) if dt == "q4_0" else orc.quantize_q8_0(w)


def _reference(orc, dt, wb, x, bias, n, m, batch):
    if dt == "q4_0":
        ref = orc.batch_matmul(wb, 3, x, n, m, batch)
    elif dt == "f16":
        ref = orc.batch_matmul(wb, 1, x, n, m, batch)
    else:
        ref = np.stack([orc.matmul_q8_0(wb, x[t], None, n, m) for t in range(batch)])
    return ref + bias if bias is not None else ref


@pytest.mark.gpu
@pytest.mark.parametrize("dt,batch,n,m,with_bias,seed", CASES)
def test_batch_dispatch_sweep(torch, lib, orc, dt, batch, n, m, with_bias, seed):
    print(f"sweep {dt} batch={batch} n={n} m={m} bias={with_bias}", flush=True)
    wb = _weights(orc, dt, n, m, seed)
    x = orc.normal_f32(seed + 1, (batch, m))
    bias = orc.normal_f32(seed + 2, n) if with_bias else None
    g = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    dw, dx = g(wb), g(x)
    db = g(bias) if bias is not None else None
    y = torch.full((batch * n,), float("nan"), dtype=torch.float32, device="cuda")
    fn = {"q4_0": lib.hypno_hip_matmul_q4_0_dev, "q8_0": lib.hypno_hip_matmul_q8_0_dev,
          "f16": lib.hypno_hip_matmul_f16_dev}[dt]
    st = fn(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(dw.data_ptr()), wb.size,
            ctypes.c_void_p(dx.data_ptr()),
            None if db is None else ctypes.c_void_p(db.data_ptr()), n, m, batch, None)
    assert st == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(batch, n)
    ref = _reference(orc, dt, wb, x, bias, n, m, batch)
    assert not np.isnan(got).any()
    if batch < 16:
        for t in range(batch):
            assert orc.normwise_err(got[t], ref[t]) <= GEMV_TOL, t
    else:
        assert orc.rel_l2(got, ref) <= GEMM_TOL
