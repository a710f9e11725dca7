"""Committed golden vectors (tests/golden/q4_0_fixtures.npz, written by
tests/golden/make_fixtures.py from the CPU restatement).

CPU: the restatement still reproduces every vector bit for bit, and the
vectors satisfy the path's invariants.  GPU (marked): libhypno_hip reproduces
the codec vectors bit for bit and the GEMV vectors within the north-star bound
(max|y - r| / max|r| <= 1e-4), through both the host-slice and the
device-pointer entry points.
"""
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "q4_0_fixtures.npz")
GEMV_CASES = [("g64x256", 64, 256), ("g37x100", 37, 100), ("g33x512", 33, 512),
              ("g5x3072", 5, 3072)]
GEMV_TOL = 1e-4


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# --- CPU: the fixtures and the oracle agree ------------------------------------------

def test_fixture_codec_reproduced(orc, fx):
    assert np.array_equal(orc.quantize_q4_0(fx["quant_in"]), fx["quant_out"])
    got = orc.dequantize_q4_0(fx["quant_out"])
    assert np.array_equal(got.view(np.uint32), fx["dequant_out"].view(np.uint32))


def test_fixture_codec_invariants(fx):
    q = fx["quant_out"].reshape(-1, 18)
    # all-zero block (quant.rs:52-56): d = 1.0 (0x3C00), every byte 0x88
    assert q[1, 0] == 0x00 and q[1, 1] == 0x3C and np.all(q[1, 2:] == 0x88)
    # the quantizer never emits nibble 0 (q >= -7): amax maps to +-7
    nib = np.concatenate([q[:, 2:] & 0xF, q[:, 2:] >> 4], axis=1)
    assert nib.min() >= 1
    # round trip (quant.rs:213-225): q = round(w / s) with s = amax / 7, so
    # |w - q*s| <= s/2, and |q| <= 8 adds at most 8*|d - s| for the stored d
    w = fx["quant_in"].reshape(-1, 32).astype(np.float64)
    dq = fx["dequant_out"].reshape(-1, 32)
    d = (q[:, 0].astype(np.uint16) | (q[:, 1].astype(np.uint16) << 8)).view(np.float16)
    d = d.astype(np.float64)
    s = (np.abs(fx["quant_in"].reshape(-1, 32)).max(axis=1) / np.float32(7)).astype(np.float64)
    err = np.abs(w - dq).max(axis=1)
    live = s > 0
    bound = 0.5 * s + 8.0 * np.abs(d - s) + 1e-12 * s
    assert np.all(err[live] <= bound[live])


@pytest.mark.parametrize("name,n,m", GEMV_CASES)
def test_fixture_gemv_reproduced(orc, fx, name, n, m):
    w, x, b = fx[f"{name}_w"], fx[f"{name}_x"], fx[f"{name}_bias"]
    assert np.array_equal(orc.matmul_q4_0_scalar(w, x, None, n, m), fx[f"{name}_y"])
    assert np.array_equal(orc.matmul_q4_0_scalar(w, x, b, n, m), fx[f"{name}_ybias"])
    assert np.array_equal(orc.matmul_q4_0_f64(w, x, None, n, m), fx[f"{name}_y64"])
    assert orc.normwise_err(fx[f"{name}_y"], fx[f"{name}_y64"]) <= 1e-5


def test_fixture_f16_and_batch_reproduced(orc, fx):
    assert np.array_equal(orc.matmul_f16_scalar(fx["f16_w"], fx["f16_x"], None, 17, 100),
                          fx["f16_y"])
    assert orc.normwise_err(fx["f16_y"], fx["f16_y64"]) <= 1e-5
    got = orc.batch_matmul(fx["batch_w"], 3, fx["batch_x"], 64, 256, 3)
    assert orc.normwise_err(got.reshape(3, 64), fx["batch_y"]) <= 1e-6


# --- GPU: libhypno_hip against the fixtures ---------------------------------------------

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


@pytest.mark.gpu
def test_gpu_fixture_codec(torch, hk, fx):
    q = hk.quantize_f32_to_q4_0(torch.from_numpy(fx["quant_in"]).cuda()).cpu().numpy()
    assert np.array_equal(q, fx["quant_out"])
    dq = hk.dequantize_q4_0(torch.from_numpy(fx["quant_out"]).cuda()).cpu().numpy()
    assert np.array_equal(dq.view(np.uint32), fx["dequant_out"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name,n,m", GEMV_CASES)
def test_gpu_fixture_gemv(torch, hk, orc, fx, name, n, m):
    w, x, b = fx[f"{name}_w"], fx[f"{name}_x"], fx[f"{name}_bias"]
    # host-slice entry point (hypno_hip_matmul_q4_0)
    y = np.empty(n, np.float32)
    hk.matmul_q4_0(y, w, x, None, n, m)
    assert orc.normwise_err(y, fx[f"{name}_y"]) <= GEMV_TOL
    assert orc.normwise_err(y, fx[f"{name}_y64"]) <= GEMV_TOL
    yb = np.empty(n, np.float32)
    hk.matmul_q4_0(yb, w, x, b, n, m)
    assert orc.normwise_err(yb, fx[f"{name}_ybias"]) <= GEMV_TOL
    # device-pointer entry point (hypno_hip_matmul_q4_0_dev)
    yd = torch.empty(n, dtype=torch.float32, device="cuda")
    hk.matmul_q4_0(yd, torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda(), None, n, m)
    torch.cuda.synchronize()
    assert orc.normwise_err(yd.cpu().numpy(), fx[f"{name}_y"]) <= GEMV_TOL


@pytest.mark.gpu
def test_gpu_fixture_f16_and_batch(torch, hk, orc, fx):
    y = np.empty(17, np.float32)
    hk.matmul_f16(y, fx["f16_w"], fx["f16_x"], None, 17, 100)
    assert orc.normwise_err(y, fx["f16_y"]) <= GEMV_TOL
    yb = np.empty(3 * 64, np.float32)
    hk.batch_matmul(yb, fx["batch_w"], hk.DType.Q4_0, fx["batch_x"].reshape(-1), 64, 256, 3)
    for t in range(3):
        assert orc.normwise_err(yb.reshape(3, 64)[t], fx["batch_y"][t]) <= GEMV_TOL
