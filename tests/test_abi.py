"""CPU checks of the C ABI: the library loads, exports every function that
include/hypno_hip.h declares, and rejects bad arguments before touching a
device.  No compute call is made here (there is no GPU in this container)."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hypno_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hypno_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from hypno_amd import _lib
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    names = _declared()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), f"{name} declared in hypno_hip.h but not exported"
    from hypno_amd import _lib
    assert sorted(_lib.SIGNATURES) == names


def test_abi_basics(lib):
    assert lib.hypno_hip_abi_version() == 1
    assert lib.hypno_hip_strerror(0) == b"ok"
    assert lib.hypno_hip_strerror(22) == b"invalid argument"
    assert lib.hypno_hip_device_count() >= 0


def test_host_validation_without_device(lib):
    y = np.zeros(4, np.float32)
    x = np.zeros(32, np.float32)
    w = np.zeros(18 * 4, np.uint8)
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    # FP32 is outside this path (ops.rs:30)
    assert lib.hypno_hip_matmul_vec_auto(vp(y), vp(w), w.size, 0, vp(x), None, 4, 32) == 95
    # Q8_0: 72 bytes hold 2 blocks = 64 elements < n*m = 128 (a panic in ops.rs:34-35)
    assert lib.hypno_hip_matmul_vec_auto(vp(y), vp(w), w.size, 2, vp(x), None, 4, 32) == 22
    assert lib.hypno_hip_matmul_q8_0(vp(y), vp(w), w.size, vp(x), None, 4, 32) == 22
    assert lib.hypno_hip_matmul_vec_auto(vp(y), vp(w), w.size, 7, vp(x), None, 4, 32) == 22
    assert b"dtype" in lib.hypno_hip_last_error()
    # NULL y / x
    assert lib.hypno_hip_matmul_q4_0(None, vp(w), w.size, vp(x), None, 4, 32) == 22
    assert lib.hypno_hip_matmul_q4_0(vp(y), vp(w), w.size, None, None, 4, 32) == 22
    # short fp16 buffer (a panic in kernels.rs:550)
    assert lib.hypno_hip_matmul_f16(vp(y), vp(w), 10, vp(x), None, 4, 32) == 22
    # empty problems succeed without a device
    assert lib.hypno_hip_matmul_q4_0(vp(y), vp(w), w.size, vp(x), None, 0, 32) == 0
    assert lib.hypno_hip_batch_matmul(vp(y), vp(w), w.size, 3, vp(x), 4, 32, 0) == 0


def test_python_mirror_validation():
    import hypno_amd as hk
    w = np.zeros(18 * 4, np.uint8)
    x = np.zeros(32, np.float32)
    with pytest.raises(ValueError):
        hk.matmul_q4_0(np.zeros(5, np.float32), w, x, None, 4, 32)   # y length != n
    with pytest.raises(ValueError):
        hk.matmul_q4_0(np.zeros(4, np.float32), w, x[:31], None, 4, 32)
    with pytest.raises(ValueError):
        hk.matmul_q4_0(np.zeros(4, np.float64), w, x, None, 4, 32)
    with pytest.raises(hk.HypnoHipError) as e:   # FP32 weights are not on this path
        hk.batch_matmul(np.zeros(8, np.float32), w, hk.DType.FP32, np.zeros(64, np.float32),
                        4, 32, 2, col_major=True)
    assert e.value.status == 95
    assert hk.DType.Q4_0.data_bytes(32) == 18 and hk.DType.Q4_0.data_bytes(33) == 36
    assert hk.DType.FP16.data_bytes(10) == 20 and int(hk.DType.Q4_0) == 3


def test_product_never_imports_oracle():
    # the oracle is test infrastructure; the package must not reference it
    pkg = os.path.join(ROOT, "hypno_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower(), f"{f} mentions the oracle"


def test_overlap_rejected_without_device(lib):
    """y may not share memory with an input (the reference's &mut y beside
    shared borrows); the check runs before any device call, so fake device
    addresses suffice here."""
    base = 1 << 40
    P = ctypes.c_void_p
    # y = x (batch 1): EINVAL
    assert lib.hypno_hip_matmul_q4_0_dev(P(base), P(base + 4096), 18 * 8, P(base), None, 4, 64, 1,
                                         None) == 22
    assert b"overlap" in lib.hypno_hip_last_error()
    # y straddles the end of w
    assert lib.hypno_hip_matmul_f16_dev(P(base + 1000), P(base), 1024, P(base + 8192), None, 4,
                                        128, 1, None) == 22
    # bias inside y
    assert lib.hypno_hip_matmul_q8_0_dev(P(base), P(base + 4096), 34 * 8, P(base + 8192),
                                         P(base + 4), 4, 64, 1, None) == 22
    assert lib.hypno_hip_matmul_q4_0_col_dev(P(base), P(base + 4096), 18 * 8, P(base + 8),
                                             None, 4, 64, 1, None) == 22


def test_plan_overlap_rejected_without_device(lib):
    from hypno_amd._lib import GemvDesc, GemvPrologue
    base = 1 << 40
    plan = ctypes.c_void_p()

    def descs(*ds):
        arr = (GemvDesc * len(ds))()
        for i, (y, w, x, n, m) in enumerate(ds):
            arr[i].y, arr[i].w_q, arr[i].w_len = base + y, base + w, n * m // 32 * 18
            arr[i].x, arr[i].bias, arr[i].n, arr[i].m = base + x, None, n, m
        return arr

    # two jobs writing overlapping y
    d = descs((0, 1 << 20, 2 << 20, 256, 256), (512, 3 << 20, 2 << 20, 256, 256))
    assert lib.hypno_hip_q4_0_gemv_plan_create(d, 2, ctypes.byref(plan)) == 22
    assert b"overlap" in lib.hypno_hip_last_error()
    # job 1 reads job 0's output as its x
    d = descs((0, 1 << 20, 2 << 20, 256, 256), (4096, 3 << 20, 0, 256, 256))
    assert lib.hypno_hip_q4_0_gemv_plan_create(d, 2, ctypes.byref(plan)) == 22
    # a prologue operand inside another job's y
    d = descs((0, 1 << 20, 2 << 20, 256, 256), (4096, 3 << 20, 2 << 20, 256, 256))
    pros = (GemvPrologue * 2)()
    pros[1].kind, pros[1].aux, pros[1].eps = 1, base + 64, 1e-5
    assert lib.hypno_hip_q4_0_gemv_plan_create_ex(d, pros, 2, ctypes.byref(plan)) == 22
    assert not plan.value
