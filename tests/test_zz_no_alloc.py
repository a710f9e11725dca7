"""hypno_hip_matmul_q4_0_dev_noalloc (the entry point for callers that cannot
allocate device memory) against hypno_hip_matmul_q4_0_dev: the same kernels on the same
inputs, so outputs must be equal bit for bit, on two calls in a row (the
second smaller, so stale scratch contents from the first would show), for
each kernel family that uses scratch memory; plus the size limit."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_SCRATCH = 64 << 20  # HYPNO_HIP_NOALLOC_SCRATCH_BYTES


@pytest.fixture(scope="module")
def env(orc):
    import torch

    import hypno_amd as hk
    from hypno_amd import _lib
    assert torch.cuda.is_available()
    return torch, hk, _lib.load()


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


def _case(torch, hk, n, m, batch, seed, bias=True):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(n * m, generator=gen, device="cuda").mul_(0.02)
    q = hk.quantize_f32_to_q4_0(w)
    x = torch.randn(batch, m, generator=gen, device="cuda")
    b = torch.randn(n, generator=gen, device="cuda") if bias else None
    return q, x, b


def _call(lib, fn, q, x, b, n, m, batch):
    import torch
    y = torch.full((batch, n), float("nan"), device="cuda")
    st = getattr(lib, fn)(_vp(y), _vp(q), q.numel(), _vp(x), None if b is None else _vp(b),
                          n, m, batch, None)
    torch.cuda.synchronize()
    return st, y


# (first call, second smaller call): few-token hi/lo rows, few-token plain rows
# with split K, prefill GEMM (folded scale, split K), prefill GEMM (fp32 block
# scale), the GEMM for m % 256 != 0, and M = 1 (no scratch)
PAIRS = [
    ((16, 4096, 4096), (5, 1000, 1024)),
    ((64, 4096, 14336), (40, 1000, 4096)),
    ((512, 3072, 8192), (300, 512, 2048)),
    ((200, 8192, 4096), (100, 4097, 512)),
    ((130, 1000, 320), (70, 300, 192)),
    ((1, 14336, 4096), (1, 300, 2048)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_dev(env, orc, first, second):
    torch, hk, lib = env
    for i, (batch, n, m) in enumerate((first, second)):
        print(f"[case] noalloc batch={batch} n={n} m={m}", flush=True)
        q, x, b = _case(torch, hk, n, m, batch, seed=batch + n + m)
        st0, y0 = _call(lib, "hypno_hip_matmul_q4_0_dev", q, x, b, n, m, batch)
        st1, y1 = _call(lib, "hypno_hip_matmul_q4_0_dev_noalloc", q, x, b, n, m, batch)
        assert st0 == 0 and st1 == 0, lib.hypno_hip_last_error()
        a0, a1 = y0.cpu().numpy(), y1.cpu().numpy()
        assert not np.isnan(a1).any()
        assert np.array_equal(a0, a1), (batch, n, m)
        if i == 1 and batch > 1:   # and right: the oracle's per-token GEMVs
            ref = orc.batch_matmul(q.cpu().numpy(), 3, x.cpu().numpy(), n, m, batch)
            ref = ref + b.cpu().numpy()
            if batch <= 16:
                assert max(orc.normwise_err(a1[t], ref[t]) for t in range(batch)) <= 1e-4
            else:
                assert orc.rel_l2(a1, ref) <= 2e-3


def test_noalloc_rejects_oversized_calls(env):
    torch, hk, lib = env
    n, m, batch = 256, 16384, 2048          # fp16 activations alone: 64 MiB
    assert batch * m * 2 >= MAX_SCRATCH
    q = torch.zeros(n * m // 32 * 18, dtype=torch.uint8, device="cuda")
    x = torch.zeros(batch, m, device="cuda")
    y = torch.full((batch, n), float("nan"), device="cuda")
    st = lib.hypno_hip_matmul_q4_0_dev_noalloc(_vp(y), _vp(q), q.numel(), _vp(x), None, n, m,
                                               batch, None)
    assert st == 22
    assert b"scratch" in lib.hypno_hip_last_error()
    torch.cuda.synchronize()
    assert bool(torch.isnan(y).all())   # nothing was launched


def test_noalloc_allocates_nothing(env):
    """The contract itself: on a stream the library has not seen (whose
    workspace the allocating entry point would have to create), noalloc
    calls of the few-token and the prefill families leave the device's free
    memory unchanged; the allocating entry point on another fresh stream is
    the control that shows such an allocation would be seen."""
    torch, hk, lib = env
    cases = [(64, 4096, 14336), (512, 3072, 8192)]
    inputs = []
    for batch, n, m in cases:
        q, x, b = _case(torch, hk, n, m, batch, seed=batch + 7)
        y = torch.empty(batch, n, device="cuda")
        inputs.append((q, x, b, y, n, m, batch))

    def run(fn, stream):
        for q, x, b, y, n, m, batch in inputs:
            st = getattr(lib, fn)(_vp(y), _vp(q), q.numel(), _vp(x), _vp(b), n, m, batch,
                                  ctypes.c_void_p(stream.cuda_stream))
            assert st == 0, lib.hypno_hip_last_error()
        torch.cuda.synchronize()

    run("hypno_hip_matmul_q4_0_dev_noalloc", torch.cuda.current_stream())  # library set up
    fresh, control = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (fresh, control):   # the streams' own first use, outside the window
        with torch.cuda.stream(s):
            inputs[0][3].zero_()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    run("hypno_hip_matmul_q4_0_dev_noalloc", fresh)
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"noalloc calls took {free0 - free1} bytes"
    run("hypno_hip_matmul_q4_0_dev", control)
    free2 = torch.cuda.mem_get_info()[0]
    assert free2 < free1, "the control's workspace allocation was not seen"
