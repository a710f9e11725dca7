"""Concurrent callers on one stream (the reference calls matmul_q4_0 from
rayon workers, turbo.rs:325-331): two host threads issue device calls on
one stream with batch sizes that alternately grow the stream's workspace
(few-token kernel, prefill GEMM, FP16 GEMM), and every output must equal,
bit for bit, what the same call gives when run alone."""
import ctypes
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_two_threads_one_stream(orc):
    import torch

    from hypno_amd import _lib
    assert torch.cuda.is_available()
    lib = _lib.load()
    n, m = 768, 2048
    gen = torch.Generator(device="cuda").manual_seed(5)
    w = torch.randn(n * m, generator=gen, device="cuda").mul_(0.02)
    import hypno_amd as hk
    q = hk.quantize_f32_to_q4_0(w)
    w16 = w.half().view(torch.uint8)
    del w
    batches = [[20, 300, 8, 600, 40, 1000], [600, 16, 1000, 64, 300, 4]]
    xs = {b: torch.randn(b, m, generator=gen, device="cuda") for bs in batches for b in bs}
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def call(kind, b, y, stream=None):
        if kind == "q4":
            return lib.hypno_hip_matmul_q4_0_dev(vp(y), vp(q), q.numel(), vp(xs[b]), None, n, m, b,
                                                 stream)
        return lib.hypno_hip_matmul_f16_dev(vp(y), vp(w16), w16.numel(), vp(xs[b]), None, n, m, b,
                                            stream)

    jobs = [[(kind, b) for b in bs for kind in ("q4", "f16")] for bs in batches]
    # alone, one call at a time
    alone = {}
    for js in jobs:
        for kind, b in js:
            y = torch.empty(b, n, device="cuda")
            assert call(kind, b, y) == 0
            torch.cuda.synchronize()
            alone[(kind, b)] = y.cpu().numpy()
    # a stream the library has not seen: its workspace starts empty and the
    # concurrent calls grow it while the other thread has work queued on it
    side = torch.cuda.Stream()
    sp = ctypes.c_void_p(side.cuda_stream)
    torch.cuda.synchronize()
    outs = [{} for _ in jobs]
    errors = []

    def worker(i):
        try:
            for rep in range(3):
                for kind, b in jobs[i]:
                    y = torch.full((b, n), float("nan"), device="cuda")
                    torch.cuda.synchronize()
                    st = call(kind, b, y, sp)
                    if st:
                        errors.append((i, kind, b, st))
                        return
                    outs[i][(kind, b, rep)] = y
        except Exception as e:  # pragma: no cover - reported below
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i, o in enumerate(outs):
        for (kind, b, rep), y in o.items():
            assert np.array_equal(y.cpu().numpy(), alone[(kind, b)]), (i, kind, b, rep)
    # and the single-call results are right
    qh = q.cpu().numpy()
    for (kind, b), got in alone.items():
        if kind == "q4" and b in (8, 300):
            xh = xs[b].cpu().numpy()
            ref = orc.batch_matmul(qh, 3, xh, n, m, b)
            if b < 16:
                assert max(orc.normwise_err(got[t], ref[t]) for t in range(b)) <= 1e-4
            else:
                assert orc.rel_l2(got, ref) <= 2e-3
