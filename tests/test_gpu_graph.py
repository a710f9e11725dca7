"""Captured HIP graphs over the newer device paths: the column-major GEMV
(k-range planes plus the reduction launch, both on the stream's workspace),
the Q8_0 few-row GEMV (one and two launches), the FP16 streaming GEMM (hi/lo
rows at 8 tokens, fp16 rows at 40) and the one-token Q4_0 and FP16 GEMVs.
Each call runs eagerly three times (bit-identical, and within its bar of the
oracle), then all of them are captured in one graph on a side stream —
consecutive calls reuse one workspace — and the graph is replayed three
times with the same calls run eagerly in between; every replay must give
the first eager result bit for bit (no kernel here clears memory with a
memset node, and every kernel's order of additions is fixed)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMV_TOL, GEMM_TOL = 1e-4, 2e-3


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


@pytest.fixture(scope="module")
def lib():
    from hypno_amd import _lib
    return _lib.load()


def _cases(orc):
    """(label, entry point, weight bytes, x, n, m, batch, reference)."""
    out = []
    n, m = 4096, 4096                      # column-major: W_col[m][n]
    wcol = orc.quantize_q4_0(orc.normal_f32(1, n * m, 0.02))
    x = orc.normal_f32(2, (1, m))
    out.append(("col", "hypno_hip_matmul_q4_0_col_dev", wcol, x, n, m, 1,
                orc.matmul_q4_0_col(wcol, x[0], None, n, m)[None]))
    for batch, nn, mm in ((5, 2000, 4096), (13, 1000, 2048)):
        wq = orc.quantize_q8_0(orc.normal_f32(3 + batch, nn * mm, 0.02))
        xb = orc.normal_f32(4 + batch, (batch, mm))
        ref = np.stack([orc.matmul_q8_0(wq, xb[t], None, nn, mm) for t in range(batch)])
        out.append((f"q8_0 x{batch}", "hypno_hip_matmul_q8_0_dev", wq, xb, nn, mm, batch, ref))
    for batch, nn, mm in ((8, 3000, 1024), (40, 1500, 2048), (1, 4096, 4096)):
        w16 = orc.normal_f32(5 + batch, nn * mm, 0.02).astype(np.float16).view(np.uint8)
        xb = orc.normal_f32(6 + batch, (batch, mm))
        out.append((f"f16 x{batch}", "hypno_hip_matmul_f16_dev", w16, xb, nn, mm, batch,
                    orc.batch_matmul(w16, 1, xb, nn, mm, batch)))
    nn, mm = 4096, 4096
    wq4 = orc.quantize_q4_0(orc.normal_f32(7, nn * mm, 0.02))
    xb = orc.normal_f32(8, (1, mm))
    out.append(("q4_0 x1", "hypno_hip_matmul_q4_0_dev", wq4, xb, nn, mm, 1,
                orc.batch_matmul(wq4, 3, xb, nn, mm, 1)))
    return out


def test_graph_replays_match_eager(torch, lib, orc):
    side = torch.cuda.Stream()
    g = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    cases = []
    for label, fn, wb, x, n, m, batch, ref in _cases(orc):
        cases.append((label, getattr(lib, fn), g(wb), wb.size, g(x), n, m, batch, ref))

    def run(case, y, stream):
        label, fn, dw, wlen, dx, n, m, batch, _ = case
        st = fn(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(dw.data_ptr()), wlen,
                ctypes.c_void_p(dx.data_ptr()), None, n, m, batch,
                ctypes.c_void_p(stream.cuda_stream))
        assert st == 0, label

    side.wait_stream(torch.cuda.current_stream())
    first = []
    for case in cases:
        label, _, _, _, _, n, m, batch, ref = case
        print(f"[case] eager {label} n={n} m={m} batch={batch}", flush=True)
        outs = []
        for _ in range(3):
            y = torch.full((batch * n,), float("nan"), device="cuda")
            with torch.cuda.stream(side):
                run(case, y, side)
            outs.append(y)
        torch.cuda.synchronize()
        got = [o.cpu().numpy().reshape(batch, n) for o in outs]
        assert np.array_equal(got[0], got[1]) and np.array_equal(got[0], got[2]), label
        if batch < 16:
            for t in range(batch):
                assert orc.normwise_err(got[0][t], ref[t]) <= GEMV_TOL, (label, t)
        else:
            assert orc.rel_l2(got[0], ref) <= GEMM_TOL, label
        first.append(got[0])
    ys = [torch.full((c[7] * c[5],), float("nan"), device="cuda") for c in cases]
    graph = torch.cuda.CUDAGraph()
    print("[case] capture", flush=True)
    with torch.cuda.graph(graph, stream=side):
        for case, y in zip(cases, ys):
            run(case, y, side)
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"[case] replay {rep}", flush=True)
        for y in ys:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for case, y, want in zip(cases, ys, first):
            label, _, _, _, _, n, _, batch, _ = case
            assert np.array_equal(y.cpu().numpy().reshape(batch, n), want), (rep, label)
        # the same calls eagerly between the replays (same workspace)
        for case in cases:
            yt = torch.full((case[7] * case[5],), float("nan"), device="cuda")
            with torch.cuda.stream(side):
                run(case, yt, side)
        torch.cuda.synchronize()
