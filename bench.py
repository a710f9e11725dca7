#!/usr/bin/env python3
"""Q4_0 matmul benchmark on one MI355X.

Headline workload: the full TinyLlama-1.1B decode
step weight stream, M = 1, Q4_0, 22 layers x {q, k, v, o, gate, up, down}
(544,997,376 weight bytes, larger than the 256 MB Infinity Cache, so every
step streams from HBM).  One step = the 154 GEMVs as one multi-GEMV plan
launch; steps are launched back to back on one stream and timed with HIP
events on that stream.  value = weight bytes / step time (GB/s).

Also reported, in the same JSON line:
  roofline      the decode GEMV kernel's weight bytes per launch / its average
                launch duration over the timed region, against the 8 TB/s HBM
                peak; traffic = measured HBM bytes per launch (rocprofv3 --pmc,
                read from the committed profile summary);
  cpu_baseline  the CPU restatement of hypno's AVX2 kernel (oracle/) on this
                host, on a bounded sample (layer 0's seven matrices);
  secondary     every other BASELINE config, GPU-timed (graph replay):
                configs[0] the single 2048x2048 GEMV, configs[2] the prefill
                GEMM at Llama-3.2-3B MLP shapes (M = 512), configs[3] the
                Mistral-7B decode stream (224 GEMVs, one plan launch) and the
                M-sweep {1, 8, 64, 512, 2048}, configs[4] the lm_head in Q4_0
                and FP16 at M = 1 and 128; model_load: a TinyLlama-shaped
                .hypno file opened with its payloads uploaded to HBM
                (pipelined pinned upload, against a pageable copy and the
                reference's host-only open); q8_0_decode and col_major: the
                Q8_0 and column-major Q4_0 GEMVs at the Mistral shapes.

Inputs are synthetic: weights N(0, 0.02) from a seeded torch generator,
quantised on the GPU by the bit-exact Q4_0 quantizer; activations N(0, 1).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "Q4_0 GEMV weight GB/s (% HBM peak); prefill GEMM TFLOPS at 7B shapes"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0

# TinyLlama-1.1B per-layer projections (n = output rows, m = input dim)
TINYLLAMA = [("q", 2048, 2048), ("k", 256, 2048), ("v", 256, 2048), ("o", 2048, 2048),
             ("gate", 5632, 2048), ("up", 5632, 2048), ("down", 2048, 5632)]
LAYERS = 22
ALIGN = 64  # .hypno tensor alignment (format.rs:10)


def q4_bytes(n, m):
    return n * m // 32 * 18


class Lib:
    def __init__(self):
        from hypno_amd import _lib
        self.lib = _lib.load()
        self.check = _lib.check

    def quantize(self, out_ptr, src, stream):
        self.check(self.lib.hypno_hip_quantize_q4_0_dev(ctypes.c_void_p(out_ptr),
                                                        ctypes.c_void_p(src.data_ptr()),
                                                        src.numel(), stream), "quantize")

    def q4(self, y, w, w_len, x, n, m, batch, stream):
        return self.lib.hypno_hip_matmul_q4_0_dev(y, w, w_len, x, None, n, m, batch, stream)


def make_q4_arena(torch, lib, shapes, seed, stream):
    """Quantised weights for `shapes` packed at 64-byte aligned offsets in one
    device buffer (the .hypno layout).  Returns (arena, [(offset, nbytes)])."""
    offs, total = [], 0
    for n, m in shapes:
        total = (total + ALIGN - 1) // ALIGN * ALIGN
        offs.append((total, q4_bytes(n, m)))
        total += q4_bytes(n, m)
    arena = torch.empty(total, dtype=torch.uint8, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(seed)
    for (n, m), (off, _) in zip(shapes, offs):
        w = torch.randn(n * m, generator=gen, device="cuda", dtype=torch.float32).mul_(0.02)
        lib.quantize(arena.data_ptr() + off, w, stream)
        del w
    torch.cuda.synchronize()
    return arena, offs


def time_graph(torch, fn, steps, warmup):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, g


def time_launches(torch, fn, steps, warmup):
    """Average ms per call of `fn` over `steps` back-to-back calls on the
    current stream, bracketed by HIP events on that stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def decode_stream(torch, lib, steps, warmup, value_only=False):
    """22 layers x 7 Q4_0 GEMVs.  Each matrix has its own output
    buffer; each layer has its own activation vectors (x for q/k/v/gate/up
    and for o share m = 2048, down has m = 5632)."""
    import hypno_amd as hk
    stream0 = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    shapes = [(n, m) for _ in range(LAYERS) for (_, n, m) in TINYLLAMA]
    arena, offs = make_q4_arena(torch, lib, shapes, seed=1234, stream=stream0)
    gen = torch.Generator(device="cuda").manual_seed(99)
    xs = [{"attn": torch.randn(2048, generator=gen, device="cuda"),
           "o": torch.randn(2048, generator=gen, device="cuda"),
           "mlp": torch.randn(2048, generator=gen, device="cuda"),
           "down": torch.randn(5632, generator=gen, device="cuda")} for _ in range(LAYERS)]
    x_of = {"q": "attn", "k": "attn", "v": "attn", "o": "o", "gate": "mlp", "up": "mlp",
            "down": "down"}
    ys = [torch.empty(n, device="cuda") for n, _ in shapes]
    jobs = []  # (layer, name, y, w view, x, n, m)
    for i, ((n, m), (off, nb)) in enumerate(zip(shapes, offs)):
        layer, (name, _, _) = divmod(i, len(TINYLLAMA))[0], TINYLLAMA[i % len(TINYLLAMA)]
        jobs.append((layer, name, ys[i], arena[off:off + nb], xs[layer][x_of[name]], n, m))
    weight_bytes = sum(nb for _, nb in offs)

    # (a) the whole weight stream as one plan: one launch per step (the value),
    # launched back to back on the current stream
    plan_all = hk.GemvPlan([(y, w, x, None, n, m) for _, _, y, w, x, n, m in jobs])
    ms_all = time_launches(torch, plan_all.run, steps, warmup)
    res = {"ms": ms_all, "weight_bytes": weight_bytes, "launches": plan_all.launches}
    host_sample = [w.cpu().numpy() for _, _, _, w, _, _, _ in jobs[:len(TINYLLAMA)]]
    res["sample"] = host_sample
    res["x_host"] = {m: jobs[0][4].cpu().numpy() if m == 2048 else jobs[6][4].cpu().numpy()
                     for m in (2048, 5632)}
    if value_only:
        return res
    # (b) dependency-respecting decode step: per layer [q,k,v] [o] [gate,up] [down]
    groups = []
    for layer in range(LAYERS):
        lj = [j for j in jobs if j[0] == layer]
        for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
            groups.append(hk.GemvPlan([(y, w, x, None, n, m)
                                       for _, nm, y, w, x, n, m in lj if nm in names]))

    def run_groups():
        for p in groups:
            p.run()

    ms_grp, g_grp = time_graph(torch, run_groups, steps, warmup)
    # (c) the drop-in path: one matmul_q4_0 call per matrix (154 launches)
    calls = [(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(w.data_ptr()), w.numel(),
              ctypes.c_void_p(x.data_ptr()), n, m) for _, _, y, w, x, n, m in jobs]

    def per_call():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for y, w, nb, x, n, m in calls:
            rc = lib.q4(y, w, nb, x, n, m, 1, st)
            if rc:
                lib.check(rc, "decode GEMV")

    ms_call, g_call = time_graph(torch, per_call, steps, warmup)
    del g_grp, g_call
    res.update({"ms_grouped": ms_grp, "launches_grouped": sum(p.launches for p in groups),
                "ms_per_call": ms_call, "launches_per_call": len(calls)})
    # (d) the same groups with the steps either side of the GEMVs: RMS norm
    # before [q,k,v] and [gate,up], silu(gate)*up before [down] — fused into
    # the GEMVs' staging, against the same work as separate kernels
    eps = 1e-5
    norms = [(1.0 + 0.1 * torch.randn(2048, generator=gen, device="cuda"),
              1.0 + 0.1 * torch.randn(2048, generator=gen, device="cuda")) for _ in range(LAYERS)]
    ups = [torch.randn(5632, generator=gen, device="cuda") for _ in range(LAYERS)]
    fused = []
    for layer in range(LAYERS):
        lj = {nm: (y, w, x, n, m) for lyr, nm, y, w, x, n, m in jobs if lyr == layer}
        n1, n2 = norms[layer]

        def j(nm, pro):
            y, w, x, n, m = lj[nm]
            return (y, w, x, None, n, m, pro)
        fused += [hk.GemvPlan([j(nm, ("rms_norm", n1, eps)) for nm in ("q", "k", "v")]),
                  hk.GemvPlan([j("o", None)]),
                  hk.GemvPlan([j(nm, ("rms_norm", n2, eps)) for nm in ("gate", "up")]),
                  hk.GemvPlan([j("down", ("silu_mul", ups[layer]))])]

    def run_fused():
        for p in fused:
            p.run()

    ms_fused, g_f = time_graph(torch, run_fused, steps, warmup)
    # separate kernels write the GEMVs' inputs from the residual stream and
    # the gate vector, as the reference's in-place norm and silu do
    hidden = torch.randn(2048, generator=gen, device="cuda")
    gate_v = torch.randn(5632, generator=gen, device="cuda")

    def run_separate():
        for layer in range(LAYERS):
            x = xs[layer]
            hk.rms_norm(hidden, norms[layer][0], eps, out=x["attn"])
            groups[4 * layer].run()
            groups[4 * layer + 1].run()
            hk.rms_norm(hidden, norms[layer][1], eps, out=x["mlp"])
            groups[4 * layer + 2].run()
            hk.silu_mul(gate_v, ups[layer], out=x["down"])
            groups[4 * layer + 3].run()

    ms_sep, g_s = time_graph(torch, run_separate, steps, warmup)
    del g_f, g_s
    res.update({"ms_fused": ms_fused, "launches_fused": sum(p.launches for p in fused),
                "ms_separate": ms_sep,
                "launches_separate": sum(p.launches for p in groups) + 3 * LAYERS})
    return res


def time_calls_graph(torch, issue, reps, replays=3):
    """GPU time per iteration of `issue(stream_ptr)` (library calls on one
    stream): one warm-up call, then `reps` iterations captured in a HIP graph
    and replayed `replays` times between HIP events, so host-side call
    overhead does not enter the figure."""
    gs = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(gs):
        issue(ctypes.c_void_p(gs.cuda_stream), 0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=gs):
        sp = ctypes.c_void_p(gs.cuda_stream)
        for i in range(reps):
            issue(sp, i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / (replays * reps) * 1e3  # us


def rotating_q4(torch, lib, n, m, seed, min_bytes=512 * 2**20):
    """Distinct Q4_0 copies of one n x m matrix, >= min_bytes in total, so that
    successive calls stream their weights from HBM, not from the 256 MB cache."""
    nb = q4_bytes(n, m)
    copies = max(2, -(-min_bytes // nb))
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    arena, offs = make_q4_arena(torch, lib, [(n, m)] * copies, seed=seed, stream=st)
    return arena, [arena.data_ptr() + off for off, _ in offs], nb


def q4_case(torch, lib, n, m, M, seed, reps):
    """GPU us per hypno_hip_matmul_q4_0_dev call of an M x m . (n x m)^T
    product (rotating weight copies when the weights are small)."""
    arena, ptrs, nb = rotating_q4(torch, lib, n, m, seed,
                                  min_bytes=512 * 2**20 if M <= 64 else 1)
    x = torch.randn(M, m, device="cuda")
    y = torch.empty(M, n, device="cuda")
    xp, yp = ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr())

    def issue(sp, i):
        rc = lib.q4(yp, ctypes.c_void_p(ptrs[i % len(ptrs)]), nb, xp, n, m, M, sp)
        if rc:
            lib.check(rc, "matmul_q4_0")

    us = time_calls_graph(torch, issue, reps)
    del arena, x, y
    torch.cuda.empty_cache()
    return {"us": round(us, 2), "weight_gbs": round(nb / us / 1e3, 1),
            "tflops": round(2.0 * M * n * m / us / 1e6, 2),
            "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4),
            "frac_fp16_peak": round(2.0 * M * n * m / us / 1e6 / FP16_PEAK_TFLOPS, 4)}


def prefill_gemm(torch, lib):
    """M = 512 tokens, Llama-3.2-3B MLP: gate/up 8192 x 3072 and
    down 3072 x 8192, activations N(0,1) with 1% of channels x20.  Each call =
    fp16 activation pre-pass + MFMA GEMM."""
    out = {}
    for name, n, m in (("gate_up", 8192, 3072), ("down", 3072, 8192)):
        out[name] = q4_case(torch, lib, n, m, 512, seed=7 + n, reps=20)
    return {"workload": "configs[2] Llama-3.2-3B MLP, M=512, Q4_0; GPU time per call incl. "
                        "the fp16 activation pre-pass", "results": out}


MISTRAL = [("q_o", 4096, 4096), ("k_v", 1024, 4096), ("gate_up", 14336, 4096),
           ("down", 4096, 14336)]


def mistral_stream(torch, lib, steps=10, warmup=3):
    """configs[3] at M = 1 as a decode step streams it: the 224 Q4_0 GEMVs of
    Mistral-7B (32 layers x q, k, v, o, gate, up, down; 3.93 GB) as one plan
    launch, launched back to back."""
    import hypno_amd as hk
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    per_layer = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096),
                 (14336, 4096), (4096, 14336)]
    shapes = per_layer * 32
    arena, offs = make_q4_arena(torch, lib, shapes, seed=11, stream=st)
    xs = {4096: torch.randn(4096, device="cuda"), 14336: torch.randn(14336, device="cuda")}
    ys = [torch.empty(n, device="cuda") for n, _ in shapes]
    plan = hk.GemvPlan([(ys[i], arena[o:o + nb], xs[m], None, n, m)
                        for i, ((n, m), (o, nb)) in enumerate(zip(shapes, offs))])
    wb = sum(nb for _, nb in offs)
    ms = time_launches(torch, plan.run, steps, warmup)
    plan.close()
    del arena, ys
    torch.cuda.empty_cache()
    gbs = wb / (ms * 1e-3) / 1e9
    return {"workload": "configs[3] M=1: Mistral-7B decode-step weight stream, 224 Q4_0 "
                        "GEMVs as one plan launch", "weight_bytes": wb, "us": round(ms * 1e3, 1),
            "weight_gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


def mistral_m_sweep(torch, lib):
    """Mistral-7B projections at M in {1, 8, 64, 512, 2048}."""
    out = {}
    for name, n, m in MISTRAL:
        for M in (1, 8, 64, 512, 2048):
            out[f"{name}_M{M}"] = q4_case(torch, lib, n, m, M, seed=n + m + M,
                                          reps=20 if M <= 64 else 4)
    return {"workload": "configs[3] Mistral-7B q/o, k/v, gate/up, down at M in "
                        "{1,8,64,512,2048}; GPU time per call (graph replay); M <= 64 "
                        "rotates >= 512 MB of weight copies", "results": out}


def lm_head(torch, lib):
    """K = 4096, N = 128256, M in {1, 128}, Q4_0 and FP16 weights."""
    n, m = 128256, 4096
    out = {}
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    arena, offs = make_q4_arena(torch, lib, [(n, m)], seed=17, stream=st)
    gen = torch.Generator(device="cuda").manual_seed(18)
    w16 = torch.randn(n * m, generator=gen, device="cuda").mul_(0.02).half()
    for M in (1, 128):
        x = torch.randn(M, m, device="cuda")
        y = torch.empty(M, n, device="cuda")
        xp, yp = ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr())
        for dt, nb in (("q4_0", offs[0][1]), ("f16", w16.numel() * 2)):
            def issue(sp, i, dt=dt, nb=nb):
                if dt == "q4_0":
                    rc = lib.lib.hypno_hip_matmul_q4_0_dev(
                        yp, ctypes.c_void_p(arena.data_ptr()), nb, xp, None, n, m, M, sp)
                else:
                    rc = lib.lib.hypno_hip_matmul_f16_dev(
                        yp, ctypes.c_void_p(w16.data_ptr()), nb, xp, None, n, m, M, sp)
                if rc:
                    lib.check(rc, "lm_head")
            us = time_calls_graph(torch, issue, reps=5)
            out[f"{dt}_M{M}"] = {"us": round(us, 1), "weight_gbs": round(nb / us / 1e3, 1),
                                 "tflops": round(2.0 * M * n * m / us / 1e6, 2),
                                 "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4),
                                 "frac_fp16_peak": round(2.0 * M * n * m / us / 1e6 /
                                                         FP16_PEAK_TFLOPS, 4)}
        del x, y
    del arena, w16
    torch.cuda.empty_cache()
    return {"workload": "configs[4] lm_head K=4096 N=128256 (N a multiple of 128 but not "
                        "of 512/1024), M in {1,128}, Q4_0 and FP16 weights", "results": out}


def q8_0_decode(torch, lib):
    """Q8_0 weights (34-byte blocks, 1.0625 B per weight) at the Mistral-7B
    projection shapes, M = 1: GPU time per hypno_hip_matmul_q8_0_dev call over
    >= 512 MB of distinct weight copies.  The reference dequantises the whole
    tensor to fp32 on every such call (ops.rs:33-36)."""
    import hypno_amd as hk
    out = {}
    gen = torch.Generator(device="cuda").manual_seed(88)
    for name, n, m in (("q_o", 4096, 4096), ("k_v", 1024, 4096), ("gate_up", 14336, 4096),
                       ("down", 4096, 14336)):
        nb = n * m // 32 * 34
        stride = (nb + 255) // 256 * 256
        copies = max(2, -(-(512 * 2**20) // nb))
        arena = torch.empty(copies * stride, dtype=torch.uint8, device="cuda")
        for c in range(copies):
            w = torch.randn(n * m, generator=gen, device="cuda").mul_(0.02)
            arena[c * stride:c * stride + nb].copy_(hk.quantize_f32_to_q8_0(w))
            del w
        x = torch.randn(m, generator=gen, device="cuda")
        y = torch.empty(n, device="cuda")
        xp, yp = ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr())
        base = arena.data_ptr()

        def issue(sp, i, base=base, stride=stride, copies=copies, nb=nb, n=n, m=m):
            rc = lib.lib.hypno_hip_matmul_q8_0_dev(yp, ctypes.c_void_p(base + (i % copies) * stride),
                                                   nb, xp, None, n, m, 1, sp)
            if rc:
                lib.check(rc, "matmul_q8_0")

        us = time_calls_graph(torch, issue, reps=copies * 4)
        out[f"{name}_M1"] = {"us": round(us, 2), "weight_gbs": round(nb / us / 1e3, 1),
                             "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
        if name == "gate_up":
            # prefill: weights expanded to fp16 once per call, fp16 MFMA GEMM
            M = 512
            xm = torch.randn(M, m, generator=gen, device="cuda")
            ym = torch.empty(M, n, device="cuda")
            xmp, ymp = ctypes.c_void_p(xm.data_ptr()), ctypes.c_void_p(ym.data_ptr())

            def issue_m(sp, i, base=base, nb=nb, n=n, m=m):
                rc = lib.lib.hypno_hip_matmul_q8_0_dev(ymp, ctypes.c_void_p(base), nb, xmp,
                                                       None, n, m, M, sp)
                if rc:
                    lib.check(rc, "matmul_q8_0 M=512")

            us = time_calls_graph(torch, issue_m, reps=5)
            out[f"{name}_M{M}"] = {"us": round(us, 2),
                                   "tflops": round(2.0 * M * n * m / us / 1e6, 2),
                                   "frac_fp16_peak": round(2.0 * M * n * m / us / 1e6 /
                                                           FP16_PEAK_TFLOPS, 4)}
            del xm, ym
        del arena, x, y
        torch.cuda.empty_cache()
    return {"workload": "Q8_0 Mistral-7B projections, M = 1, one call per matrix, rotating "
                        ">= 512 MB of weight copies; gate/up also at M = 512 (prefill: fp16 "
                        "expansion + fp16 GEMM, per call)", "results": out}


def col_major(torch, lib):
    """Column-major Q4_0 (kernels.rs:403-535) at the Mistral-7B shapes, M = 1:
    W_col[m][n] streamed once per call (plus the fixed-order split
    reduction), rotating >= 512 MB of weight copies."""
    out = {}
    for name, n, m in (("q_o", 4096, 4096), ("gate_up", 14336, 4096), ("down", 4096, 14336)):
        arena, ptrs, nb = rotating_q4(torch, lib, m, n, seed=n + m)  # m columns of n outputs
        x = torch.randn(m, device="cuda")
        y = torch.empty(n, device="cuda")
        xp, yp = ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr())

        def issue(sp, i, ptrs=ptrs, nb=nb, n=n, m=m):
            rc = lib.lib.hypno_hip_matmul_q4_0_col_dev(yp, ctypes.c_void_p(ptrs[i % len(ptrs)]),
                                                       nb, xp, None, n, m, 1, sp)
            if rc:
                lib.check(rc, "matmul_q4_0_col")

        us = time_calls_graph(torch, issue, reps=len(ptrs) * 2)
        out[f"{name}_M1"] = {"us": round(us, 2), "weight_gbs": round(nb / us / 1e3, 1),
                             "frac_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS, 4)}
        del arena, x, y
        torch.cuda.empty_cache()
    return {"workload": "column-major Q4_0 Mistral-7B projections, M = 1, rotating >= 512 MB "
                        "of weight copies", "results": out}


PCIE_PEAK_GBS = 64.0  # MI355X host link: PCIe 5.0 x16, one direction


def write_hypno(path, metadata, tensors):
    """Write (name, shape, dtype code, bytes-like payload) tensors as a .hypno
    file with the converter's layout (format.rs:13-24, sft_convert.rs:121-289):
    header, metadata pairs, tensor table, payloads at 64-byte boundaries."""
    import struct
    head = bytearray(struct.pack("<4sIII", b"HYPN", 1, len(metadata), len(tensors)))
    for k, v in metadata:
        kb, vb = k.encode(), v.encode()
        head += struct.pack("<I", len(kb)) + kb + struct.pack("<I", len(vb)) + vb
    table = sum(4 + len(n.encode()) + 4 + 8 * len(s) + 20 for n, s, _, _ in tensors)
    cur = (len(head) + table + ALIGN - 1) // ALIGN * ALIGN
    offs = []
    for _, _, _, payload in tensors:
        offs.append(cur)
        cur = (cur + len(payload) + ALIGN - 1) // ALIGN * ALIGN
    for (name, shape, dtype, payload), off in zip(tensors, offs):
        nb = name.encode()
        head += struct.pack("<I", len(nb)) + nb + struct.pack("<I", len(shape))
        head += b"".join(struct.pack("<Q", d) for d in shape)
        head += struct.pack("<IQQ", dtype, off, len(payload))
    with open(path, "wb") as f:
        f.write(head)
        for (_, _, _, payload), off in zip(tensors, offs):
            f.seek(off)
            f.write(payload)
        f.truncate(cur)
    return cur


def model_load(torch, lib):
    """A TinyLlama-1.1B-shaped .hypno file (22 layers x 7 Q4_0 projections and
    two FP32 norms per layer) in the page cache, opened with every payload
    uploaded to HBM (hypno_hip_model_open), beside a host-only open (what
    HypnoModel::open costs: map + parse) and one pageable host-to-device copy
    of the mapped payload span (torch tensor over the mapping, .to("cuda"))."""
    import mmap
    import shutil
    import tempfile
    import warnings

    import numpy as np

    import hypno_amd as hk
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    shapes = [(n, m) for _ in range(LAYERS) for (_, n, m) in TINYLLAMA]
    arena, offs = make_q4_arena(torch, lib, shapes, seed=4321, stream=st)
    host = arena.cpu().numpy()
    del arena
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
             "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
             "down": "mlp.down_proj"}
    ones = np.ones(2048, np.float32).tobytes()
    tensors = []
    for i, ((n, m), (off, nb)) in enumerate(zip(shapes, offs)):
        layer, short = divmod(i, len(TINYLLAMA))[0], TINYLLAMA[i % len(TINYLLAMA)][0]
        if short == "q":
            for norm in ("input_layernorm", "post_attention_layernorm"):
                tensors.append((f"model.layers.{layer}.{norm}.weight", (2048,), 0, ones))
        tensors.append((f"model.layers.{layer}.{names[short]}.weight", (n, m), 3,
                        memoryview(host[off:off + nb])))
    tmp = tempfile.mkdtemp(prefix="hypno_bench_")
    try:
        path = os.path.join(tmp, "tinyllama_q4_0.hypno")
        size = write_hypno(path, [("architecture", "LlamaForCausalLM"),
                                  ("num_hidden_layers", str(LAYERS)),
                                  ("weight_layout", "row_major")], tensors)
        hk.HypnoModel.open(path, device=False).close()
        up, parse = [], []
        for _ in range(3):
            t0 = time.perf_counter()
            m = hk.HypnoModel.open(path)
            up.append(time.perf_counter() - t0)
            infos = m.manifest.tensors
            span = infos[-1].offset + infos[-1].data_len - (infos[0].offset // ALIGN * ALIGN)
            m.close()
            t0 = time.perf_counter()
            hk.HypnoModel.open(path, device=False).close()
            parse.append(time.perf_counter() - t0)
        with open(path, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
            with warnings.catch_warnings():
                warnings.simplefilter("ignore")
                src = torch.frombuffer(mm, dtype=torch.uint8)[infos[0].offset // ALIGN * ALIGN:]
            naive = []
            for _ in range(2):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                dev = src.to("cuda")
                torch.cuda.synchronize()
                naive.append(time.perf_counter() - t0)
                del dev
            del src
            mm.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    t_up, t_naive = sorted(up)[1], min(naive)
    return {"workload": "TinyLlama-1.1B-shaped .hypno file (154 Q4_0 projections + 44 FP32 "
                        "norms) from the page cache to HBM: hypno_hip_model_open, median of 3 (the "
                        "first also creates the pinned staging pool)",
            "file_bytes": size, "payload_span_bytes": span,
            "open_upload_ms": round(t_up * 1e3, 2),
            "first_open_ms": round(up[0] * 1e3, 2),
            "upload_gbs": round(span / t_up / 1e9, 2),
            "frac_pcie_peak": round(span / t_up / 1e9 / PCIE_PEAK_GBS, 3),
            "host_only_open_ms": round(sorted(parse)[1] * 1e3, 3),
            "pageable_copy_gbs": round(span / t_naive / 1e9, 2)}


def single_gemv(torch, lib):
    """one 2048 x 2048 Q4_0 GEMV (TinyLlama q_proj), M = 1."""
    r = q4_case(torch, lib, 2048, 2048, 1, seed=2048, reps=50)
    r["workload"] = ("configs[0] 2048x2048 Q4_0 GEMV, M=1; GPU time per call, >= 512 MB "
                     "of rotating weight copies")
    return r


def copy_probe(torch, nbytes=1 << 30, reps=20):
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE per
    dispatch calibrate the HBM counters (expected nbytes each way)."""
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ms = time_launches(torch, lambda: dst.copy_(src), reps, 2)
    print(json.dumps({"copy_probe_bytes": nbytes, "ms": round(ms, 4),
                      "gbs_each_way": round(nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_0_gemv_jobs_kernel_tinyllama_stream_traffic.txt")


def stream_traffic():
    """HBM bytes per launch of the decode-stream GEMV, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE per dispatch, each divided
    by the factor the same counter reads on a plain copy of known size)."""
    try:
        kv = {}
        with open(TRAFFIC_FILE) as f:
            for ln in f:
                if "=" in ln and not ln.startswith("#"):
                    k, v = ln.split("=", 1)
                    kv[k.strip()] = v.strip()
        return int(float(kv["traffic_bytes_per_launch"]))
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(sample, x_host, seconds):
    """hypno's AVX2 Q4_0 kernel (restated in oracle/) on this host's cores."""
    from oracle import oracle as orc
    threads = max(1, min(16, os.cpu_count() or 1))
    orc.set_threads(threads)
    mats = list(zip(sample, TINYLLAMA))
    for q, (_, n, m) in mats:  # warm-up (bench.rs:121)
        orc.matmul_q4_0(q, x_host[m], None, n, m)
    reps, t0 = 0, time.perf_counter()
    while True:
        for q, (_, n, m) in mats:
            orc.matmul_q4_0(q, x_host[m], None, n, m)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds and reps >= 3:
            break
    layer_bytes = sum(q.size for q in sample)
    gbs = layer_bytes * reps / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "avx2": orc.have_avx2_fma(),
            "sample": f"TinyLlama layer 0 (7 GEMVs, {layer_bytes} weight bytes) x {reps} reps "
                      f"in {el:.1f} s, OpenMP row-parallel"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--value-only", action="store_true",
                    help="time only the value's launches (no grouped/per-call variants, "
                         "no secondary, no CPU baseline)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run only a plain 1 GiB device copy, 20 times (HBM counter "
                         "calibration under rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(every GPU box here has one GPU)", file=sys.stderr)
        sys.exit(2)

    if args.value_only:
        args.no_secondary = args.no_cpu_baseline = True

    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.copy_probe:
        copy_probe(torch)
        return
    lib = Lib()

    print("[bench] decode stream: building 545 MB of Q4_0 weights", file=sys.stderr, flush=True)
    d = decode_stream(torch, lib, args.steps, args.warmup, value_only=args.value_only)
    value = d["weight_bytes"] / (d["ms"] * 1e-3) / 1e9
    print(f"[bench] decode stream {d['ms']:.4f} ms/step, {value:.1f} GB/s", file=sys.stderr,
          flush=True)
    config = {
        "workload": "TinyLlama-1.1B decode-step Q4_0 weight stream (configs[1]): 22 layers "
                    "x {q,k,v,o,gate,up,down} GEMV, M=1, all 154 GEMVs as one "
                    "multi-GEMV plan launch",
        "weight_bytes": d["weight_bytes"],
        "launches_per_step": d["launches"],
        "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
    }
    if "ms_grouped" in d:
        config["decode_step_grouped"] = {
            "desc": "dependency-respecting decode step: per layer [q,k,v], [o], [gate,up], "
                    "[down] plans, replayed as one HIP graph",
            "launches": d["launches_grouped"],
            "ms_per_step": round(d["ms_grouped"], 5),
            "gbs": round(d["weight_bytes"] / (d["ms_grouped"] * 1e-3) / 1e9, 2)}
        config["decode_step_fused"] = {
            "desc": "the grouped decode step with RMS norm before [q,k,v] and [gate,up] and "
                    "silu(gate)*up before [down] applied inside the GEMVs' activation staging",
            "launches": d["launches_fused"],
            "ms_per_step": round(d["ms_fused"], 5),
            "vs_separate_kernels_ms": round(d["ms_separate"], 5),
            "separate_launches": d["launches_separate"]}
        config["per_call"] = {
            "desc": "drop-in path: one hypno_hip_matmul_q4_0_dev call per matrix, "
                    "replayed as one HIP graph",
            "launches": d["launches_per_call"],
            "ms_per_step": round(d["ms_per_call"], 5),
            "gbs": round(d["weight_bytes"] / (d["ms_per_call"] * 1e-3) / 1e9, 2)}
    # One kernel launch per step: the launch's average duration over the timed
    # region is the step time (it includes the few-microsecond gap between
    # back-to-back launches).
    launch_ms = d["ms"] / d["launches"]
    achieved = d["weight_bytes"] / d["launches"] / (launch_ms * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: weights N(0,0.02) seeded, Q4_0-quantised on GPU; x N(0,1)",
        "config": config,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": stream_traffic(),
            "kernel": "q4_0_gemv_jobs_kernel",
            "launch_us": round(launch_ms * 1e3, 2),
            "bytes_per_launch": d["weight_bytes"] // d["launches"],
        },
    }
    if not args.no_secondary:
        sec = {}
        for key, fn in (("c0_single_gemv", single_gemv), ("c2_prefill_gemm", prefill_gemm),
                        ("c3_mistral_stream", mistral_stream), ("c3_m_sweep", mistral_m_sweep),
                        ("c4_lm_head", lm_head), ("model_load", model_load),
                        ("q8_0_decode", q8_0_decode), ("col_major", col_major)):
            print(f"[bench] secondary: {key}", file=sys.stderr, flush=True)
            sec[key] = fn(torch, lib)
        line["secondary"] = sec
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(d["sample"], d["x_host"], args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
