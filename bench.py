#!/usr/bin/env python3
"""Q4_0 matmul benchmark on one MI355X.

Headline workload (BASELINE.json configs[3] at M = 1, the 7B shapes the
metric and the north star quote): the Mistral-7B decode-step weight stream,
32 layers x {q, k, v, o, gate, up, down} Q4_0 GEMVs (3,925,868,544 weight
bytes, fifteen times the 256 MB Infinity Cache, so every step streams from
HBM).  One step = the 224 GEMVs as one multi-GEMV plan launch; steps are
launched back to back on one stream and timed with HIP events on that
stream.  value = weight bytes / step time (GB/s).

Also reported, in the same JSON line:
  roofline      the decode GEMV kernel's weight bytes per launch / its average
                launch duration over the timed region (HIP events on the
                launch stream), against the 8 TB/s HBM peak, with the
                first-launches ("burst") and last-launches ("sustained")
                averages; traffic = measured HBM bytes per launch (rocprofv3
                --pmc, read from the committed profile summary);
  cpu_baseline  the CPU restatement of hypno's AVX2 kernel (oracle/) on this
                host, on the same 224-matrix stream: the host's CPU share
                and 8 threads, OMP_PROC_BIND=close, 3 warm-ups + 10 timed
                passes, median (bench.rs:115-133);
  secondary     every other BASELINE config, GPU-timed (graph replay):
                configs[0] the single 2048x2048 GEMV, configs[1] the
                TinyLlama decode stream (with its own roofline block, and as
                grouped / fused / per-call decode steps), configs[2] the
                prefill GEMM at Llama-3.2-3B MLP shapes (M = 512), configs[3]
                the Mistral M-sweep {1, 2, 4, 8, 64, 512, 2048} and its
                decode step in dependency order (per layer [q,k,v], [o],
                [gate,up], [down] plans, one HIP graph), configs[4] the
                lm_head in Q4_0 and FP16 at M = 1 and 128; prefill GEMMs in
                the default exact-nibble arithmetic and again with the opt-in
                folded scales (hypno_hip_set_gemm_numerics FOLDED);
                model_load, q8_0_decode, col_major.  The final line holds
                them as a flat map "workload.case" -> {us, frac, ok} (frac =
                the binding roofline's fraction, ok = output checked); the
                full result tree goes to --detail FILE only, so the line
                stays ~6 KB and stderr a few progress lines.
Every workload's output is checked once, untimed, against an fp64 reference
computed here from the same packed bytes (sampled rows or columns; GEMV
bar 1e-4 normwise, GEMM bar 2e-3 relative L2): each carries "checked".
Each result also carries the reference bench's fields (bench.rs:14-16,35-46):
time_ms, gflops, bandwidth_gbps (weight bytes / time).

Inputs are synthetic: weights N(0, 0.02) from a seeded torch generator,
quantised on the GPU by the bit-exact Q4_0 quantizer; activations N(0, 1).
"""
from __future__ import annotations

import argparse
import ctypes
import glob
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "Q4_0 GEMV weight GB/s (% HBM peak); prefill GEMM TFLOPS at 7B shapes"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
GEMV_TOL = 1e-4
GEMM_TOL = 2e-3

# (name, n = output rows, m = input dim) per layer
TINYLLAMA = [("q", 2048, 2048), ("k", 256, 2048), ("v", 256, 2048), ("o", 2048, 2048),
             ("gate", 5632, 2048), ("up", 5632, 2048), ("down", 2048, 5632)]
TINYLLAMA_LAYERS = 22
MISTRAL = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
           ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
MISTRAL_LAYERS = 32
MISTRAL_SHAPES = [("q_o", 4096, 4096), ("k_v", 1024, 4096), ("gate_up", 14336, 4096),
                  ("down", 4096, 14336)]
ALIGN = 64  # .hypno tensor alignment (format.rs:10)
X_OF = {"q": "attn", "k": "attn", "v": "attn", "o": "o", "gate": "mlp", "up": "mlp",
        "down": "down"}


def q4_bytes(n, m):
    return n * m // 32 * 18


# --- fp64 reference checks (untimed; numpy over the packed bytes) ---------------------

def q4_rows_f64(raw):
    """Q4_0 rows [r, B*18] -> weights [r, B*32] in fp64: byte i of a block holds
    element 2i (low nibble) and 2i+1 (high); w = (nibble - 8) * d."""
    import numpy as np
    r = raw.shape[0]
    blk = raw.reshape(r, -1, 18)
    d = blk[:, :, :2].copy().view(np.float16).astype(np.float64)  # [r, B, 1]
    qs = blk[:, :, 2:].astype(np.int16)
    vals = np.stack([(qs & 15) - 8, (qs >> 4) - 8], axis=-1).reshape(r, -1, 32)
    return (vals * d).reshape(r, -1)


def q8_rows_f64(raw):
    """Q8_0 rows [r, B*34] -> fp64 weights: w = (u - 128) * d."""
    import numpy as np
    r = raw.shape[0]
    blk = raw.reshape(r, -1, 34)
    d = blk[:, :, :2].copy().view(np.float16).astype(np.float64)
    return ((blk[:, :, 2:].astype(np.float64) - 128.0) * d).reshape(r, -1)


def sample_idx(n, count, seed):
    import numpy as np
    rng = np.random.default_rng(seed)
    s = set(rng.choice(n, size=min(n, count), replace=False).tolist())
    s.update({0, n - 1})
    return np.array(sorted(s))


def gather_rows(torch, buf, off, n, row_bytes, rows):
    """Bytes of weight rows `rows` of the matrix at buf[off:] (rows of
    row_bytes bytes), gathered on the device and copied to the host."""
    mat = buf[off:off + n * row_bytes].view(n, row_bytes)
    return mat[torch.as_tensor(rows, device=buf.device)].cpu().numpy()


def normwise(got, ref):
    import numpy as np
    den = float(np.max(np.abs(ref)))
    err = float(np.max(np.abs(got.astype(np.float64) - ref)))
    return err / den if den > 0 else err


def rel_l2(got, ref):
    import numpy as np
    den = float(np.linalg.norm(ref))
    err = float(np.linalg.norm(got.astype(np.float64) - ref))
    return err / den if den > 0 else err


def check_q4(torch, buf, off, n, m, x, y, M, seed, count=64):
    """y [M][n] from W at buf[off:] and x [M][m] (device) against fp64 over
    sampled weight rows (GEMV: normwise; M > 16: relative L2 over all tokens of
    the sampled columns)."""
    cols = sample_idx(n, count, seed)
    w = q4_rows_f64(gather_rows(torch, buf, off, n, m // 32 * 18, cols))
    xh = x.reshape(M, m).cpu().numpy().astype("float64")
    ref = xh @ w.T
    got = y.reshape(M, n)[:, torch.as_tensor(cols, device=y.device)].cpu().numpy()
    if M <= 16:
        err = max(normwise(got[t], ref[t]) for t in range(M))
        return {"checked": err <= GEMV_TOL, "max_err": float(f"{err:.3g}"), "bar": "normwise 1e-4",
                "sampled_cols": len(cols)}
    err = rel_l2(got, ref)
    return {"checked": err <= GEMM_TOL, "max_err": float(f"{err:.3g}"), "bar": "rel-L2 2e-3",
            "sampled_cols": len(cols)}


def merge_checks(checks):
    """One check record for a workload made of several outputs."""
    checks = list(checks)
    return {"checked": all(c["checked"] for c in checks),
            "max_err": max(c["max_err"] for c in checks), "bar": checks[0]["bar"],
            "outputs_checked": len(checks)}


def ref_fields(us, flops, nbytes):
    """The reference bench's BenchResult fields (bench.rs:14-16)."""
    return {"time_ms": round(us * 1e-3, 6), "gflops": round(flops / us * 1e-3, 1),
            "bandwidth_gbps": round(nbytes / us * 1e-3, 1)}


SHORT = {"c0_single_gemv": "c0", "c1_tinyllama_stream": "c1", "c2_prefill_gemm": "c2",
         "c3_m_sweep": "c3", "c4_lm_head": "c4", "c4_next_token": "tok", "model_load": "load",
         "q8_0_decode": "q8", "col_major": "col", "c3_decode_step": "c3.decode_step_grouped"}


def compact(sec):
    """Flat map of every timed result in the secondary tree: "path" -> {us,
    frac, ok}, the compact record the final line carries (one entry per
    result, like bench.rs:35-46's BenchResult).  frac is the fraction of the
    roofline that binds the call: the larger of its HBM and fp16-MFMA
    fractions (the bound whose minimum time is the longer)."""
    flat = {}

    def walk(o, path):
        if not isinstance(o, dict):
            return
        us = o.get("us")
        if us is None and "ms_per_step" in o:
            us = o["ms_per_step"] * 1e3
        if us is None and "open_upload_ms" in o:
            us = o["open_upload_ms"] * 1e3
        if isinstance(us, (int, float)):
            fr = [o[k] for k in ("frac_hbm_peak", "frac_fp16_peak") if k in o]
            if not fr and "gbs" in o:
                fr = [o["gbs"] / HBM_PEAK_GBS]
            if not fr and isinstance(o.get("roofline"), dict):
                fr = [o["roofline"]["frac"]]
            ent = {"us": round(us, 2)}
            if fr:
                ent["frac"] = round(max(fr), 4)
            if isinstance(o.get("check"), dict):
                ent["ok"] = bool(o["check"].get("checked"))
            flat[path] = ent
        for k, v in o.items():
            if isinstance(v, dict) and k not in ("check", "separate_check", "roofline"):
                k = "folded" if k == "folded_scales" else k
                walk(v, f"{path}.{k}" if path and k != "results" else (path or k))
    for key, val in sec.items():
        walk(val, SHORT.get(key, key))
    return flat


# --- library and inputs ----------------------------------------------------------------

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


def time_launches(torch, fn, steps, warmup, per_launch=False):
    """Back-to-back calls of `fn` (one kernel launch each) on the current
    stream, timed by one event before the first launch and one after the
    last.  With per_launch, a second pass of `steps` launches follows the
    timed region with an event after every launch, for the launch-to-launch
    profile; an event between two launches leaves the GPU idle for ~6 us
    (the next kernel starts only after the marker), so that pass is not used
    for the average.  Returns (average ms over the timed region, per-launch
    ms of the second pass or None)."""
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
    ms = e0.elapsed_time(e1) / steps
    if not per_launch:
        return ms, None
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    return ms, [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]


def launch_stats(per_ms, bytes_per_launch):
    """Launch-to-launch profile of the pass after the timed region."""
    k = max(1, min(5, len(per_ms) // 4))
    first, last = per_ms[:k], per_ms[-k:]
    us = lambda v: round(v * 1e3, 2)  # noqa: E731
    gbs = lambda ms: round(bytes_per_launch / (ms * 1e-3) / 1e9, 1)  # noqa: E731
    return {"pass": "after the timed region, one event per launch",
            "launches": len(per_ms), "median_us": us(statistics.median(per_ms)),
            "min_us": us(min(per_ms)), "max_us": us(max(per_ms)),
            f"burst_first{k}_us": us(sum(first) / k), f"sustained_last{k}_us": us(sum(last) / k),
            f"burst_first{k}_gbs": gbs(sum(first) / k),
            f"sustained_last{k}_gbs": gbs(sum(last) / k)}


# --- decode-step weight streams (configs[1], configs[3] at M = 1) -----------------------

def build_stream(torch, lib, per_layer, layers, seed):
    """All layers' Q4_0 matrices in one arena, one output per matrix and, per
    layer, one activation vector per input kind (q/k/v and gate/up share)."""
    stream0 = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    shapes = [(n, m) for _ in range(layers) for (_, n, m) in per_layer]
    arena, offs = make_q4_arena(torch, lib, shapes, seed=seed, stream=stream0)
    gen = torch.Generator(device="cuda").manual_seed(seed + 1)
    dm = {"attn": per_layer[0][2], "o": per_layer[3][2], "mlp": per_layer[4][2],
          "down": per_layer[6][2]}
    xs = [{k: torch.randn(v, generator=gen, device="cuda") for k, v in dm.items()}
          for _ in range(layers)]
    ys = [torch.empty(n, device="cuda") for n, _ in shapes]
    jobs = []  # (layer, name, y, offset, x, n, m)
    for i, ((n, m), (off, nb)) in enumerate(zip(shapes, offs)):
        layer, name = i // len(per_layer), per_layer[i % len(per_layer)][0]
        jobs.append((layer, name, ys[i], off, xs[layer][X_OF[name]], n, m))
    return arena, offs, xs, jobs


def check_jobs(torch, arena, jobs, seed, count=16):
    return merge_checks(check_q4(torch, arena, off, n, m, x, y, 1, seed + i, count)
                        for i, (_, _, y, off, x, n, m) in enumerate(jobs))


def plan_of(hk, arena, jobs, names=None, layer=None, pro=None):
    sel = [j for j in jobs if (names is None or j[1] in names) and (layer is None or j[0] == layer)]
    return hk.GemvPlan([(y, arena[off:off + q4_bytes(n, m)], x, None, n, m) +
                        ((pro(name),) if pro else ())
                        for _, name, y, off, x, n, m in sel])


def mistral_stream(torch, lib, steps, warmup):
    """The value: Mistral-7B's 224 Q4_0 GEMVs as one plan launch per step."""
    import hypno_amd as hk
    arena, offs, xs, jobs = build_stream(torch, lib, MISTRAL, MISTRAL_LAYERS, seed=11)
    plan = plan_of(hk, arena, jobs)
    wb = sum(nb for _, nb in offs)
    ms, per = time_launches(torch, plan.run, steps, warmup, per_launch=True)
    for _, _, y, *_ in jobs:
        y.fill_(float("nan"))
    plan.run()
    torch.cuda.synchronize()
    chk = check_jobs(torch, arena, jobs, seed=3)
    res = {"ms": ms, "per": per, "weight_bytes": wb, "launches": plan.launches, "check": chk,
           "arena": arena, "offs": offs, "jobs": jobs}
    plan.close()
    return res


def mistral_decode_step(torch, d, steps, warmup):
    """The Mistral stream's weights as a real decode step runs them: per layer
    the dependency-respecting plans [q,k,v], [o], [gate,up], [down]
    (transformer.rs:296-453's order), 128 plan launches replayed as one HIP
    graph; the fraction is the weight bytes over the step time against the
    HBM peak."""
    import hypno_amd as hk
    arena, jobs, wb = d["arena"], d["jobs"], d["weight_bytes"]
    groups = [plan_of(hk, arena, jobs, names, layer)
              for layer in range(MISTRAL_LAYERS)
              for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",))]

    def run_groups():
        for p in groups:
            p.run()

    ms, g = time_graph(torch, run_groups, steps, warmup)
    for _, _, y, *_ in jobs:
        y.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    del g
    gbs = wb / (ms * 1e-3) / 1e9
    out = {"workload": "configs[3] Mistral-7B decode step at M=1 in dependency order: per "
                       "layer [q,k,v], [o], [gate,up], [down] plans, replayed as one HIP graph",
           "launches": sum(p.launches for p in groups), "ms_per_step": round(ms, 5),
           "gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
           "check": check_jobs(torch, arena, jobs, seed=13)}
    for p in groups:
        p.close()
    return out


def tinyllama_stream(torch, lib, steps, warmup):
    """TinyLlama's 154 GEMVs as one plan launch (with its own
    roofline block), and the same weights as a real decode step runs them:
    dependency-respecting plans per layer, those plans with RMS norm and
    silu(gate)*up fused into their activation staging (beside the same work
    as separate kernels), and one drop-in call per matrix."""
    import numpy as np

    import hypno_amd as hk
    arena, offs, xs, jobs = build_stream(torch, lib, TINYLLAMA, TINYLLAMA_LAYERS, seed=1234)
    wb = sum(nb for _, nb in offs)
    out = {"workload": "configs[1] TinyLlama-1.1B decode-step Q4_0 weight stream: 22 layers x "
                       "{q,k,v,o,gate,up,down}, M=1, 154 GEMVs as one plan launch, back to back",
           "weight_bytes": wb}

    def reset():
        for _, _, y, *_ in jobs:
            y.fill_(float("nan"))

    plan = plan_of(hk, arena, jobs)
    ms, per = time_launches(torch, plan.run, steps, warmup, per_launch=True)
    reset()
    plan.run()
    torch.cuda.synchronize()
    out["check"] = check_jobs(torch, arena, jobs, seed=5)
    gbs = wb / (ms * 1e-3) / 1e9
    out.update({"us": round(ms * 1e3, 2), "weight_gbs": round(gbs, 1),
                "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                "roofline": {"bound": "hbm", "kernel": "q4_0_gemv_jobs_kernel",
                             "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(gbs / HBM_PEAK_GBS, 4),
                             "traffic": stream_traffic(TINY_TRAFFIC_FILE),
                             "per_launch": launch_stats(per, wb)},
                **ref_fields(ms * 1e3, 2.0 * sum(n * m for *_, n, m in jobs), wb)})
    plan.close()
    # dependency-respecting decode step: per layer [q,k,v] [o] [gate,up] [down]
    groups = [plan_of(hk, arena, jobs, names, layer)
              for layer in range(TINYLLAMA_LAYERS)
              for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",))]

    def run_groups():
        for p in groups:
            p.run()

    ms_grp, g = time_graph(torch, run_groups, steps, warmup)
    reset()
    g.replay()
    torch.cuda.synchronize()
    del g
    out["decode_step_grouped"] = {
        "desc": "dependency-respecting decode step: per layer [q,k,v], [o], [gate,up], [down] "
                "plans, replayed as one HIP graph",
        "launches": sum(p.launches for p in groups), "ms_per_step": round(ms_grp, 5),
        "gbs": round(wb / (ms_grp * 1e-3) / 1e9, 2), "check": check_jobs(torch, arena, jobs, 7)}
    # one drop-in call per matrix
    calls = [(ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(arena.data_ptr() + off),
              q4_bytes(n, m), ctypes.c_void_p(x.data_ptr()), n, m)
             for _, _, y, off, x, n, m in jobs]

    def per_call():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for y, w, nb, x, n, m in calls:
            rc = lib.q4(y, w, nb, x, n, m, 1, st)
            if rc:
                lib.check(rc, "decode GEMV")

    ms_call, g = time_graph(torch, per_call, steps, warmup)
    reset()
    g.replay()
    torch.cuda.synchronize()
    del g
    out["per_call"] = {
        "desc": "drop-in path: one hypno_hip_matmul_q4_0_dev call per matrix, replayed as one "
                "HIP graph", "launches": len(calls), "ms_per_step": round(ms_call, 5),
        "gbs": round(wb / (ms_call * 1e-3) / 1e9, 2), "check": check_jobs(torch, arena, jobs, 9)}
    # RMS norm before [q,k,v] and [gate,up], silu(gate)*up before [down], fused
    eps = 1e-5
    gen = torch.Generator(device="cuda").manual_seed(77)
    norms = [(1.0 + 0.1 * torch.randn(2048, generator=gen, device="cuda"),
              1.0 + 0.1 * torch.randn(2048, generator=gen, device="cuda"))
             for _ in range(TINYLLAMA_LAYERS)]
    ups = [torch.randn(5632, generator=gen, device="cuda") for _ in range(TINYLLAMA_LAYERS)]

    def pro_of(layer):
        return lambda name: (("rms_norm", norms[layer][0], eps) if name in ("q", "k", "v") else
                             ("rms_norm", norms[layer][1], eps) if name in ("gate", "up") else
                             ("silu_mul", ups[layer]) if name == "down" else None)

    fused = []
    for layer in range(TINYLLAMA_LAYERS):
        for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
            pf = pro_of(layer)
            if names == ("o",):
                fused.append(plan_of(hk, arena, jobs, names, layer))
            else:
                fused.append(plan_of(hk, arena, jobs, names, layer, pro=pf))

    def run_fused():
        for p in fused:
            p.run()

    ms_fused, g = time_graph(torch, run_fused, steps, warmup)
    reset()
    g.replay()
    torch.cuda.synchronize()
    del g
    # fp64 reference of the fused step: the GEMV of the normed / gated input
    fchecks = []
    for i, (layer, name, y, off, x, n, m) in enumerate(jobs):
        if i % 7 == 0 or name in ("down", "gate"):  # a sample of the 154 jobs
            xv = x.cpu().numpy().astype(np.float64)
            if name in ("q", "k", "v", "gate", "up"):
                nw = norms[layer][0 if name in ("q", "k", "v") else 1].cpu().numpy()
                xv = xv / np.sqrt(np.mean(xv * xv) + eps) * nw
            elif name == "down":
                xv = xv / (1.0 + np.exp(-xv)) * ups[layer].cpu().numpy()
            cols = sample_idx(n, 16, 100 + i)
            wv = q4_rows_f64(gather_rows(torch, arena, off, n, m // 32 * 18, cols))
            got = y[torch.as_tensor(cols, device="cuda")].cpu().numpy()
            err = normwise(got, wv @ xv)
            fchecks.append({"checked": err <= GEMV_TOL, "max_err": float(f"{err:.3g}"),
                            "bar": "normwise 1e-4"})
    # the same work as separate kernels (norm / silu write the GEMVs' inputs)
    hidden = torch.randn(2048, generator=gen, device="cuda")
    gate_v = torch.randn(5632, generator=gen, device="cuda")

    def run_separate():
        for layer in range(TINYLLAMA_LAYERS):
            x = xs[layer]
            hk.rms_norm(hidden, norms[layer][0], eps, out=x["attn"])
            groups[4 * layer].run()
            groups[4 * layer + 1].run()
            hk.rms_norm(hidden, norms[layer][1], eps, out=x["mlp"])
            groups[4 * layer + 2].run()
            hk.silu_mul(gate_v, ups[layer], out=x["down"])
            groups[4 * layer + 3].run()

    ms_sep, g = time_graph(torch, run_separate, steps, warmup)
    reset()
    g.replay()
    torch.cuda.synchronize()
    del g
    out["decode_step_fused"] = {
        "desc": "the grouped decode step with RMS norm before [q,k,v] and [gate,up] and "
                "silu(gate)*up before [down] applied inside the GEMVs' activation staging",
        "launches": sum(p.launches for p in fused), "ms_per_step": round(ms_fused, 5),
        "vs_separate_kernels_ms": round(ms_sep, 5),
        "separate_launches": sum(p.launches for p in groups) + 3 * TINYLLAMA_LAYERS,
        "check": merge_checks(fchecks), "separate_check": check_jobs(torch, arena, jobs, 11)}
    for p in groups + fused:
        p.close()
    del arena
    torch.cuda.empty_cache()
    return out


# --- single calls (graph replay) -------------------------------------------------------

def time_calls_graph(torch, issue, reps, replays=3):
    """GPU time per iteration of `issue(stream_ptr, i)` (library calls on one
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


def result(us, M, n, m, nbytes):
    flops = 2.0 * M * n * m
    return {"us": round(us, 2), "weight_gbs": round(nbytes / us / 1e3, 1),
            "tflops": round(flops / us / 1e6, 2),
            "frac_hbm_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "frac_fp16_peak": round(flops / us / 1e6 / FP16_PEAK_TFLOPS, 4),
            **ref_fields(us, flops, nbytes)}


def q4_case(torch, lib, n, m, M, seed, reps, folded_too=False):
    """GPU us per hypno_hip_matmul_q4_0_dev call of an M x m . (n x m)^T
    product, over >= 512 MB of distinct weight copies when M <= 64 (so the
    weights stream from HBM), checked once against fp64.  With folded_too,
    the same call again with the opt-in folded-scale GEMM arithmetic."""
    import hypno_amd as hk
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nb = q4_bytes(n, m)
    copies = max(2, -(-(512 * 2**20) // nb)) if M <= 64 else 1
    arena, offs = make_q4_arena(torch, lib, [(n, m)] * copies, seed=seed, stream=st)
    ptrs = [arena.data_ptr() + off for off, _ in offs]
    gen = torch.Generator(device="cuda").manual_seed(seed + 1)
    x = torch.randn(M, m, generator=gen, device="cuda")
    y = torch.empty(M, n, device="cuda")
    xp, yp = ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr())

    def issue(sp, i):
        rc = lib.q4(yp, ctypes.c_void_p(ptrs[i % len(ptrs)]), nb, xp, n, m, M, sp)
        if rc:
            lib.check(rc, "matmul_q4_0")

    def checked():
        y.fill_(float("nan"))
        issue(st, 0)
        torch.cuda.synchronize()
        return check_q4(torch, arena, offs[0][0], n, m, x, y, M, seed)

    out = result(time_calls_graph(torch, issue, reps), M, n, m, nb)
    out["check"] = checked()
    if folded_too:
        prev = hk.set_gemm_numerics(hk.GEMM_FOLDED)
        try:
            ex = result(time_calls_graph(torch, issue, reps), M, n, m, nb)
            ex["check"] = checked()
        finally:
            hk.set_gemm_numerics(prev)
        out["folded_scales"] = ex
    del arena, x, y
    torch.cuda.empty_cache()
    return out


def single_gemv(torch, lib):
    """one 2048 x 2048 Q4_0 GEMV (TinyLlama q_proj), M = 1."""
    r = q4_case(torch, lib, 2048, 2048, 1, seed=2048, reps=50)
    r["workload"] = ("configs[0] 2048x2048 Q4_0 GEMV, M=1; GPU time per call, >= 512 MB "
                     "of rotating weight copies")
    return r


def prefill_gemm(torch, lib):
    """M = 512 tokens, Llama-3.2-3B MLP: gate/up 8192 x 3072 and
    down 3072 x 8192.  Each call = fp16 activation pre-pass + MFMA GEMM (+ a
    split-K reduction when the tile grid is small)."""
    out = {}
    for name, n, m in (("gate_up", 8192, 3072), ("down", 3072, 8192)):
        out[name] = q4_case(torch, lib, n, m, 512, seed=7 + n, reps=20, folded_too=True)
    return {"workload": "configs[2] Llama-3.2-3B MLP, M=512, Q4_0; GPU time per call incl. "
                        "the fp16 activation pre-pass (the BASELINE outlier channels are "
                        "exercised by the parity tests)", "results": out}


def mistral_m_sweep(torch, lib):
    """Mistral-7B projections at M in {1, 8, 64, 512, 2048}, and at
    M = 2 and 4 (the few-row GEMV: every matrix at M = 2, q/o and k/v at M = 4)."""
    out = {}
    for name, n, m in MISTRAL_SHAPES:
        for M in (1, 2, 4, 8, 64, 512, 2048):
            out[f"{name}_M{M}"] = q4_case(torch, lib, n, m, M, seed=n + m + M,
                                          reps=20 if M <= 64 else 4, folded_too=M >= 512)
    return {"workload": "configs[3] Mistral-7B q/o, k/v, gate/up, down at M in "
                        "{1,2,4,8,64,512,2048}; GPU time per call (graph replay); M <= 64 "
                        "rotates >= 512 MB of weight copies; M >= 512 also with the "
                        "opt-in folded scales", "results": out}


def lm_head(torch, lib):
    """K = 4096, N = 128256, M in {1, 128}, Q4_0 and FP16 weights;
    also M = 8 (a few tokens: the few-token Q4_0 kernel, the FP16 GEMM on
    hi/lo activation rows), held to the GEMV bar."""
    import numpy as np
    n, m = 128256, 4096
    out = {}
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    arena, offs = make_q4_arena(torch, lib, [(n, m)], seed=17, stream=st)
    gen = torch.Generator(device="cuda").manual_seed(18)
    w16 = torch.randn(n * m, generator=gen, device="cuda").mul_(0.02).half()
    for M in (1, 8, 128):
        x = torch.randn(M, m, generator=gen, device="cuda")
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
            r = result(time_calls_graph(torch, issue, reps=5), M, n, m, nb)
            y.fill_(float("nan"))
            issue(st, 0)
            torch.cuda.synchronize()
            if dt == "q4_0":
                r["check"] = check_q4(torch, arena, 0, n, m, x, y, M, seed=M, count=256)
            else:
                cols = np.union1d(sample_idx(n, 256, M), np.arange(n - 64, n))
                wv = w16.view(n, m)[torch.as_tensor(cols, device="cuda")].double().cpu().numpy()
                ref = x.double().cpu().numpy() @ wv.T
                got = y[:, torch.as_tensor(cols, device="cuda")].cpu().numpy()
                err = (max(normwise(got[t], ref[t]) for t in range(M)) if M <= 16
                       else rel_l2(got, ref))
                tol = GEMV_TOL if M <= 16 else GEMM_TOL
                r["check"] = {"checked": err <= tol, "max_err": float(f"{err:.3g}"),
                              "bar": "normwise 1e-4" if M <= 16 else "rel-L2 2e-3",
                              "sampled_cols": len(cols)}
            out[f"{dt}_M{M}"] = r
        del x, y
    del arena, w16
    torch.cuda.empty_cache()
    return {"workload": "configs[4] lm_head K=4096 N=128256 (N a multiple of 128 but not "
                        "of 512/1024), M in {1,128} (and 8), Q4_0 and FP16 weights",
            "results": out}


def next_token(torch, lib):
    """The step after the lm_head on its N = 128256 logits (run.rs:203-251):
    greedy argmax and sample_token at typical settings, GPU us per call (graph
    replay), each result checked against an independent host evaluation of
    the same logits (argmax; the temperature-0 sampling arithmetic in numpy
    float32)."""
    import numpy as np

    import hypno_amd as hk
    n = 128256
    gen = torch.Generator(device="cuda").manual_seed(31)
    logits = torch.randn(n, generator=gen, device="cuda").mul_(3.0)
    lh = logits.cpu().numpy()
    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    state = torch.tensor([88172645463325252], dtype=torch.int64, device="cuda")
    lp, tp, sp = (ctypes.c_void_p(t.data_ptr()) for t in (logits, tok, state))
    out = {}
    cases = {"argmax": None, "T0.7_topk40_topp0.9": (0.7, 0.9, 40),
             "T1.0_topp0.9_no_topk": (1.0, 0.9, 0), "T1.0_no_filters": (1.0, 1.0, 0)}
    for name, cfg in cases.items():
        def issue(st, i, cfg=cfg):
            rc = (lib.lib.hypno_hip_argmax_dev(tp, lp, n, st) if cfg is None else
                  lib.lib.hypno_hip_sample_token_dev(tp, sp, lp, n, cfg[0], cfg[1], cfg[2], st))
            if rc:
                lib.check(rc, "next token")
        us = time_calls_graph(torch, issue, reps=10)
        out[name] = {"us": round(us, 2)}
    # checks: the argmax, and a temperature-0 draw over positive logits,
    # against numpy
    issue_st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.lib.hypno_hip_argmax_dev(tp, lp, n, issue_st)
    torch.cuda.synchronize()
    ok = rc == 0 and int(tok.item()) == int(n - 1 - np.argmax(lh[::-1]))
    p = np.abs(lh)
    pg = torch.from_numpy(p).cuda()
    st0 = 987654321
    state.fill_(st0)
    hk.sample_token(pg, 0.0, 1.0, 0, state)
    torch.cuda.synchronize()
    f = np.float32
    s = f(-0.0)
    for v in p:
        s = f(s + v)
    x = st0
    M = (1 << 64) - 1
    x ^= (x << 13) & M
    x ^= x >> 7
    x ^= (x << 17) & M
    r = f((x >> 40) / 2.0**24)
    want, cum = None, f(0)
    for i, v in enumerate(p):
        cum = f(cum + f(v / s))
        if r < cum:
            want = i
            break
    got = hk.sample_token(pg, 0.0, 1.0, 0, torch.tensor([st0], dtype=torch.int64,
                                                        device="cuda"))
    torch.cuda.synchronize()
    ok = ok and want is not None and int(got.item()) == want
    return {"workload": "next token from K=4096 x N=128256 lm_head logits: greedy argmax and "
                        "sample_token (a launch over 63 ranges of the logits, then one "
                        "work-group; the reference's sequential fp32 sums and walks "
                        "reproduced bit for bit by integer prefix sums on the running "
                        "sum's binade grid); GPU us per call", "results": out,
            "check": {"checked": bool(ok), "bar": "token equal to a host evaluation"}}


def q8_0_decode(torch, lib):
    """Q8_0 weights (34-byte blocks, 1.0625 B per weight) at the Mistral-7B
    projection shapes, M = 1 (gate/up and down also at M = 8): GPU time per
    hypno_hip_matmul_q8_0_dev call over >= 512 MB of distinct weight copies.  The reference dequantises the whole
    tensor to fp32 on every such call (ops.rs:33-36)."""
    import hypno_amd as hk
    out = {}
    gen = torch.Generator(device="cuda").manual_seed(88)

    def chk(arena, n, m, x, y, M, seed):
        cols = sample_idx(n, 64, seed)
        raw = gather_rows(torch, arena, 0, n, m // 32 * 34, cols)
        ref = x.reshape(M, m).double().cpu().numpy() @ q8_rows_f64(raw).T
        got = y.reshape(M, n)[:, torch.as_tensor(cols, device="cuda")].cpu().numpy()
        err = (max(normwise(got[t], ref[t]) for t in range(M)) if M < 16
               else rel_l2(got, ref))
        tol = GEMV_TOL if M < 16 else GEMM_TOL
        return {"checked": err <= tol, "max_err": float(f"{err:.3g}"),
                "bar": "normwise 1e-4" if M < 16 else "rel-L2 2e-3", "sampled_cols": len(cols)}

    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for name, n, m in MISTRAL_SHAPES:
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

        r = result(time_calls_graph(torch, issue, reps=copies * 4), 1, n, m, nb)
        issue(st, 0)
        torch.cuda.synchronize()
        r["check"] = chk(arena, n, m, x, y, 1, n)
        out[f"{name}_M1"] = r
        if name in ("gate_up", "down"):
            # a few tokens: the few-row GEMV, one launch of 8 rows
            M = 8
            x8 = torch.randn(M, m, generator=gen, device="cuda")
            y8 = torch.empty(M, n, device="cuda")
            x8p, y8p = ctypes.c_void_p(x8.data_ptr()), ctypes.c_void_p(y8.data_ptr())

            def issue_8(sp, i, base=base, stride=stride, copies=copies, nb=nb, n=n, m=m):
                rc = lib.lib.hypno_hip_matmul_q8_0_dev(
                    y8p, ctypes.c_void_p(base + (i % copies) * stride), nb, x8p, None, n, m, M, sp)
                if rc:
                    lib.check(rc, "matmul_q8_0 M=8")

            r = result(time_calls_graph(torch, issue_8, reps=copies * 4), M, n, m, nb)
            issue_8(st, 0)
            torch.cuda.synchronize()
            r["check"] = chk(arena, n, m, x8, y8, M, n + 2)
            out[f"{name}_M{M}"] = r
            del x8, y8
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

            r = result(time_calls_graph(torch, issue_m, reps=5), M, n, m, nb)
            issue_m(st, 0)
            torch.cuda.synchronize()
            r["check"] = chk(arena, n, m, xm, ym, M, n + 1)
            out[f"{name}_M{M}"] = r
            del xm, ym
        del arena, x, y
        torch.cuda.empty_cache()
    return {"workload": "Q8_0 Mistral-7B projections, M = 1, one call per matrix, rotating "
                        ">= 512 MB of weight copies; gate/up and down also at M = 8 (few-row "
                        "GEMV), gate/up at M = 512 (prefill: fp16 expansion + fp16 GEMM, per "
                        "call)", "results": out}


def col_major(torch, lib):
    """Column-major Q4_0 (kernels.rs:403-535) at the Mistral-7B shapes, M = 1:
    W_col[m][n] streamed once per call (plus the fixed-order split
    reduction), rotating >= 512 MB of weight copies."""
    import numpy as np
    out = {}
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for name, n, m in (("q_o", 4096, 4096), ("gate_up", 14336, 4096), ("down", 4096, 14336)):
        nb = q4_bytes(m, n)  # m columns of n outputs
        copies = max(2, -(-(512 * 2**20) // nb))
        arena, offs = make_q4_arena(torch, lib, [(m, n)] * copies, seed=n + m, stream=st)
        ptrs = [arena.data_ptr() + off for off, _ in offs]
        x = torch.randn(m, device="cuda")
        y = torch.empty(n, device="cuda")
        xp, yp = ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr())

        def issue(sp, i, ptrs=ptrs, nb=nb, n=n, m=m):
            rc = lib.lib.hypno_hip_matmul_q4_0_col_dev(yp, ctypes.c_void_p(ptrs[i % len(ptrs)]),
                                                       nb, xp, None, n, m, 1, sp)
            if rc:
                lib.check(rc, "matmul_q4_0_col")

        r = result(time_calls_graph(torch, issue, reps=len(ptrs) * 2), 1, n, m, nb)
        issue(st, 0)
        torch.cuda.synchronize()
        # outputs of a few block columns: block b of every input row k
        nbk = n // 32
        blocks = sample_idx(nbk, 8, n)
        view = arena[:nb].view(m, nbk, 18)
        raw = view[:, torch.as_tensor(blocks, device="cuda"), :].cpu().numpy()  # [m, b, 18]
        w = q4_rows_f64(raw.reshape(m * len(blocks), 18)).reshape(m, len(blocks), 32)
        ref = np.einsum("kbj,k->bj", w, x.double().cpu().numpy()).ravel()
        cols = (blocks[:, None] * 32 + np.arange(32)[None, :]).ravel()
        got = y[torch.as_tensor(cols, device="cuda")].cpu().numpy()
        err = normwise(got, ref)
        r["check"] = {"checked": err <= GEMV_TOL, "max_err": float(f"{err:.3g}"),
                      "bar": "normwise 1e-4", "sampled_cols": len(cols)}
        out[f"{name}_M1"] = r
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
    shapes = [(n, m) for _ in range(TINYLLAMA_LAYERS) for (_, n, m) in TINYLLAMA]
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
                                  ("num_hidden_layers", str(TINYLLAMA_LAYERS)),
                                  ("weight_layout", "row_major")], tensors)
        hk.HypnoModel.open(path, device=False).close()
        up, parse = [], []
        for it in range(3):
            t0 = time.perf_counter()
            mdl = hk.HypnoModel.open(path)
            up.append(time.perf_counter() - t0)
            infos = mdl.manifest.tensors
            span = infos[-1].offset + infos[-1].data_len - (infos[0].offset // ALIGN * ALIGN)
            if it == 0:  # the uploaded payloads are the file's bytes (a sample of tensors)
                ok, picked = True, list(range(0, len(infos), 17)) + [len(infos) - 1]
                for ti in picked:
                    name = infos[ti].name
                    ptr, nbytes, _ = mdl.device_tensor(name)
                    dev = torch.empty(nbytes, dtype=torch.uint8)
                    torch.cuda.synchronize()
                    if hip_memcpy_d2h(dev.data_ptr(), ptr, nbytes) != 0:
                        ok = False
                        continue
                    hb = np.frombuffer(mdl.get_tensor_data(name)[0], np.uint8)
                    ok &= bool(np.array_equal(dev.numpy(), hb))
                load_check = {"checked": ok, "bar": "uploaded bytes equal the file's",
                              "tensors_compared": len(picked)}
            mdl.close()
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
            "pageable_copy_gbs": round(span / t_naive / 1e9, 2), "check": load_check}


def hip_memcpy_d2h(dst, src, nbytes):
    """hipMemcpy device -> host through the HIP runtime that torch loaded."""
    for name in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6",
                 "/opt/rocm/lib/libamdhip64.so"):
        try:
            h = ctypes.CDLL(name)
        except OSError:
            continue
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        return h.hipMemcpy(ctypes.c_void_p(dst), ctypes.c_void_p(src), nbytes, 2)
    return -1


def copy_probe(torch, nbytes=1 << 30, reps=20):
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE per
    dispatch calibrate the HBM counters (expected nbytes each way)."""
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ms, _ = time_launches(torch, lambda: dst.copy_(src), reps, 2)
    print(json.dumps({"copy_probe_bytes": nbytes, "ms": round(ms, 4),
                      "gbs_each_way": round(nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)


MISTRAL_TRAFFIC_FILE = os.path.join(ROOT, "profiles",
                                    "q4_0_gemv_jobs_kernel_mistral7b_stream_traffic.txt")
TINY_TRAFFIC_FILE = os.path.join(ROOT, "profiles",
                                 "q4_0_gemv_jobs_kernel_tinyllama_stream_traffic.txt")


def stream_traffic(path):
    """HBM bytes per launch of a decode-stream GEMV, from a committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE per dispatch, each divided
    by the factor the same counter reads on a plain copy of known size)."""
    try:
        kv = {}
        with open(path) as f:
            for ln in f:
                if "=" in ln and not ln.startswith("#"):
                    k, v = ln.split("=", 1)
                    kv[k.strip()] = v.strip()
        return int(float(kv["traffic_bytes_per_launch"]))
    except (OSError, KeyError, ValueError):
        return None


# --- CPU baseline: the oracle's GEMVs on the host cores ---------------------------------

def host_description():
    """nproc, CPU share, sockets, NUMA nodes and CPU model of this host."""
    d = {"nproc": len(os.sched_getaffinity(0)), "host_cpus": os.cpu_count()}
    try:
        with open("/proc/cpuinfo") as f:
            info = f.read()
        models = {ln.split(":", 1)[1].strip() for ln in info.splitlines()
                  if ln.startswith("model name")}
        d["cpu_model"] = "; ".join(sorted(models))
        sockets = {ln.split(":", 1)[1].strip() for ln in info.splitlines()
                   if ln.startswith("physical id")}
        d["sockets"] = len(sockets) or None
    except OSError:
        pass
    d["numa_nodes"] = len(glob.glob("/sys/devices/system/node/node[0-9]*")) or None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()[:2]
        d["cgroup_cpu_quota"] = None if q == "max" else round(int(q) / int(per), 2)
    except (OSError, ValueError):
        d["cgroup_cpu_quota"] = None
    d["omp_num_threads_env"] = os.environ.get("OMP_NUM_THREADS")
    return d


def cpu_baseline(mats, x_host):
    """hypno's AVX2 Q4_0 kernel (restated in oracle/, kernels.rs:270-359) on
    this host, over the same 224-matrix Mistral-7B stream as the value: one
    pass = one matmul_q4_0 call per matrix (row-parallel with OpenMP, as
    rayon's par_iter_mut, kernels.rs:279).  Method of bench.rs:115-133: 3
    warm-up passes, 10 timed, median; GB/s = weight bytes / time.  Runs on the
    CPU share this process has (all host cores when nothing limits it) and on
    8 threads (the published figures' thread count), threads bound
    OMP_PROC_BIND=close, OMP_PLACES=cores (set before the oracle's OpenMP
    runtime loads)."""
    os.environ["OMP_PROC_BIND"] = "close"
    os.environ["OMP_PLACES"] = "cores"
    from oracle import oracle as orc
    host = host_description()
    share = host["nproc"]
    if host.get("cgroup_cpu_quota"):
        share = min(share, max(1, int(host["cgroup_cpu_quota"])))
    if host.get("omp_num_threads_env", "").isdigit():
        share = min(share, int(host["omp_num_threads_env"]))
    total = sum(q.size for q, _, _ in mats)

    def run(threads):
        orc.set_threads(threads)
        times = []
        for it in range(13):
            t0 = time.perf_counter()
            for q, n, m in mats:
                orc.matmul_q4_0(q, x_host[m], None, n, m)
            if it >= 3:
                times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        return {"threads": threads, "median_s": round(med, 4), "gbs": round(total / med / 1e9, 3),
                "gflops": round(2.0 * sum(n * m for _, n, m in mats) / med / 1e9, 2)}

    t0 = time.perf_counter()
    share_run = run(share)
    t8 = run(8) if share != 8 else share_run
    elapsed = time.perf_counter() - t0
    return {"value": share_run["gbs"], "unit": "GB/s", "cores": share, "kind": "port",
            "avx2": orc.have_avx2_fma(), "threads_8": t8, "all_share": share_run,
            "omp_proc_bind": "close", "omp_places": "cores", "host": host,
            "sample": f"the full Mistral-7B decode stream ({len(mats)} matrices, {total} weight "
                      f"bytes, above any host LLC) per pass; 3 warm-up + 10 timed passes per "
                      f"thread count, median; {elapsed:.1f} s in all"}


# --- main -------------------------------------------------------------------------------

# Secondary workloads in the order the full run times them (None: the TinyLlama
# stream, which takes the run's --steps/--warmup).
SECONDARY = (("c0_single_gemv", single_gemv), ("c1_tinyllama_stream", None),
             ("c2_prefill_gemm", prefill_gemm), ("c3_m_sweep", mistral_m_sweep),
             ("c4_lm_head", lm_head), ("c4_next_token", next_token),
             ("model_load", model_load),
             ("q8_0_decode", q8_0_decode), ("col_major", col_major))


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--value-only", action="store_true",
                    help="time only the value's launches (no secondary, no CPU baseline)")
    ap.add_argument("--tinyllama-only", action="store_true",
                    help="time only the TinyLlama stream plan (profiling its traffic)")
    ap.add_argument("--only", metavar="WORKLOAD", default=None,
                    help="run only this secondary workload and print its result "
                         "(c0_single_gemv, c1_tinyllama_stream, c2_prefill_gemm, c3_m_sweep, "
                         "c3_decode_step, c4_lm_head, "
                         "c4_next_token, model_load, q8_0_decode, col_major); used to "
                         "profile one workload's kernels")
    ap.add_argument("--detail", metavar="FILE", default=None,
                    help="write every secondary workload's full result tree to FILE "
                         "(the final stdout line carries a compact us/frac/ok map)")
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
    if args.only == "c1_tinyllama_stream":
        print(json.dumps({args.only: tinyllama_stream(torch, lib, args.steps, args.warmup)}),
              flush=True)
        return
    if args.only == "c3_decode_step":
        arena, offs, xs, jobs = build_stream(torch, lib, MISTRAL, MISTRAL_LAYERS, seed=11)
        d = {"arena": arena, "jobs": jobs, "weight_bytes": sum(nb for _, nb in offs)}
        print(json.dumps({args.only: mistral_decode_step(torch, d, args.steps, args.warmup)}),
              flush=True)
        return
    if args.only is not None:
        fns = dict(SECONDARY)
        if fns.get(args.only) is None:
            print(f"--only: unknown workload {args.only!r}", file=sys.stderr)
            sys.exit(2)
        print(json.dumps({args.only: fns[args.only](torch, lib)}), flush=True)
        return
    if args.tinyllama_only:
        import hypno_amd as hk
        arena, offs, xs, jobs = build_stream(torch, lib, TINYLLAMA, TINYLLAMA_LAYERS, seed=1234)
        plan = plan_of(hk, arena, jobs)
        ms, _ = time_launches(torch, plan.run, args.steps, args.warmup)
        print(json.dumps({"tinyllama_stream_ms": round(ms, 5)}), flush=True)
        return

    print("[bench] Mistral-7B decode stream: building 3.93 GB of Q4_0 weights", file=sys.stderr,
          flush=True)
    d = mistral_stream(torch, lib, args.steps, args.warmup)
    wb = d["weight_bytes"]
    value = wb / (d["ms"] * 1e-3) / 1e9
    print(f"[bench] decode stream {d['ms']:.4f} ms/step, {value:.1f} GB/s, checked "
          f"{d['check']['checked']}", file=sys.stderr, flush=True)
    # One kernel launch per step: the launch's average duration over the timed
    # region is the step time (back-to-back launches, no event between them).
    launch_ms = d["ms"] / d["launches"]
    achieved = wb / d["launches"] / (launch_ms * 1e-3) / 1e9
    n_mats = len(d["jobs"])
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
        "dtype": "i4 weights x i19 activation limbs (i32 dots), f32 accumulate",
        "data": "synthetic: weights N(0,0.02) seeded, Q4_0-quantised on GPU; x N(0,1)",
        "config": {
            "workload": "Mistral-7B decode-step Q4_0 weight stream (configs[3] at M=1): 32 "
                        "layers x {q,k,v,o,gate,up,down} GEMV, all 224 GEMVs as one "
                        "multi-GEMV plan launch, launched back to back",
            "weight_bytes": wb,
            "matrices": n_mats,
            "launches_per_step": d["launches"],
            "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
            "check": d["check"],
            **ref_fields(d["ms"] * 1e3, 2.0 * sum(n * m for *_, n, m in d["jobs"]), wb),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": stream_traffic(MISTRAL_TRAFFIC_FILE),
            "kernel": "q4_0_gemv_jobs_kernel",
            "launch_us": round(launch_ms * 1e3, 2),
            "bytes_per_launch": wb // d["launches"],
            "per_launch": launch_stats(d["per"], wb),
        },
    }
    step = None
    if not args.no_secondary:
        print("[bench] secondary: c3_decode_step", file=sys.stderr, flush=True)
        step = mistral_decode_step(torch, d, args.steps, args.warmup)
    cpu_mats = None
    if not args.no_cpu_baseline:
        arena = d["arena"]
        cpu_mats = [(arena[off:off + nb].cpu().numpy(), n, m)
                    for (off, nb), (_, _, _, _, _, n, m) in zip(d["offs"], d["jobs"])]
        x_host = {m: x.cpu().numpy() for *_, x, n, m in d["jobs"][:7]}
    del d
    torch.cuda.empty_cache()
    if not args.no_secondary:
        sec = {"c3_decode_step": step}
        for key, fn in SECONDARY:
            print(f"[bench] secondary: {key}", file=sys.stderr, flush=True)
            if fn is None:
                sec[key] = tinyllama_stream(torch, lib, args.steps, args.warmup)
            else:
                sec[key] = fn(torch, lib)
        line["secondary"] = compact(sec)
        # The full tree goes only to --detail FILE: the final stdout line and
        # the few progress lines on stderr stay small enough for a log tail
        # of stdout and stderr together to hold the line whole.
        if args.detail:
            with open(args.detail, "w") as f:
                f.write(json.dumps({"secondary": sec}) + "\n")
        checks = []

        def walk(o):
            if isinstance(o, dict):
                for k, v in o.items():
                    if k in ("check", "separate_check") and isinstance(v, dict):
                        checks.append(v.get("checked", False))
                    else:
                        walk(v)
        walk(sec)
        line["all_checked"] = bool(checks) and all(checks) and line["config"]["check"]["checked"]
        line["checks_run"] = len(checks) + 1
    if cpu_mats is not None:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(cpu_mats, x_host)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
