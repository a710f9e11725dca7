"""The decode step's neighbours of the GEMV: RMS norm (kernels.rs:592-625)
and silu(gate) * up (transformer.rs:446-449), stand-alone and as prologues of
the plan GEMV.

CPU tests pin the oracle restatements (oracle/q4_0_oracle.c) with the
reference's own known-answer tests and closed forms; GPU tests compare the
device kernels and the fused plans with the oracle through the C ABI."""
import numpy as np
import pytest

EPS = 1e-5


# --- oracle pins (CPU) ----------------------------------------------------------------

@pytest.mark.parametrize("kind", ["avx2", "scalar"])
def test_rms_norm_reference_kat(orc, kind):
    """ops.rs:131-136: [2, 2, 2, 2] with unit weight -> ~1.0."""
    y = orc.rms_norm_variant(np.full(4, 2.0, np.float32), np.ones(4, np.float32), EPS, kind)
    assert np.all(np.abs(y - 1.0) < 1e-3)


def test_rms_norm_batch_form_matches_simd_form(orc):
    """turbo.rs:716-735: the f64 batch_rms_norm and the SIMD rms_norm agree
    within 1e-6 on x = (i+1)*0.1, w = 1 + 0.01 i, dim 64."""
    i = np.arange(64, dtype=np.float32)
    x = (i + 1).astype(np.float32) * np.float32(0.1)
    w = np.float32(1.0) + i * np.float32(0.01)
    a = orc.batch_rms_norm(x, w, 64, 1, EPS)
    b = orc.rms_norm(x, w, EPS)
    assert np.max(np.abs(a - b)) < 1e-6


def test_batch_rms_norm_reference_kats(orc):
    """turbo.rs:924-951."""
    out = orc.batch_rms_norm(np.full(8, 2.0, np.float32), np.ones(4, np.float32), 4, 2, EPS)
    assert np.all(np.abs(out - 1.0) < 0.01)
    out = orc.batch_rms_norm(np.array([1, 2, 3, 4], np.float32), np.full(2, 0.5, np.float32),
                             2, 2, EPS)
    r0, r1 = np.sqrt(np.float32(2.5)), np.sqrt(np.float32(12.5))
    want = [1 * 0.5 / r0, 2 * 0.5 / r0, 3 * 0.5 / r1, 4 * 0.5 / r1]
    assert np.all(np.abs(out - np.array(want)) < 0.01)


def test_rms_norm_closed_form_and_tail(orc):
    """Constant rows make every sum exact, so each output is fixed bit for bit:
    the first n - n % 8 elements are (c * (1 / r)) * w, the tail c / r * w
    (kernels.rs:611-616), with r = sqrt(c^2 + eps) in f32.  c = 3 is a value
    where the two forms give different f32 results, so a tail computed with
    the multiply form fails here."""
    c, n = np.float32(3.0), 13
    w = np.float32(1.0)
    r = np.sqrt(np.float32(c * c) + np.float32(EPS))
    main = (c * (np.float32(1.0) / r)) * w
    tail = (c / r) * w
    assert main != tail
    for kind in ("avx2",):
        y = orc.rms_norm_variant(np.full(n, c, np.float32), np.ones(n, np.float32), EPS, kind)
        assert np.all(y[:8] == main) and np.all(y[8:] == tail)
    y = orc.rms_norm_variant(np.full(n, c, np.float32), np.ones(n, np.float32), EPS, "scalar")
    assert np.all(y == main)


def test_rms_norm_against_f64(orc):
    rng = np.random.default_rng(3)
    for n in (7, 100, 2048, 5632):
        x = rng.standard_normal(n).astype(np.float32)
        w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + EPS) * w
        got = orc.rms_norm(x, w, EPS)
        assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-6, n


def test_silu_reference_kat_and_identity(orc):
    """turbo.rs:979-990, and silu(v) - silu(-v) = v (sigma(v) + sigma(-v) = 1),
    which fails for a sign or exponent mistake."""
    s = orc.silu_mul(np.array([0.0, -1.0, 1.0], np.float32), np.ones(3, np.float32))
    assert abs(s[0]) < 1e-3 and abs(s[1] + 0.2689) < 0.01 and abs(s[2] - 0.7311) < 0.01
    rng = np.random.default_rng(4)
    v = (rng.standard_normal(4096) * 4).astype(np.float32)
    up = rng.standard_normal(4096).astype(np.float32)
    one = np.ones_like(v)
    d = orc.silu_mul(v, one).astype(np.float64) - orc.silu_mul(-v, one).astype(np.float64)
    assert np.max(np.abs(d - v) / np.maximum(np.abs(v), 1.0)) < 1e-6
    ref = v.astype(np.float64) / (1.0 + np.exp(-v.astype(np.float64))) * up
    got = orc.silu_mul(v, up)
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) < 1e-6


# --- device kernels (GPU) -------------------------------------------------------------

@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


@pytest.fixture(scope="module")
def hk():
    import hypno_amd
    return hypno_amd


@pytest.mark.gpu
@pytest.mark.parametrize("n,rows", [(4, 1), (7, 1), (64, 3), (100, 2), (2048, 1), (5632, 1),
                                    (4096, 5)])
def test_rms_norm_dev(torch, hk, orc, n, rows):
    print(f"rms_norm n={n} rows={rows}", flush=True)
    rng = np.random.default_rng(n + rows)
    x = rng.standard_normal(n * rows).astype(np.float32) * 3
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    ref = orc.rms_norm(x, w, EPS, rows)
    dx, dw = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    got = hk.rms_norm(dx, dw, EPS, rows)
    hk.rms_norm_in_place(dx, dw, EPS, rows)
    torch.cuda.synchronize()
    g = got.cpu().numpy()
    assert np.array_equal(g, dx.cpu().numpy())  # in place == out of place
    tol = 1e-5  # fp32 reductions in a different order than the AVX2 chain
    assert np.max(np.abs(g - ref)) / np.max(np.abs(ref)) <= tol


@pytest.mark.gpu
def test_silu_mul_dev(torch, hk, orc):
    rng = np.random.default_rng(9)
    g = np.concatenate([np.array([0, -1, 1, 20, -20, 88, -88, 1e-30], np.float32),
                        (rng.standard_normal(14336 * 2) * 4).astype(np.float32)])
    u = rng.standard_normal(g.size).astype(np.float32)
    ref = orc.silu_mul(g, u)
    dg, du = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    got = hk.silu_mul(dg, du).cpu().numpy()
    tol = 1e-6  # elementwise, relative: expf and the divide differ by a few ulp
    assert np.all(np.abs(got - ref) <= tol * np.abs(ref) + 1e-37)
    hk.silu_mul(dg, du, out=dg)  # in place (silu_in_place then gate *= up)
    torch.cuda.synchronize()
    assert np.array_equal(dg.cpu().numpy(), got)


def _q4(orc, seed, n, m):
    return orc.quantize_q4_0(orc.normal_f32(seed, n * m, 0.02))


@pytest.mark.gpu
def test_plan_prologues_decode_layer(torch, hk, orc):
    """One TinyLlama layer as the four dependency groups of a decode step,
    each a plan: [q, k, v] after input_layernorm, [o], [gate, up] after
    post_attention_layernorm, [down] on silu(gate) * up — every norm and
    silu applied inside the GEMV's staging.  Against the oracle's rms_norm /
    silu_mul followed by matmul_q4_0; normwise <= 1e-4, repeat bit-exact,
    inputs left unchanged."""
    rng = np.random.default_rng(21)
    hd, im = 2048, 5632
    shapes = {"q": (2048, hd), "k": (256, hd), "v": (256, hd), "o": (2048, hd),
              "gate": (im, hd), "up": (im, hd), "down": (hd, im)}
    W = {k: _q4(orc, 300 + i, n, m) for i, (k, (n, m)) in enumerate(shapes.items())}
    hidden = (rng.standard_normal(hd) * 2).astype(np.float32)
    attn = rng.standard_normal(hd).astype(np.float32)
    gate = (rng.standard_normal(im) * 3).astype(np.float32)
    up = rng.standard_normal(im).astype(np.float32)
    n1 = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    n2 = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    d = {k: torch.from_numpy(v).cuda() for k, v in
         dict(hidden=hidden, attn=attn, gate=gate, up=up, n1=n1, n2=n2).items()}
    dw = {k: torch.from_numpy(v).cuda() for k, v in W.items()}
    ys = {k: torch.empty(n, device="cuda") for k, (n, _) in shapes.items()}
    src = {"q": ("hidden", ("rms_norm", "n1")), "k": ("hidden", ("rms_norm", "n1")),
           "v": ("hidden", ("rms_norm", "n1")), "o": ("attn", None),
           "gate": ("hidden", ("rms_norm", "n2")), "up": ("hidden", ("rms_norm", "n2")),
           "down": ("gate", ("silu_mul", "up"))}

    def job(k):
        n, m = shapes[k]
        xname, pro = src[k]
        p = None
        if pro and pro[0] == "rms_norm":
            p = ("rms_norm", d[pro[1]], EPS)
        elif pro:
            p = ("silu_mul", d[pro[1]])
        return (ys[k], dw[k], d[xname], None, n, m, p)

    plans = [hk.GemvPlan([job(k) for k in grp])
             for grp in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",))]
    assert all(p.launches == 1 for p in plans)
    for p in plans:
        p.run()
    torch.cuda.synchronize()
    first = {k: y.cpu().numpy().copy() for k, y in ys.items()}
    for p in plans:
        p.run()
    torch.cuda.synchronize()
    xin = {"hidden": hidden, "attn": attn, "gate": gate}
    for k, (n, m) in shapes.items():
        assert np.array_equal(first[k], ys[k].cpu().numpy()), k
        xname, pro = src[k]
        x = xin[xname]
        if pro and pro[0] == "rms_norm":
            x = orc.rms_norm(x, n1 if pro[1] == "n1" else n2, EPS)
        elif pro:
            x = orc.silu_mul(x, up)
        ref = orc.matmul_q4_0(W[k], x, None, n, m)
        err = np.max(np.abs(first[k] - ref)) / np.max(np.abs(ref))
        assert err <= 1e-4, (k, err)
    for name, v in (("hidden", hidden), ("gate", gate)):
        assert np.array_equal(d[name].cpu().numpy(), v)


@pytest.mark.gpu
@pytest.mark.parametrize("m,offset", [(320, 0), (96, 0), (2048, 1)])
def test_plan_prologues_generic_path(torch, hk, orc, m, offset):
    """Jobs the streaming kernel cannot take (K % 256 != 0, or an operand not
    16-byte aligned) run the stand-alone prologue into a plan buffer, then
    the generic GEMV."""
    n = 37
    rng = np.random.default_rng(m + offset)
    wq = _q4(orc, 77, n, m)
    x = rng.standard_normal(m + offset).astype(np.float32)
    a = (1 + 0.1 * rng.standard_normal(m + offset)).astype(np.float32)
    dx = torch.from_numpy(x).cuda()[offset:]
    da = torch.from_numpy(a).cuda()[offset:]
    dw = torch.from_numpy(wq).cuda()
    y1, y2 = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    plan = hk.GemvPlan([(y1, dw, dx, None, n, m, ("rms_norm", da, EPS)),
                        (y2, dw, dx, None, n, m, ("silu_mul", da))])
    assert plan.launches == 4
    plan.run()
    torch.cuda.synchronize()
    xs, as_ = x[offset:], a[offset:]
    for y, xin in ((y1, orc.rms_norm(xs, as_, EPS)), (y2, orc.silu_mul(xs, as_))):
        ref = orc.matmul_q4_0(wq, xin, None, n, m)
        err = np.max(np.abs(y.cpu().numpy() - ref)) / np.max(np.abs(ref))
        assert err <= 1e-4, err


@pytest.mark.gpu
def test_prologue_errors(torch, hk):
    y = torch.empty(4, device="cuda")
    w = torch.zeros(4 * 8 * 18, dtype=torch.uint8, device="cuda")
    x = torch.zeros(256, device="cuda")
    with pytest.raises(ValueError):
        hk.GemvPlan([(y, w, x, None, 4, 256, ("gelu", x))])
    with pytest.raises(ValueError):
        hk.GemvPlan([(y, w, x, None, 4, 256, ("silu_mul", x[:10]))])
