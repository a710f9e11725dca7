"""GPU parity of the steps either side of the decode GEMVs that touch whole
rows: the token-embedding gather (q4_0_extract_row quant.rs:139-153,
q8_0_extract_row :158-175, transformer.rs:476-497) bit-exact against the
oracle's dequantisers, and the next-token choice after the lm_head (argmax
and sample_token, run.rs:203-278) against the oracle's restatement:
  * temperature 0 (p = the logits themselves, no exp): the top-k threshold,
    the top-p walk, the fp32 sums and the draw are the reference's
    operations in its order, so token and generator state must match
    exactly, over many seeds and N = 128256 (the lm_head of configs[4]);
  * temperature > 0: exp is evaluated differently (fp64 rounded once against
    libm's expf), so the token is checked to match on fixed seeds."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

VOCAB = 128256


@pytest.fixture(scope="module")
def env(orc):
    import torch

    import hypno_amd as hk
    from hypno_amd import _lib
    assert torch.cuda.is_available()
    return torch, hk, _lib.load()


def _gpu_sample(torch, hk, logits_g, temperature, top_p, top_k, state):
    st = torch.tensor([np.uint64(state).astype(np.int64)], dtype=torch.int64, device="cuda")
    tok = hk.sample_token(logits_g, temperature, top_p, top_k, st)
    torch.cuda.synchronize()
    return int(tok.item()), int(np.int64(st.item()).astype(np.uint64))


# --- embedding rows -----------------------------------------------------------------

@pytest.mark.parametrize("dtype", ["fp32", "fp16", "q8_0", "q4_0"])
def test_embed_tokens_bit_exact(env, orc, dtype):
    torch, hk, lib = env
    vocab, hd = 1000, 4096
    print(f"[case] embed {dtype}", flush=True)
    w = orc.normal_f32(61, vocab * hd, 0.02)
    if dtype == "fp32":
        table, ref = w.view(np.uint8), w.reshape(vocab, hd)
    elif dtype == "fp16":
        h = w.astype(np.float16)
        table, ref = h.view(np.uint8), h.astype(np.float32).reshape(vocab, hd)
    elif dtype == "q8_0":
        table = orc.quantize_q8_0(w)
        ref = orc.dequantize_q8_0(table).reshape(vocab, hd)
    else:
        table = orc.quantize_q4_0(w)
        ref = orc.dequantize_q4_0(table).reshape(vocab, hd)
    code = {"fp32": 0, "fp16": 1, "q8_0": 2, "q4_0": 3}[dtype]
    ids = np.random.default_rng(62).integers(0, vocab, size=37).astype(np.int32)
    ids[0], ids[-1] = 0, vocab - 1
    tg = torch.from_numpy(table).cuda()
    out = hk.embed_tokens(tg, code, torch.from_numpy(ids).cuda(), hd)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref[ids].view(np.uint32))
    # a token id past the table: a NaN row (the reference panics)
    bad = hk.embed_tokens(tg, code, torch.tensor([vocab], dtype=torch.int32, device="cuda"), hd)
    torch.cuda.synchronize()
    assert bool(torch.isnan(bad).all())


@pytest.mark.parametrize("width", [4096, 100])
def test_extract_row(env, orc, width):
    torch, hk, lib = env
    rows = 50
    bpr = width // 32
    w = orc.normal_f32(63, rows * bpr * 32, 0.02)
    q4, q8 = orc.quantize_q4_0(w), orc.quantize_q8_0(w)
    for fn, q, deq in ((hk.q4_0_extract_row, q4, orc.dequantize_q4_0),
                       (hk.q8_0_extract_row, q8, orc.dequantize_q8_0)):
        qg = torch.from_numpy(q).cuda()
        for r in (0, 17, rows - 1):
            got = fn(qg, r, width).cpu().numpy()
            want = np.zeros(width, np.float32)
            want[: bpr * 32] = deq(q).reshape(rows, bpr * 32)[r]
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (fn, r)
        with pytest.raises(hk.HypnoHipError):   # past the end: a panic in the reference
            fn(qg, rows, width)


# --- next token -----------------------------------------------------------------------

def test_argmax(env, orc):
    torch, hk, lib = env
    rng = np.random.default_rng(64)
    cases = []
    x = rng.standard_normal(VOCAB).astype(np.float32)
    cases.append(x)
    y = x.copy()
    y[[5, 700, 99999]] = 50.0          # ties: the last one
    cases.append(y)
    z = y.copy()
    z[123] = np.nan                    # a NaN: argmax of what follows
    cases.append(z)
    w = y.copy()
    w[-1] = np.nan                     # a final NaN: that index
    cases.append(w)
    cases.append(np.array([0.0, -0.0], np.float32))
    cases.append(np.array([-1.0], np.float32))
    # the device splits the logits into consecutive ranges: NaNs and maxima
    # on either side of range boundaries, a maximum before the last NaN,
    # every element NaN, and sizes with one, two and three ranges
    u = x.copy()
    u[3] = 100.0                       # larger than anything after the NaN
    u[[10, 64000]] = np.nan
    cases.append(u)
    for b in (2035, 2036, 4071, 4072, 126220):  # near 128256 * g / 63
        v = x.copy()
        v[b] = np.nan
        v[b - 1] = 60.0
        v[b + 1] = 40.0
        cases.append(v)
    cases.append(np.full(5000, np.nan, np.float32))
    for n in (2047, 2049, 5000):
        s = rng.standard_normal(n).astype(np.float32)
        s[[0, n - 1]] = s.max()
        cases.append(s)
    for c in cases:
        got = hk.argmax(torch.from_numpy(c).cuda())
        torch.cuda.synchronize()
        assert int(got.item()) == orc.argmax(c)
    # empty input: 0
    out = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    assert lib.hypno_hip_argmax_dev(ctypes.c_void_p(out.data_ptr()), None, 0, None) == 0
    torch.cuda.synchronize()
    assert int(out.item()) == 0



def test_argmax_unaligned_and_edges(env, orc):
    """One-launch greedy argmax: starts 0-3 floats past a 16-byte boundary
    (the leading elements and the tail are read one by one), ties between
    the leading elements, the 16-byte body and the tail, signed zeros, all
    -inf, short lengths, and a NaN (the exact scan)."""
    torch, hk, lib = env
    rng = np.random.default_rng(66)
    base = torch.from_numpy(rng.standard_normal(VOCAB + 8).astype(np.float32)).cuda()
    for off in range(4):
        for n in (1, 2, 3, 5, 7, 4099, VOCAB):
            src = base[off:off + n].clone()
            for variant in range(4):
                c = src.clone()
                if variant == 1 and n > 2:   # the same maximum at the start, middle and end
                    c[[0, n // 2, n - 1]] = 9.0
                elif variant == 2:           # +0 and -0 tie: the later index
                    c[:] = -1.0
                    c[0] = 0.0
                    c[n - 1] = -0.0
                elif variant == 3:
                    c[:] = -float("inf")
                buf = torch.empty(n + off, device="cuda")
                buf[off:] = c
                view = buf[off:]
                assert view.data_ptr() % 16 == (4 * off) % 16
                got = hk.argmax(view)
                torch.cuda.synchronize()
                want = orc.argmax(view.cpu().numpy())
                assert int(got.item()) == want, (off, n, variant)
    c = base[1:VOCAB + 1].clone()
    c[77777] = float("nan")
    buf = torch.empty(VOCAB + 1, device="cuda")
    buf[1:] = c
    got = hk.argmax(buf[1:])
    torch.cuda.synchronize()
    assert int(got.item()) == orc.argmax(c.cpu().numpy())


EXACT_CASES = [  # (top_p, top_k)
    (1.0, 0), (1.0, 40), (0.9, 0), (0.9, 40), (0.5, 1000), (0.95, 1), (0.999, 50000),
    # without top-k: the key bins from the top (0.5), and every p sorted
    # (0.99: top_p plus the margin of the fp32 sums reaches 1)
    (0.5, 0), (0.99, 0),
    # k around the length of the device's per-range candidate lists (128256
    # logits in 63 ranges of 2035-2036) and k = n - 1
    (0.9, 2035), (1.0, 2036), (0.8, 3000), (1.0, VOCAB - 1),
]


@pytest.mark.parametrize("top_p,top_k", EXACT_CASES)
def test_sample_exact_temperature0(env, orc, top_p, top_k):
    """p = the logits: every step is the reference's fp32 arithmetic in its
    order, so tokens and generator states match bit for bit."""
    torch, hk, lib = env
    print(f"[case] sample exact top_p={top_p} top_k={top_k}", flush=True)
    rng = np.random.default_rng(65 + top_k)
    for trial in range(6):
        # positive "probabilities" with a long tail and some exact ties
        p = np.exp(rng.standard_normal(VOCAB) * 2.0).astype(np.float32)
        p[rng.integers(0, VOCAB, 50)] = p[0]
        g = torch.from_numpy(p).cuda()
        seed = int(rng.integers(1, 1 << 62))
        want = orc.sample_token(p, 0.0, top_p, top_k, seed)
        assert _gpu_sample(torch, hk, g, 0.0, top_p, top_k, seed) == want, trial


def _edge_value_lists():
    rng = np.random.default_rng(91)
    f = np.float32
    out = []
    # 2^24, then ones: every later addition lies exactly halfway (round to even)
    out.append(np.concatenate([[2.0 ** 24], np.ones(20000), rng.random(30000)]).astype(f))
    out.append(np.full(40000, 0.5, f))                    # halves: ties while the sum is small
    out.append(np.concatenate([rng.random(20000) * 2.0 ** -140,       # subnormal values,
                               rng.random(20000)]).astype(f))        # then normal ones
    out.append(np.full(60000, 3.0, f))                    # the sum doubles many times
    c = rng.random(50000).astype(f)
    c[::3] = 0.0
    c[40000] = 1e30                                       # zeros, and one huge value late
    out.append(c)
    out.append((rng.integers(0, 8, 50000) * 0.25).astype(f))  # a coarse grid: many ties
    n = rng.random(30000).astype(f) + 0.5
    n[[17, 9000, 29000]] = -2.0                           # negative values amid positive ones
    out.append(n)
    i = rng.random(20000).astype(f)
    i[12345] = np.inf                                     # an infinity
    out.append(i)
    return out


@pytest.mark.parametrize("which", range(8))
@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_sample_exact_sum_edge_values(env, orc, which, top_p):
    """The sums and walks run as an exact integer emulation of the sequential
    fp32 additions over runs of values, with the additions it cannot emulate
    (ties, leaving a binade, negative or non-finite values) done one at a
    time: values built to hit each of those, at temperature 0 (p = the
    values), token and generator state bit for bit."""
    torch, hk, lib = env
    p = _edge_value_lists()[which]
    print(f"[case] edge values {which} top_p={top_p}", flush=True)
    g = torch.from_numpy(p).cuda()
    for seed in (4544772189918439317, 261738794409030371, 3524332833679783468):  # r 0.13, 0.53, 0.92
        want = orc.sample_token(p, 0.0, top_p, 0, seed)
        assert _gpu_sample(torch, hk, g, 0.0, top_p, 0, seed) == want, seed


@pytest.mark.parametrize("temperature,top_p,top_k", [
    (0.7, 0.9, 40), (1.0, 1.0, 0), (0.8, 0.95, 0), (1.2, 1.0, 100), (0.3, 0.5, 0)])
def test_sample_tokens_match(env, orc, temperature, top_p, top_k):
    torch, hk, lib = env
    print(f"[case] sample T={temperature} top_p={top_p} top_k={top_k}", flush=True)
    rng = np.random.default_rng(int(temperature * 100) + top_k)
    for trial in range(8):
        logits = (rng.standard_normal(VOCAB) * 3.0).astype(np.float32)
        g = torch.from_numpy(logits).cuda()
        seed = int(rng.integers(1, 1 << 62))
        want = orc.sample_token(logits, temperature, top_p, top_k, seed)
        assert _gpu_sample(torch, hk, g, temperature, top_p, top_k, seed) == want, trial


def test_sample_fallbacks(env, orc):
    """sum <= 0 (temperature 0, negative logits): the argmax of the logits and
    no draw; small vocabularies; a single logit."""
    torch, hk, lib = env
    neg = -np.abs(np.random.default_rng(66).standard_normal(1000)).astype(np.float32)
    for args in ((0.0, 1.0, 0), (0.0, 0.9, 10), (-1.0, 1.0, 0)):
        want = orc.sample_token(neg, *args, 12345)
        assert _gpu_sample(torch, hk, torch.from_numpy(neg).cuda(), *args, 12345) == want
    for n in (1, 2, 3, 17):
        lg = np.random.default_rng(n).standard_normal(n).astype(np.float32)
        for args in ((1.0, 1.0, 0), (0.5, 0.5, 1), (1.0, 0.9, n)):
            want = orc.sample_token(lg, *args, 777)
            assert _gpu_sample(torch, hk, torch.from_numpy(lg).cuda(), *args, 777) == want


@pytest.mark.parametrize("top_k", [1000, VOCAB - 1])
@pytest.mark.parametrize("top_p", [0.9, 1.0])
def test_sample_temperature0_topk_mixed_signs(env, orc, top_k, top_p):
    """Temperature 0 keeps p = logit: with N(0, 1) logits the k-th largest p
    is negative for top_k = VOCAB - 1, so negative p stay in the compacted
    list and its sums add them one at a time (run.rs:212-245); the sum stays
    positive, so a draw is made.  Token and generator state bit-exact."""
    torch, hk, lib = env
    print(f"[case] sample T=0 top_k={top_k} top_p={top_p}", flush=True)
    rng = np.random.default_rng(top_k + int(top_p * 10))
    for trial in range(3):
        # mean 0.05: a positive total (about 6400 +- 360) over mixed signs
        logits = (rng.standard_normal(VOCAB) + 0.05).astype(np.float32)
        g = torch.from_numpy(logits).cuda()
        seed = int(rng.integers(1, 1 << 62))
        want = orc.sample_token(logits, 0.0, top_p, top_k, seed)
        assert want[1] != seed   # a draw was made
        assert _gpu_sample(torch, hk, g, 0.0, top_p, top_k, seed) == want, trial
