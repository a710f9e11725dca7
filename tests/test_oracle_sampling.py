"""Pins of the oracle's restatement of the next-token choice (run.rs:203-278):
XorShift64 against Marsaglia's published sequence, the argmax fold against
hand-built cases, and sample_token against draws whose outcome follows from
exact decimal interval bounds, from reductions to the argmax or to floor(r n),
and from an independent numpy float32 restatement (CPU only)."""
import numpy as np

M64 = (1 << 64) - 1


def _xs(x):
    x ^= (x << 13) & M64
    x ^= x >> 7
    x ^= (x << 17) & M64
    return x


def test_xorshift64_marsaglia_sequence(orc):
    # G. Marsaglia, "Xorshift RNGs" (2003): xor64 from 88172645463325252
    st = 88172645463325252
    got = []
    for _ in range(3):
        v, st = orc.xorshift64_next(st)
        got.append(v)
    assert got == [8748534153485358512, 3040900993826735515, 3453997556048239312]
    assert orc.xorshift64_seed(0) == 1 and orc.xorshift64_seed(7) == 7
    r, st2 = orc.xorshift64_next_f32(12345)
    x = _xs(12345)
    assert st2 == x and r == (x >> 40) / 2.0**24


def test_argmax_fold(orc):
    nan = float("nan")
    assert orc.argmax([1.0, 3.0, 3.0, 2.0]) == 2          # last of equal maxima
    assert orc.argmax([nan, 1.0, 0.0]) == 1               # NaN handed over
    assert orc.argmax([1.0, 5.0, nan]) == 2               # a final NaN wins
    assert orc.argmax([1.0, nan, 0.5]) == 2               # argmax after the last NaN
    assert orc.argmax([-0.0, 0.0]) == 1 and orc.argmax([0.0, -0.0]) == 1
    assert orc.argmax([]) == 0


def _state_with_r(lo, hi, seed=1):
    """A state whose first draw r lies in (lo, hi), away from both ends."""
    rng = np.random.default_rng(seed)
    while True:
        s = int(rng.integers(1, 1 << 63))
        x = _xs(s)
        r = (x >> 40) / 2.0**24
        if lo < r < hi:
            return s, r


def test_sample_intervals(orc):
    # temperature 0: p = logits; cumulative shares 0.1, 0.3, 0.6, 1.0
    logits = np.array([0.1, 0.2, 0.3, 0.4], np.float32)
    for lo, hi, want in ((0.0, 0.099, 0), (0.101, 0.299, 1), (0.301, 0.599, 2),
                         (0.601, 0.999, 3)):
        s, _ = _state_with_r(lo, hi)
        tok, st = orc.sample_token(logits, 0.0, 1.0, 0, s)
        assert tok == want and st == _xs(s)


def test_sample_reductions(orc):
    rng = np.random.default_rng(5)
    logits = (rng.standard_normal(1000) * 3).astype(np.float32)
    am = int(np.argmax(logits))
    for seed in range(1, 20):
        assert orc.sample_token(logits, 0.8, 1.0, 1, seed)[0] == am      # top-k 1
        assert orc.sample_token(logits, 0.8, 1e-7, 0, seed)[0] == am     # tiny top-p
    # uniform logits: token = floor(r n) for r away from the boundaries
    n = 8
    for seed in np.random.default_rng(6).integers(1, 1 << 63, size=200).tolist():
        x = _xs(seed)
        r = (x >> 40) / 2.0**24
        if abs(r * n - round(r * n)) < 1e-4:
            continue
        assert orc.sample_token(np.zeros(n, np.float32), 1.0, 1.0, 0, seed)[0] == int(r * n)
    # sum <= 0 (temperature 0, negative logits): the logits' argmax, no draw
    neg = np.array([-3.0, -1.0, -2.0, -1.0], np.float32)
    assert orc.sample_token(neg, 0.0, 1.0, 0, 99) == (3, 99)
    # top-p never crossed: every p zeroed (threshold = f32::MAX) -> argmax of
    # the logits, no draw
    f = np.float32
    found = 0
    for trial in range(2000):
        p = np.random.default_rng(trial).random(7).astype(np.float32)
        tot = f(-0.0)
        for v in p:
            tot = f(tot + v)
        cum = f(0)
        for v in np.sort(p)[::-1]:
            cum = f(cum + f(v / tot))
        tp = np.nextafter(cum, f(2))   # just above the final running sum
        if tp < 1.0:
            found += 1
            want = 6 - int(np.argmax(p[::-1]))
            assert orc.sample_token(p, 0.0, float(tp), 0, 99) == (want, 99)
    assert found > 0


def _np_sample(logits, temperature, top_p, top_k, state):
    """numpy float32 restatement of run.rs:203-251 (small n only)."""
    f = np.float32
    p = logits.astype(np.float32).copy()
    n = p.size
    if temperature > 0:
        inv = f(1.0) / f(temperature)
        p = np.exp((p * inv).astype(np.float32)).astype(np.float32)
    if 0 < top_k < n:
        thr = np.sort(p)[::-1][top_k - 1]
        p[p < thr] = 0
    if top_p < 1.0:
        s = f(-0.0)
        for v in p:
            s = f(s + v)
        if s > 0:
            cum, thr = f(0), f(np.finfo(np.float32).max)
            for v in np.sort(p)[::-1]:
                cum = f(cum + f(v / s))
                if cum > f(top_p):
                    thr = v
                    break
            p[p < thr] = 0
    s = f(-0.0)
    for v in p:
        s = f(s + v)
    if s <= 0:
        return int(n - 1 - np.argmax(logits[::-1])), state
    x = _xs(state)
    r = f((x >> 40) / 2.0**24)
    cum = f(0)
    for i, v in enumerate(p):
        cum = f(cum + f(v / s))
        if r < cum:
            return i, x
    return int(n - 1 - np.argmax(p[::-1])), x


def test_sample_matches_numpy_restatement(orc):
    rng = np.random.default_rng(11)
    for trial in range(40):
        n = int(rng.integers(2, 300))
        logits = (rng.standard_normal(n) * 2).astype(np.float32)
        temperature = [0.0, 0.5, 1.0, 1.3][trial % 4]
        if temperature == 0.0:
            logits = np.abs(logits)
        top_k = [0, 1, 5, n // 2, n][trial % 5]
        top_p = [1.0, 0.9, 0.5, 0.99][trial % 4 if trial % 3 else 0]
        seed = int(rng.integers(1, 1 << 62))
        want = _np_sample(logits, temperature, top_p, top_k, seed)
        assert orc.sample_token(logits, temperature, top_p, top_k, seed) == want, trial
