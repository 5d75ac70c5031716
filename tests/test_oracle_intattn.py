"""Pins the oracle's integer attention (intmath.mojo, int_attention.mojo)
before it checks the GPU kernels.  The reference holds no golden vectors for
it (its tests draw inputs from Mojo's RNG), so the oracle is checked against
what the mathematics fixes and against the reference's own two tests, with
their tolerances:

- exp2_neg: exact powers of two where the fraction is zero, 2^30 at d = 0,
  monotone, and within the polynomial's stated error of 2^30 e^(-d s)
  (intmath.mojo:38-39, 53-65);
- masked_softmax: tests/int_softmax.mojo's sweep against float64 softmax
  (max |p - exact| < 1e-4, KL < 2e-3, padding exactly 0), and its scalar
  spec masked_softmax_ref (intmath.mojo:143-172) on small cases;
- IntAttnKV: the cache codes and Q24 scales against a NumPy quantizer, and
  tests/int_attention_check.mojo's sweep against exact float64 attention on
  the same quantized data (max error < 5e-3 of max |out|).
"""
import math

import numpy as np
import pytest

SCALE = 1.0 / 65536  # scores with 16 fraction bits (int_attention.mojo:55)


def round_away64(x):
    """Mojo's round(), half away from zero (the oracle's default tie rule),
    evaluated exactly in float64."""
    x = np.asarray(x, np.float64)
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


# ----------------------------------------------------------------- exp2_neg

def test_exp_multiplier_scales_the_exponent(orc):
    # ((m - x) * M) >> MB is the base-2 exponent with 16 fraction bits:
    # one unit of score (2^16 at SCALE) is log2(e) in that exponent.
    m = orc.exp_multiplier(SCALE)
    assert abs(m * 65536 / 2 ** 40 - math.log2(math.e)) < 2 ** -23
    assert orc.exp_multiplier(1.0 / 1024) == orc.exp_multiplier(SCALE) * 64 or \
        abs(orc.exp_multiplier(1.0 / 1024) - 64 * orc.exp_multiplier(SCALE)) <= 64


def test_exp2_neg_exact_points(orc):
    # With M = 2^24 the exponent is d itself: integer exponents k (r = 0)
    # give C0 >> k = 2^(30 - k) exactly, and 0 from k = 31 on.
    for k in range(0, 40):
        got = orc.exp2_neg(k << 16, 1 << 24)
        assert got == (2 ** (30 - k) if k < 31 else 0), k
    # the fraction's polynomial ends at 2^29 as r -> 1 (coefficients sum to 2^29)
    assert abs(orc.exp2_neg(65535, 1 << 24) - 2 ** 29) <= 2 ** 29 * 2e-4
    # differences past D_CAP = 2^31 are capped (and underflow to 0 anyway)
    assert orc.exp2_neg(1 << 40, orc.exp_multiplier(SCALE)) == 0


def test_exp2_neg_accuracy_and_monotone(orc):
    mult = orc.exp_multiplier(SCALE)
    d = np.unique(np.concatenate([np.arange(0, 70000, 7), np.geomspace(1, 2 ** 31, 3000).astype(np.int64)]))
    got = np.array([orc.exp2_neg(int(v), mult) for v in d], np.float64)
    want = 2.0 ** 30 * np.exp(-d * SCALE)
    # polynomial relative error 1.4e-4, the exponent's truncation to 16
    # fraction bits (2^-16 ln 2 = 1.06e-5 relative), and the Q30 truncations
    assert np.all(np.abs(got - want) <= want * 1.52e-4 + 4)
    assert np.all(np.diff(got) <= 0)


# ----------------------------------------------------------- masked_softmax

def softmax_ref_scalar(x, mask, n, mult):
    """masked_softmax_ref (intmath.mojo:143-172), the reference's own scalar
    spec, one element at a time in Python integers."""
    FB, MB, C = 16, 24, (1073741824, -742598100, 248207216, -42480028)
    use = [mask is None or mask[i] != -(1 << 31) for i in range(n)]
    vals = [int(x[i]) + (int(mask[i]) if mask is not None else 0) for i in range(n)]
    m = max((v for v, u in zip(vals, use) if u), default=None)
    e = [0] * n
    for i in range(n):
        if use[i]:
            y = (min(m - vals[i], 1 << 31) * mult) >> MB
            q, r = y >> FB, y & ((1 << FB) - 1)
            p = C[3]
            p = ((p * r) >> FB) + C[2]
            p = ((p * r) >> FB) + C[1]
            p = ((p * r) >> FB) + C[0]
            e[i] = 0 if q >= 31 else p >> q
    t = sum(e)
    inv = (1 << 61) // t if t > 0 else 0
    return [(v * inv + (1 << 45)) >> 46 for v in e]


def softmax_cases(seed=11):
    rng = np.random.default_rng(seed)
    for n in [1, 7, 16, 33, 100, 511, 1024]:
        for spread in [1.0, 4.0, 10.0]:
            for use_mask in [False, True]:
                nr = (n + 15) // 16 * 16
                x = (rng.normal(0, spread, nr) / SCALE).astype(np.int64).astype(np.int32)
                mask = None
                if use_mask:
                    mask = (rng.normal(0, 0.5, nr) / SCALE).astype(np.int64).astype(np.int32)
                    masked = (rng.random(nr) < 0.3) & (np.arange(nr) > 0)
                    mask[masked] = -(1 << 31)
                yield n, spread, x, mask


def test_masked_softmax_vs_float64(orc):
    """tests/int_softmax.mojo's sweep and bounds."""
    mult = orc.exp_multiplier(SCALE)
    worst_abs, worst_kl, cases = 0.0, 0.0, 0
    for n, spread, x, mask in softmax_cases():
        p = orc.masked_softmax(x, n, mult, mask)
        assert np.all(p[n:] == 0), "padding must get probability 0"
        live = np.ones(n, bool) if mask is None else mask[:n] != -(1 << 31)
        v = x[:n].astype(np.float64) + (0 if mask is None else mask[:n].astype(np.float64))
        m = v[live].max() * SCALE
        want = np.where(live, np.exp(v * SCALE - m), 0.0)
        want /= want.sum()
        got = p[:n].astype(np.float64) / 32768
        worst_abs = max(worst_abs, np.abs(got - want).max())
        w = want > 0
        kl = np.sum(want[w] * (np.log(want[w]) - np.log(np.maximum(got[w], 0.5 / 32768))))
        worst_kl = max(worst_kl, kl)
        cases += 1
    assert cases == 42
    assert worst_abs < 1e-4 and worst_kl < 2e-3, (worst_abs, worst_kl)


def test_masked_softmax_matches_scalar_spec(orc):
    mult = orc.exp_multiplier(SCALE)
    for n, spread, x, mask in softmax_cases(seed=3):
        if n > 100:
            continue
        got = orc.masked_softmax(x, n, mult, mask)
        assert list(got[:n]) == softmax_ref_scalar(x, mask, n, mult), (n, spread, mask is not None)


def test_masked_exp_total_and_peak(orc):
    mult = orc.exp_multiplier(SCALE)
    rng = np.random.default_rng(1)
    x = (rng.normal(0, 3, 77) / SCALE).astype(np.int32)
    e, t = orc.masked_exp(x, 77, mult)
    assert e[int(np.argmax(x))] == 1 << 30  # the largest is exactly 1.0
    assert t == int(e.astype(np.int64).sum()) and np.all(e[77:] == 0)


# --------------------------------------------------------------- IntAttnKV

NH, HS, MAXT = 12, 64, 1024
C = NH * HS


def quantize_np(x, qmax):
    """Per-head symmetric quantization the way int_attention.mojo:140-168
    (and step 1, 183-197) states it: float32 scale max|x| / qmax (1 when
    zero), codes round(x * (1 / s)) in float32."""
    x = np.asarray(x, np.float32)
    s = np.float32(np.abs(x).max()) / np.float32(qmax)
    s = np.float32(1.0) if s == 0 else s
    codes = round_away64(x * (np.float32(1.0) / s))
    return codes, s


def exact_attention(kf, vf, q, npos):
    """int_attention_check.mojo:54-87: float64 attention over the same
    quantized keys, values and query, for one head."""
    qi, sq = quantize_np(q, 32767)
    sc = np.empty(npos)
    vdq = np.empty((npos, HS))
    for s in range(npos):
        ki, sk = quantize_np(kf[s], 127)
        sc[s] = float(qi @ ki) * float(sq) * float(sk) / math.sqrt(HS)
        vi, sv = quantize_np(vf[s], 127)
        vdq[s] = vi * float(sv)
    p = np.exp(sc - sc.max())
    return (p / p.sum()) @ vdq


def test_ikv_store_codes_and_scales(orc):
    rng = np.random.default_rng(2)
    kv = orc.IntAttnKV(2, 32, NH, HS)
    k = rng.normal(0, 2.0, C).astype(np.float32)
    v = rng.normal(0, 1.0, C).astype(np.float32)
    k[HS:2 * HS] = 0  # an all-zero head: scale 1
    kv.store(1, 5, k, v)
    for h in range(NH):
        sl = (1 * 32 + 5) * NH + h
        for src, codes, q in ((k, kv.k, kv.kq), (v, kv.v, kv.vq)):
            want, s = quantize_np(src[h * HS:(h + 1) * HS], 127)
            assert np.array_equal(codes[sl * HS:(sl + 1) * HS], want.astype(np.int8))
            assert q[sl] == int(round_away64(float(s) * 2 ** 24))
    assert kv.kq[(32 + 5) * NH + 1] == 1 << 24


@pytest.mark.parametrize("spread", [0.5, 2.0])
def test_ikv_attend_vs_exact(orc, spread):
    """tests/int_attention_check.mojo: cases and the 5e-3 bound."""
    rng = np.random.default_rng(5 if spread == 0.5 else 6)
    worst = 0.0
    for npos0, T in [(0, 1), (0, 5), (15, 1), (16, 1), (99, 1), (200, 7), (511, 1), (1000, 3)]:
        n = npos0 + T
        kv = orc.IntAttnKV(1, MAXT, NH, HS)
        kf = rng.normal(0, spread, (n, C)).astype(np.float32)
        vf = rng.normal(0, 1, (n, C)).astype(np.float32)
        for pos in range(n):
            kv.store(0, pos, kf[pos], vf[pos])
        qkv = rng.normal(0, spread, (T, 3 * C)).astype(np.float32)
        out = kv.attend(qkv, 0, T, npos0)
        err, big = 0.0, 0.0
        for t in range(T):
            npos = npos0 + t + 1
            for h in range(NH):
                sl = slice(h * HS, (h + 1) * HS)
                want = exact_attention(kf[:npos, sl], vf[:npos, sl], qkv[t, sl], npos)
                err = max(err, np.abs(out[t, sl] - want).max())
                big = max(big, np.abs(want).max())
        worst = max(worst, err / big)
    assert worst < 5e-3, worst


def test_ikv_attend_layers_are_separate(orc):
    # attention reads only its own layer's slots: a second layer filled with
    # other data leaves layer 0's output unchanged
    rng = np.random.default_rng(9)
    a = orc.IntAttnKV(2, 32, NH, HS)
    b = orc.IntAttnKV(2, 32, NH, HS)
    for pos in range(20):
        k, v = rng.normal(0, 1, C), rng.normal(0, 1, C)
        a.store(0, pos, k, v)
        b.store(0, pos, k, v)
        b.store(1, pos, rng.normal(0, 1, C), rng.normal(0, 1, C))
    qkv = rng.normal(0, 1, (4, 3 * C)).astype(np.float32)
    assert np.array_equal(a.attend(qkv, 0, 4, 16), b.attend(qkv, 0, 4, 16))
