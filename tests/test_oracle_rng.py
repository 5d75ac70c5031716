"""Pins the oracle's Rng (gpt2t.mojo:777-789, a xorshift64* generator) and
its second restatement in llm_mojo_amd/synth.py, which draws every prompt.

* The state step x ^= x >> 12; x ^= x << 25; x ^= x >> 27 is a linear map T
  over GF(2)^64.  Marsaglia's (12, 25, 27) is a full-period triple: T has
  order exactly 2^64 - 1, i.e. T^(2^64 - 1) = I and T^((2^64 - 1) / p) != I
  for each prime p of 2^64 - 1 = 3 * 5 * 17 * 257 * 641 * 65537 * 6700417.
  A wrong shift (the planted triples below) fails that check.
* The oracle's state after every draw equals T applied to the state before
  (read through its ctypes structure), so its step is that map; its output
  is ((state * M) mod 2^64) >> 40 over 2^24 with M the xorshift64*
  multiplier, published in decimal as 2685821657736338717 (Vigna, "An
  experimental exploration of Marsaglia's xorshift generators, scrambled").
* The C oracle and the Python restatement agree over 10^5 draws and several
  seeds; draws lie in [0, 1) on the 2^-24 grid with mean ~1/2.
"""
import numpy as np
import pytest

MASK = (1 << 64) - 1
ORDER = MASK  # 2^64 - 1
PRIMES = [3, 5, 17, 257, 641, 65537, 6700417]
M_PUBLISHED = 2685821657736338717


def step(x, a=12, b=25, c=27):
    x ^= x >> a
    x ^= (x << b) & MASK
    x ^= x >> c
    return x


def as_columns(f):
    """The linear map f as the images of the 64 basis vectors."""
    return [f(1 << i) for i in range(64)]


def apply(cols, v):
    r = 0
    i = 0
    while v:
        if v & 1:
            r ^= cols[i]
        v >>= 1
        i += 1
    return r


def compose(A, B):  # A after B
    return [apply(A, b) for b in B]


def power(cols, n):
    result = [1 << i for i in range(64)]
    base = cols
    while n:
        if n & 1:
            result = compose(base, result)
        base = compose(base, base)
        n >>= 1
    return result


def is_identity(cols):
    return all(c == 1 << i for i, c in enumerate(cols))


def full_period(a, b, c):
    T = as_columns(lambda v: step(v, a, b, c))
    if not is_identity(power(T, ORDER)):
        return False
    return all(not is_identity(power(T, ORDER // p)) for p in PRIMES)


def test_factorization():
    prod = 1
    for p in PRIMES:
        prod *= p
        assert all(p % q for q in range(2, int(p ** 0.5) + 1))
    assert prod == ORDER


def test_shift_triple_has_full_period():
    assert full_period(12, 25, 27)


@pytest.mark.parametrize("triple", [(12, 25, 26), (13, 25, 27), (12, 24, 27)])
def test_planted_wrong_triples_fail(triple):
    assert not full_period(*triple)


def test_oracle_rng_steps_and_output(orc):
    assert 0x2545F4914F6CDD1D == M_PUBLISHED
    for seed in (0, 1, 1337, 2 ** 40 + 3):
        r = orc.Rng(seed)
        state = r.s.state
        assert state == (seed * 0x9E3779B97F4A7C15 + 1) & MASK
        for _ in range(2000):
            u = r.uniform()
            nxt = step(state)
            assert r.s.state == nxt
            assert u == np.float32(((nxt * M_PUBLISHED) & MASK) >> 40) / np.float32(1 << 24)
            state = nxt


def test_oracle_and_synth_rng_agree(orc):
    from llm_mojo_amd import synth

    for seed in (7, 1001, 4004):
        a, b = orc.Rng(seed), synth.Rng(seed)
        draws = np.array([a.uniform() for _ in range(100_000)], np.float32)
        want = np.array([b.uniform() for _ in range(100_000)], np.float32)
        assert np.array_equal(draws, want)
        assert draws.min() >= 0 and draws.max() < 1
        assert np.array_equal(draws * (1 << 24), np.floor(draws * (1 << 24)))
        assert abs(float(draws.mean()) - 0.5) < 0.005
