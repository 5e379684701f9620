"""CPU tier: the integer identities the default-list reconstruction kernel
rests on, checked against exact big-integer arithmetic.

- Mixed radix: the balanced digits of X (the reference's Garner digits,
  fp64_emu_cuda/fp64_emu.cu:849-952) equal the digits of X + M/2 in [0, p)
  minus p >> 1, because M/2 = sum_t (p_t >> 1) W_t for the default list
  (256, then odd moduli); X + M/2 has X's residues except r_0 + 128.
- Per group of seven digits, the balanced group value is the unsigned one
  minus the group's digit offset (the kernel's default_digit_offset).
- floor(y / p) = mulhi(y, ceil(2^32 / p)) for every y < 2^24, and the Garner
  accumulator y = 128 p_t + r_t minv_t + sum d_u f_u stays in [0, 2^21).
- The 128-bit conversion's redundant-sign-bit count k (leading zeros of
  ((hi ^ s) << 1) | ((lo ^ s) >> 63), capped at 64) and its shifted window
  with the sticky tail round to the same double as the exact value.
"""
import math
import random
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

P_ALL = O.PRIMES


def _balanced_digits(X, primes):
    """Balanced mixed-radix digits of X in [-M/2, M/2) by exact division."""
    d = []
    W = 1
    rem = X
    for p in primes:
        r = rem % p
        if r > (p - 1) // 2 if p % 2 else r >= p // 2:
            r -= p
        d.append(r)
        rem = (rem - r) // p
        W *= p
    assert rem == 0
    return d


def _unsigned_digits(Y, primes):
    d = []
    for p in primes:
        d.append(Y % p)
        Y //= p
    assert Y == 0
    return d


@pytest.mark.parametrize("P", [1, 2, 7, 8, 13, 14, 15, 16, 20])
def test_balanced_digits_are_shifted_unsigned_digits(P):
    primes = P_ALL[:P]
    M = math.prod(primes)
    assert sum((p >> 1) * math.prod(primes[:t]) for t, p in enumerate(primes)) == M // 2
    rng = random.Random(P)
    for X in [-(M // 2), M // 2 - 1, 0, -1, 1] + [rng.randrange(-(M // 2), M // 2) for _ in range(300)]:
        bal = _balanced_digits(X, primes)
        uns = _unsigned_digits(X + M // 2, primes)
        assert bal == [u - (p >> 1) for u, p in zip(uns, primes)]
        # X + M/2 keeps X's residues except r_0 + 128 (mod 256).
        for t, p in enumerate(primes):
            assert (X + M // 2) % p == (X + (128 if t == 0 else 0)) % p


@pytest.mark.parametrize("P", [1, 3, 7, 9, 14, 15, 20])
def test_group_offsets(P):
    primes = P_ALL[:P]
    rng = random.Random(100 + P)
    for _ in range(200):
        M = math.prod(primes)
        X = rng.randrange(-(M // 2), M // 2)
        bal = _balanced_digits(X, primes)
        uns = _unsigned_digits(X + M // 2, primes)
        for g in range((P + 6) // 7):
            ts = range(7 * g, min(7 * g + 7, P))
            w = 1
            vb = vu = off = 0
            for t in ts:
                vb += bal[t] * w
                vu += uns[t] * w
                off += (primes[t] >> 1) * w
                w *= primes[t]
            assert vb == vu - off
            # The kernel's halves: positions 3..6 (H) below 2^32 unsigned,
            # positions 0..2 (L) below 2^24, partial H below 2^24.
            lo = [t for t in ts if t - 7 * g < 3]
            hi = [t for t in ts if t - 7 * g >= 3]
            assert math.prod(primes[t] for t in lo) < 2 ** 24
            assert math.prod(primes[t] for t in hi) < 2 ** 32
            assert math.prod(primes[t] for t in hi[1:]) < 2 ** 24


def test_high_multiply_quotient():
    y = np.arange(1 << 24, dtype=np.uint64)
    for p in P_ALL[1:]:
        mq = ((1 << 32) + p - 1) // p
        assert np.array_equal((y * np.uint64(mq)) >> np.uint64(32), y // np.uint64(p)), p


def test_garner_accumulator_range():
    """y = 128 p + r minv + sum_u d_u f_u with r, minv balanced bytes and
    d_u, f_u in [0, 255]: positive and below 2^21 for every digit position."""
    minv, _, _, _ = O.tables(P_ALL)
    for t in range(1, 20):
        p = P_ALL[t]
        mi = int(minv[t])
        mib = mi - p if 2 * mi > p else mi
        assert abs(mib) <= 127
        lo = 128 * p - 127 * abs(mib)
        hi = 128 * p + 127 * abs(mib) + t * 255 * (p - 1)
        assert lo > 0 and hi < 2 ** 21


def _convert(hi, lo):
    """The kernel's branchless round-to-odd conversion of hi:lo (k >= 1)."""
    M64 = (1 << 64) - 1
    s = M64 if hi < 0 else 0
    hu = hi & M64
    V = ((((hu ^ s) << 1) & M64) | (((lo ^ s) >> 63) & 1))
    k = 64 if V == 0 else 64 - V.bit_length()
    assert k >= 1
    kk = min(k, 63)
    dropped = (lo << kk) & M64
    top = (((hu << kk) & M64) | (lo >> (64 - k))) | (1 if dropped else 0)
    if top >= 1 << 63:
        top -= 1 << 64
    return float(top) * 2.0 ** (64 - k)   # int -> float rounds to nearest even


def test_branchless_conversion_matches_exact_rounding():
    rng = random.Random(7)
    vals = [0, 1, -1, 5, -5, 2 ** 53 + 1, -(2 ** 53 + 1), 2 ** 55 + 3, 2 ** 63 - 1, -(2 ** 63),
            2 ** 63, -(2 ** 63) - 1, 2 ** 64 + 1, 2 ** 125 - 1, -(2 ** 125) + 7, 2 ** 126 - 1, -(2 ** 126)]
    for bits in range(1, 127):
        for _ in range(20):
            v = rng.getrandbits(bits) | (1 << (bits - 1))
            vals.append(v if rng.random() < 0.5 else -v)
            # ties and near-ties at the double's rounding position
            if bits > 54:
                base = (v >> (bits - 54)) << (bits - 54)
                vals += [base + (1 << (bits - 55)), base + (1 << (bits - 55)) - 1]
    for X in vals:
        hi, lo = X >> 64, X & ((1 << 64) - 1)
        assert _convert(hi, lo) == float(Fraction(X)), X


def _fastdiv(d):
    """make_fastdiv (fp64emu.hip): l = ceil(log2 d), m = floor(2^32 (2^l - d)
    / d) + 1, as 32-bit words."""
    d = max(int(d), 1)
    l = 0
    while (1 << l) < d:
        l += 1
    m = ((1 << 32) * ((1 << l) - d)) // d + 1
    assert 0 < m < (1 << 32) or d == 1
    return np.uint64(m & 0xFFFFFFFF), np.uint64(l)


def _fastdiv_q(m, l, n):
    """FastDiv::div in 32-bit words: (mulhi(m, n) + n) >> l, the add wrapping
    like the kernel's uint32 arithmetic."""
    s = (((m * n) >> np.uint64(32)) + n) & np.uint64(0xFFFFFFFF)
    return s >> l


def test_fastdiv_quotients():
    """The round-up Granlund-Montgomery division that maps work-group indices
    to (member, row group, k tile) and output blocks: q == n // d for every
    divisor 1 .. 2^16 on sampled indices in [0, 2^24) (the 32-bit work-item
    bound of a 256-thread launch) with each divisor's edge values, every
    index below 2^24 for a few divisors, and random divisors up to 2^31 with
    indices up to 2^31 - 1 (the range the kernel's sum stays below 2^32)."""
    rng = np.random.default_rng(2024)
    top = np.uint64(1 << 24)
    sample = rng.integers(0, 1 << 24, 2048, dtype=np.uint64)
    for d in range(1, (1 << 16) + 1):
        m, l = _fastdiv(d)
        du = np.uint64(d)
        edges = np.array([0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d], dtype=np.uint64)
        last = (top - np.uint64(1)) // du * du
        edges = np.concatenate([edges, [last - np.uint64(1), last, top - np.uint64(1)]])
        n = np.concatenate([sample, edges[edges < top]])
        assert np.array_equal(_fastdiv_q(m, l, n), n // du), d
    n = np.arange(1 << 24, dtype=np.uint64)
    for d in (3, 7, 100, 641, 4095, 65537, 1 << 20, (1 << 24) - 1):
        m, l = _fastdiv(d)
        assert np.array_equal(_fastdiv_q(m, l, n), n // np.uint64(d)), d
    big = rng.integers(0, 1 << 31, 4096, dtype=np.uint64)
    big = np.concatenate([big, np.array([(1 << 31) - 1, (1 << 31) - 2], dtype=np.uint64)])
    for d in np.concatenate([rng.integers(1 << 16, 1 << 31, 512), [(1 << 31) - 1, 1 << 30]]):
        m, l = _fastdiv(int(d))
        assert np.array_equal(_fastdiv_q(m, l, big), big // np.uint64(d)), int(d)
