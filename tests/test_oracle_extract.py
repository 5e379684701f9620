"""CPU tier: the oracle's extraction (integer-only RNE scaling, three-limb
Barrett residues, hi7/q7 correction summaries) and its Barrett reductions,
pinned by exact rational arithmetic and exhaustive modular checks."""
import json
import math
import os
import random

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_rne_shift_exhaustive_small():
    """rne_shr(m, s) == round-half-even(m / 2^s) for all m < 2^12, s in 0..13,
    and the left-shift / zero branches."""
    for s in range(0, 14):
        for m in range(0, 1 << 12):
            assert O.lib().or_rne_shr(m, s) == O.rne_int(O.Fraction(m, 1 << s))
    assert O.lib().or_rne_shr(5, -3) == 40
    assert O.lib().or_rne_shr(5, -64) == 0
    assert O.lib().or_rne_shr((1 << 53) - 1, 64) == 0


def test_extraction_golden_kats():
    cases = json.load(open(os.path.join(GOLD, "extract_kat.json")))
    by_be = {}
    for c in cases:
        by_be.setdefault(c["be"], []).append(c)
    n = 0
    for be, cs in by_be.items():
        x = np.array([float.fromhex(c["x"]) for c in cs])
        sh = np.array([c["shift"] for c in cs], np.int32)
        td, res, hi, q = O.extract_array(x, sh, be, O.PRIMES)
        for i, c in enumerate(cs):
            assert int(td[i]) == c["td"], c
            assert res[i].tolist() == c["res"], c
            assert int(hi[i]) == c["hi"] and int(q[i]) == c["q"], c
            n += 1
    assert n == len(cases) and n > 300


def test_extraction_random_vs_fraction():
    rng = random.Random(7)
    xs, shs, bes = [], [], []
    for _ in range(2000):
        be = rng.choice([16, 33, 49, 50, 53])
        x = rng.uniform(-1, 1) * 2.0 ** rng.randint(-1000, 1000)
        e = math.frexp(abs(x))[1]
        xs.append(x)
        shs.append((be - 1) - (e - 1) - rng.randint(0, 40))
        bes.append(be)
    for be in set(bes):
        idx = [i for i, b in enumerate(bes) if b == be]
        td, res, hi, q = O.extract_array(np.array([xs[i] for i in idx]),
                                         np.array([shs[i] for i in idx], np.int32), be, O.PRIMES)
        for k, i in enumerate(idx):
            tde, h, qq = O.exact_split(xs[i], shs[i], be)
            assert int(td[k]) == tde
            assert int(hi[k]) == h and int(q[k]) == qq
            assert res[k].tolist() == [O.balanced(tde, p) for p in O.PRIMES]


def test_residue_p256_edge_and_balance():
    """p = 256: the balanced range is [-128, 127]; 128 (mod 256) maps to -128."""
    td, res, _, _ = O.extract_array(np.array([128.0, -128.0, 384.0, 127.0, -129.0]), 0, 50,
                                    O.PRIMES[:1])
    assert res[:, 0].tolist() == [-128, -128, -128, 127, 127]


@pytest.mark.parametrize("p", O.PRIMES)
def test_bal8_exhaustive_window(p):
    """The GEMM epilogue's 31-bit Barrett equals the balanced residue on every
    int32 in [-2^20, 2^20] and across the single-launch range |C| <= K 2^14,
    K <= 131071 (the offset floor(2^31/p) p keeps v + offset non-negative
    there)."""
    lim = 131071 * 128 * 128
    v = np.arange(-2 ** 20, 2 ** 20 + 1, dtype=np.int64)
    extremes = np.array([lim, -lim, lim - 1, -lim + 1, lim - 255, -lim + 256], np.int64)
    rng = np.random.default_rng(p)
    v = np.concatenate([v, extremes, rng.integers(-lim, lim + 1, 200000)])
    got = O.bal8_array(v.astype(np.int32), p)
    r = np.mod(v, p)
    exp = np.where(r > p // 2, r - p, r)            # bal8's threshold p/2
    assert np.array_equal(got.astype(np.int64), exp.astype(np.int8).astype(np.int64))


@pytest.mark.parametrize("p", O.PRIMES)
def test_barrett_bal32_garner_range(p):
    """barrett_bal32 with bias p << 21 on the Garner range |y| < 2^27."""
    y = np.arange(-2 ** 18, 2 ** 18 + 1, dtype=np.int64)
    rng = np.random.default_rng(1000 + p)
    y = np.concatenate([y, rng.integers(-2 ** 27 + 1, 2 ** 27, 100000), [2 ** 27 - 1, -2 ** 27 + 1]])
    got = O.barrett_bal32_array(y.astype(np.int32), p)
    r = np.mod(y, p)
    exp = np.where(r > (p - 1) // 2, r - p, r)
    assert np.array_equal(got.astype(np.int64), exp)
