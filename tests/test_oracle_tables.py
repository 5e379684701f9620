"""CPU tier: the oracle's modulus tables and the planner, pinned by golden
fixtures computed from exact big-integer definitions (tests/golden/) and by
invariants (modular inverses, CRT round trip)."""
import json
import math
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def test_moduli_pairwise_coprime():
    P = O.PRIMES
    assert len(P) == 20 and max(P) == 256 and P == sorted(P, reverse=True)
    for i in range(20):
        for j in range(i):
            assert math.gcd(P[i], P[j]) == 1
    composites = [p for p in P if any(p % d == 0 for d in range(2, int(p ** 0.5) + 1))]
    assert composites == [256, 255, 253, 247, 217]


@pytest.mark.parametrize("entry", _load("tables.json"), ids=lambda e: f"P{e['P']}")
def test_tables_match_golden(entry):
    P = entry["P"]
    minv, mppack, m64, l2 = O.tables(O.PRIMES[:P])
    assert minv.tolist() == entry["minv"]
    assert mppack.tolist() == entry["mppack"]
    assert m64.tolist() == entry["m64"]
    assert np.float32(l2) == np.float32(entry["log2M"])


@pytest.mark.parametrize("P", [1, 5, 13, 14, 15, 20])
def test_tables_invariants(P):
    pr = O.PRIMES[:P]
    minv, mppack, m64, _ = O.tables(pr)
    for t in range(P):
        Mt = math.prod(pr[:t])
        assert (Mt * int(minv[t])) % pr[t] == 1 % pr[t]
        for u in range(4 * O.GROUPS):
            word = int(mppack[t * O.GROUPS + u // 4]) & 0xFFFFFFFF
            byte = (word >> (8 * (u % 4))) & 0xFF
            f = byte - 256 if byte >= 128 else byte
            if u < t:
                assert (f - math.prod(pr[:u])) % pr[t] == 0
                assert -(pr[t] // 2) <= f <= (pr[t] - 1) // 2
            else:
                assert f == 0
    assert m64[0] == math.prod(pr[:min(P, 7)])
    assert m64[0] < 2 ** 57 and m64[1] < 2 ** 57


def test_planner_matches_golden_and_survey_appendix():
    g = _load("planner.json")
    for n, v in g["range_bits"].items():
        assert abs(O.range_bits(int(n)) - v) < 1e-9
    # independent table of range_bits (survey appendix, 2 decimals)
    appendix = {12: 93.80, 13: 101.53, 14: 109.16, 15: 116.78, 16: 124.38, 17: 131.95,
                18: 139.45, 19: 146.94, 20: 154.37}
    for n, v in appendix.items():
        assert abs(O.range_bits(n) - v) < 0.011
    for K, n in g["plan_config"].items():
        assert O.plan_config(int(K)) == (n, True)
    for key, n in g["plan"].items():
        K, b = map(int, key.split(","))
        if n is None:
            with pytest.raises(ValueError):
                O.plan(K, b)
        else:
            assert O.plan(K, b) == n
    # closed-form statements of the survey appendix
    assert all(O.plan_config(K)[0] == 14 for K in (64, 256, 1024, 4096, 8192))
    assert all(O.plan_config(K)[0] == 15 for K in (16384, 32769, 131071, 200000))
    assert O.plan(512, 53) == 15 and O.plan(1024, 53) == 16 and O.plan(131071, 53) == 16
    assert O.plan(200000, 53) == 17


def test_package_planner_is_the_reference_planner():
    """The product's pure-Python planner (fp64_emu.plan_config/plan/range_bits)
    against the golden values; importing the package needs only the built
    extension, no GPU."""
    fp64_emu = pytest.importorskip("fp64_emu")
    g = _load("planner.json")
    for n, v in g["range_bits"].items():
        assert abs(fp64_emu.range_bits(int(n)) - v) < 1e-9
    for K, n in g["plan_config"].items():
        assert fp64_emu.plan_config(int(K)) == (n, True)
    for key, n in g["plan"].items():
        K, b = map(int, key.split(","))
        if n is not None:
            assert fp64_emu.plan(K, b) == n
    assert fp64_emu._PRIMES == O.PRIMES


@pytest.mark.parametrize("P", [7, 14, 20])
def test_crt_round_trip(P):
    """Residues of random integers in the balanced range (capped at 2^125,
    the pipeline's usable range) reconstruct to the integer (exact path, no
    correction, zero shifts): float(X) exactly."""
    rng = np.random.default_rng(P)
    pr = O.PRIMES[:P]
    M = math.prod(pr)
    xs = [int(v) for v in rng.integers(-2 ** 62, 2 ** 62, 30)]
    xs += [M // 2 - 1, -(M // 2), 0, 1, -1, 2 ** 53 + 1]
    lim = min(M // 2, 2 ** 125)
    xs += [lim - 1, -lim]
    xs = [x for x in xs if -lim <= x < lim]
    res = np.array([[O.balanced(x, p) for x in xs] for p in pr], np.int8).reshape(P, 1, len(xs))
    out = O.reconstruct(res, None, None, pr, 53, np.zeros(1, np.int16), np.zeros(len(xs), np.int16))
    assert out.ravel().tolist() == [float(x) for x in xs]
