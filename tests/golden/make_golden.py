"""Generate the golden fixtures under tests/golden/ from first principles.

Nothing here runs the reference (it is CUDA + a remote hub loader and cannot
run in this image) or the oracle: every expected value is computed with exact
Python integers and Fractions from the definitions the reference implements
(fp64_emu_cuda/fp64_emu.cu, torch-ext/fp64_emu/__init__.py), so the fixtures
pin both the CPU oracle and the HIP path independently.

    python tests/golden/make_golden.py      # rewrites the *.json / *.npz files

Fixtures:
  tables.json       Garner tables (minv, packed balanced factors, group
                    products, float log2M) per modulus count.
  planner.json      range_bits / plan_config / plan values.
  extract_kat.json  per-element extraction: (x, shift, bits_eff) -> signed
                    scaled integer, residues mod all 20 moduli, hi7, q7.
  crt_kat.json      reconstruction: residues of X (+ correction, shifts) ->
                    correctly rounded double.
  int_gemm.npz      small integer GEMMs with exact int64 products.
"""
import json
import math
import os
import random
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PRIMES = [256, 255, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199,
          197, 193, 191, 181, 179, 173]
GROUPS = 5


def balanced(v, p):
    """Balanced representative in [-(p//2), (p-1)//2]."""
    r = v % p
    return r - p if r > (p - 1) // 2 else r


def tables(P):
    pr = PRIMES[:P]
    minv, mppack = [], [0] * (P * GROUPS)
    for t in range(P):
        Mt = math.prod(pr[:t])
        minv.append(pow(Mt % pr[t], -1, pr[t]))
        for u in range(t):
            f = balanced(math.prod(pr[:u]), pr[t]) & 0xFF
            mppack[t * GROUPS + u // 4] |= f << (8 * (u % 4))
    mppack = [w - (1 << 32) if w >= (1 << 31) else w for w in mppack]   # as int32
    m64 = [math.prod(pr[0:min(7, P)]) if P > 0 else 1, math.prod(pr[7:min(14, P)]) if P > 7 else 1]
    l2 = np.float32(0.0)
    for p in pr:
        l2 = np.float32(l2 + np.float32(math.log2(p)))
    return {"P": P, "minv": minv, "mppack": mppack, "m64": m64, "log2M": float(l2)}


def range_bits_exact(n):
    # log2 of the exact product (one rounding), not the sum of log2s
    return math.log2(math.prod(PRIMES[:n])) - 1.0


def planner():
    rb = {n: range_bits_exact(n) for n in range(1, 21)}

    def plan_config(K):
        need = 2 * 49 + math.ceil(math.log2(max(K, 1))) + 1 - 3.4
        return next((n for n in range(1, 21) if rb[n] >= need), 20)

    def plan(K, bits):
        need = 2 * bits + math.ceil(math.log2(max(K, 1))) + 1
        return next((n for n in range(1, 21) if rb[n] >= need), None)

    Ks = [1, 2, 64, 128, 512, 513, 1024, 4096, 8192, 8193, 16384, 32769, 65536, 131071, 200000]
    return {"range_bits": {str(n): rb[n] for n in rb},
            "plan_config": {str(K): plan_config(K) for K in Ks},
            "plan": {f"{K},{b}": plan(K, b) for K in Ks for b in (53, 50, 44, 40, 32, 20)}}


def rne(fr):
    return round(fr)  # Fraction rounds half to even


def exact_extract(x, shift, be):
    fx = Fraction(x)
    mag = abs(fx) * Fraction(2) ** shift
    Tu = rne(mag)
    neg = math.copysign(1.0, x) < 0
    td = -Tu if neg else Tu
    h8 = rne(Fraction(Tu) * Fraction(2) ** (7 - be))
    r8 = rne(mag * 256) - 256 * Tu
    hs, qs = (-h8, -r8) if neg else (h8, r8)
    clamp = lambda v: max(-127, min(127, v))  # noqa: E731
    return {"x": x.hex(), "shift": shift, "be": be, "td": td,
            "res": [balanced(td, p) for p in PRIMES], "hi": clamp(hs), "q": clamp(qs)}


def extract_kats(rng):
    cases = []
    be = 50
    # zeros, subnormals, smallest normal
    for x in (0.0, -0.0, 5e-324, -5e-324, 2.2250738585072009e-308, 2.2250738585072014e-308):
        for sh in (0, 1074, 1100):
            cases.append((x, sh, be))
    # ties of the scaled integer: (k + 1/2) * 2^-s scaled by 2^s
    for k in (0, 1, 2, 3, 4, 5, 1000, 2**40 + 1):
        for s in (1, 3, 10):
            x = (k + 0.5) * 2.0 ** -s
            cases.append((x, s, be))
            cases.append((-x, s, be))
    # the p = 256 edge: scaled integer congruent to 128 (mod 256)
    for k in (128, 384, -128, -384, 128 + 256 * 12345):
        cases.append((float(k), 0, be))
    # hi7 clamp: scaled max element at 2^be - 1 rounds to 2^7 in hi7
    for e in (53, 50, 40, 16):
        cases.append((2.0 ** e - 1.0, 0, e))
        cases.append((-(2.0 ** e - 1.0), 0, e))
    # q7 clamp: residual of exactly 1/2 scales to 128
    for k in (7, 8):
        cases.append((k + 0.5, 0, be))
    # random values, shifts placing the row max in [2^(be-1), 2^be)
    for _ in range(300):
        be_r = rng.choice([16, 30, 43, 49, 50, 51, 53])
        x = rng.uniform(-1, 1) * 2.0 ** rng.randint(-30, 30)
        e = math.frexp(abs(x))[1] if x != 0 else 0
        sh = (be_r - 1) - (e - 1) - rng.randint(0, 12)
        cases.append((x, sh, be_r))
    # sizing guarantees |x| 2^shift < 2^be; cases outside that contract are dropped
    ok = [(x, s, b) for x, s, b in cases if abs(Fraction(x)) * Fraction(2) ** s < Fraction(2) ** b]
    return [exact_extract(x, s, b) for x, s, b in ok]


def crt_kats(rng):
    out = []
    for P in (7, 13, 14, 15, 20):
        pr = PRIMES[:P]
        M = math.prod(pr)
        half = M // 2
        for _ in range(40):
            kind = rng.random()
            if kind < 0.2:
                X = rng.randint(-2**60, 2**60)
            elif kind < 0.3:
                X = rng.choice([half - 1, -half, 0, 1, -1])
            else:
                X = rng.randint(-half, half - 1)
            X = max(-half, min(half - 1, X))
            be = rng.choice([16, 40, 49, 50, 53])
            cs = be - 15
            corr = rng.randint(-2**32 + 2, 2**32 - 2) if rng.random() < 0.7 else 0   # two int32 planes
            V = X + corr * 2**cs
            if abs(V) >= 2**126:
                continue
            sA, sB = rng.randint(-60, 60), rng.randint(-60, 60)
            val = math.ldexp(float(V), -(sA + sB)) if V != 0 else 0.0
            out.append({"P": P, "res": [balanced(X, p) for p in pr], "X": str(X), "corr": corr,
                        "be": be, "sftA": sA, "sftB": sB, "out": val.hex()})
    return out


def int_gemms(rng_np):
    g = {}
    A = rng_np.integers(-4096, 4097, (48, 96))
    B = rng_np.integers(-4096, 4097, (32, 96))
    g["i4096_A"], g["i4096_B"], g["i4096_C"] = A, B, A @ B.T
    A = rng_np.integers(-2**20, 2**20 + 1, (40, 256))
    B = rng_np.integers(-2**20, 2**20 + 1, (24, 256))
    g["i2p20_A"], g["i2p20_B"], g["i2p20_C"] = A, B, A @ B.T
    # dyadic: integers under per-k power-of-two scales 2^-12 .. 2^0 (test:66-83)
    ek = rng_np.integers(-12, 1, 64)
    Ai = rng_np.integers(-256, 257, (16, 64))
    Bi = rng_np.integers(-256, 257, (12, 64))
    g["dy_A"] = (Ai * (2.0 ** ek)).astype(np.float64)
    g["dy_B"] = (Bi * (2.0 ** ek)).astype(np.float64)
    w = (4 ** (ek + 12)).astype(np.int64)
    g["dy_C"] = ((Ai * w) @ Bi.T).astype(np.float64) * 2.0 ** -24
    return g


def main():
    rng = random.Random(20261201)
    rng_np = np.random.default_rng(20261201)
    with open(os.path.join(HERE, "tables.json"), "w") as f:
        json.dump([tables(P) for P in (1, 2, 7, 8, 13, 14, 15, 20)], f)
    with open(os.path.join(HERE, "planner.json"), "w") as f:
        json.dump(planner(), f)
    with open(os.path.join(HERE, "extract_kat.json"), "w") as f:
        json.dump(extract_kats(rng), f)
    with open(os.path.join(HERE, "crt_kat.json"), "w") as f:
        json.dump(crt_kats(rng), f)
    np.savez_compressed(os.path.join(HERE, "int_gemm.npz"), **int_gemms(rng_np))


if __name__ == "__main__":
    main()
