"""CPU tier: the oracle's modular GEMM, reconstruction and whole pipeline.

Pins: numpy int64 products; big-integer CRT with correctly rounded
conversion (crt_kat.json); exact integer GEMMs (the reference test suite's
integer KATs re-expressed with CPU seeds, int_gemm.npz); the double-double
oracle against exact rationals; the Prop. 3.3 accuracy bound with exact
Fractions; correct-bit floors against native float64.
"""
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("p", [256, 253, 173, 0])
def test_modgemm_vs_numpy(p):
    rng = np.random.default_rng(p + 1)
    A = rng.integers(-128, 128, (37, 300)).astype(np.int8)
    B = rng.integers(-128, 128, (29, 300)).astype(np.int8)
    C = A.astype(np.int64) @ B.astype(np.int64).T
    got = O.modgemm(A, B, p)
    if p == 0:
        assert np.array_equal(got, C)
    else:
        r = np.mod(C, p)
        exp = np.where(r > p // 2, r - p, r).astype(np.int8)
        assert np.array_equal(got, exp)


def test_modgemm_overflow_detected():
    A = np.full((1, 131072), -128, np.int8)
    with pytest.raises(OverflowError):
        O.modgemm(A, A, 0)
    O.modgemm(A[:, :131071], A[:, :131071], 0)   # the single-launch bound holds


def test_reconstruct_golden_crt():
    """Residues of X plus a correction split over two int32 planes (as the
    two cross GEMMs deliver it) reconstruct to RN(X + corr 2^(be-15)) rescaled
    by 2^-(sftA+sftB) (crt_kat.json, exact big-integer ground truth)."""
    cases = json.load(open(os.path.join(GOLD, "crt_kat.json")))
    assert len(cases) > 150
    for c in cases:
        P = c["P"]
        res = np.array(c["res"], np.int8).reshape(P, 1, 1)
        c1 = c["corr"] // 2
        c2 = c["corr"] - c1
        out = O.reconstruct(res, np.array([[c1]], np.int32), np.array([[c2]], np.int32),
                            O.PRIMES[:P], c["be"], np.array([c["sftA"]], np.int16),
                            np.array([c["sftB"]], np.int16))
        assert out[0, 0] == float.fromhex(c["out"]), c


def test_i128_to_double_correct_rounding():
    vals = [0, 1, -1, 2 ** 53 + 1, 2 ** 60 + 2 ** 7, 2 ** 60 + 2 ** 7 + 1, 2 ** 60 + 3 * 2 ** 7,
            -(2 ** 100) - 1, 2 ** 126 - 1, -(2 ** 126) + 1, (2 ** 64 + 1) * 2 ** 40]
    rng = np.random.default_rng(3)
    for _ in range(2000):
        b = int(rng.integers(1, 126))
        vals.append(int(rng.integers(0, 2 ** 62)) << max(0, b - 62) | int(rng.integers(0, 2 ** 20)))
        vals.append(-vals[-1])
    got = O.i128_to_double(vals)
    assert got.tolist() == [float(v) for v in vals]   # Python int -> float rounds half-even


def _int_case(name):
    g = np.load(os.path.join(GOLD, "int_gemm.npz"))
    return g[name + "_A"], g[name + "_B"], g[name + "_C"]


def test_integer_exact_nprimes20():
    """test_fp64_emu.py:28-36 re-expressed: integers in [-4096, 4096], exact."""
    A, B, C = _int_case("i4096")
    out, _ = O.mm(A.astype(np.float64), B.astype(np.float64), 0, O.PRIMES[:20])
    assert np.array_equal(out, C.astype(np.float64))


def test_integer_exact_default_plan_2p20():
    """c3b in small: integers in [-2^20, 2^20] at the default plan are exact and
    both correction products vanish."""
    A, B, C = _int_case("i2p20")
    P, corr = O.plan_config(A.shape[1])
    out, info = O.mm(A.astype(np.float64), B.astype(np.float64), 0, O.PRIMES[:P], use_corr=corr)
    assert np.array_equal(out, C.astype(np.float64))
    _, hi, q = O.extract_operand(A.astype(np.float64), 0, info["sftA"], info["bits_eff"], O.PRIMES[:P])
    assert not q.any()


def test_dyadic_dynamic_range_exact():
    """test_fp64_emu.py:66-83 re-expressed: integers under per-k scales."""
    A, B, C = _int_case("dy")
    out, _ = O.mm(A, B, 0, O.PRIMES[:14])
    assert np.array_equal(out, C)


def test_all_ones_range_rule():
    """test_fp64_emu.py:53-63: all-ones K=2048 reconstructs exactly at defaults."""
    A = np.ones((64, 2048))
    Bt = np.ones((2048, 48))
    P, c = O.plan_config(2048)
    out, info = O.mm(A, Bt, 1, O.PRIMES[:P], use_corr=c)
    assert np.all(out == 2048.0)


def test_bmm_integer_exact():
    rng = np.random.default_rng(6)
    A = rng.integers(-4096, 4097, (3, 20, 64))
    B = rng.integers(-4096, 4097, (3, 12, 64))
    out, _ = O.mm(A.astype(np.float64), B.astype(np.float64), 0, O.PRIMES[:20])
    exp = np.stack([A[b] @ B[b].T for b in range(3)]).astype(np.float64)
    assert np.array_equal(out, exp)


def test_mm_nt_equals_mm_layouts():
    """The [K, N] and [N, K] layouts of B give the same output when the sizing
    decision agrees (it does here: the column sums are far from a width
    boundary)."""
    rng = np.random.default_rng(11)
    A = rng.standard_normal((33, 200))
    B = rng.standard_normal((41, 200))
    o1, i1 = O.mm(A, B, 0, O.PRIMES[:14])
    o2, i2 = O.mm(A, np.ascontiguousarray(B.T), 1, O.PRIMES[:14])
    assert i1["bits_eff"] == i2["bits_eff"]
    assert np.array_equal(o1, o2)


def _frac_matmul_nt(A, Bt):
    M, K = A.shape
    N = Bt.shape[1]
    return [[sum(Fraction(A[i, k]) * Fraction(Bt[k, j]) for k in range(K)) for j in range(N)]
            for i in range(M)]


@pytest.mark.parametrize("dist", ["wide8", "illcond40"])
def test_dd_oracle_vs_exact_rationals(dist):
    """bench/accuracy.py:124-132: the double-double reference within ~2^-100
    of the exact rational product on 8x128x8."""
    rng = np.random.default_rng(7)
    A = rng.standard_normal((8, 128))
    Bt = rng.standard_normal((128, 8))
    if dist == "wide8":
        A *= 2.0 ** rng.integers(-8, 9, A.shape)
        Bt *= 2.0 ** rng.integers(-8, 9, Bt.shape)
    else:
        s = 2.0 ** (-40 * rng.random(128))
        A *= s[None, :]
        Bt *= s[:, None]
    hi, lo = O.ddgemm_nt(A, Bt)
    ex = _frac_matmul_nt(A, Bt)
    worst = max(abs(ex[i][j] - (Fraction(hi[i, j]) + Fraction(lo[i, j])))
                for i in range(8) for j in range(8))
    scale = max(abs(ex[i][j]) for i in range(8) for j in range(8))
    assert worst / scale < Fraction(1, 2 ** 95)


def test_c1_plumbing_accuracy():
    """Config c1 (128x128x4096 randn, default plan) through the oracle: correct
    bits against the dd reference at least native float64's, >= 52."""
    rng = np.random.default_rng(1000)
    A = rng.standard_normal((128, 4096))
    Bt = rng.standard_normal((4096, 128))
    P, c = O.plan_config(4096)
    assert (P, c) == (14, True)
    out, info = O.mm(A, Bt, 1, O.PRIMES[:P], use_corr=c)
    hi, lo = O.ddgemm_nt(A, Bt)
    emu = O.correct_bits(out, hi, lo)
    nat = O.correct_bits(A @ Bt, hi, lo)
    assert emu >= nat and emu >= 52.0, (emu, nat)
    assert info["bits_eff"] == 50
    red, _ = O.mm(A, Bt, 1, O.PRIMES[:13], use_corr=False)
    assert 42.0 <= O.correct_bits(red, hi, lo) < emu


def test_prop33_error_bound_exact():
    """Prop. 3.3 (paper): |V - S| <= K (3 2^(be-7) + 9/2 2^(be-15) + 1/4) in
    the scaled integer domain, checked with exact Fractions; the output is
    V rounded once and rescaled."""
    rng = np.random.default_rng(5)
    M, K, N = 6, 96, 5
    A = rng.standard_normal((M, K)) * 2.0 ** rng.integers(-6, 7, (M, K))
    B = rng.standard_normal((N, K))
    P = 14
    out, info = O.mm(A, B, 0, O.PRIMES[:P])
    be, sA, sB = info["bits_eff"], info["sftA"], info["sftB"]
    bound = K * (3 * Fraction(2) ** (be - 7) + Fraction(9, 2) * Fraction(2) ** (be - 15) + Fraction(1, 4))
    for i in range(M):
        for j in range(N):
            S = sum(Fraction(A[i, k]) * Fraction(B[j, k]) for k in range(K)) * Fraction(2) ** (int(sA[i]) + int(sB[j]))
            V = Fraction(out[i, j]) * Fraction(2) ** (int(sA[i]) + int(sB[j]))
            ulp = Fraction(2) ** (math.frexp(float(V))[1] - 53) if V != 0 else Fraction(0)
            assert abs(V - S) <= bound + ulp


def test_bits_sweep_degrades_gracefully():
    """bench/accuracy.py:143-151: narrower operand widths with their planned
    modulus counts lose accuracy monotonically-ish but stay near the width."""
    rng = np.random.default_rng(9)
    A = rng.standard_normal((32, 512))
    Bt = rng.standard_normal((512, 32))
    hi, lo = O.ddgemm_nt(A, Bt)
    prev = 60.0
    for b in (53, 44, 36, 28):
        out, info = O.mm(A, Bt, 1, O.PRIMES[:O.plan(512, b)], bits=b)
        cb = O.correct_bits(out, hi, lo)
        assert cb <= prev + 1.0 and cb >= b - 6, (b, cb)
        prev = cb


def test_inexact_recombine_close_to_exact():
    rng = np.random.default_rng(12)
    A = rng.standard_normal((40, 700))
    B = rng.standard_normal((30, 700))
    o1, _ = O.mm(A, B, 0, O.PRIMES[:14], exact=True)
    o2, _ = O.mm(A, B, 0, O.PRIMES[:14], exact=False)
    hi, lo = O.ddgemm_nt(A, np.ascontiguousarray(B.T))
    assert O.correct_bits(o2, hi, lo) >= 50.0
    assert np.max(np.abs(o1 - o2) / np.abs(hi).max()) < 2.0 ** -50


def test_segment_fold_is_the_balanced_residue():
    """The fold of K-segmented residue sums (barrett_bal32, bias
    p ceil((p/2)^2/p)) equals the balanced residue of the sum over the
    reachable range of up to 86 segments, for every modulus."""
    for p in O.PRIMES:
        lim = 86 * (p // 2)
        for acc in list(range(-lim, lim + 1, 7)) + [-lim, lim, 0, 1, -1]:
            assert O.fold_residue(acc, p) == O.balanced(acc, p), (p, acc)


def test_deep_k_integer_bitexact():
    """test_fp64_emu.py:122-131 re-expressed: K = 200000 entries in {-1,0,1}
    through the K-segmented path (4 segments), exact."""
    rng = np.random.default_rng(16)
    K = 200_000
    A = rng.integers(-1, 2, (12, K))
    B = rng.integers(-1, 2, (8, K))
    P, corr = O.plan_config(K)
    out, _ = O.mm(A.astype(np.float64), B.astype(np.float64), 0, O.PRIMES[:P], use_corr=corr)
    assert np.array_equal(out, (A @ B.T).astype(np.float64))


def test_deep_k_segmentation_is_transparent():
    """Segmented residues and int64 correction sums equal the single-pass
    values computed with int64 products (numpy): the K-segmented output is
    the full-depth CRT value."""
    rng = np.random.default_rng(17)
    K = 140_000
    A = rng.standard_normal((6, K))
    B = rng.standard_normal((5, K))
    P = 15
    pr = O.PRIMES[:P]
    out, info = O.mm(A, B, 0, pr)
    be = info["bits_eff"]
    rA, hA, qA = O.extract_operand(A[None], 0, info["sftA"], be, pr)
    rB, hB, qB = O.extract_operand(B[None], 0, info["sftB"], be, pr)
    res = np.zeros((P, 6, 5), np.int8)
    for t, p in enumerate(pr):
        full = rA[0, t].astype(np.int64) @ rB[0, t].astype(np.int64).T
        r = np.mod(full, p)
        res[t] = np.where(r > (p - 1) // 2, r - p, r)
    d1 = hA[0].astype(np.int64) @ qB[0].astype(np.int64).T
    d2 = qA[0].astype(np.int64) @ hB[0].astype(np.int64).T
    rec = O.reconstruct64(res, d1, d2, pr, be, info["sftA"], info["sftB"])
    assert np.array_equal(out.view(np.uint64), rec.view(np.uint64))


def test_int_gemm_is_exact_at_the_extremes():
    """int_gemm stays exact at the largest sums: every entry
    -128 over the deepest single launch (sum 131071 * 2^14 < 2^31), against
    numpy int64 products, and random planes against or_modgemm's int32."""
    A = np.full((3, 131071), -128, np.int8)
    assert np.array_equal(O.int_gemm(A, A), np.full((3, 3), 131071 * 16384, np.int64))
    rng = np.random.default_rng(5)
    A = rng.integers(-128, 128, (41, 5000)).astype(np.int8)
    B = rng.integers(-128, 128, (33, 5000)).astype(np.int8)
    assert np.array_equal(O.int_gemm(A, B), A.astype(np.int64) @ B.astype(np.int64).T)
    assert np.array_equal(O.int_gemm(A, B).astype(np.int32), O.modgemm(A, B, 0))


@pytest.mark.parametrize("kind,shape,P,corr,exact", [
    ("mm_nt", (1, 130, 70, 1500), 14, True, True),
    ("mm", (1, 257, 129, 2049), 15, True, False),
    ("bmm_nt", (3, 33, 65, 700), 13, False, True),
    ("bmm", (2, 64, 31, 1025), 20, True, True),
])
def test_mm_blas_matches_mm(kind, shape, P, corr, exact):
    """The whole-output checker of the full-size GPU configs (BLAS modular
    products) is bit-identical to the oracle's pipeline on ragged, batched,
    reduced and inexact cases, with rows spanning 2^-30 .. 2^30."""
    batch, M, N, K = shape
    rng = np.random.default_rng(M * N + K)
    A = rng.standard_normal((batch, M, K)) * np.exp2(rng.integers(-30, 31, (batch, M, 1)))
    b_kn = kind.endswith("_nt")
    B = rng.standard_normal((batch, K, N) if b_kn else (batch, N, K))
    if kind in ("mm", "mm_nt"):
        A, B = A[0], B[0]
    primes = O.PRIMES[:P]
    ref, info = O.mm(A, B, int(b_kn), primes, exact=exact, use_corr=corr)
    got, info2 = O.mm_blas(A, B, int(b_kn), primes, exact=exact, use_corr=corr)
    assert info["bits_eff"] == info2["bits_eff"]
    assert np.array_equal(ref.view(np.uint64), got.view(np.uint64))
