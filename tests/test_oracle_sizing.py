"""CPU tier: the oracle's Cauchy-Schwarz sizing, pinned by closed forms
(the shift is bits - 1 - ilogb(max|x|), bits - 1 for an all-zero row; the
log2-norm is 0.5 log2(sum x^2) plus the shift), by the row/column duality, and by the invariant it exists
for (Prop. 3.1 of the reference paper, paper/paper.tex:463-499): after the
width pick every scaled dot product lies strictly inside the balanced CRT
range, checked with exact integers on adversarial and random inputs."""
import math

import numpy as np
import pytest

import oracle as O


def _dists(rng, R, K):
    yield "randn", rng.standard_normal((R, K))
    yield "wide", rng.choice([-1, 1], (R, K)) * (1 + rng.random((R, K))) * 2.0 ** rng.integers(-20, 21, (R, K))
    yield "aligned", 1 + 0.001 * rng.standard_normal((R, K))
    A = rng.standard_normal((R, K))
    A[1] = 0.0
    A[2, :] = 0.0
    A[2, 5] = 5e-324        # a subnormal alone in its row
    yield "zeros+subnormal", A


@pytest.mark.parametrize("bits", [53, 40, 16])
def test_size_rows_closed_form(bits):
    rng = np.random.default_rng(bits)
    for name, X in _dists(rng, 12, 300):
        sft, lg = O.size_rows(X, bits)
        for r in range(X.shape[0]):
            m = np.abs(X[r]).max()
            if m == 0:    # ilogb taken as 0 (fp64_emu_cuda/fp64_emu.cu:139-141)
                assert sft[r] == bits - 1 and lg[r] == -np.inf, name
                continue
            e = math.frexp(m)[1] - 1                   # ilogb
            assert sft[r] == bits - 1 - e, name
            s2 = float(np.sum(X[r] ** 2))
            if s2 > 0:
                exp = 0.5 * math.log2(s2) + sft[r]
                assert abs(float(lg[r]) - exp) <= 4e-6 * max(1.0, abs(exp)), name
            else:
                assert lg[r] == np.inf, name           # nonzero max, underflowed square sum


def test_size_cols_is_size_rows_of_the_transpose():
    rng = np.random.default_rng(4)
    for name, X in _dists(rng, 40, 700):
        Bt = np.ascontiguousarray(X.T)                 # [K, N] layout
        s1, l1 = O.size_rows(X, 53)
        s2, l2 = O.size_cols(Bt, 53)
        assert np.array_equal(s1, s2), name
        fin = np.isfinite(l1)
        assert np.array_equal(fin, np.isfinite(l2)) and np.array_equal(l1[~fin], l2[~fin])
        ulp = np.abs(l1[fin].view(np.int32).astype(np.int64) - l2[fin].view(np.int32).astype(np.int64))
        assert ulp.max(initial=0) <= 2, name           # different summation order only


@pytest.mark.parametrize("P", [8, 13, 14, 15, 16, 20])
def test_width_pick_is_range_safe(P):
    """Every |sum_k T_A[i,k] T_B[j,k]| < M/2 after the pick, exactly,
    unless the width is clamped at its floor of 16 bits."""
    rng = np.random.default_rng(100 + P)
    pr = O.PRIMES[:P]
    M = math.prod(pr)
    _, _, _, log2M = O.tables(pr)
    for name, A in _dists(rng, 6, 160):
        B = next(d for n, d in _dists(rng, 5, 160) if n == name)
        sA, lA = O.size_rows(A, 53)
        sB, lB = O.size_rows(B, 53)
        be, sA2, sB2 = O.pick_bits(lA, lB, min(log2M, 126.0), 53, sA, sB)
        assert 16 <= be <= 53
        worst_case = not np.isfinite(np.max(lA) + np.max(lB))
        if worst_case:
            # a square sum underflowed (lg = +inf): no narrowing, be = bits,
            # and only a worst-case modulus count is range-safe
            # (fp64_emu_cuda/fp64_emu.cu:213-216)
            assert be == 53
            if P < O.plan(A.shape[1], 53):
                continue
        TA = [[O.exact_split(float(x), int(sA2[i]), be)[0] for x in A[i]] for i in range(A.shape[0])]
        TB = [[O.exact_split(float(x), int(sB2[j]), be)[0] for x in B[j]] for j in range(B.shape[0])]
        for i in range(len(TA)):
            assert max(abs(t) for t in TA[i]) <= 2 ** be   # scaled row max below 2^be (+ rounding)
            for j in range(len(TB)):
                X = sum(a * b for a, b in zip(TA[i], TB[j]))
                if be > 16:
                    assert abs(X) < M // 2, (name, i, j)


def test_width_examples_from_the_survey_appendix():
    """c1 (128x128x4096 randn, 14 moduli) sizes to be = 50; integers in
    [-2^20, 2^20] at K=4096 to be = 49 (independent appendix values)."""
    rng = np.random.default_rng(1000)
    A = rng.standard_normal((128, 4096))
    Bt = rng.standard_normal((4096, 128))
    _, _, _, log2M = O.tables(O.PRIMES[:14])
    sA, lA = O.size_rows(A, 53)
    sB, lB = O.size_cols(Bt, 53)
    assert O.pick_bits(lA, lB, min(log2M, 126.0), 53, sA, sB)[0] == 50
    Ai = rng.integers(-2 ** 20, 2 ** 20 + 1, (64, 4096)).astype(np.float64)
    Bi = rng.integers(-2 ** 20, 2 ** 20 + 1, (64, 4096)).astype(np.float64)
    sA, lA = O.size_rows(Ai, 53)
    sB, lB = O.size_rows(Bi, 53)
    assert O.pick_bits(lA, lB, min(log2M, 126.0), 53, sA, sB)[0] == 49
