"""TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Python face of the CPU oracle (fp64emu_oracle.c, a restatement of the
reference RARE pipeline): ctypes wrappers over numpy arrays, the reference's
planner restated in pure Python (torch-ext/fp64_emu/__init__.py:20-45,
152-177), and exact big-integer / rational checkers used to pin the oracle.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module.
"""
import ctypes
import math
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_fp64emu.so")

# torch-ext/fp64_emu/__init__.py:20-22
PRIMES = [256, 255, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199,
          197, 193, 191, 181, 179, 173]
MAXP = 20
GROUPS = (MAXP + 3) // 4


# ---- planner: torch-ext/fp64_emu/__init__.py:152-177 ----------------------

def range_bits(n):
    r = 0.0
    for p in PRIMES[:n]:
        r += math.log2(p)
    return r - 1.0


def plan_config(K):
    need = 2 * 49 + math.ceil(math.log2(max(K, 1))) + 1 - 3.4
    for n in range(1, MAXP + 1):
        if range_bits(n) >= need:
            return n, True
    return MAXP, True


def plan(K, bits=53):
    need = 2 * bits + math.ceil(math.log2(max(K, 1))) + 1
    for n in range(1, MAXP + 1):
        if range_bits(n) >= need:
            return n
    raise ValueError(f"K={K} at bits={bits} needs more range than {MAXP} primes give")


# ---- ctypes ---------------------------------------------------------------

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"oracle not built: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.or_tables.argtypes = [vp, i32, vp, vp, vp, vp]
        L.or_size_rows.argtypes = [vp, i64, i64, i32, vp, vp]
        L.or_size_cols.argtypes = [vp, i64, i64, i64, i32, vp, vp]
        L.or_pick_bits.argtypes = [vp, i64, vp, i64, ctypes.c_float, i32, vp, vp]
        L.or_pick_bits.restype = i32
        L.or_rne_shr.argtypes = [ctypes.c_uint64, i32]
        L.or_rne_shr.restype = ctypes.c_uint64
        L.or_split.argtypes = [ctypes.c_double, i32, i32, i32, vp, vp]
        L.or_split.restype = ctypes.c_uint64
        L.or_residue.argtypes = [ctypes.c_uint64, i32, i32]
        L.or_residue.restype = ctypes.c_int8
        L.or_extract_operand.argtypes = [vp, i64, i64, i64, i32, vp, i32, vp, i32, i32, vp, vp, vp]
        L.or_bal8.argtypes = [ctypes.c_int32, i32]
        L.or_bal8.restype = ctypes.c_int8
        L.or_barrett_bal32.argtypes = [i32, i32, ctypes.c_uint32, ctypes.c_uint32]
        L.or_barrett_bal32.restype = i32
        L.or_modgemm.argtypes = [vp, vp, i64, i64, i64, i32, vp, vp, i32]
        L.or_modgemm.restype = i32
        L.or_reconstruct.argtypes = [vp, vp, vp, i64, i64, vp, i32, i32, vp, vp, i32, vp]
        L.or_reconstruct64.argtypes = [vp, vp, vp, i64, i64, vp, i32, i32, vp, vp, i32, vp]
        L.or_fold_residue.argtypes = [ctypes.c_int32, i32]
        L.or_fold_residue.restype = i32
        L.or_mm.argtypes = [vp, vp, vp, i64, i64, i64, i64, i32, vp, i32, i32, i32, i32, i32,
                            vp, vp, vp, vp, vp]
        L.or_mm.restype = i32
        L.or_ddgemm_nt.argtypes = [vp, vp, vp, vp, i64, i64, i64, i32]
        L.or_i128_to_double.restype = ctypes.c_double
        L.or_bal8_array.argtypes = [vp, i64, i32, vp]
        L.or_barrett_bal32_array.argtypes = [vp, i64, i32, vp]
        L.or_extract_array.argtypes = [vp, vp, i64, i32, vp, i32, vp, vp, vp, vp]
        L.or_i128_array_to_double.argtypes = [vp, vp, i64, vp]
        _LIB = L
    return _LIB


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _c(a, dtype):
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def tables(primes):
    primes = _c(primes, np.int32)
    P = primes.size
    minv = np.zeros(P, np.int32)
    mppack = np.zeros(P * GROUPS, np.int32)
    m64 = np.zeros(2, np.int64)
    l2 = ctypes.c_float()
    lib().or_tables(_p(primes), P, _p(minv), _p(mppack), _p(m64), ctypes.byref(l2))
    return minv, mppack, m64, l2.value


def size_rows(X, bits):
    X = _c(X, np.float64)
    rows, cols = X.shape[0] if X.ndim == 2 else int(np.prod(X.shape[:-1])), X.shape[-1]
    sft = np.zeros(rows, np.int16)
    lg = np.zeros(rows, np.float32)
    lib().or_size_rows(_p(X), rows, cols, bits, _p(sft), _p(lg))
    return sft, lg


def size_cols(X, bits):
    """X [batch, K, N] (or [K, N])."""
    X = _c(X, np.float64)
    if X.ndim == 2:
        X = X[None]
    batch, K, N = X.shape
    sft = np.zeros(batch * N, np.int16)
    lg = np.zeros(batch * N, np.float32)
    lib().or_size_cols(_p(X), batch, K, N, bits, _p(sft), _p(lg))
    return sft, lg


def pick_bits(lgA, lgB, log2M, bits, sftA, sftB):
    lgA, lgB = _c(lgA, np.float32), _c(lgB, np.float32)
    sA, sB = _c(sftA, np.int16).copy(), _c(sftB, np.int16).copy()
    be = lib().or_pick_bits(_p(lgA), lgA.size, _p(lgB), lgB.size, ctypes.c_float(log2M), bits,
                            _p(sA), _p(sB))
    return be, sA, sB


def split(x, shift, bits_eff, do_corr=True):
    h = ctypes.c_int8()
    q = ctypes.c_int8()
    uu = lib().or_split(float(x), int(shift), int(bits_eff), int(do_corr), ctypes.byref(h),
                        ctypes.byref(q))
    return uu, h.value, q.value


def residue(uu, p, bits_eff):
    return lib().or_residue(int(uu), int(p), int(bits_eff))


def extract_operand(X, kn, sft, bits_eff, primes, do_corr=True):
    """X [batch, R, K] (kn=0) or [batch, K, R] (kn=1) -> res [batch, P, R, K],
    hi, q [batch, R, K]."""
    X = _c(X, np.float64)
    if X.ndim == 2:
        X = X[None]
    batch = X.shape[0]
    R, K = (X.shape[2], X.shape[1]) if kn else (X.shape[1], X.shape[2])
    primes = _c(primes, np.int32)
    P = primes.size
    res = np.zeros((batch, P, R, K), np.int8)
    hi = np.zeros((batch, R, K), np.int8)
    q = np.zeros((batch, R, K), np.int8)
    sft = _c(sft, np.int16)
    lib().or_extract_operand(_p(X), batch, R, K, int(kn), _p(sft), int(bits_eff), _p(primes), P,
                             int(do_corr), _p(res), _p(hi), _p(q))
    return res, hi, q


def bal8_array(v, p):
    """The GEMM epilogue's 31-bit Barrett (fp64_emu.cu:613-620) on an int32 array."""
    v = _c(v, np.int32)
    out = np.zeros(v.shape, np.int8)
    lib().or_bal8_array(_p(v), v.size, int(p), _p(out))
    return out


def barrett_bal32_array(y, p):
    """barrett_bal32 (fp64_emu.cu:42-51) with the Garner bias p << 21."""
    y = _c(y, np.int32)
    out = np.zeros(y.shape, np.int32)
    lib().or_barrett_bal32_array(_p(y), y.size, int(p), _p(out))
    return out


def extract_array(x, shift, bits_eff, primes):
    """Per-element extraction: (td int64, res [n, P] int8, hi int8, q int8)."""
    x = _c(x, np.float64).ravel()
    shift = _c(np.broadcast_to(np.asarray(shift, np.int32), x.shape), np.int32)
    primes = _c(primes, np.int32)
    n, P = x.size, primes.size
    td = np.zeros(n, np.int64)
    res = np.zeros((n, P), np.int8)
    hi = np.zeros(n, np.int8)
    q = np.zeros(n, np.int8)
    lib().or_extract_array(_p(x), _p(shift), n, int(bits_eff), _p(primes), P, _p(td), _p(res),
                           _p(hi), _p(q))
    return td, res, hi, q


def i128_to_double(values):
    """Correctly rounded conversion of Python ints in the signed 128-bit range."""
    hi = np.array([(v >> 64) for v in values], dtype=np.int64)
    lo = np.array([v & ((1 << 64) - 1) for v in values], dtype=np.uint64)
    out = np.zeros(len(values), np.float64)
    lib().or_i128_array_to_double(_p(hi), _p(lo), len(values), _p(out))
    return out


def modgemm(A8, B8, p, nthreads=0):
    """A8 [M,K], B8 [N,K] int8: p > 0 -> balanced int8 residues of A B^T;
    p == 0 -> raw int32."""
    A8, B8 = _c(A8, np.int8), _c(B8, np.int8)
    M, K = A8.shape
    N = B8.shape[0]
    if p > 0:
        out = np.zeros((M, N), np.int8)
        ov = lib().or_modgemm(_p(A8), _p(B8), M, N, K, p, _p(out), None, nthreads)
    else:
        out = np.zeros((M, N), np.int32)
        ov = lib().or_modgemm(_p(A8), _p(B8), M, N, K, 0, None, _p(out), nthreads)
    if ov:
        raise OverflowError("int32 accumulator bound exceeded")
    return out


def reconstruct(res, c1, c2, primes, bits_eff, sftA, sftB, exact=True):
    """res [P, M, N] int8; c1, c2 [M, N] int32 or None."""
    res = _c(res, np.int8)
    P, M, N = res.shape
    primes = _c(primes, np.int32)
    c1 = _c(c1, np.int32) if c1 is not None else None
    c2 = _c(c2, np.int32) if c2 is not None else None
    out = np.zeros((M, N), np.float64)
    lib().or_reconstruct(_p(res), _p(c1), _p(c2), M, N, _p(primes), P, int(bits_eff),
                         _p(_c(sftA, np.int16)), _p(_c(sftB, np.int16)), int(bool(exact)), _p(out))
    return out


def reconstruct64(res, d1, d2, primes, bits_eff, sftA, sftB, exact=True):
    """reconstruct with int64 correction planes (the K-segmented path)."""
    res = _c(res, np.int8)
    P, M, N = res.shape
    primes = _c(primes, np.int32)
    d1 = _c(d1, np.int64) if d1 is not None else None
    d2 = _c(d2, np.int64) if d2 is not None else None
    out = np.zeros((M, N), np.float64)
    lib().or_reconstruct64(_p(res), _p(d1), _p(d2), M, N, _p(primes), P, int(bits_eff),
                           _p(_c(sftA, np.int16)), _p(_c(sftB, np.int16)), int(bool(exact)),
                           _p(out))
    return out


def fold_residue(acc, p):
    """The K-segmented path's fold of an int32 residue sum (barrett_bal32)."""
    return lib().or_fold_residue(int(acc), int(p))


def mm(A, B, b_kn, primes, exact=True, bits=53, use_corr=True, nthreads=0):
    """Whole pipeline.  A [batch,M,K] or [M,K]; B [batch,N,K] (b_kn=0) or
    [batch,K,N] (b_kn=1).  K > 131071 with b_kn=0 runs the K-segmented path.
    Returns (out, sizing dict)."""
    A = _c(A, np.float64)
    B = _c(B, np.float64)
    squeeze = A.ndim == 2
    if squeeze:
        A, B = A[None], B[None]
    batch, M, K = A.shape
    N = B.shape[2] if b_kn else B.shape[1]
    primes = _c(primes, np.int32)
    out = np.zeros((batch, M, N), np.float64)
    sA = np.zeros(batch * M, np.int16)
    sB = np.zeros(batch * N, np.int16)
    lA = np.zeros(batch * M, np.float32)
    lB = np.zeros(batch * N, np.float32)
    be = ctypes.c_int()
    st = lib().or_mm(_p(out), _p(A), _p(B), batch, M, N, K, int(b_kn), _p(primes), primes.size,
                     int(bool(exact)), int(bits), int(bool(use_corr)), nthreads, _p(sA), _p(sB),
                     _p(lA), _p(lB), ctypes.byref(be))
    if st != 0:
        raise MemoryError("oracle allocation failed")
    info = dict(sftA=sA, sftB=sB, lgA=lA, lgB=lB, bits_eff=be.value)
    return (out[0] if squeeze else out), info


def int_gemm(A8, B8):
    """Exact A8 @ B8^T of int8 planes A8 [M, K], B8 [N, K], as int64: one
    float64 BLAS product (every partial sum, in any order, is an integer of
    magnitude at most K * 128^2 < 2^53, so each operation is exact).  The
    same integers as or_modgemm's sums, many times faster, for whole-output
    checks at the benchmark sizes."""
    A8, B8 = np.asarray(A8), np.asarray(B8)
    assert A8.shape[1] * 128 * 128 < 2 ** 53
    return (A8.astype(np.float64) @ B8.astype(np.float64).T).astype(np.int64)


def mm_blas(A, B, b_kn, primes, exact=True, bits=53, use_corr=True):
    """The whole pipeline of mm() (single launch depth, K <= 131071) with
    the modular GEMMs as int_gemm products and the reference's bal8 on
    their int32 sums: or_size_rows / or_size_cols / or_pick_bits,
    or_extract_operand, int_gemm + or_bal8 (fp64_emu.cu:494-657),
    or_reconstruct.  Bit-identical to mm() (the CPU tests check it);
    returns (out, sizing dict)."""
    A = _c(A, np.float64)
    B = _c(B, np.float64)
    squeeze = A.ndim == 2
    if squeeze:
        A, B = A[None], B[None]
    batch, M, K = A.shape
    if K > 131071:
        raise ValueError("mm_blas: single-launch depth only (K <= 131071)")
    N = B.shape[2] if b_kn else B.shape[1]
    primes = _c(primes, np.int32)
    P = primes.size
    sA, lA = size_rows(A.reshape(-1, K), bits)
    if b_kn:
        sB, lB = size_cols(B, bits)
    else:
        sB, lB = size_rows(B.reshape(-1, K), bits)
    _, _, _, log2M = tables(primes)
    be, sA, sB = pick_bits(lA, lB, min(log2M, 126.0), bits, sA, sB)
    out = np.zeros((batch, M, N), np.float64)
    for b in range(batch):
        rA, hA, qA = extract_operand(A[b:b + 1], 0, sA[b * M:(b + 1) * M], be, primes, use_corr)
        rB, hB, qB = extract_operand(B[b:b + 1], 1 if b_kn else 0, sB[b * N:(b + 1) * N], be,
                                     primes, use_corr)
        res = np.zeros((P, M, N), np.int8)
        for t in range(P):
            res[t] = bal8_array(int_gemm(rA[0, t], rB[0, t]), int(primes[t]))
        c1 = int_gemm(hA[0], qB[0]).astype(np.int32) if use_corr else None
        c2 = int_gemm(qA[0], hB[0]).astype(np.int32) if use_corr else None
        del rA, rB
        out[b] = reconstruct(res, c1, c2, primes, be, sA[b * M:(b + 1) * M],
                             sB[b * N:(b + 1) * N], exact)
    info = dict(sftA=sA, sftB=sB, lgA=lA, lgB=lB, bits_eff=be)
    return (out[0] if squeeze else out), info


def ddgemm_nt(A, Bt, nthreads=0):
    """Double-double A [M,K] @ Bt [K,N] (bench/accuracy.py:21-50)."""
    A, Bt = _c(A, np.float64), _c(Bt, np.float64)
    M, K = A.shape
    N = Bt.shape[1]
    hi = np.zeros((M, N), np.float64)
    lo = np.zeros((M, N), np.float64)
    lib().or_ddgemm_nt(_p(hi), _p(lo), _p(A), _p(Bt), M, N, K, nthreads)
    return hi, lo


def correct_bits(C, hi, lo):
    """-log2(max|C - (hi+lo)| / max|hi|), bench/accuracy.py:75-82."""
    C, hi, lo = (np.asarray(x, dtype=np.float64) for x in (C, hi, lo))
    err = float(np.max(np.abs((C - hi) - lo))) if C.size else 0.0
    scale = float(np.max(np.abs(hi))) if C.size else 0.0
    if err == 0.0:
        return 53.0
    return -math.log2(err / scale)


# ---- exact checkers (pure Python) -----------------------------------------

def rne_int(fr):
    """Round a Fraction to the nearest integer, ties to even."""
    return round(fr)   # Fraction.__round__ rounds half to even


def balanced(v, p):
    """Balanced residue in [-(p//2), (p-1)//2] (p = 256: [-128, 127])."""
    r = v % p
    if r > (p - 1) // 2:
        r -= p
    return r


def exact_split(x, shift, bits_eff):
    """Exact rational form of the reference's split (fp64_emu.cu:300-321):
    (td, h7, q7) from Fraction arithmetic, independent of the bit tricks."""
    fx = Fraction(x)
    mag = abs(fx) * Fraction(2) ** shift
    Tu = rne_int(mag)
    neg = x < 0 or (x == 0 and math.copysign(1.0, x) < 0)
    td = -Tu if neg else Tu
    h8 = rne_int(Fraction(Tu) * Fraction(2) ** (7 - bits_eff))
    r8 = rne_int(mag * 256) - 256 * Tu
    hs, qs = (-h8, -r8) if neg else (h8, r8)
    clamp = lambda v: max(-127, min(127, v))  # noqa: E731
    return td, clamp(hs), clamp(qs)


def crt_value(res, primes):
    """The integer in the balanced range with the given residues (big-int CRT)."""
    M = 1
    for p in primes:
        M *= p
    x = 0
    for r, p in zip(res, primes):
        Mi = M // p
        x += int(r) * Mi * pow(Mi, -1, p)
    x %= M
    if x >= (M + 1) // 2:
        x -= M
    return x
