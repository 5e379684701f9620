"""Double-precision matrix products on MI355X's INT8 matrix cores.

Each operand is scaled by powers of two, per row of A and per column of B,
to integers of at most 53 bits.  Their product is then known exactly
through its remainders modulo a list of small pairwise-coprime moduli, and
each remainder costs one INT8 MFMA GEMM of balanced residues.  A mixed-radix
(Garner) recombination of those remainders, plus two int8 GEMMs of the
rounding residue that correct the scaling's first-order error, gives the
float64 result.  How many moduli suffice is decided from K by the planner
below, and a norm bound computed on the device narrows the integers until
the product fits their range.  Integer inputs whose products are exact in
float64 come out identical to the native product.

The functions, keywords, defaults and planner are those of the reference
package (torch-ext/fp64_emu/__init__.py, cited line by line), so callers
switch by import.  The work runs in hand-written gfx950 HIP kernels; without
the built extension the import raises.
"""
import math
from functools import lru_cache

import torch

from ._ops import ops
from . import _meta  # noqa: F401  (fake kernels for torch.compile)

# Pairwise-coprime moduli up to the balanced int8 ceiling of 256, largest
# first; torch-ext/fp64_emu/__init__.py:20-22.
_PRIMES = [256, 255, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199,
           197, 193, 191, 181, 179, 173]
_MAXP = 20

# Single-launch depth bound of the int32 modular GEMM (K * 128^2 < 2^31).
_KMAX_SINGLE = 131071


def _modinv(a, m):
    """Inverse of a modulo m (torch-ext/fp64_emu/__init__.py:25-30)."""
    return pow(a % m, -1, m)


@lru_cache(maxsize=None)
def _tables(nprimes):
    """(primes, inv, mu) CPU tensors, torch-ext/fp64_emu/__init__.py:33-45.
    Only `primes` is used by the kernels; inv (pairwise inverses) and mu
    (2^62 Barrett reciprocals) are kept for interface compatibility."""
    primes = _PRIMES[:nprimes]
    P = len(primes)
    inv = [0] * (P * P)
    for a in range(P):
        for b in range(a + 1, P):
            inv[a * P + b] = _modinv(primes[a] % primes[b], primes[b])
    mu = [(1 << 62) // p for p in primes]
    return (torch.tensor(primes, dtype=torch.int32),
            torch.tensor(inv, dtype=torch.int32),
            torch.tensor(mu, dtype=torch.int64))


def _defaults(K, nprimes, corr):
    if nprimes is None or corr is None:
        dp, dc = plan_config(K)
        nprimes = dp if nprimes is None else nprimes
        corr = dc if corr is None else corr
    return nprimes, corr


def mm(A: torch.Tensor, B: torch.Tensor, nprimes: int = None,
       exact: bool = True, bits: int = 53, corr: bool = None) -> torch.Tensor:
    """C = A @ B^T in float64 for A [M, K] and B [N, K]
    (torch-ext/fp64_emu/__init__.py:48-70).

    nprimes: how many moduli, i.e. INT8 GEMMs; None lets plan_config(K)
      choose.
    exact: True recombines in 128-bit integers and rounds once; False
      recombines in float64, slightly faster and a fraction of a bit less
      accurate.
    bits: the operands' integer width before the device narrows it; 53
      keeps every bit of a float64 significand.
    corr: whether to run the two INT8 GEMMs of the rounding residue that
      remove the scaling's first-order error; None lets plan_config(K)
      choose.
    """
    assert A.dim() == 2 and B.dim() == 2 and A.size(1) == B.size(1)
    M, K = A.shape
    N = B.size(0)
    nprimes, corr = _defaults(K, nprimes, corr)
    primes, inv, mu = _tables(nprimes)
    out = torch.empty(M, N, dtype=torch.float64, device=A.device)
    Ac = A if A.is_contiguous() else A.contiguous()
    Bc = B if B.is_contiguous() else B.contiguous()
    ops.fp64_emu_mm(out, Ac, Bc, primes, inv, mu, exact, bits, corr)
    return out


def mm_nt(A: torch.Tensor, Bt: torch.Tensor, nprimes: int = None,
          exact: bool = True, bits: int = 53, corr: bool = None) -> torch.Tensor:
    """C = A @ Bt with Bt given as [K, N], consumed in place: the extraction
    kernel reads it column-wise, no transpose copy
    (torch-ext/fp64_emu/__init__.py:73-90)."""
    assert A.dim() == 2 and Bt.dim() == 2 and A.size(1) == Bt.size(0)
    K = A.size(1)
    if K > _KMAX_SINGLE:
        return mm(A, Bt.t().contiguous(), nprimes, exact, bits, corr)
    nprimes, corr = _defaults(K, nprimes, corr)
    primes, inv, mu = _tables(nprimes)
    out = torch.empty(A.size(0), Bt.size(1), dtype=torch.float64, device=A.device)
    Ac = A if A.is_contiguous() else A.contiguous()
    Bc = Bt if Bt.is_contiguous() else Bt.contiguous()
    ops.fp64_emu_mm_nt(out, Ac, Bc, primes, inv, mu, exact, bits, corr)
    return out


def bmm(A: torch.Tensor, B: torch.Tensor, nprimes: int = None,
        exact: bool = True, bits: int = 53, corr: bool = None) -> torch.Tensor:
    """Batched C[b] = A[b] @ B[b]^T with B given as [batch, N, K]
    (torch-ext/fp64_emu/__init__.py:93-112).  One operand width serves the
    whole batch; every GEMM of the batch runs in one launch."""
    assert A.dim() == 3 and B.dim() == 3 and A.size(0) == B.size(0) and A.size(2) == B.size(2)
    K = A.size(2)
    nprimes, corr = _defaults(K, nprimes, corr)
    primes, inv, mu = _tables(nprimes)
    out = torch.empty(A.size(0), A.size(1), B.size(1), dtype=torch.float64, device=A.device)
    Ac = A if A.is_contiguous() else A.contiguous()
    Bc = B if B.is_contiguous() else B.contiguous()
    ops.fp64_emu_bmm(out, Ac, Bc, primes, inv, mu, exact, bits, corr)
    return out


def bmm_nt(A: torch.Tensor, Bt: torch.Tensor, nprimes: int = None,
           exact: bool = True, bits: int = 53, corr: bool = None) -> torch.Tensor:
    """C[b] = A[b] @ Bt[b] with Bt given as [batch, K, N] (torch.bmm layout),
    consumed in place (torch-ext/fp64_emu/__init__.py:115-132)."""
    assert A.dim() == 3 and Bt.dim() == 3 and A.size(0) == Bt.size(0) and A.size(2) == Bt.size(1)
    K = A.size(2)
    if K > _KMAX_SINGLE:
        return bmm(A, Bt.transpose(1, 2).contiguous(), nprimes, exact, bits, corr)
    nprimes, corr = _defaults(K, nprimes, corr)
    primes, inv, mu = _tables(nprimes)
    out = torch.empty(A.size(0), A.size(1), Bt.size(2), dtype=torch.float64, device=A.device)
    Ac = A if A.is_contiguous() else A.contiguous()
    Bc = Bt if Bt.is_contiguous() else Bt.contiguous()
    ops.fp64_emu_bmm_nt(out, Ac, Bc, primes, inv, mu, exact, bits, corr)
    return out


def mm_timed(A: torch.Tensor, B: torch.Tensor, nprimes: int = None, exact: bool = True,
             bits: int = 53, corr: bool = None):
    """(C, phase_ms[4]) = [scale+extract, gemms, marker, reconstruct], B as
    [N, K] (torch-ext/fp64_emu/__init__.py:135-149)."""
    M, K = A.shape
    N = B.size(0)
    nprimes, corr = _defaults(K, nprimes, corr)
    primes, inv, mu = _tables(nprimes)
    out = torch.empty(M, N, dtype=torch.float64, device=A.device)
    times = torch.zeros(4, dtype=torch.float32)
    ops.fp64_emu_mm_timed(out, times, A.contiguous(), B.contiguous(), primes, inv, mu,
                          exact, bits, corr)
    return out, times.tolist()


def range_bits(nprimes: int) -> float:
    """Signed CRT range of the first `nprimes` moduli in bits
    (torch-ext/fp64_emu/__init__.py:152-157)."""
    r = 0.0
    for p in _PRIMES[:nprimes]:
        r += math.log2(p)
    return r - 1.0


def plan_config(K: int) -> tuple:
    """(nprimes, corr) reaching FP64-equivalent accuracy at depth K
    (torch-ext/fp64_emu/__init__.py:160-167); the device sizing pass keeps
    the choice range-safe."""
    need = 2 * 49 + math.ceil(math.log2(max(K, 1))) + 1 - 3.4
    for n in range(1, _MAXP + 1):
        if range_bits(n) >= need:
            return n, True
    return _MAXP, True


def plan(K: int, bits: int = 53) -> int:
    """Smallest worst-case range-safe nprimes at depth K and width bits
    (torch-ext/fp64_emu/__init__.py:170-177): 2*bits + ceil(log2 K) + 1."""
    need = 2 * bits + math.ceil(math.log2(max(K, 1))) + 1
    for n in range(1, _MAXP + 1):
        if range_bits(n) >= need:
            return n
    raise ValueError(f"K={K} at bits={bits} needs more range than {_MAXP} primes give")


__all__ = ["mm", "mm_nt", "bmm", "bmm_nt", "mm_timed", "plan", "plan_config", "range_bits"]
