"""GPU parity over a seeded sweep of small shapes: every stage of the HIP
path against the CPU oracle (through the C ABI, on a pattern-filled
workspace), for kinds, batch counts, ragged M / N / K, modulus counts,
correction on and off and both combines drawn from a fixed generator.  The
draws reach every GEMM launch form (256 x 256, 256 x 128, 128 x 128 and
mixed tiles; K-splits; slot runs), as a CPU-tier test of the draws checks."""
import numpy as np
import pytest
import torch

import oracle as O
from parity_util import check_call

pytestmark = pytest.mark.gpu

N_CASES = 40


def _cases():
    rng = np.random.default_rng(20261202)
    out = []
    for i in range(N_CASES):
        kind = ["mm", "mm_nt", "bmm", "bmm_nt"][rng.integers(4)]
        batch = int(rng.integers(1, 5)) if kind.startswith("bmm") else 1
        M = int(rng.integers(1, 600))
        N = int(rng.integers(1, 1400 if i % 3 == 0 else 600))
        K = int(rng.integers(1, 3000 if i % 4 else 24000))
        P = int(rng.integers(1, 21))
        corr = bool(rng.integers(2))
        exact = bool(rng.integers(4))          # mostly exact
        out.append((i, kind, batch, M, N, K, P, corr, exact))
    return out


CASES = _cases()


@pytest.mark.parametrize("i,kind,batch,M,N,K,P,corr,exact", CASES)
def test_sweep_parity(dev, i, kind, batch, M, N, K, P, corr, exact):
    print(f"case sweep {i}: {kind} b={batch} {M}x{N}x{K} P={P} corr={corr} exact={exact}", flush=True)
    g = torch.Generator().manual_seed(5000 + i)
    if kind.startswith("bmm"):
        A = torch.randn((batch, M, K), dtype=torch.float64, generator=g)
        B = torch.randn((batch, K, N) if kind == "bmm_nt" else (batch, N, K), dtype=torch.float64, generator=g)
    else:
        A = torch.randn((M, K), dtype=torch.float64, generator=g)
        B = torch.randn((K, N) if kind == "mm_nt" else (N, K), dtype=torch.float64, generator=g)
    check_call(kind, A.to(dev), B.to(dev), O.PRIMES[:P], exact=exact, use_corr=corr)

