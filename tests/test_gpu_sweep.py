"""GPU parity over seeded sweeps of small shapes: every stage of the HIP
path against the CPU oracle (through the C ABI, on a pattern-filled
workspace), for kinds, batch counts, ragged M / N / K, modulus counts,
correction on and off and both combines drawn from a fixed generator.  The
draws, with a few shallow ones of 256 and more 256 x 256 tiles, reach every GEMM launch form
(256 x 256, 256 x 128, 128 x 128 and mixed tiles; K-splits; slot runs), as a
CPU-tier test of the draws checks.
A second sweep draws the reference accuracy study's input distributions
(wide exponent ranges, ill-conditioned scalings, spikes) at ragged shapes."""
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


def _run_cases():
    """Shallow products on 256 x 256 output tiles, the launches that run each
    tile's residue slots back to back: batched members of one tile each
    (256..290 members: one run per tile at 256 tiles, three above), and
    single products of 16..18 tile rows and columns (columns whose last tile
    holds more than 128 of them, so that no mixed launch takes them); ragged
    K, modulus counts, correction on and off.  Then one shallow product of as
    many tiles whose last tile column holds at most 128 columns: the mixed
    launch, one slot per group."""
    rng = np.random.default_rng(20261205)
    out = []
    for i in range(6):
        P = int(rng.integers(3, 21))
        corr = bool(rng.integers(2))
        exact = bool(rng.integers(4))
        if i % 2 == 0:
            kind = ["bmm", "bmm_nt"][rng.integers(2)]
            batch = int(rng.choice([int(rng.integers(257, 291)), 256, int(rng.integers(257, 291))]))
            M = int(rng.integers(233, 257))
            N = int(rng.integers(233, 257))
            K = int(rng.integers(1, 131))
        else:
            kind = ["mm", "mm_nt"][rng.integers(2)]
            batch = 1
            M = 256 * int(rng.integers(16, 19)) - int(rng.integers(0, 128))
            N = 256 * int(rng.integers(16, 19)) - int(rng.integers(0, 128))
            K = int(rng.integers(1, 121))
        out.append((100 + i, kind, batch, M, N, K, P, corr, exact))
    M = 256 * int(rng.integers(16, 19)) - int(rng.integers(0, 128))
    N = 256 * int(rng.integers(16, 19)) - int(rng.integers(128, 256))
    out.append((106, ["mm", "mm_nt"][rng.integers(2)], 1, M, N, int(rng.integers(1, 121)),
                int(rng.integers(3, 21)), bool(rng.integers(2)), True))
    return out


RUN_CASES = _run_cases()


@pytest.mark.parametrize("i,kind,batch,M,N,K,P,corr,exact", CASES + RUN_CASES)
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



def _dist_cases():
    """Seeded draws over the reference accuracy study's input distributions
    (tests/distributions.py) at ragged shapes, modulus counts and plans."""
    from distributions import DISTS
    rng = np.random.default_rng(20261203)
    out = []
    for i in range(18):
        dist = DISTS[i % len(DISTS)]
        kind = ["mm", "mm_nt"][rng.integers(2)]
        M = int(rng.integers(1, 500))
        N = int(rng.integers(1, 700))
        K = int(rng.integers(1, 6000))
        P = int(rng.integers(12, 21))
        corr = bool(rng.integers(4))           # mostly with the correction
        exact = bool(rng.integers(4))
        out.append((i, dist, kind, M, N, K, P, corr, exact))
    return out


@pytest.mark.parametrize("i,dist,kind,M,N,K,P,corr,exact", _dist_cases())
def test_sweep_distributions(dev, i, dist, kind, M, N, K, P, corr, exact):
    from distributions import make
    print(f"case dist-sweep {i}: {dist} {kind} {M}x{N}x{K} P={P} corr={corr} exact={exact}", flush=True)
    A, Bt = make(dist, M, K, N, 9000 + i)
    B = Bt if kind == "mm_nt" else Bt.t().contiguous()
    check_call(kind, A.to(dev), B.to(dev), O.PRIMES[:P], exact=exact, use_corr=corr)
