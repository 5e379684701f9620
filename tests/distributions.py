"""Input distributions of the reference's accuracy study, generated on the CPU
from a seed so that the HIP path and the CPU oracle see identical bits.

bench/accuracy.py:85-107 (reference) defines them on the CUDA generator;
the same transformations are applied here to CPU draws:
  randn      iid N(0, 1)
  wide8/16   each element of A and Bt times 2^e, e uniform in [-w, w]
  illcond    columns of A and rows of Bt (the k index) scaled by a shared
             2^(-span U(0,1)), span 20 (illcond) or 40 (illcond40)
  spike      one element per row of A (at a uniform k) times 2^30
"""
import torch

DISTS = ("randn", "wide8", "wide16", "illcond", "illcond40", "spike")


def make(dist, M, K, N, seed):
    """A [M, K] and Bt [K, N], float64 on the CPU."""
    g = torch.Generator().manual_seed(seed)
    f64 = torch.float64
    A = torch.randn(M, K, dtype=f64, generator=g)
    Bt = torch.randn(K, N, dtype=f64, generator=g)
    if dist == "randn":
        pass
    elif dist in ("wide8", "wide16"):
        w = 8 if dist == "wide8" else 16
        A *= torch.exp2(torch.randint(-w, w + 1, A.shape, generator=g).to(f64))
        Bt *= torch.exp2(torch.randint(-w, w + 1, Bt.shape, generator=g).to(f64))
    elif dist in ("illcond", "illcond40"):
        span = 20 if dist == "illcond" else 40
        s = torch.exp2(-span * torch.rand(K, generator=g, dtype=f64))
        A *= s[None, :]
        Bt *= s[:, None]
    elif dist == "spike":
        idx = torch.randint(0, K, (M,), generator=g)
        A[torch.arange(M), idx] *= 2.0 ** 30
    else:
        raise ValueError(dist)
    return A, Bt


def seed_of(dist, K):
    """A fixed seed per (distribution, depth)."""
    return 7000 + 100 * DISTS.index(dist) + (K % 97)
