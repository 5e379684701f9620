"""GPU tier: fp64emu_mm_nt_noalloc, the allocation-free variant of
fp64emu_mm_nt (its scratch is the library's static device array), against
fp64emu_mm_nt bit for bit on two calls in a row, the second with a smaller
input, so the second call runs over the first call's leftover scratch.  The
first product's full workspace exceeds the static scratch, so it runs in row
chunks."""
import numpy as np
import pytest
import torch

import oracle as O
from fp64_emu import capi
from parity_util import sampled_parity

pytestmark = pytest.mark.gpu


def _randn(shape, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, dtype=torch.float64, generator=g).to(dev)


@pytest.mark.parametrize("shapes", [
    ((2000, 500, 2500), (300, 200, 1000)),     # chunked (full workspace > scratch), then small
    ((3000, 400, 2000), (64, 48, 256)),
])
def test_noalloc_matches_mm_nt(dev, shapes):
    P = 14
    primes = O.PRIMES[:P]
    for i, (M, N, K) in enumerate(shapes):
        print(f"case noalloc call {i}: mm_nt {M}x{N}x{K} P={P}", flush=True)
        A = _randn((M, K), 700 + 10 * i + M, dev)
        Bt = _randn((K, N), 701 + 10 * i + N, dev)
        ref, _, _ = capi.run("mm_nt", A, Bt, primes)
        got = capi.mm_nt_noalloc(A, Bt, primes)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int64), ref.view(torch.int64)), f"call {i} differs"
    # The first call ran in row chunks: its full workspace exceeds the scratch.
    assert capi.workspace_size(1, *shapes[0], P, True) > capi.NOALLOC_SCRATCH_BYTES


def test_noalloc_inexact_and_reduced(dev):
    """exact=False and the reduced plan (13 moduli, no correction)."""
    M, N, K = 700, 300, 2500
    print(f"case noalloc inexact/reduced mm_nt {M}x{N}x{K}", flush=True)
    A = _randn((M, K), 811, dev)
    Bt = _randn((K, N), 812, dev)
    for P, corr, exact in ((14, True, False), (13, False, True)):
        ref, _, _ = capi.run("mm_nt", A, Bt, O.PRIMES[:P], exact=exact, use_corr=corr)
        got = capi.mm_nt_noalloc(A, Bt, O.PRIMES[:P], exact=exact, use_corr=corr)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int64), ref.view(torch.int64)), (P, corr, exact)


def test_noalloc_rejects_oversize(dev):
    """A product whose smallest workspace exceeds the scratch is refused
    with the workspace status, and nothing runs."""
    print("case noalloc oversize", flush=True)
    A = torch.zeros((256, 8192), dtype=torch.float64, device=dev)
    Bt = torch.zeros((8192, 4096), dtype=torch.float64, device=dev)
    with pytest.raises(capi.CapiError, match="too large for the static scratch"):
        capi.mm_nt_noalloc(A, Bt, O.PRIMES[:14])


def test_noalloc_oracle_sample(dev):
    """The chunked no-alloc output at sampled rows and columns against the
    oracle pipeline (the entry point's own result, not only the ordinary
    entry point's)."""
    M, N, K = 2000, 500, 2500
    print(f"case noalloc oracle sample mm_nt {M}x{N}x{K}", flush=True)
    A = _randn((M, K), 821, dev)
    Bt = _randn((K, N), 822, dev)
    primes = np.asarray(O.PRIMES[:14], dtype=np.int32)
    got = capi.mm_nt_noalloc(A, Bt, primes)
    out, _, _, _ = sampled_parity("mm_nt", A, Bt, primes, rows=[0, 1, 255, 256, 1024, 1999],
                                  cols=[0, 5, 333, 499])
    assert torch.equal(got.view(torch.int64), out.view(torch.int64))


def test_noalloc_under_graph_capture(dev):
    """Callers under HIP graph capture: after one call on the device outside
    any capture (it looks up the scratch's device address), a call of a
    fresh shape is captured.  Each of three replays, with eager calls of
    both entry points between them (the eager no-alloc call overwrites the
    scratch), equals fp64emu_mm_nt bit for bit."""
    primes = O.PRIMES[:14]
    A0, B0 = _randn((64, 256), 830, dev), _randn((256, 48), 831, dev)
    first = capi.mm_nt_noalloc(A0, B0, primes)
    torch.cuda.synchronize()
    M, N, K = 700, 300, 2500
    print(f"case noalloc graph capture mm_nt {M}x{N}x{K}", flush=True)
    A, Bt = _randn((M, K), 832, dev), _randn((K, N), 833, dev)
    ref, _, _ = capi.run("mm_nt", A, Bt, primes)
    out = torch.empty((M, N), dtype=torch.float64, device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        capi.mm_nt_noalloc(A, Bt, primes, out=out)
    torch.cuda.synchronize()
    for r in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int64), ref.view(torch.int64)), f"replay {r}"
        again = capi.mm_nt_noalloc(A0, B0, primes)
        capi.run("mm_nt", A0, B0, primes)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int64), first.view(torch.int64))
