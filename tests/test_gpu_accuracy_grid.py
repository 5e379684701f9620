"""GPU tier: the reference's accuracy study and edge shapes, stage by stage
against the CPU oracle.

- The six input distributions of bench/accuracy.py:85-107 (randn, wide8,
  wide16, illcond, illcond40, spike) at M = N = 128, K in {512, 4096}
  (accuracy.py:117-118), at the default plan and at the reduced operating
  point (13 moduli, no correction): every stage bit-exact, and at the
  default plan correct bits against a double-double product at least those
  of native float64 on the GPU (the claim of README.md:200-215).
- bench/defaultcheck.py:12-20: the out-of-box mm call at K in
  {64, 256, 1024, 4096} on randn, wide16, illcond40 and spike.
- bench/edgecheck.py:12-13 and bench/make_job.py:104: the named odd and
  edge shapes (M x K x N), through mm like the reference scripts.
Inputs come from CPU seeds (distributions.py), so the oracle sees the same
bits."""
import numpy as np
import pytest
import torch

import oracle as O
from distributions import DISTS, make, seed_of
from parity_util import check_call

pytestmark = pytest.mark.gpu

GRID = [(d, K, plan) for d in DISTS for K in (512, 4096) for plan in ("default", "reduced")]


def _bits(C, hi, lo):
    return O.correct_bits(np.asarray(C), hi, lo)


@pytest.mark.parametrize("dist,K,plan", GRID)
def test_accuracy_grid(dev, dist, K, plan):
    P, corr = O.plan_config(K) if plan == "default" else (13, False)
    print(f"case grid {dist} K={K} {plan} (P={P}, corr={corr}) mm_nt 128x128x{K}", flush=True)
    A, Bt = make(dist, 128, K, 128, seed_of(dist, K))
    Ad, Btd = A.to(dev), Bt.to(dev)
    out, _, _ = check_call("mm_nt", Ad, Btd, O.PRIMES[:P], use_corr=corr)
    hi, lo = O.ddgemm_nt(A.numpy(), Bt.numpy())
    emu_bits = _bits(out.cpu().numpy(), hi, lo)
    native_bits = _bits((Ad @ Btd).cpu().numpy(), hi, lo)
    print(f"  correct bits emu {emu_bits:.2f} native {native_bits:.2f}", flush=True)
    if plan == "default":
        assert emu_bits >= native_bits
    else:
        # README.md:202-213 reports 43.3-48.6 bits for the reduced point.
        assert emu_bits >= 40.0


@pytest.mark.parametrize("K", [64, 256, 1024, 4096])
@pytest.mark.parametrize("dist", ["randn", "wide16", "illcond40", "spike"])
def test_default_call_depths(dev, dist, K):
    P, corr = O.plan_config(K)
    print(f"case default-call {dist} K={K} mm 128x128x{K}", flush=True)
    A, Bt = make(dist, 128, K, 128, seed_of(dist, K) + 1)
    B = Bt.t().contiguous()
    Ad, Bd = A.to(dev), B.to(dev)
    out, _, _ = check_call("mm", Ad, Bd, O.PRIMES[:P], use_corr=corr)
    hi, lo = O.ddgemm_nt(A.numpy(), Bt.numpy())
    emu_bits = _bits(out.cpu().numpy(), hi, lo)
    native_bits = _bits((Ad @ Bd.t()).cpu().numpy(), hi, lo)
    print(f"  correct bits emu {emu_bits:.2f} native {native_bits:.2f}", flush=True)
    assert emu_bits >= native_bits


EDGE_SHAPES = [(129, 4095, 127), (17, 23, 29), (256, 511, 254), (255, 1000, 999),
               (1000, 1000, 1000), (128, 64, 256), (384, 8192, 512), (512, 2047, 33)]


@pytest.mark.parametrize("M,K,N", EDGE_SHAPES)
def test_edge_shapes(dev, M, K, N):
    P, corr = O.plan_config(K)
    print(f"case edge shape mm {M}x{K}x{N} (M x K x N)", flush=True)
    g = torch.Generator().manual_seed(M * 7 + K * 5 + N)
    A = torch.randn(M, K, dtype=torch.float64, generator=g)
    B = torch.randn(N, K, dtype=torch.float64, generator=g)
    Ad, Bd = A.to(dev), B.to(dev)
    out, _, _ = check_call("mm", Ad, Bd, O.PRIMES[:P], use_corr=corr)
    ref = Ad @ Bd.t()
    rel = ((out - ref).abs().max() / ref.abs().max()).item()
    assert rel < 1e-11     # the reference scripts' bar (edgecheck.py:18)
