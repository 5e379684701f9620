"""GPU tier at the benchmark configurations' full sizes (c2..c5), with the
inputs generated on the CPU from fixed seeds (1000*cfg, 1000*cfg + 1):

- sizing (per-row/column shifts and the global width) bit-exact against the
  oracle on the full operands;
- every output element bit-exact against the oracle's pipeline (its modular
  products as exact BLAS products, O.mm_blas, pinned to O.mm on the CPU);
- correct bits against the device double-double GEMM at least native
  float64's (torch matmul on the same GPU);
- the effective width within one bit of the values computed independently
  from the distributions (c2 49, c3a 50, c3b 49, c5 51, c5 reduced 43);
- c3b: the integer product bit for bit, with both correction products zero;
- c4: every stage of all 64 members against the oracle.
"""
import numpy as np
import pytest
import torch

import fp64_emu as emu
import oracle as O
from fp64_emu import capi
from parity_util import check_call, whole_parity

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _rows(n, seed, k=24):
    rng = np.random.default_rng(seed)
    return np.concatenate([[0, 1, n - 2, n - 1], rng.integers(0, n, k)])


def _dd_bits(C, A, Bt_nk):
    hi, lo = capi.ddgemm_nt(A, Bt_nk)
    torch.cuda.synchronize()
    return O.correct_bits(C.cpu().numpy(), hi.cpu().numpy(), lo.cpu().numpy())


def _native_and_emu_bits(C, A, Bt):
    Bnk = Bt.t().contiguous()
    native = A @ Bt
    hi, lo = capi.ddgemm_nt(A, Bnk)
    torch.cuda.synchronize()
    h, l = hi.cpu().numpy(), lo.cpu().numpy()
    return O.correct_bits(C.cpu().numpy(), h, l), O.correct_bits(native.cpu().numpy(), h, l)


def test_c2_square_8192(dev):
    print("case c2 mm_nt 8192^3 default plan", flush=True)
    n = 8192
    A = torch.randn((n, n), dtype=torch.float64, generator=_gen(2000)).to(dev)
    Bt = torch.randn((n, n), dtype=torch.float64, generator=_gen(2001)).to(dev)
    P, corr = emu.plan_config(n)
    assert (P, corr) == (14, True)
    out, be, lay, ws = whole_parity("mm_nt", A, Bt, O.PRIMES[:P])
    del ws
    assert be == 49
    assert torch.equal(out, emu.mm_nt(A, Bt))
    emu_bits, nat_bits = _native_and_emu_bits(out, A, Bt)
    print(f"c2 correct bits emu {emu_bits:.2f} native {nat_bits:.2f}", flush=True)
    assert emu_bits >= nat_bits


def _wide(shape, g):
    s = torch.randint(0, 2, shape, generator=g) * 2 - 1
    m = 1 + torch.rand(shape, generator=g, dtype=torch.float64)
    e = torch.randint(-20, 21, shape, generator=g)
    return s * torch.ldexp(m, e)


def test_c3a_wide_range_4096(dev):
    print("case c3a mm_nt 4096^3 wide range", flush=True)
    n = 4096
    A = _wide((n, n), _gen(3000)).to(dev)
    Bt = _wide((n, n), _gen(3001)).to(dev)
    out, be, _, ws = whole_parity("mm_nt", A, Bt, O.PRIMES[:14])
    del ws
    assert abs(be - 50) <= 1
    emu_bits, nat_bits = _native_and_emu_bits(out, A, Bt)
    print(f"c3a bits_eff {be} correct bits emu {emu_bits:.2f} native {nat_bits:.2f}", flush=True)
    assert emu_bits >= nat_bits


def test_c3b_integer_exact_4096(dev):
    """Integers in [-2^20, 2^20]: |C| <= 2^52, so every partial sum of the
    native product is an exact integer too; the emulated output is bit-exact
    and the correction products are all zero."""
    print("case c3b mm_nt 4096^3 integers", flush=True)
    n = 4096
    A = torch.randint(-2 ** 20, 2 ** 20 + 1, (n, n), generator=_gen(3100)).double().to(dev)
    Bt = torch.randint(-2 ** 20, 2 ** 20 + 1, (n, n), generator=_gen(3101)).double().to(dev)
    out, be, lay, ws = whole_parity("mm_nt", A, Bt, O.PRIMES[:14])
    assert abs(be - 49) <= 1
    assert torch.equal(out, A @ Bt)
    rows = _rows(n, 7, 8)
    exact = A.cpu().numpy()[rows].astype(np.int64) @ Bt.cpu().numpy().astype(np.int64)
    assert np.array_equal(out.cpu().numpy()[rows], exact.astype(np.float64))
    cz = ws[lay.off_corr:lay.off_corr + 4 * lay.ncorr * lay.outplane_bytes]
    assert lay.ncorr >= 1 and not cz.any().item(), "correction products must vanish"


def test_c4_bmm_64x512(dev):
    print("case c4 bmm_nt 64 x 512^3", flush=True)
    A = torch.randn((64, 512, 512), dtype=torch.float64, generator=_gen(4000)).to(dev)
    Bt = torch.randn((64, 512, 512), dtype=torch.float64, generator=_gen(4001)).to(dev)
    P, corr = emu.plan_config(512)
    out, _, lay = check_call("bmm_nt", A, Bt, O.PRIMES[:P], use_corr=corr, full_oracle=False)
    assert torch.equal(out, emu.bmm_nt(A, Bt))
    ref = torch.bmm(A, Bt)
    for b in (0, 31, 63):
        hi, lo = capi.ddgemm_nt(A[b], Bt[b].t().contiguous())
        torch.cuda.synchronize()
        h, l = hi.cpu().numpy(), lo.cpu().numpy()
        assert O.correct_bits(out[b].cpu().numpy(), h, l) >= O.correct_bits(ref[b].cpu().numpy(), h, l)


@pytest.mark.parametrize("P,corr", [(15, True), (13, False)])
def test_c5_ragged_deep_k(dev, P, corr):
    print(f"case c5 mm_nt 1023x2049x32769 P={P} corr={corr}", flush=True)
    M, N, K = 1023, 2049, 32769
    A = (torch.rand((M, K), dtype=torch.float64, generator=_gen(5000)) * 2 - 1).to(dev)
    Bt = (torch.rand((K, N), dtype=torch.float64, generator=_gen(5001)) * 2 - 1).to(dev)
    if corr:
        assert emu.plan_config(K) == (P, corr)
    expect_be = 51 if corr else 43
    out, be, lay, ws = whole_parity("mm_nt", A, Bt, O.PRIMES[:P], use_corr=corr)
    del ws
    assert abs(be - expect_be) <= 1
    assert torch.equal(out, emu.mm_nt(A, Bt, nprimes=P, corr=corr))
    emu_bits, nat_bits = _native_and_emu_bits(out, A, Bt)
    print(f"c5 P={P} bits_eff {be} correct bits emu {emu_bits:.2f} native {nat_bits:.2f}",
          flush=True)
    if corr:
        assert emu_bits >= nat_bits
    else:
        assert emu_bits >= 40.0
