"""GPU parity of every stage of the HIP path against the CPU oracle, through
the C ABI, on seeded CPU-generated inputs (configs c1, odd and ragged shapes,
batched layouts, reduced and inexact operating points)."""
import numpy as np
import pytest
import torch

import oracle as O
from parity_util import check_call, sampled_parity

pytestmark = pytest.mark.gpu


def _randn(shape, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, dtype=torch.float64, generator=g).to(dev)


CASES = [
    # kind, batch, M, N, K, nprimes, corr
    ("mm_nt", 1, 128, 128, 4096, 14, True),     # c1 plumbing config
    ("mm_nt", 1, 17, 29, 23, 14, True),
    ("mm", 1, 129, 127, 4095, 14, True),
    ("mm", 1, 300, 520, 200, 15, True),
    ("mm_nt", 1, 257, 255, 129, 13, False),     # reduced operating point
    ("bmm_nt", 3, 100, 77, 333, 14, True),
    ("bmm", 5, 96, 64, 256, 14, True),
    ("mm", 1, 64, 48, 64, 20, True),
    ("mm_nt", 1, 64, 40, 100_000, 15, True),    # two int32 correction planes, K-split 16
    # >= 4096 short rows (one wave per row in the sizing), odd row counts
    ("bmm", 9, 301, 256, 300, 14, True),         # A and B rows, 5013 in all
    ("bmm_nt", 17, 257, 100, 448, 13, True),     # A's 4369 rows beside the column slabs
]


@pytest.mark.parametrize("kind,batch,M,N,K,P,corr", CASES)
def test_stage_parity(dev, kind, batch, M, N, K, P, corr):
    print(f"case {kind} b={batch} {M}x{N}x{K} P={P} corr={corr}", flush=True)
    seed = 1000 * batch + M + 7 * N + 13 * K
    if kind in ("bmm", "bmm_nt"):
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, K, N) if kind == "bmm_nt" else (batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, O.PRIMES[:P], use_corr=corr)


MODULI_ORDERS = [
    # odd first modulus, 256 later: an even digit past the first
    [255, 256, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199],
    # even first modulus other than 256: the first digit's own balancing
    [254, 255, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199],
    # small moduli (largest quotients in the digit steps), 16 in the middle
    [7, 11, 13, 16, 9, 5, 17, 19, 23, 29, 31, 37, 41, 43],
]


@pytest.mark.parametrize("order", range(len(MODULI_ORDERS)))
@pytest.mark.parametrize("kind,M,N,K", [("mm_nt", 70, 90, 700), ("mm_nt", 33, 40, 40_000)])
def test_moduli_orders(dev, order, kind, M, N, K):
    """Admissible modulus sets outside the default order run the generic
    reconstruction, whose digits keep barrett_bal32's balanced range for even
    moduli; the second shape goes through the K-split fold."""
    primes = MODULI_ORDERS[order]
    print(f"case moduli order {order} {kind} {M}x{N}x{K}", flush=True)
    A = _randn((M, K), 50 + order, dev)
    B = _randn((K, N), 60 + order, dev)
    check_call(kind, A, B, primes)


def test_inexact_parity(dev):
    print("case inexact mm_nt 96x80x1000", flush=True)
    A = _randn((96, 1000), 5, dev)
    B = _randn((1000, 80), 6, dev)
    check_call("mm_nt", A, B, O.PRIMES[:14], exact=False)


def test_narrow_bits_parity(dev):
    print("case bits=40 mm 64x64x512", flush=True)
    A = _randn((64, 512), 7, dev)
    B = _randn((64, 512), 8, dev)
    check_call("mm", A, B, O.PRIMES[:O.plan(512, 40)], bits=40)


def test_wide_range_parity(dev):
    """c3a-style entries sign * U[1,2) * 2^e, e in [-20, 20]."""
    print("case wide-range mm_nt 200x150x700", flush=True)
    g = torch.Generator().manual_seed(31)
    def wide(shape):
        s = torch.randint(0, 2, shape, generator=g) * 2 - 1
        m = 1 + torch.rand(shape, generator=g, dtype=torch.float64)
        e = torch.randint(-20, 21, shape, generator=g)
        return (s * m * torch.pow(2.0, e.double())).to(dev)
    check_call("mm_nt", wide((200, 700)), wide((700, 150)), O.PRIMES[:14])


@pytest.mark.parametrize("P", list(range(1, 21)))
def test_full_range_every_modulus_count(dev, P):
    """Aligned operands (entries 1 + small noise, rows of either sign) make
    the Cauchy-Schwarz bound nearly tight, so the products reach the top of
    the CRT range and the highest Garner digit is nonzero: every group split
    of the reconstruction (1..20 moduli) against the oracle."""
    print(f"case full-range mm_nt 96x80x512 P={P}", flush=True)
    g = torch.Generator().manual_seed(700 + P)
    A = 1 + 0.01 * torch.randn((96, 512), dtype=torch.float64, generator=g)
    A[::3] *= -1
    B = 1 + 0.01 * torch.randn((512, 80), dtype=torch.float64, generator=g)
    B[:, ::5] *= -1
    check_call("mm_nt", A.to(dev), B.to(dev), O.PRIMES[:P], use_corr=P >= 12)


DEEP_CASES = [
    # kind, batch, M, N, K, nprimes, corr, exact
    ("mm", 1, 40, 24, 140_000, 15, True, True),        # 3 segments, ragged last
    ("mm", 1, 33, 17, 196_609, 16, True, True),        # last segment one column deep
    ("mm", 1, 29, 31, 131_072, 15, False, True),       # first K past the single-launch bound
    ("bmm", 2, 24, 16, 135_000, 15, True, False),
]


@pytest.mark.parametrize("kind,batch,M,N,K,P,corr,exact", DEEP_CASES)
def test_deep_k_parity(dev, kind, batch, M, N, K, P, corr, exact):
    """K-segmented path (K > 131071, B as [N, K]): sizing and the whole
    output bit-exact against the oracle's segmented pipeline."""
    from parity_util import bits_equal, oracle_sizing
    from fp64_emu import capi
    print(f"case deep-K {kind} b={batch} {M}x{N}x{K} P={P} corr={corr} exact={exact}", flush=True)
    shapeA = (batch, M, K) if kind == "bmm" else (M, K)
    shapeB = (batch, N, K) if kind == "bmm" else (N, K)
    A = _randn(shapeA, K + M, dev)
    B = _randn(shapeB, K + N, dev)
    out, ws, lay = capi.run(kind, A, B, O.PRIMES[:P], exact=exact, use_corr=corr)
    torch.cuda.synchronize()
    assert lay.deep == 1 and lay.nseg == (K + 65535) // 65536
    gsA, gsB, _, _, gbe = capi.sizing(ws[:lay.off_planesA].cpu().numpy(), lay)
    Ah, Bh = A.cpu().numpy(), B.cpu().numpy()
    obe, osA, osB, _, _ = oracle_sizing(Ah, Bh, False, O.PRIMES[:P], 53)
    assert gbe == obe and np.array_equal(gsA, osA) and np.array_equal(gsB, osB)
    oout, info = O.mm(Ah, Bh, 0, O.PRIMES[:P], exact=exact, use_corr=corr)
    assert info["bits_eff"] == gbe
    assert bits_equal(out.cpu().numpy(), oout), "deep-K output differs from the oracle"


@pytest.mark.parametrize("kind,M,N,K", [("mm_nt", 1000, 700, 3000), ("mm", 777, 300, 1500),
                                        ("mm_nt", 2000, 100, 4096),
                                        ("mm_nt", 1300, 900, 700),    # shallow: slot runs
                                        ("mm_nt", 4096, 2048, 3000)])  # item streams (full run)
def test_row_chunks_match_full(dev, kind, M, N, K):
    """A workspace below the full size runs the rows of A in chunks against
    one extraction of B; the output is bit-identical to the full run, at
    the minimum workspace and at one in between."""
    from fp64_emu import capi
    print(f"case row-chunks {kind} {M}x{N}x{K}", flush=True)
    A = _randn((M, K), M + K, dev)
    B = _randn((K, N) if kind == "mm_nt" else (N, K), N + K, dev)
    P = 14
    full, _, _ = capi.run(kind, A, B, O.PRIMES[:P])
    wfull = capi.workspace_size(1, M, N, K, P, True)
    wmin = capi.workspace_size_min(1, M, N, K, P, True)
    assert wmin < wfull
    for wbytes in (wmin, (wmin + wfull) // 2):
        ws = torch.empty(wbytes, dtype=torch.uint8, device=dev)
        out, _, _ = capi.run(kind, A, B, O.PRIMES[:P], ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(out, full), f"workspace {wbytes}"
    # The chunked run at the minimum workspace against the oracle itself, at
    # rows across chunk boundaries (256-row multiples) and both ends.
    ws = torch.empty(wmin, dtype=torch.uint8, device=dev)
    rows = sorted({0, 1, 255, 256, 511, 512, M // 2, M - 2, M - 1} & set(range(M)))
    cols = sorted({0, 1, N // 3, N - 1})
    out, _, lay, _ = sampled_parity(kind, A, B, O.PRIMES[:P], rows, cols, ws=ws)
    assert torch.equal(out, full)
    with pytest.raises(capi.CapiError, match="workspace too small"):
        capi.run(kind, A, B, O.PRIMES[:P], ws=torch.empty(wmin - 256, dtype=torch.uint8, device=dev))


@pytest.mark.parametrize("order", [1, 2])
def test_deep_k_moduli_orders(dev, order):
    """K-segmented path with a modulus list outside the default: the
    segment residue sums fold in the generic reconstruction (an even first
    modulus other than 256; small moduli)."""
    from parity_util import bits_equal
    from fp64_emu import capi
    primes = MODULI_ORDERS[order]
    M, N, K = 8, 12, 140_000
    print(f"case deep-K moduli order {order} mm {M}x{N}x{K}", flush=True)
    A = _randn((M, K), 90 + order, dev)
    B = _randn((N, K), 95 + order, dev)
    out, ws, lay = capi.run("mm", A, B, primes)
    torch.cuda.synchronize()
    assert lay.deep == 1
    oout, info = O.mm(A.cpu().numpy(), B.cpu().numpy(), 0, primes)
    assert bits_equal(out.cpu().numpy(), oout), "deep-K output differs from the oracle"


def test_non_finite_entries(dev):
    """Infinities and NaNs contribute 0, as the reference's integer split of
    their encoding (fp64_emu_cuda/fp64_emu.cu:300-321) gives; the rows and
    columns holding them keep the unnarrowed shift (bits - 1, fp64_emu.cu:138)
    and fall back to the worst-case width (:213-216).  Entries here stay below
    4 in magnitude, where the reference's 64-bit split of such rows does not
    wrap, so every stage matches the oracle."""
    print("case non-finite entries mm_nt 48x40x300", flush=True)
    g = torch.Generator().manual_seed(77)
    A = 0.5 * torch.randn((48, 300), dtype=torch.float64, generator=g)
    B = 0.5 * torch.randn((300, 40), dtype=torch.float64, generator=g)
    A[3, 10] = float("inf")
    A[5, :] = float("inf")
    A[7, 20] = float("nan")
    A[9, 1] = float("-inf")
    B[2, 7] = float("nan")
    B[:, 11] = float("-inf")
    B[40, 3] = float("inf")
    out, _, _ = check_call("mm_nt", A.to(dev), B.to(dev), O.PRIMES[:14])
    assert torch.isfinite(out).all()


def test_extreme_magnitudes(dev):
    """Rows scaled by 2^±990 (shifts far outside int8 widths): products that
    overflow to infinity or underflow to subnormals and zero after the final
    ldexp, against the oracle bit for bit."""
    print("case extreme magnitudes mm_nt 40x36x200", flush=True)
    g = torch.Generator().manual_seed(88)
    A = torch.randn((40, 200), dtype=torch.float64, generator=g)
    B = torch.randn((200, 36), dtype=torch.float64, generator=g)
    A[:10] *= 2.0 ** 990
    A[10:20] *= 2.0 ** -990
    A[20:24] *= 2.0 ** -1060            # subnormal rows
    B[:, :9] *= 2.0 ** 990
    B[:, 9:18] *= 2.0 ** -990
    out, _, _ = check_call("mm_nt", A.to(dev), B.to(dev), O.PRIMES[:14])
    o = out.cpu()
    assert torch.isinf(o[:10, :9]).any() and (o[10:20, 9:18] == 0).any()


@pytest.mark.parametrize("kind", ["mm_nt", "mm"])
def test_int32_accumulation_bound(dev, kind):
    """K = 131071, the deepest single launch, with every residue modulo 256
    at -128: the p = 256 slot accumulates K * 2^14 = 2^31 - 2^14, the largest
    sum the int32 GEMM must hold (fp64_emu.cu's K bound).  x = 1 + 2^-42 puts
    its lowest set bit at 2^7 after the shift the plan gives (be = 50)."""
    from parity_util import oracle_sizing
    M = N = 16
    K = 131071
    print(f"case int32 bound {kind} {M}x{N}x{K}", flush=True)
    x = 1.0 + 2.0 ** -42
    A = torch.full((M, K), x, dtype=torch.float64)
    Bt = torch.full((K, N), x, dtype=torch.float64)
    A[::2] *= -1.0
    Bt[:, ::3] *= -1.0
    primes = O.PRIMES[:15]                      # plan_config(131071)
    be, sA, _, _, _ = oracle_sizing(A.numpy(), Bt.numpy(), True, np.asarray(primes, np.int32), 53)
    res = np.asarray(O.extract_operand(A.numpy()[None], 0, sA, be, np.asarray(primes, np.int32),
                                       True)[0])
    assert be == 50 and np.all(np.abs(res[0, 0].astype(np.int32)) == 128)
    B = Bt if kind == "mm_nt" else Bt.t().contiguous()
    out, _, _ = check_call(kind, A.to(dev), B.to(dev), primes)
    sign = torch.outer(torch.tensor([-1.0 if i % 2 == 0 else 1.0 for i in range(M)], dtype=torch.float64),
                       torch.tensor([-1.0 if j % 3 == 0 else 1.0 for j in range(N)], dtype=torch.float64))
    assert torch.equal(out.cpu(), sign * (K * x * x))


def _slab_rows(NF, K):
    """Rows per column slab of a [K, NF] operand (the reference's slab split)."""
    nsl0 = min(max(131072 // NF, 1), 128)
    return -(-K // nsl0)


SIZING_FORM_CASES = [
    # kind, batch, M, N, K -- the sizing form in the comment
    ("mm_nt", 1, 8, 1024, 32768),    # slabs of 256 rows: one launch (row and column groups)
    ("mm_nt", 1, 8, 1024, 32769),    # 257 rows: slab partials, then their fold
    ("bmm_nt", 3, 5, 77, 700),       # 117 slabs, 8 columns per group straddling members
    ("bmm_nt", 2, 300, 1, 2000),     # one column per member
    ("mm_nt", 1, 4500, 40, 9),       # rows past 4096: a wave per row, 16 rows per group
    ("mm_nt", 1, 2048, 2048, 64),    # 4096 rows and columns: the width pick in the extraction
    ("mm_nt", 1, 2049, 2048, 64),    # 4097: the width pick's own launch
    ("mm", 1, 1000, 3000, 100),      # rows of both operands, pick in the extraction
]


@pytest.mark.parametrize("kind,batch,M,N,K", SIZING_FORM_CASES)
def test_sizing_forms(dev, kind, batch, M, N, K):
    """Each form of the sizing (one launch for rows and shallow column slabs
    folded in LDS, or slab partials then their fold; the width pick in its
    own launch or inside the extraction) against the oracle, on operands
    whose rows and columns span 2^-40 .. 2^40, so that every row and column
    takes its own shift."""
    from fp64_emu import capi
    print(f"case sizing form {kind} b={batch} {M}x{N}x{K}", flush=True)
    if kind.endswith("_nt"):
        fused = _slab_rows(batch * N, K) <= 256
        print(f"  column slabs of {_slab_rows(batch * N, K)} rows: {'one launch' if fused else 'two'}",
              flush=True)
    g = torch.Generator().manual_seed(4100 + M + N + K)
    sa = torch.pow(2.0, torch.randint(-40, 41, (batch, M, 1), generator=g).double())
    sb = torch.pow(2.0, torch.randint(-40, 41, (batch, 1, N), generator=g).double())
    A = torch.randn((batch, M, K), dtype=torch.float64, generator=g) * sa
    Bt = torch.randn((batch, K, N), dtype=torch.float64, generator=g) * sb
    B = Bt if kind.endswith("_nt") else Bt.transpose(1, 2).contiguous()
    if batch == 1 and not kind.startswith("bmm"):
        A, B = A[0], B[0]
    check_call(kind, A.to(dev), B.to(dev), O.PRIMES[:14])


@pytest.mark.parametrize("kind,batch,M,N,K,P,exact", [
    ("bmm", 2, 40, 30, 5000, 14, True),       # K-split with batch > 1 (split-major planes)
    ("mm_nt", 1, 50, 60, 20000, 15, False),   # K-split, inexact combine
    ("mm_nt", 1, 33, 20, 6000, 10, True),     # K-split, generic reconstruction (10 moduli)
])
def test_ksplit_variants(dev, kind, batch, M, N, K, P, exact):
    from fp64_emu import capi
    print(f"case K-split {kind} b={batch} {M}x{N}x{K} P={P} exact={exact}", flush=True)
    if kind == "bmm":
        A = _randn((batch, M, K), 300 + M, dev)
        B = _randn((batch, N, K), 301 + N, dev)
    else:
        A = _randn((M, K), 300 + M, dev)
        B = _randn((K, N), 301 + N, dev)
    assert capi.layout(batch, M, N, K, P, True).ksplit > 1
    check_call(kind, A, B, O.PRIMES[:P], exact=exact)


NARROW_CASES = [
    # kind, batch, M, N, K, moduli, corr -- k-steps per residue group in the comment
    ("bmm_nt", 40, 100, 100, 64, O.PRIMES[:14], True),     # 1 (corr 2), one column tile
    ("bmm", 6, 300, 260, 200, O.PRIMES[:14], True),        # 4 (corr 8), three column tiles
    ("bmm", 8, 260, 300, 1000, O.PRIMES[:14], True),       # 16 (corr 32), steady loop
    ("mm_nt", 1, 1536, 1100, 700, O.PRIMES[:15], True),    # 11, odd step count
    ("bmm_nt", 20, 256, 380, 320, O.PRIMES[:13], False),   # 5, no correction
    ("mm_nt", 1, 1536, 1100, 2000, O.PRIMES[:14], True),   # 32: one slot per group
    ("bmm", 40, 64, 64, 128, MODULI_ORDERS[1], True),      # 2, even modulus 254 (tie fix)
]


@pytest.mark.parametrize("kind,batch,M,N,K,primes,corr", NARROW_CASES)
def test_narrow_tile_parity(dev, kind, batch, M, N, K, primes, corr):
    """Products whose 256-column tiles would be mostly padding run 128-column
    tiles (two work groups per CU, one residue slot each): every stage
    against the oracle."""
    from fp64_emu import capi
    print(f"case narrow GEMM {kind} b={batch} {M}x{N}x{K} P={len(primes)} corr={corr}", flush=True)
    assert capi.layout(batch, M, N, K, len(primes), corr).gemm_tile_cols == 128
    seed = 700 + batch + M + N + K
    if kind in ("bmm", "bmm_nt"):
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, K, N) if kind == "bmm_nt" else (batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, primes, use_corr=corr)


@pytest.mark.parametrize("kind,batch,M,N,K", [
    ("mm", 1, 300, 1290, 2200),       # last tile column: 10 of 256 columns
    ("mm_nt", 1, 64, 1300, 20000),    # the same under a K-split
    ("bmm", 48, 60, 1408, 130),       # 128 of 256: the narrow half exactly full
])
def test_mixed_tile_parity(dev, kind, batch, M, N, K):
    """Wide GEMM tiles whose last tile column holds at most 128 columns of N
    run that column as 128-column tiles in the same launch."""
    from fp64_emu import capi
    print(f"case mixed tiles {kind} b={batch} {M}x{N}x{K}", flush=True)
    L = capi.layout(batch, M, N, K, 14, True)
    assert L.gemm_tile_cols == 256 and 0 < N % 256 <= 128 and L.Np // 256 >= 2
    seed = 900 + M + N + K
    if kind == "bmm":
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, O.PRIMES[:14])


@pytest.mark.parametrize("kind,batch,M,N,K", [
    ("mm_nt", 1, 128, 128, 4096),     # c1: one 128 x 128 tile, K-split 8
    ("bmm", 3, 100, 77, 333),         # batched, ragged
    ("mm", 1, 300, 520, 200),         # 3 x 5 tiles of 128 x 128
])
def test_small_tile_parity(dev, kind, batch, M, N, K):
    """128 x 128 GEMM tiles where both 128-row and 128-column tiles cut the
    padded work: every stage against the oracle."""
    from fp64_emu import capi
    print(f"case small tiles {kind} b={batch} {M}x{N}x{K}", flush=True)
    L = capi.layout(batch, M, N, K, 14, True)
    assert L.gemm_tile_rows == 128 and L.gemm_tile_cols == 128
    seed = 1300 + M + N + K
    if kind == "bmm":
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, O.PRIMES[:14])


RUN_CASES = [
    # kind, batch, M, N, K, moduli, corr, tile (rows, cols) -- k-steps per slot in the comment.
    # One run of every residue slot per tile: 256 x 256 output tiles in whole rounds of the
    # 256 CUs, hence the batch counts and sizes.
    ("bmm_nt", 128, 300, 200, 256, O.PRIMES[:14], True, (256, 256)),   # 4
    ("mm", 1, 4000, 4000, 150, O.PRIMES[:13], False, None),            # 3, odd stream of 39 steps
    ("mm_nt", 1, 4096, 4096, 64, O.PRIMES[:20], True, (256, 256)),     # 1, every modulus
    ("mm", 1, 4096, 4096, 50, O.PRIMES[:2], True, None),               # 1, a run of two slots
    ("bmm", 256, 200, 200, 200, MODULI_ORDERS[1], True, None),         # 4, even modulus 254
    ("bmm_nt", 256, 240, 250, 64, O.PRIMES[:14], True, (256, 256)),   # 1, one tile per member
    # Deeper slots (the c4 shape's 8 k-steps and more): streams of 9 to 32 k-steps per slot.
    ("bmm_nt", 16, 1024, 1000, 1000, O.PRIMES[:14], True, (256, 256)),  # 16, ragged K and N
    ("mm", 1, 4096, 4096, 520, O.PRIMES[:13], False, None),            # 9, no correction slot
    ("bmm", 256, 200, 200, 700, MODULI_ORDERS[1], True, None),         # 11, even modulus 254
    ("mm_nt", 1, 4096, 4096, 2048, O.PRIMES[:3], True, (256, 256)),    # 32, a run of three slots
]


@pytest.mark.parametrize("kind,batch,M,N,K,primes,corr,tile", RUN_CASES)
def test_slot_run_parity(dev, kind, batch, M, N, K, primes, corr, tile):
    """Shallow products run each tile's residue slots back to back in one
    work group (one stream of operand copies across the slots; residues
    stored at each slot's end): every stage against the oracle."""
    from fp64_emu import capi
    P = len(primes)
    print(f"case slot runs {kind} b={batch} {M}x{N}x{K} P={P} corr={corr}", flush=True)
    L = capi.layout(batch, M, N, K, P, corr)
    assert L.gemm_run == P and L.ksplit == 1
    if tile is not None:
        assert (L.gemm_tile_rows, L.gemm_tile_cols) == tile
    seed = 1700 + batch + M + N + K + P
    if kind in ("bmm", "bmm_nt"):
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, K, N) if kind == "bmm_nt" else (batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, primes, use_corr=corr)



THREE_RUN_CASES = [
    # kind, batch, M, N, K, moduli, corr, expected slots per run.
    # Past 256 output tiles of 256 x 256 and off whole rounds of CUs: each tile's slots
    # split into three runs, the last one shorter.
    ("bmm_nt", 300, 240, 250, 64, O.PRIMES[:14], True, 5),             # 300 tiles: 5, 5, 4
    ("bmm", 270, 250, 250, 100, MODULI_ORDERS[1], True, 5),            # even modulus 254
    ("mm", 1, 4352, 4352, 100, O.PRIMES[:13], False, 5),               # 289 tiles: 5, 5, 3
    ("mm_nt", 1, 4200, 4500, 120, O.PRIMES[:20], True, 7),             # 306 tiles: 7, 7, 6
    ("bmm_nt", 300, 240, 250, 512, O.PRIMES[:14], True, 5),            # 8 k-steps per slot
]


@pytest.mark.parametrize("kind,batch,M,N,K,primes,corr,run", THREE_RUN_CASES)
def test_split_slot_run_parity(dev, kind, batch, M, N, K, primes, corr, run):
    """Shallow products whose output tiles do not fill whole rounds of CUs:
    each tile's residue slots split over three run groups (every group
    starts its own operand stream at its run's first plane): every stage
    against the oracle."""
    from fp64_emu import capi
    P = len(primes)
    print(f"case split slot runs {kind} b={batch} {M}x{N}x{K} P={P} corr={corr} run={run}", flush=True)
    L = capi.layout(batch, M, N, K, P, corr)
    assert (L.gemm_run, L.ksplit, L.gemm_tile_rows, L.gemm_tile_cols) == (run, 1, 256, 256)
    seed = 2700 + batch + M + N + K + P
    if kind in ("bmm", "bmm_nt"):
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, K, N) if kind == "bmm_nt" else (batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, primes, use_corr=corr)


FEW_TILE_CASES = [
    # kind, batch, M, N, K, moduli, corr, (tile rows, cols).
    # Shallow products of fewer than 256 output tiles of 256 x 256: one slot per group on
    # 256 x 128 tiles, on 128 x 128 tiles at 40 tiles or fewer.
    ("mm_nt", 1, 1792, 2560, 256, O.PRIMES[:14], True, (256, 128)),    # 70 tiles
    ("mm", 1, 2560, 2560, 200, O.PRIMES[:13], False, (256, 128)),      # 100 tiles
    ("mm_nt", 1, 1280, 2048, 320, O.PRIMES[:20], True, (128, 128)),    # 40 tiles
    ("bmm", 8, 300, 400, 256, O.PRIMES[:14], True, (128, 128)),        # 32 tiles
    ("bmm_nt", 32, 500, 500, 128, O.PRIMES[:14], True, (256, 128)),    # 128 tiles
    ("bmm", 90, 240, 250, 192, MODULI_ORDERS[1], True, (256, 128)),    # even modulus 254
    ("bmm", 20, 240, 240, 1800, O.PRIMES[:14], True, (128, 128)),      # 29 k-steps per slot
]


@pytest.mark.parametrize("kind,batch,M,N,K,primes,corr,tile", FEW_TILE_CASES)
def test_few_tile_parity(dev, kind, batch, M, N, K, primes, corr, tile):
    """Shallow products with fewer output tiles than CUs run one residue slot
    per work group on the narrow launches: every stage against the oracle."""
    from fp64_emu import capi
    P = len(primes)
    print(f"case few tiles {kind} b={batch} {M}x{N}x{K} P={P} corr={corr} tile={tile}", flush=True)
    L = capi.layout(batch, M, N, K, P, corr)
    assert (L.gemm_run, L.ksplit, L.gemm_tile_rows, L.gemm_tile_cols) == (1, 1) + tile
    seed = 2700 + batch + M + N + K + P
    if kind in ("bmm", "bmm_nt"):
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, K, N) if kind == "bmm_nt" else (batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, primes, use_corr=corr)


def test_deep_slot_runs_sampled(dev):
    """Slot runs at their depth limit on 256 x 256 tiles (4096 x 4096 x 2048:
    256 tiles, one run of 14 slots of 32 k-steps each): the sizing and
    sampled outputs against the oracle, first and last rows and columns
    included."""
    from fp64_emu import capi
    from parity_util import sampled_parity
    n, K = 4096, 2048
    print(f"case deep slot runs mm_nt {n}x{n}x{K} sampled", flush=True)
    L = capi.layout(1, n, n, K, 14, True)
    assert (L.gemm_run, L.ksplit, L.gemm_tile_rows, L.gemm_tile_cols) == (14, 1, 256, 256)
    A = _randn((n, K), 2801, dev)
    Bt = _randn((K, n), 2802, dev)
    rng = np.random.default_rng(2803)
    rows = [0, 255, 256, n - 1] + list(rng.integers(0, n, 12))
    cols = [0, 255, 256, n - 1] + list(rng.integers(0, n, 12))
    sampled_parity("mm_nt", A, Bt, O.PRIMES[:14], rows, cols)


def _item_stream(L, N):
    """The GEMM launch runs work groups of several items, each over its items
    as one stream (256 x 256 tiles, one slot per item of at most 64 k-steps,
    no K-split, at least 512 items)."""
    Np = -(-N // 256) * 256
    mixed = Np // 256 >= 2 and N % 256 != 0 and N % 256 <= 128
    items = (L.nprimes + L.ncorr) * L.batch * (L.chunk_rows // 256) * (Np // 256)
    return (not L.deep and L.gemm_run == 1 and L.ksplit == 1 and not mixed
            and (L.gemm_tile_rows, L.gemm_tile_cols) == (256, 256) and items >= 512
            and -(-L.K // 64) <= 64)


STREAM_CASES = [
    # kind, batch, M, N, K, moduli, corr -- items (tiles x slots) in the comment.
    ("mm", 1, 2304, 2560, 3000, O.PRIMES[:14], True),     # 1350: five whole rounds and 70
    ("bmm", 3, 1024, 1024, 2500, MODULI_ORDERS[1], True),  # 720, even modulus 254
    ("bmm_nt", 2, 1536, 1792, 2100, O.PRIMES[:13], False), # 1092, no correction slot
    ("mm_nt", 1, 2048, 2048, 2200, O.PRIMES[:20], True),  # 1344, every modulus
    ("mm_nt", 1, 3072, 2048, 4096, O.PRIMES[:14], True),  # 1440, 64 k-steps (the limit)
]


@pytest.mark.parametrize("kind,batch,M,N,K,primes,corr", STREAM_CASES)
def test_item_stream_parity(dev, kind, batch, M, N, K, primes, corr):
    """Products of many 256 x 256 tiles at 33 to 64 k-steps per slot run the
    GEMM in work groups of eight items, each over its items as one stream of
    operand copies (the items of a group in different tiles, slots and
    members; correction items twice as deep; the last groups with fewer
    items): every stage against the oracle."""
    from fp64_emu import capi
    P = len(primes)
    print(f"case item stream {kind} b={batch} {M}x{N}x{K} P={P} corr={corr}", flush=True)
    assert _item_stream(capi.layout(batch, M, N, K, P, corr), N)
    seed = 3700 + batch + M + N + K + P
    if kind in ("bmm", "bmm_nt"):
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, K, N) if kind == "bmm_nt" else (batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, primes, use_corr=corr)



def test_item_stream_random_whole_parity(dev):
    """Eight seeded random products that take the item stream (mm and mm_nt,
    12 to 20 moduli, with and without the correction, exact and fp64
    combines; normal, wide-range and integer entries): every output element
    bit for bit against the oracle pipeline (BLAS modular products)."""
    from fp64_emu import capi
    from parity_util import whole_parity
    rng = np.random.default_rng(4711)
    done = 0
    while done < 8:
        kind = str(rng.choice(["mm", "mm_nt"]))
        M, N = (int(x) for x in rng.integers(1300, 3400, 2))
        K = int(rng.integers(2060, 4097))
        P = int(rng.integers(12, 21))
        corr, exact = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
        dist = int(rng.integers(0, 3))
        seed = int(rng.integers(1 << 30))
        if not _item_stream(capi.layout(1, M, N, K, P, corr), N):
            continue
        print(f"case random item stream {kind} {M}x{N}x{K} P={P} corr={corr} exact={exact} "
              f"dist={dist}", flush=True)
        g = torch.Generator().manual_seed(seed)

        def gen(shape):
            if dist == 0:
                return torch.randn(shape, dtype=torch.float64, generator=g)
            if dist == 1:
                s = torch.randint(0, 2, shape, generator=g) * 2 - 1
                m = 1 + torch.rand(shape, generator=g, dtype=torch.float64)
                return s * torch.ldexp(m, torch.randint(-30, 31, shape, generator=g))
            return torch.randint(-2 ** 20, 2 ** 20 + 1, shape, generator=g).double()
        A = gen((M, K)).to(dev)
        B = gen((K, N) if kind == "mm_nt" else (N, K)).to(dev)
        whole_parity(kind, A, B, O.PRIMES[:P], exact=exact, use_corr=corr)
        done += 1
        del A, B


def _split_stream(L):
    """The GEMM runs split streams: one work group per CU, each XCD's groups
    over an eighth of the K-deep (tile, slot) units' k-steps in blocks of 32
    units, with two K-split planes."""
    return L.gemm_split == 1 and L.ksplit == 2 and not L.deep


SPLIT_CASES = [
    # kind, batch, M, N, K, moduli, corr -- units (tiles x slots) in the comment.
    ("mm_nt", 1, 1000, 1000, 16384, O.PRIMES[:14], True),     # 256: 8 blocks, the fewest
    ("mm", 1, 300, 2000, 17000, O.PRIMES[:15], True),         # 272: a last block of 16 units
    ("bmm_nt", 2, 300, 1000, 20000, MODULI_ORDERS[1], True),  # 256 over 2 members, modulus 254
    ("mm_nt", 1, 1000, 2000, 16384, O.PRIMES[:13], False),    # 416, no correction slots
    ("mm", 1, 1000, 1000, 16384, O.PRIMES[:20], True),        # 352, every modulus
    ("bmm", 2, 300, 1000, 20000, O.PRIMES[:15], True),        # 272 of 313 k-steps
]


@pytest.mark.parametrize("kind,batch,M,N,K,primes,corr", SPLIT_CASES)
def test_split_stream_parity(dev, kind, batch, M, N, K, primes, corr):
    """Deep products of few tiles run split streams (each unit in one or two
    K ranges, a unit taken whole also storing zeros as its second split; the
    workspace is filled with a nonzero byte first): every stage against the
    oracle."""
    from fp64_emu import capi
    P = len(primes)
    print(f"case split stream {kind} b={batch} {M}x{N}x{K} P={P} corr={corr}", flush=True)
    assert _split_stream(capi.layout(batch, M, N, K, P, corr))
    seed = 5100 + batch + M + N + K + P
    if kind in ("bmm", "bmm_nt"):
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, K, N) if kind == "bmm_nt" else (batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, primes, use_corr=corr)


@pytest.mark.parametrize("P,corr", [(15, True), (13, False)])
def test_split_stream_deep_whole_parity(dev, P, corr):
    """c5's depth with 2048 columns (mm_nt 1023 x 2048 x 32769: 4 x 8 tiles,
    units of 513 k-steps, 17 or 13 blocks of 32): the whole output bit for bit
    against the oracle, the default plan and the reduced one."""
    from fp64_emu import capi
    from parity_util import whole_parity
    M, N, K = 1023, 2048, 32769
    print(f"case split stream whole mm_nt {M}x{N}x{K} P={P} corr={corr}", flush=True)
    assert _split_stream(capi.layout(1, M, N, K, P, corr))
    whole_parity("mm_nt", _randn((M, K), 6101, dev), _randn((K, N), 6102, dev), O.PRIMES[:P],
                 use_corr=corr)


def test_split_stream_random_whole_parity(dev):
    """Six seeded random products that take split streams (mm and mm_nt, 12
    to 20 moduli, with and without the correction, exact and fp64 combines;
    normal, wide-range and integer entries): every output element bit for
    bit against the oracle pipeline."""
    from fp64_emu import capi
    from parity_util import whole_parity
    rng = np.random.default_rng(5301)
    done = 0
    while done < 6:
        kind = str(rng.choice(["mm", "mm_nt"]))
        M, N = int(rng.integers(250, 1100)), int(rng.integers(500, 2100))
        K = int(rng.integers(16400, 33000))
        P = int(rng.integers(12, 21))
        corr, exact = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
        dist = int(rng.integers(0, 3))
        seed = int(rng.integers(1 << 30))
        if not _split_stream(capi.layout(1, M, N, K, P, corr)):
            continue
        print(f"case random split stream {kind} {M}x{N}x{K} P={P} corr={corr} exact={exact} "
              f"dist={dist}", flush=True)
        g = torch.Generator().manual_seed(seed)

        def gen(shape):
            if dist == 0:
                return torch.randn(shape, dtype=torch.float64, generator=g)
            if dist == 1:
                s = torch.randint(0, 2, shape, generator=g) * 2 - 1
                m = 1 + torch.rand(shape, generator=g, dtype=torch.float64)
                return s * torch.ldexp(m, torch.randint(-30, 31, shape, generator=g))
            return torch.randint(-2 ** 20, 2 ** 20 + 1, shape, generator=g).double()
        A = gen((M, K)).to(dev)
        B = gen((K, N) if kind == "mm_nt" else (N, K)).to(dev)
        whole_parity(kind, A, B, O.PRIMES[:P], exact=exact, use_corr=corr)
        done += 1
        del A, B


SPLIT_X_CASES = [
    # kind, batch, M, N, K, moduli, corr -- extra columns past the wide tiles in the comment.
    ("mm_nt", 1, 1000, 1025, 16384, O.PRIMES[:14], True),     # 1 past 4 tile columns
    ("mm", 1, 500, 2050, 17000, O.PRIMES[:15], True),         # 2 past 8
    ("bmm_nt", 2, 512, 1025, 20000, MODULI_ORDERS[1], True),  # 1, two members, modulus 254
    ("mm_nt", 1, 1000, 2049, 16384, O.PRIMES[:13], False),    # 1 past 8, no correction slots
    ("mm", 1, 1000, 1026, 16384, O.PRIMES[:20], True),        # 2, every modulus
]


@pytest.mark.parametrize("kind,batch,M,N,K,primes,corr", SPLIT_X_CASES)
def test_split_stream_extra_column_parity(dev, kind, batch, M, N, K, primes, corr):
    """A last tile column of one or two columns of N under split streams:
    the units of the last wide tile column compute those columns beside
    their tiles (VALU dot products over the same A fragments, the columns'
    B fragment copied with each stage): every stage against the oracle, on a
    workspace filled with a nonzero byte first."""
    from fp64_emu import capi
    P = len(primes)
    print(f"case split stream extra columns {kind} b={batch} {M}x{N}x{K} P={P} corr={corr}",
          flush=True)
    L = capi.layout(batch, M, N, K, P, corr)
    assert _split_stream(L) and 1 <= N % 256 <= 2
    seed = 5700 + batch + M + N + K + P
    if kind in ("bmm", "bmm_nt"):
        A = _randn((batch, M, K), seed, dev)
        B = _randn((batch, K, N) if kind == "bmm_nt" else (batch, N, K), seed + 1, dev)
    else:
        A = _randn((M, K), seed, dev)
        B = _randn((K, N) if kind == "mm_nt" else (N, K), seed + 1, dev)
    check_call(kind, A, B, primes, use_corr=corr)


def test_split_stream_extra_column_random_whole_parity(dev):
    """Six seeded random products with one or two columns past their wide
    tiles under split streams (mm and mm_nt, 12 to 20 moduli, with and
    without the correction, exact and fp64 combines; normal, wide-range and
    integer entries): every output element bit for bit against the oracle
    pipeline."""
    from fp64_emu import capi
    from parity_util import whole_parity
    rng = np.random.default_rng(5417)
    done = 0
    while done < 6:
        kind = str(rng.choice(["mm", "mm_nt"]))
        M = int(rng.integers(250, 1100))
        N = 256 * int(rng.integers(2, 9)) + int(rng.integers(1, 3))
        K = int(rng.integers(16400, 33000))
        P = int(rng.integers(12, 21))
        corr, exact = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
        dist = int(rng.integers(0, 3))
        seed = int(rng.integers(1 << 30))
        if not _split_stream(capi.layout(1, M, N, K, P, corr)):
            continue
        print(f"case random split stream extra columns {kind} {M}x{N}x{K} P={P} corr={corr} "
              f"exact={exact} dist={dist}", flush=True)
        g = torch.Generator().manual_seed(seed)

        def gen(shape):
            if dist == 0:
                return torch.randn(shape, dtype=torch.float64, generator=g)
            if dist == 1:
                s = torch.randint(0, 2, shape, generator=g) * 2 - 1
                m = 1 + torch.rand(shape, generator=g, dtype=torch.float64)
                return s * torch.ldexp(m, torch.randint(-30, 31, shape, generator=g))
            return torch.randint(-2 ** 20, 2 ** 20 + 1, shape, generator=g).double()
        A = gen((M, K)).to(dev)
        B = gen((K, N) if kind == "mm_nt" else (N, K)).to(dev)
        whole_parity(kind, A, B, O.PRIMES[:P], exact=exact, use_corr=corr)
        done += 1
        del A, B
