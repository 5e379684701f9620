"""GPU tier: the reference's own test suite (tests/test_fp64_emu.py),
re-expressed with CPU-seeded inputs, through the drop-in Python API and torch
ops; plus graph capture, streams, mm_timed, error messages and empty shapes.

Where the reference asserts a statistical floor (>= 45 bits against torch's
float64 matmul) the same floor is kept and, where the inputs make the product
exactly representable, the exact result is asserted as well.
"""
import math

import numpy as np
import pytest
import torch

import fp64_emu as emu
import oracle as O
from fp64_emu import capi

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _randn(shape, seed, dev):
    return torch.randn(shape, dtype=torch.float64, generator=_gen(seed)).to(dev)


def _randint(lo, hi, shape, seed, dev):
    return torch.randint(lo, hi, shape, generator=_gen(seed), dtype=torch.int64).double().to(dev)


def _bits_vs(C, ref):
    rel = (C - ref).abs().max().item() / ref.abs().max().item()
    return -math.log2(rel) if rel > 0 else 53.0


def _dd_bits(C, A, Bt):
    hi, lo = capi.ddgemm_nt(A, Bt.t().contiguous())
    torch.cuda.synchronize()
    return O.correct_bits(C.cpu().numpy(), hi.cpu().numpy(), lo.cpu().numpy())


def test_integer_products_accurate(dev):
    """test_fp64_emu.py:14-25: integers in [-1000, 1000], nprimes=18."""
    print("case integer_products_accurate", flush=True)
    A = _randint(-1000, 1001, (128, 256), 0, dev)
    Bt = _randint(-1000, 1001, (256, 96), 1, dev)
    ref = torch.from_numpy(A.cpu().numpy().astype(np.int64) @ Bt.cpu().numpy().astype(np.int64))
    C = emu.mm_nt(A, Bt, nprimes=18)
    assert _bits_vs(C, ref.double().to(dev)) >= 45.0
    assert torch.equal(C.cpu(), ref.double())


def test_exact_mode_bitwise_integer_oracle(dev):
    """test_fp64_emu.py:28-39: integers in [-4096, 4096], nprimes=20, exact."""
    print("case exact_mode_bitwise_integer_oracle", flush=True)
    A = _randint(-4096, 4097, (128, 256), 2, dev)
    Bt = _randint(-4096, 4097, (256, 96), 3, dev)
    ref = (A.cpu().long() @ Bt.cpu().long()).double()
    assert torch.equal(emu.mm_nt(A, Bt, nprimes=20, exact=True).cpu(), ref)


@pytest.mark.parametrize("nprimes", [18, 20])
def test_random_fp64_accuracy(dev, nprimes):
    """test_fp64_emu.py:42-50, plus correct bits against the double-double
    reference at least native float64's."""
    print(f"case random_fp64_accuracy nprimes={nprimes}", flush=True)
    A = _randn((512, 1024), 4, dev)
    Bt = _randn((1024, 512), 5, dev)
    native = A @ Bt
    C = emu.mm_nt(A, Bt, nprimes=nprimes)
    assert _bits_vs(C, native) >= 45.0
    assert _dd_bits(C, A, Bt) >= _dd_bits(native, A, Bt)


def test_range_rule_adversarial_aligned(dev):
    """test_fp64_emu.py:53-63: all-ones, K=2048, every dot product K 2^104
    in the scaled domain, exact at the default plan."""
    print("case range_rule_adversarial_aligned", flush=True)
    K = 2048
    A = torch.ones(64, K, dtype=torch.float64, device=dev)
    Bt = torch.ones(K, 48, dtype=torch.float64, device=dev)
    C = emu.mm_nt(A, Bt, exact=True)
    assert torch.equal(C, torch.full((64, 48), float(K), dtype=torch.float64, device=dev))


def test_dyadic_dynamic_range_bitexact(dev):
    """test_fp64_emu.py:66-83: integers under per-k power-of-two scales
    2^-12..2^0; exact at defaults through mm."""
    print("case dyadic_dynamic_range_bitexact", flush=True)
    g = _gen(6)
    M, K, N = 64, 512, 48
    ek = torch.randint(-12, 1, (K,), generator=g)
    Ai = torch.randint(-256, 257, (M, K), generator=g)
    Bi = torch.randint(-256, 257, (N, K), generator=g)
    A = (torch.bitwise_left_shift(Ai, ek + 12).double() * 2.0 ** -12).to(dev)
    B = (torch.bitwise_left_shift(Bi, ek + 12).double() * 2.0 ** -12).to(dev)
    w = 4 ** (ek + 12)
    ref = ((Ai * w) @ Bi.T).double() * 2.0 ** -24
    assert torch.equal(emu.mm(A, B).cpu(), ref)


def test_bmm_single_batch_matches_mm(dev):
    """test_fp64_emu.py:86-94."""
    print("case bmm_single_batch_matches_mm", flush=True)
    A = _randn((192, 384), 7, dev)
    B = _randn((160, 384), 8, dev)
    assert torch.equal(emu.bmm(A[None], B[None])[0], emu.mm(A, B))


def test_bmm_integer_oracle_bitexact(dev):
    """test_fp64_emu.py:97-104."""
    print("case bmm_integer_oracle_bitexact", flush=True)
    A = _randint(-4096, 4097, (5, 96, 256), 9, dev)
    B = _randint(-4096, 4097, (5, 64, 256), 10, dev)
    ref = torch.stack([(A[b].cpu().long() @ B[b].cpu().long().T).double() for b in range(5)])
    assert torch.equal(emu.bmm(A, B).cpu(), ref)


def test_bmm_odd_shapes_accuracy(dev):
    """test_fp64_emu.py:107-119."""
    print("case bmm_odd_shapes_accuracy", flush=True)
    A = _randn((3, 100, 333), 11, dev)
    Bt = _randn((3, 333, 77), 12, dev)
    ref = torch.bmm(A, Bt)
    C = emu.bmm_nt(A, Bt)
    assert _bits_vs(C, ref) >= 45.0


def test_mm_nt_and_mm_layouts_agree(dev):
    """test_fp64_emu.py:147-161 in this build's terms: the [K, N] layout read
    in place and the [N, K] layout give identical bits (the shifts are exact
    and the width decision agrees)."""
    print("case mm_nt_and_mm_layouts_agree", flush=True)
    A = _randn((256, 1024), 13, dev)
    Bt = _randn((1024, 200), 14, dev)
    assert torch.equal(emu.mm_nt(A, Bt), emu.mm(A, Bt.t().contiguous()))


@pytest.mark.parametrize("kind,M,N,K", [
    ("mm", 128, 96, 256),          # row sizing, small GEMM tiles as slot runs
    ("mm_nt", 64, 1300, 20000),    # fused row/column sizing, mixed tiles, K-split
])
def test_graph_capture_replays(dev, kind, M, N, K):
    """test_fp64_emu.py:164-182, strengthened: several replays with eager work
    and synchronisation between them; each replay equals the eager result on
    the buffers' current contents."""
    print(f"case graph_capture_replays {kind} {M}x{N}x{K}", flush=True)
    shapeB = (N, K) if kind == "mm" else (K, N)
    fn = emu.mm if kind == "mm" else emu.mm_nt
    A = _randn((M, K), 15, dev)
    B = _randn(shapeB, 16, dev)
    for _ in range(3):
        fn(A, B)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        C = fn(A, B)
    for r in range(4):
        A.copy_(_randn((M, K), 100 + r, dev))
        B.copy_(_randn(shapeB, 200 + r, dev))
        g.replay()
        torch.cuda.synchronize()
        eager = fn(A, B)
        torch.cuda.synchronize()
        assert torch.equal(C, eager), f"replay {r}"
        emu.mm_nt(A, _randn((K, 40), 300 + r, dev))   # unrelated eager work between replays


@pytest.mark.parametrize("kind,batch,M,N,K,nprimes", [
    ("mm_nt", 1, 200, 136, 3000, 17),    # shapes and modulus counts no earlier test runs
    ("bmm", 3, 72, 40, 1500, 19),
])
def test_graph_capture_first_call(dev, kind, batch, M, N, K, nprimes):
    """The first call of a fresh shape and plan runs inside torch.cuda.graph
    (no warm-up, no probe): the capture holds the whole call, and each replay
    equals the eager result and the oracle's."""
    print(f"case graph_capture_first_call {kind} b={batch} {M}x{N}x{K} P={nprimes}", flush=True)
    batched = kind == "bmm"
    shapeA = (batch, M, K) if batched else (M, K)
    shapeB = (batch, N, K) if batched else (K, N)
    fn = (lambda X, Y: emu.bmm(X, Y, nprimes=nprimes)) if batched else \
        (lambda X, Y: emu.mm_nt(X, Y, nprimes=nprimes))
    A = _randn(shapeA, 61, dev)
    B = _randn(shapeB, 62, dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        C = fn(A, B)
    for r in range(3):
        A.copy_(_randn(shapeA, 400 + r, dev))
        B.copy_(_randn(shapeB, 500 + r, dev))
        g.replay()
        torch.cuda.synchronize()
        eager = fn(A, B)
        torch.cuda.synchronize()
        assert torch.equal(C, eager), f"replay {r}"
    Ah, Bh, Ch = A.cpu().numpy(), B.cpu().numpy(), C.cpu().numpy()
    for i in range(batch):
        ref, _ = O.mm(Ah[i] if batched else Ah, Bh[i] if batched else Bh, 0 if batched else 1,
                      O.PRIMES[:nprimes])
        got = Ch[i] if batched else Ch
        assert np.array_equal(got.view(np.uint64), ref.view(np.uint64)), f"member {i}"


def test_torch_compile_traces(dev):
    """test_fp64_emu.py:185-193."""
    print("case torch_compile_traces", flush=True)
    A = _randn((64, 128), 17, dev)
    B = _randn((48, 128), 18, dev)
    eager = emu.mm(A, B)
    compiled = torch.compile(emu.mm, dynamic=False)
    assert torch.equal(compiled(A, B), eager)


def test_deterministic(dev):
    """test_fp64_emu.py:196-211."""
    print("case deterministic", flush=True)
    A = _randn((4, 128, 512), 19, dev)
    B = _randn((4, 96, 512), 20, dev)
    assert torch.equal(emu.bmm(A, B), emu.bmm(A, B))
    A = _randn((256, 512), 21, dev)
    Bt = _randn((512, 256), 22, dev)
    assert torch.equal(emu.mm_nt(A, Bt, nprimes=18), emu.mm_nt(A, Bt, nprimes=18))


def test_side_stream(dev):
    """Work is enqueued on the caller's current stream."""
    print("case side_stream", flush=True)
    A = _randn((300, 700), 23, dev)
    Bt = _randn((700, 200), 24, dev)
    ref = emu.mm_nt(A, Bt)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C = emu.mm_nt(A, Bt)
    s.synchronize()
    assert torch.equal(C, ref)


def test_concurrent_host_threads(dev):
    """Calls from several host threads, each on its own stream, give the
    results of the same calls made one after another (the library keeps no
    per-call state outside its workspace; the reference guards its table
    caches with mutexes, fp64_emu_cuda/fp64_emu.cu:1038-1040)."""
    import threading
    print("case concurrent_host_threads", flush=True)
    shapes = [("mm_nt", 300, 200, 700), ("mm", 129, 257, 1000), ("bmm_nt", 96, 80, 600),
              ("mm_nt", 40, 513, 3000)]
    inputs = []
    for i, (kind, M, N, K) in enumerate(shapes):
        if kind == "bmm_nt":
            inputs.append((kind, _randn((3, M, K), 400 + i, dev), _randn((3, K, N), 410 + i, dev)))
        elif kind == "mm":
            inputs.append((kind, _randn((M, K), 400 + i, dev), _randn((N, K), 410 + i, dev)))
        else:
            inputs.append((kind, _randn((M, K), 400 + i, dev), _randn((K, N), 410 + i, dev)))
    fn = {"mm": emu.mm, "mm_nt": emu.mm_nt, "bmm_nt": emu.bmm_nt}
    ref = [fn[k](A, B) for k, A, B in inputs]
    torch.cuda.synchronize()
    out = [[None] * 3 for _ in inputs]
    errors = []

    def work(t):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for r in range(3):
                    k, A, B = inputs[t]
                    out[t][r] = fn[k](A, B)
            s.synchronize()
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=work, args=(t,)) for t in range(len(inputs))]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    hung = [i for i, th in enumerate(threads) if th.is_alive()]
    assert not hung, f"threads {hung} ({[shapes[i] for i in hung]}) still running after 60 s"
    assert not errors, errors
    for t in range(len(inputs)):
        for r in range(3):
            assert torch.equal(out[t][r], ref[t]), (t, r)


def test_batch_beyond_reference_z_extent(dev):
    """The reference refuses (nprimes + 2) * batch > 65535, its GEMM launch's
    z-extent (fp64_emu_cuda/fp64_emu.cu:1652, 1680); this build's launches are
    one-dimensional, so such a batch runs, bit-identical to the oracle."""
    print("case batch beyond z-extent: bmm_nt 4200 x 8x8x8 and bmm 4200 x 5x7x9", flush=True)
    assert (14 + 2) * 4200 > 65535
    A = _randn((4200, 8, 8), 430, dev)
    Bt = _randn((4200, 8, 8), 431, dev)
    C = emu.bmm_nt(A, Bt, nprimes=14)
    ref, _ = O.mm(A.cpu().numpy(), Bt.cpu().numpy(), 1, O.PRIMES[:14])
    assert np.array_equal(C.cpu().numpy().view(np.uint64), ref.view(np.uint64))
    A = _randn((4200, 5, 9), 432, dev)
    B = _randn((4200, 7, 9), 433, dev)
    C = emu.bmm(A, B, nprimes=14)
    ref, _ = O.mm(A.cpu().numpy(), B.cpu().numpy(), 0, O.PRIMES[:14])
    assert np.array_equal(C.cpu().numpy().view(np.uint64), ref.view(np.uint64))


def test_mm_timed_contract(dev):
    """torch-ext/fp64_emu/__init__.py:135-149: (C, [extract, gemms, 0, reconstruct])."""
    print("case mm_timed_contract", flush=True)
    A = _randn((512, 2048), 25, dev)
    B = _randn((384, 2048), 26, dev)
    C, t = emu.mm_timed(A, B)
    assert isinstance(t, list) and len(t) == 4
    # t[2] spans two back-to-back events (the reference's 0-marker)
    assert t[0] > 0 and t[1] > 0 and t[3] > 0 and 0.0 <= t[2] < t[1]
    assert torch.equal(C, emu.mm(A, B))
    P, corr = emu.plan_config(2048)
    ref, _ = O.mm(A.cpu().numpy(), B.cpu().numpy(), 0, O.PRIMES[:P], use_corr=corr)
    assert np.array_equal(C.cpu().numpy().view(np.uint64), ref.view(np.uint64)), \
        "mm_timed output differs from the oracle"


def test_op_error_messages(dev):
    """The reference's TORCH_CHECK messages (fp64_emu_cuda/fp64_emu.cu:1586-1693)
    surface as RuntimeError."""
    print("case op_error_messages", flush=True)
    ops = torch.ops.fp64_emu
    primes, inv, mu = emu._tables(14)
    A = _randn((8, 16), 27, dev)
    Bt = _randn((16, 8), 28, dev)
    out = torch.empty(8, 8, dtype=torch.float64, device=dev)
    with pytest.raises(RuntimeError, match=r"bits must be in \[16, 53\]"):
        ops.fp64_emu_mm_nt(out, A, Bt, primes, inv, mu, True, 15, True)
    with pytest.raises(RuntimeError, match="f64"):
        ops.fp64_emu_mm_nt(out, A.float(), Bt, primes, inv, mu, True, 53, True)
    with pytest.raises(RuntimeError, match="contig"):
        ops.fp64_emu_mm_nt(out, A.t(), Bt, primes, inv, mu, True, 53, True)
    with pytest.raises(RuntimeError):
        ops.fp64_emu_mm_nt(out, A, Bt[:8], primes, inv, mu, True, 53, True)
    bad = torch.tensor(list(range(2, 24)), dtype=torch.int32)
    with pytest.raises(RuntimeError, match="too many primes"):
        ops.fp64_emu_mm_nt(out, A, Bt, bad, inv, mu, True, 53, True)
    with pytest.raises(AssertionError):
        emu.mm_nt(A, Bt.t().contiguous())   # Python dim checks are asserts


def test_empty_and_degenerate_shapes(dev):
    print("case empty_and_degenerate_shapes", flush=True)
    A = _randn((0, 16), 29, dev)
    Bt = _randn((16, 8), 30, dev)
    assert emu.mm_nt(A, Bt).shape == (0, 8)
    A = torch.empty(5, 0, dtype=torch.float64, device=dev)
    Bt = torch.empty(0, 7, dtype=torch.float64, device=dev)
    C = emu.mm_nt(A, Bt)
    assert C.shape == (5, 7) and not C.any()
    A = torch.zeros(33, 40, dtype=torch.float64, device=dev)
    A[3] = _randn((40,), 31, dev)
    B = _randn((9, 40), 32, dev)
    C = emu.mm(A, B)
    assert not C[:3].any() and not C[4:].any()
    assert _bits_vs(C[3], A[3] @ B.t()) >= 50.0
    one = emu.mm(_randn((1, 1), 33, dev), _randn((1, 1), 34, dev))
    assert one.shape == (1, 1)


def test_inexact_recombine_accuracy(dev):
    """exact=False (the fp64 combine): correct bits within a bit of exact."""
    print("case inexact_recombine_accuracy", flush=True)
    A = _randn((256, 2048), 35, dev)
    Bt = _randn((2048, 256), 36, dev)
    ce = emu.mm_nt(A, Bt, exact=True)
    ci = emu.mm_nt(A, Bt, exact=False)
    assert _dd_bits(ci, A, Bt) >= _dd_bits(ce, A, Bt) - 1.0


@pytest.mark.parametrize("bits", [53, 50, 44, 40, 36, 32])
def test_bits_sweep(dev, bits):
    """bench/accuracy.py:143-151: each width at plan(K, bits) reaches about
    its width in correct bits."""
    print(f"case bits_sweep bits={bits}", flush=True)
    A = _randn((256, 1024), 37, dev)
    Bt = _randn((1024, 256), 38, dev)
    C = emu.mm_nt(A, Bt, nprimes=emu.plan(1024, bits), bits=bits)
    assert _dd_bits(C, A, Bt) >= bits - 6


@pytest.mark.parametrize("M,N,K", [(37, 53, 1001), (16, 16, 16), (129, 7, 333)])
def test_ddgemm_matches_oracle(dev, M, N, K):
    """The device double-double GEMM, the yardstick of every correct-bits
    check here and in the bench, against the oracle's (bench/accuracy.py:21-50
    restated on the CPU, itself pinned to exact rationals): the same k order
    and an exact two-product (FMA here, Dekker's split there), so hi and lo
    agree bit for bit on ragged shapes."""
    print(f"case ddgemm vs oracle {M}x{N}x{K}", flush=True)
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, dtype=torch.float64, generator=g)
    Bt = torch.randn(K, N, dtype=torch.float64, generator=g)
    A[:, ::7] *= 2.0 ** 30             # wide range: the tails matter
    hi, lo = capi.ddgemm_nt(A.to(dev), Bt.t().contiguous().to(dev))
    ohi, olo = O.ddgemm_nt(A.numpy(), Bt.numpy())
    assert np.array_equal(hi.cpu().numpy().view(np.uint64), ohi.view(np.uint64))
    assert np.array_equal(lo.cpu().numpy().view(np.uint64), olo.view(np.uint64))


def test_deep_k_integer_bitexact(dev):
    """test_fp64_emu.py:122-131: K = 200000 (four 65536 segments), entries
    in {-1, 0, 1}, exact at defaults."""
    print("case deep_k_integer_bitexact", flush=True)
    K = 200_000
    A = _randint(-1, 2, (48, K), 41, dev)
    B = _randint(-1, 2, (32, K), 42, dev)
    ref = (A.cpu().long() @ B.cpu().long().T).double()
    assert torch.equal(emu.mm(A, B).cpu(), ref)


def test_deep_k_randn_accuracy(dev):
    """test_fp64_emu.py:134-144 (>= 40 bits vs native), plus correct bits at
    least native float64's against the double-double reference."""
    print("case deep_k_randn_accuracy", flush=True)
    K = 150_000
    A = _randn((64, K), 43, dev)
    B = _randn((48, K), 44, dev)
    native = A @ B.t()
    C = emu.mm(A, B)
    assert _bits_vs(C, native) >= 40.0
    assert _dd_bits(C, A, B.t().contiguous()) >= _dd_bits(native, A, B.t().contiguous())


def test_deep_k_mm_nt_reroutes(dev):
    """mm_nt / bmm_nt past the single-launch bound run as mm / bmm on the
    transposed operand (torch-ext/fp64_emu/__init__.py:79-80, 121-122)."""
    print("case deep_k_mm_nt_reroutes", flush=True)
    K = 140_000
    A = _randn((20, K), 45, dev)
    Bt = _randn((K, 12), 46, dev)
    assert torch.equal(emu.mm_nt(A, Bt), emu.mm(A, Bt.t().contiguous()))
    assert torch.equal(emu.bmm_nt(A[None], Bt[None])[0], emu.mm(A, Bt.t().contiguous()))
    with pytest.raises(RuntimeError, match="K bound for int32 modular GEMM"):
        torch.ops.fp64_emu.fp64_emu_mm_nt(torch.empty(20, 12, dtype=torch.float64, device=dev),
                                          A, Bt, *emu._tables(15), True, 53, True)
