"""CPU tier: the drop-in boundary without a GPU.

- libfp64emu.so loads and exports every function include/fp64emu.h declares;
- the workspace map is consistent (padding, alignment, no overlap, sizes);
- argument validation returns the documented error codes and messages before
  any device work (so it runs here, with no GPU);
- the torch op library registers the reference's schemas verbatim
  (torch-ext/torch_binding.cpp:7-12) with CUDA-only kernels: CPU tensors are
  refused, never computed on a fallback;
- the package refuses to import when the extension is not built.
"""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fp64emu.h")

torch = pytest.importorskip("torch")
fp64_emu = pytest.importorskip("fp64_emu")
from fp64_emu import capi  # noqa: E402

EINVAL, EWORKSPACE = 1, 2


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(fp64emu_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_exactly_the_exported_api():
    declared = _declared_functions()
    assert declared == sorted(capi.EXPORTS)
    text = open(HEADER).read()
    assert "extern \"C\"" in text
    code = re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", text, flags=re.S))
    for torch_type in ("Tensor", "at::", "c10", "torch"):
        assert torch_type not in code, torch_type   # plain pointers and sizes only


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(capi.CAPI_PATH)
    for name in _declared_functions():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", capi.CAPI_PATH], capture_output=True,
                         text=True, check=True).stdout
    syms = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    for name in _declared_functions():
        assert name in syms, name


def test_maxp_and_status_codes():
    L = capi.lib()
    assert L.fp64emu_maxp() == 20
    text = open(HEADER).read()
    for name, val in (("FP64EMU_OK", 0), ("FP64EMU_EINVAL", 1), ("FP64EMU_EWORKSPACE", 2),
                      ("FP64EMU_EHIP", 3)):
        assert re.search(rf"{name}\s*=\s*{val}\b", text), name


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (1, 128, 128, 4096), (1, 1023, 2049, 32769),
                                   (64, 512, 512, 512), (1, 300, 7, 65537), (3, 0, 5, 10),
                                   (1, 48, 32, 200000), (2, 24, 16, 131072),
                                   (1, 8192, 8192, 8192)])
@pytest.mark.parametrize("P,corr", [(14, True), (13, False), (20, True)])
def test_layout_consistency(shape, P, corr):
    batch, M, N, K = shape
    L = capi.layout(batch, M, N, K, P, corr)
    assert L.Mp % 256 == 0 and L.Np % 256 == 0 and L.Kp % 64 == 0
    assert L.Mp >= max(M, 1) and L.Mp - max(M, 1) < 256
    assert L.Np >= max(N, 1) and L.Np - max(N, 1) < 256
    assert L.Kp >= L.kseg and L.Kp - L.kseg < 64
    deep = K > 131071
    assert L.deep == int(deep) and L.nseg == ((K + 65535) // 65536 if deep else 1)
    assert L.kseg == (65536 if deep else K)
    assert L.ncorr == (0 if not corr else (1 if (L.ksplit == 1 and (deep or K <= 65536)) else 2))
    nplanes = P + (2 if corr else 0)
    assert L.planeA_bytes == L.Mp * L.Kp and L.planeB_bytes == L.Np * L.Kp
    assert L.memberA_bytes == nplanes * L.planeA_bytes
    assert L.memberB_bytes == nplanes * L.planeB_bytes
    assert L.outplane_bytes == L.Mp * L.Np
    # Extracted plane rows: every operand row, a multiple of 128, within the
    # padded plane; short of it only where GEMM tiles are 128 wide.
    # (B also under mixed tiles, whose last tile column is read 128 wide,
    # and to a multiple of 64 under split streams with extra columns, which
    # read 16 rows of the last tile.)
    xcols = L.gemm_split and L.Np // 256 >= 2 and 1 <= N % 256 <= 2
    for ext, R, Rp, short_ok, q in ((L.ext_rowsA, M, L.chunk_rows, L.gemm_tile_rows == 128, 128),
                                    (L.ext_rowsB, N, L.Np, not deep, 64 if xcols else 128)):
        assert ext % q == 0 and min(max(R, 1), Rp) <= ext <= Rp
        assert ext == Rp or (short_ok and ext == -(-max(R, 1) // q) * q)
    sizes = [("off_sftA", 2 * batch * M), ("off_sftB", 2 * batch * N), ("off_lgA", 4 * batch * M),
             ("off_lgB", 4 * batch * N), ("off_bits", 16), ("off_pmax", 8 * L.nslab * batch * N),
             ("off_pss", 8 * L.nslab * batch * N), ("off_planesA", batch * L.memberA_bytes),
             ("off_planesB", batch * L.memberB_bytes),
             ("off_res8", (4 if deep else 1) * L.ksplit * batch * P * L.outplane_bytes),
             ("off_corr", (8 if deep else 4) * L.ksplit * batch * L.ncorr * L.outplane_bytes)]
    prev_end = 0
    for name, size in sizes:
        off = getattr(L, name)
        assert off % 256 == 0, name
        assert off >= prev_end, name
        prev_end = off + size
    assert L.total >= prev_end
    assert capi.workspace_size(batch, M, N, K, P, corr) == L.total


def test_layout_choices_fuzz():
    """The layout's launch choices over 3000 seeded shapes (log-uniform
    sizes, batches, depths through the K-segmented range, every modulus
    count, correction on and off): no failure, and each choice within the
    ranges the GEMM launches assume."""
    rng = np.random.default_rng(20261206)
    for _ in range(3000):
        batch = int(np.exp(rng.uniform(0, np.log(2000)))) if rng.random() < 0.5 else 1
        M = int(np.exp(rng.uniform(0, np.log(20000))))
        N = int(np.exp(rng.uniform(0, np.log(20000))))
        K = int(np.exp(rng.uniform(0, np.log(400000))))
        if batch * M * K > 2 ** 33 or batch * N * K > 2 ** 33:
            continue
        P = int(rng.integers(1, 21))
        corr = bool(rng.integers(2))
        L = capi.layout(batch, M, N, K, P, corr)
        case = (batch, M, N, K, P, corr)
        assert L.ksplit in (1, 2, 4, 8, 16), case
        assert L.ksplit == 1 or (L.Kp // 64) // L.ksplit >= 8, case
        assert 1 <= L.gemm_run <= max(P, 1), case
        tiles = batch * (L.Mp // 256) * (L.Np // 256)
        if L.gemm_run > 1:
            assert (L.gemm_tile_rows, L.gemm_tile_cols, L.ksplit, L.deep) == (256, 256, 1, 0), case
            assert L.Kp // 64 <= 32 and P >= 2 and tiles >= 256, case
        if not L.deep and L.ksplit == 1 and P >= 2 and L.Kp // 64 <= 32 and 0 < tiles < 256:
            assert L.gemm_tile_cols == 128, case
        assert (L.gemm_tile_rows, L.gemm_tile_cols) in ((256, 256), (256, 128), (128, 128)), case
        if L.gemm_split:
            xc = N % 256 if (L.Np // 256 >= 2 and 1 <= N % 256 <= 2) else 0
            T = (L.Mp // 256) * (L.Np // 256 - (1 if xc else 0))
            assert (L.ksplit, L.gemm_run, L.deep, L.nchunk) == (2, 1, 0, 1), case
            assert (L.gemm_tile_rows, L.gemm_tile_cols) == (256, 256), case
            assert L.ncorr == (2 if corr else 0) and L.Kp // 64 >= 256, case
            assert T % 32 == 0 or 32 % T == 0, case
            assert -(-(P + L.ncorr) * batch * T // 32) >= 8, case
        assert capi.workspace_size_min(batch, M, N, K, P, corr) <= L.total, case


def test_layout_rejects_bad_arguments():
    with pytest.raises(capi.CapiError):
        capi.layout(1, -1, 4, 4, 14, True)
    with pytest.raises(capi.CapiError):
        capi.layout(1, 4, 4, 4, 21, True)
    assert capi.workspace_size(1, 4, 4, 4, 0, True) == 0
    assert capi.workspace_size(1, 4, 4, 4, 21, True) == 0


def _call(kind="mm_nt", M=8, N=8, K=16, primes=None, bits=53, ws_bytes=None, null_ops=False,
          batch=1, ws_addr=0x2000):
    """Invoke a C entry point with host-side dummies; every case here fails
    validation (or is empty) before any pointer is dereferenced or any HIP
    call is made."""
    L = capi.lib()
    pr = np.asarray(capi_primes(14) if primes is None else primes, np.int32)
    pp = pr.ctypes.data_as(ctypes.c_void_p)
    dummy = None if null_ops else ctypes.c_void_p(0x1000)
    ws_size = capi.workspace_size(batch, max(M, 0), max(N, 0), max(K, 0), max(1, min(pr.size, 20)),
                                  True)
    ws_bytes = ws_size if ws_bytes is None else ws_bytes
    ws = ctypes.c_void_p(ws_addr)
    if kind in ("mm", "mm_nt"):
        st = getattr(L, "fp64emu_" + kind)(dummy, dummy, dummy, M, N, K, pp, None, None, pr.size, 1,
                                           bits, 1, ws, ws_bytes, None)
    else:
        st = getattr(L, "fp64emu_" + kind)(dummy, dummy, dummy, batch, M, N, K, pp, None, None,
                                           pr.size, 1, bits, 1, ws, ws_bytes, None)
    return st, L.fp64emu_last_error().decode()


def capi_primes(n):
    return fp64_emu._PRIMES[:n]


@pytest.mark.parametrize("kind", ["mm", "mm_nt", "bmm", "bmm_nt"])
def test_validation_messages(kind):
    assert _call(kind, bits=15) == (EINVAL, "bits must be in [16, 53]")
    assert _call(kind, bits=54) == (EINVAL, "bits must be in [16, 53]")
    assert _call(kind, primes=list(range(2, 23))) == (EINVAL, "too many primes")
    assert _call(kind, primes=[256, 128]) == (EINVAL, "moduli must be pairwise coprime")
    assert _call(kind, primes=[257, 255]) == (EINVAL, "moduli must be in [2, 256]")
    assert _call(kind, primes=[1]) == (EINVAL, "moduli must be in [2, 256]")
    if kind.endswith("_nt"):
        assert _call(kind, K=131072) == (EINVAL, "K bound for int32 modular GEMM")
    else:   # mm / bmm run K-segmented past 131071, to 128 segments of 65536
        assert _call(kind, K=128 * 65536 + 1) == (EINVAL, "K bound: 128 segments of 65536")
    assert _call(kind, M=-1) == (EINVAL, "shapes must be non-negative")
    assert _call(kind, ws_bytes=100) == (EWORKSPACE, "workspace too small")
    assert _call(kind, ws_addr=0x2008) == (EINVAL, "workspace must be 256-byte aligned")
    assert _call(kind, null_ops=True)[0] == EINVAL


def test_noalloc_validation_before_device_work():
    """fp64emu_mm_nt_noalloc checks its arguments and the static scratch's
    limit before any HIP call, so the refusals show here without a GPU."""
    L = capi.lib()
    pr = np.asarray(capi_primes(14), dtype=np.int32)
    pp = pr.ctypes.data_as(ctypes.c_void_p)

    def call(M, N, K, P=14, bits=53, primes=pp):
        st = L.fp64emu_mm_nt_noalloc(None, None, None, M, N, K, primes, None, None, P, 1, bits,
                                     1, None)
        return st, L.fp64emu_last_error().decode()

    assert call(64, 64, 64, bits=15) == (EINVAL, "bits must be in [16, 53]")
    assert call(64, 64, 131072) == (EINVAL, "K bound for int32 modular GEMM")
    assert call(-1, 64, 64) == (EINVAL, "shapes must be non-negative")
    st, msg = call(256, 4096, 8192)     # B's planes alone are 512 MiB
    assert st == EWORKSPACE and "too large for the static scratch" in msg
    need = capi.workspace_size_min(1, 256, 4096, 8192, 14, True)
    assert str(need) in msg and need > capi.NOALLOC_SCRATCH_BYTES
    assert call(0, 64, 64) == (0, "")   # empty: nothing to do, no device touched


def test_empty_shapes_are_a_no_op():
    assert _call("mm_nt", M=0)[0] == 0
    assert _call("mm", N=0)[0] == 0
    assert _call("bmm_nt", batch=0)[0] == 0


def test_torch_schemas_match_reference():
    """The reference's op definitions (torch-ext/torch_binding.cpp:7-12),
    parsed, equal the registered schemas."""
    ref = [
        "fp64_emu_mm(Tensor! out, Tensor A, Tensor B, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()",
        "fp64_emu_bmm(Tensor! out, Tensor A, Tensor B, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()",
        "fp64_emu_mm_nt(Tensor! out, Tensor A, Tensor Bt, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()",
        "fp64_emu_bmm_nt(Tensor! out, Tensor A, Tensor Bt, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()",
        "fp64_emu_mm_timed(Tensor! out, Tensor! times, Tensor A, Tensor B, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()",
        "fp64_emu_maxp() -> int",
    ]
    for d in ref:
        name = d.split("(")[0]
        want = torch._C.parse_schema("fp64_emu::" + d)
        got = getattr(torch.ops.fp64_emu, name).default._schema
        assert str(got) == str(want), name
    assert torch.ops.fp64_emu.fp64_emu_maxp() == 20


def test_fakes_registered_for_compile():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        primes = torch.tensor(capi_primes(14), dtype=torch.int32)
        A = torch.empty(4, 8, dtype=torch.float64, device="cuda")
        B = torch.empty(6, 8, dtype=torch.float64, device="cuda")
        out = torch.empty(4, 6, dtype=torch.float64, device="cuda")
        torch.ops.fp64_emu.fp64_emu_mm_nt(out, A, B, primes, primes, primes, True, 53, True)


def test_cpu_tensors_are_refused_not_computed():
    """The product has no CPU path: host tensors hit no kernel."""
    A = torch.randn(4, 8, dtype=torch.float64)
    B = torch.randn(6, 8, dtype=torch.float64)
    with pytest.raises((RuntimeError, NotImplementedError)):
        fp64_emu.mm(A, B)                       # B as [N, K]
    with pytest.raises((RuntimeError, NotImplementedError)):
        fp64_emu.mm_nt(A, B.T.contiguous())     # Bt as [K, N]
    with pytest.raises((RuntimeError, NotImplementedError)):
        fp64_emu.bmm(A[None], B[None])


def test_python_api_surface_mirrors_reference():
    """torch-ext/fp64_emu/__init__.py: mm_nt, mm, bmm_nt, bmm, plan_config,
    mm_timed (+ plan, range_bits helpers)."""
    for name in ("mm_nt", "mm", "bmm_nt", "bmm", "plan_config", "mm_timed", "plan", "range_bits"):
        assert callable(getattr(fp64_emu, name)), name
    assert fp64_emu.plan_config(8192) == (14, True)
    assert fp64_emu.plan_config(32769) == (15, True)


def test_import_fails_loudly_without_extension(tmp_path):
    """A copy of the package without the built .so files must not import."""
    import shutil
    src = os.path.dirname(fp64_emu.__file__)
    dst = tmp_path / "fp64_emu"
    shutil.copytree(src, dst, ignore=shutil.ignore_patterns("*.so", "__pycache__"))
    code = ("import sys; sys.path.insert(0, %r)\n"
            "try:\n    import fp64_emu\nexcept ImportError as e:\n"
            "    print('IMPORT_ERROR', e); sys.exit(0)\n"
            "sys.exit(3)\n" % str(tmp_path))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "not built" in r.stdout


@pytest.mark.parametrize("shape", [(1, 1000, 700, 3000), (1, 8192, 8192, 8192), (1, 300, 20, 65537),
                                   (4, 600, 500, 700), (1, 900, 800, 140000)])
def test_minimum_workspace(shape):
    """Batch-1 products with K <= 131071 accept a workspace down to one
    256-row chunk of A; batched and K-segmented products need the full size."""
    batch, M, N, K = shape
    full = capi.workspace_size(batch, M, N, K, 14, True)
    wmin = capi.workspace_size_min(batch, M, N, K, 14, True)
    L = capi.layout(batch, M, N, K, 14, True)
    assert L.nchunk == 1 and L.chunk_rows == L.Mp
    if batch == 1 and K <= 131071 and L.Mp > 256:
        assert 0 < wmin < full
    else:
        assert wmin == full


def test_split_streams_only_for_deep_products_of_few_tiles():
    """Split streams replace a K-split the planner chose for products of at
    least 256 k-steps whose wide tiles per member and slot divide or are
    divided by 32, with at least eight blocks of 32 units; a last tile column
    of one or two columns rides on the wide tiles (c5), one of 3 to 128
    columns keeps the mixed launch.  Their two K ranges per unit are a
    K-split of 2."""
    for shape in [(1, 1024, 2048, 32768, 15, True), (1, 1024, 1024, 32768, 15, True),
                  (1, 1024, 2048, 16384, 14, True), (4, 512, 1024, 16384, 14, True),
                  (1, 1023, 2048, 32769, 13, False), (1, 300, 2000, 17000, 15, True),
                  (1, 1023, 2049, 32769, 15, True), (1, 1023, 2049, 32769, 13, False),
                  (1, 500, 2050, 17000, 15, True), (2, 512, 1025, 20000, 14, True)]:
        L = capi.layout(*shape)
        assert (L.gemm_split, L.ksplit, L.gemm_run) == (1, 2, 1), shape
    assert capi.layout(1, 1023, 2049, 32769, 15, True).ext_rowsB == 2112   # B rows to 64 past N
    for shape in [(1, 1023, 2051, 32769, 15, True),    # three columns past: mixed tiles
                  (1, 1024, 1024, 8192, 14, True),     # 128 k-steps
                  (1, 1500, 1500, 30000, 15, True),    # 36 tiles per slot
                  (1, 3000, 1000, 20000, 14, True),    # 48 tiles per slot
                  (1, 8192, 8192, 8192, 14, True),     # c2: no K-split
                  (1, 512, 512, 65536, 15, True),      # 68 units: 3 blocks
                  (1, 64, 40, 100_000, 15, True)]:     # narrow tiles
        assert capi.layout(*shape).gemm_split == 0, shape


def test_slot_runs_only_for_shallow_products():
    """Runs are chosen from the shapes alone: shallow products without a
    K-split with at least 256 output tiles of 256 x 256, one run at whole
    multiples of 256 tiles, three runs otherwise; deep, K-split, mixed-tile
    and one-modulus launches keep one slot per group, and shallow products
    with fewer tiles run one slot per group on 256 x 128 tiles (128 x 128 at
    40 tiles or fewer)."""
    assert capi.layout(64, 512, 512, 512, 14, True).gemm_run == 14        # c4: 256 tiles
    assert capi.layout(1, 8192, 8192, 8192, 14, True).gemm_run == 1       # c2: 128 k-steps
    assert capi.layout(1, 128, 128, 4096, 14, True).gemm_run == 1         # c1: K-split
    assert capi.layout(1, 300, 1290, 200, 14, True).gemm_run == 1         # mixed tiles
    assert capi.layout(1, 500, 500, 1024, 1, True).gemm_run == 1          # one modulus
    assert capi.layout(128, 512, 512, 512, 14, True).gemm_run == 14       # 512 tiles: whole rounds
    assert capi.layout(80, 512, 512, 512, 14, True).gemm_run == 5         # 320 tiles: 3 runs
    assert capi.layout(300, 256, 256, 256, 20, True).gemm_run == 7        # 300 tiles: 3 runs
    assert capi.layout(1, 4096, 4096, 1024, 14, True).gemm_run == 14      # 256 tiles, 16 k-steps
    assert capi.layout(1, 4096, 4096, 4096, 14, True).gemm_run == 1       # 64 k-steps
    # fewer than 256 tiles: one slot per group on narrow tiles
    for shape, tile in [((32, 500, 500, 128, 14, True), (256, 128)),      # 128 tiles
                        ((1, 2560, 2560, 200, 13, False), (256, 128)),    # 100 tiles
                        ((64, 256, 256, 256, 14, True), (256, 128)),      # 64 tiles
                        ((48, 512, 512, 512, 14, True), (256, 128)),      # 192 tiles
                        ((1, 2048, 2048, 2048, 14, True), (256, 128)),    # 64 tiles, 32 k-steps
                        ((40, 256, 256, 320, 20, True), (128, 128)),      # 40 tiles
                        ((8, 512, 512, 512, 14, True), (128, 128)),       # 32 tiles
                        ((16, 256, 256, 256, 14, True), (128, 128)),      # 16 tiles
                        ((1, 1500, 1500, 1500, 14, True), (128, 128)),    # 36 tiles
                        ((128, 40, 40, 256, 14, True), (128, 128)),
                        ((64, 512, 300, 1000, 14, True), (256, 128))]:
        L = capi.layout(*shape)
        assert (L.gemm_run, L.gemm_tile_rows, L.gemm_tile_cols) == (1,) + tile, shape


def test_sweep_reaches_every_gemm_form():
    """The GPU sweep's shapes (tests/test_gpu_sweep.py) cover each launch
    form of the modular GEMM."""
    from test_gpu_sweep import CASES, RUN_CASES
    forms = set()
    for (_, kind, batch, M, N, K, P, corr, _) in CASES + RUN_CASES:
        L = capi.layout(batch, M, N, K, P, corr)
        mixed = (L.gemm_tile_cols == 256 and L.Np // 256 >= 2 and 0 < N % 256 <= 128)
        forms.add(("tile", L.gemm_tile_rows, L.gemm_tile_cols, mixed))
        forms.add(("ksplit", L.ksplit > 1))
        forms.add(("run", L.gemm_run > 1))
    for f in [("tile", 256, 256, False), ("tile", 256, 256, True), ("tile", 256, 128, False),
              ("tile", 128, 128, False), ("ksplit", True), ("ksplit", False), ("run", True),
              ("run", False)]:
        assert f in forms, f


def test_run_checks_operand_extents():
    """The C entry points read every extent from their arguments: the
    ctypes helper refuses operands whose shapes disagree before any call."""
    A = torch.zeros(2, 3, 5, dtype=torch.float64)
    with pytest.raises(ValueError, match="K of A"):
        capi.run("bmm", A, torch.zeros(2, 5, 3, dtype=torch.float64), capi_primes(3))
    with pytest.raises(ValueError, match="batch"):
        capi.run("bmm_nt", A, torch.zeros(3, 5, 4, dtype=torch.float64), capi_primes(3))
    with pytest.raises(ValueError, match="K of A"):
        capi.run("mm_nt", A[0], torch.zeros(4, 5, dtype=torch.float64), capi_primes(3))
    with pytest.raises(ValueError, match="dims"):
        capi.run("mm", A, torch.zeros(4, 5, dtype=torch.float64), capi_primes(3))
    with pytest.raises(ValueError, match="contiguous float64"):
        capi.run("mm", A[0], torch.zeros(4, 5, dtype=torch.float32), capi_primes(3))


def test_baseline_config_launch_forms():
    """The launch forms of the BASELINE configs, which the profiles and the
    bench figures were measured with (K-split, GEMM tile, slot run, correction
    planes, sizing slabs): a layout change that moves one of them is a
    deliberate one."""
    forms = {
        "c1": ((1, 128, 128, 4096, 14, True), (8, 128, 128, 1, 2, 128)),
        "c2": ((1, 8192, 8192, 8192, 14, True), (1, 256, 256, 1, 1, 16)),
        "c2r": ((1, 8192, 8192, 8192, 13, False), (1, 256, 256, 1, 0, 16)),
        "c3": ((1, 4096, 4096, 4096, 14, True), (1, 256, 256, 1, 1, 32)),
        "c4": ((64, 512, 512, 512, 14, True), (1, 256, 256, 14, 1, 4)),
        "c5": ((1, 1023, 2049, 32769, 15, True), (2, 256, 256, 1, 2, 63)),
        "c5r": ((1, 1023, 2049, 32769, 13, False), (2, 256, 256, 1, 0, 63)),
    }
    for name, (shape, want) in forms.items():
        L = capi.layout(*shape)
        got = (L.ksplit, L.gemm_tile_rows, L.gemm_tile_cols, L.gemm_run, L.ncorr, L.nslab)
        assert got == want, (name, got, want)


def test_nt_helpers_check_operand_extents():
    """mm_nt_events, mm_nt_noalloc and ddgemm_nt hand bare pointers to the
    library: their ctypes helpers refuse mismatched shapes, dtypes, layouts
    and host tensors before any call."""
    A = torch.zeros(4, 5, dtype=torch.float64)
    pr = capi_primes(3)
    with pytest.raises(ValueError, match="K of A"):
        capi.mm_nt_noalloc(A, torch.zeros(6, 3, dtype=torch.float64), pr)
    with pytest.raises(ValueError, match="2-D"):
        capi.mm_nt_noalloc(A, torch.zeros(1, 5, 3, dtype=torch.float64), pr)
    with pytest.raises(ValueError, match="contiguous float64 on one GPU"):
        capi.mm_nt_noalloc(A, torch.zeros(5, 3, dtype=torch.float64), pr)   # host tensors
    with pytest.raises(ValueError, match="contiguous float64 on one GPU"):
        capi.mm_nt_noalloc(A, torch.zeros(3, 5, dtype=torch.float64).t(), pr)
    with pytest.raises(ValueError, match="K of A"):
        capi.mm_nt_events(A, torch.zeros(4, 3, dtype=torch.float64), pr,
                          torch.zeros(4, 3, dtype=torch.float64), None, None)
    with pytest.raises(ValueError, match="K of A"):
        capi.ddgemm_nt(A, torch.zeros(3, 6, dtype=torch.float64))


def test_probe_source_and_expected_layout():
    """The ceiling probe's source: balanced residues, stage 1 = (-A0, B0).
    The expected accumulators decode the planes' fragment order and the
    accumulator order: a single product of ones lands where they place it."""
    src = capi.probe_source(1)
    t = capi.TILE_R * capi.TILE_K
    assert src.size == capi.PROBE_SOURCE_BYTES == 4 * t
    assert src.min() >= -127 and src.max() <= 127
    assert np.array_equal(src[2 * t:3 * t], -src[:t]) and np.array_equal(src[3 * t:], src[t:2 * t])
    one = np.zeros(capi.PROBE_SOURCE_BYTES, np.int8)
    # A fragment 0: row 5, k = 16 * 2 + 3 (lane 2 * 16 + 5, byte 3); B fragment
    # 9 (wave wn = 1, y = 1): column 11, the same k (lane 2 * 16 + 11, byte 3).
    one[16 * (2 * 16 + 5) + 3] = 3
    one[t + 9 * capi.FRAG + 16 * (2 * 16 + 11) + 3] = -2
    exp = capi.probe_expected(one)
    nz = np.argwhere(exp)
    # wave 1 (wm 0, wn 1), x 0, y 1; row 5 = 4 (l / 16) + v -> l / 16 = 1,
    # v = 1; column 11 = l mod 16 -> lane 27, element 4 * 27 + 1.
    assert nz.tolist() == [[1, 0, 1, 4 * 27 + 1]] and exp[1, 0, 1, 109] == -6
