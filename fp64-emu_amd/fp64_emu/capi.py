"""ctypes binding of the C ABI (include/fp64emu.h) plus host-side decoders of
the workspace map, for stage-level inspection by tests and the bench.

Calls go straight to libfp64emu.so with device pointers from torch tensors
and the current torch stream; no torch C++ is involved.  Decoders turn the
tile-blocked operand planes and the blocked output planes back into logical
[rows, K] / [M, N] arrays (numpy).
"""
import ctypes
import os

import numpy as np
import torch  # loads torch's HIP runtime before libfp64emu.so binds to it

from . import _ops  # noqa: F401  (fails loudly when the extension is missing)

_HERE = os.path.dirname(os.path.abspath(__file__))
CAPI_PATH = os.path.join(_HERE, "libfp64emu.so")

TILE_R, TILE_K, FRAG = 256, 64, 1024

# Every function declared in include/fp64emu.h.
EXPORTS = ("fp64emu_maxp", "fp64emu_last_error", "fp64emu_workspace_size",
           "fp64emu_workspace_size_min", "fp64emu_mm",
           "fp64emu_mm_nt", "fp64emu_bmm", "fp64emu_bmm_nt", "fp64emu_mm_timed",
           "fp64emu_mm_nt_events", "fp64emu_bmm_nt_events", "fp64emu_mm_nt_noalloc",
           "fp64emu_layout",
           "fp64emu_ddgemm_nt", "fp64emu_probe_mfma", "fp64emu_probe_stream")

NOALLOC_SCRATCH_BYTES = 64 << 20   # FP64EMU_NOALLOC_SCRATCH_BYTES


class Layout(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int64), ("M", ctypes.c_int64), ("N", ctypes.c_int64),
                ("K", ctypes.c_int64), ("nprimes", ctypes.c_int), ("use_corr", ctypes.c_int),
                ("ncorr", ctypes.c_int), ("nslab", ctypes.c_int), ("deep", ctypes.c_int),
                ("nseg", ctypes.c_int), ("kseg", ctypes.c_int64), ("ksplit", ctypes.c_int),
                ("nchunk", ctypes.c_int), ("chunk_rows", ctypes.c_int64), ("Mp", ctypes.c_int64),
                ("Np", ctypes.c_int64), ("Kp", ctypes.c_int64), ("planeA_bytes", ctypes.c_int64),
                ("planeB_bytes", ctypes.c_int64), ("memberA_bytes", ctypes.c_int64),
                ("memberB_bytes", ctypes.c_int64), ("outplane_bytes", ctypes.c_int64)] + [
                   (n, ctypes.c_size_t) for n in (
                       "off_sftA", "off_sftB", "off_lgA", "off_lgB", "off_bits", "off_pmax",
                       "off_pss", "off_planesA", "off_planesB", "off_res8", "off_corr", "total")] + [
                   ("gemm_tile_cols", ctypes.c_int), ("gemm_tile_rows", ctypes.c_int),
                   ("gemm_run", ctypes.c_int), ("ext_rowsA", ctypes.c_int64),
                   ("ext_rowsB", ctypes.c_int64), ("gemm_split", ctypes.c_int)]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


_LIB = None


def lib():
    global _LIB
    if _LIB is not None:
        return _LIB
    L = ctypes.CDLL(CAPI_PATH)
    i64, i32, vp, sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
    L.fp64emu_maxp.restype = i32
    L.fp64emu_last_error.restype = ctypes.c_char_p
    L.fp64emu_workspace_size.argtypes = [i64, i64, i64, i64, i32, i32]
    L.fp64emu_workspace_size.restype = sz
    L.fp64emu_workspace_size_min.argtypes = [i64, i64, i64, i64, i32, i32]
    L.fp64emu_workspace_size_min.restype = sz
    mm_args = [vp, vp, vp, i64, i64, i64, vp, vp, vp, i32, i32, i64, i32, vp, sz, vp]
    for name in ("fp64emu_mm", "fp64emu_mm_nt"):
        getattr(L, name).argtypes = mm_args
        getattr(L, name).restype = i32
    bmm_args = [vp, vp, vp, i64, i64, i64, i64, vp, vp, vp, i32, i32, i64, i32, vp, sz, vp]
    for name in ("fp64emu_bmm", "fp64emu_bmm_nt"):
        getattr(L, name).argtypes = bmm_args
        getattr(L, name).restype = i32
    L.fp64emu_mm_timed.argtypes = [vp, vp, vp, vp, i64, i64, i64, vp, vp, vp, i32, i32, i64, i32,
                                   vp, sz, vp]
    L.fp64emu_mm_timed.restype = i32
    L.fp64emu_mm_nt_events.argtypes = mm_args + [ctypes.POINTER(ctypes.c_void_p)]
    L.fp64emu_mm_nt_events.restype = i32
    L.fp64emu_bmm_nt_events.argtypes = bmm_args + [ctypes.POINTER(ctypes.c_void_p)]
    L.fp64emu_bmm_nt_events.restype = i32
    L.fp64emu_mm_nt_noalloc.argtypes = [vp, vp, vp, i64, i64, i64, vp, vp, vp, i32, i32, i64,
                                        i32, vp]
    L.fp64emu_mm_nt_noalloc.restype = i32
    L.fp64emu_layout.argtypes = [i64, i64, i64, i64, i32, i32, ctypes.POINTER(Layout)]
    L.fp64emu_layout.restype = i32
    L.fp64emu_ddgemm_nt.argtypes = [vp, vp, vp, vp, i64, i64, i64, vp]
    L.fp64emu_ddgemm_nt.restype = i32
    L.fp64emu_probe_mfma.argtypes = [vp, vp, vp, i64, i64, i32, vp]
    L.fp64emu_probe_mfma.restype = i32
    L.fp64emu_probe_stream.argtypes = [vp, vp, i64, i32, vp]
    L.fp64emu_probe_stream.restype = i32
    _LIB = L
    return L


class CapiError(RuntimeError):
    pass


def _check(st):
    if st != 0:
        raise CapiError(lib().fp64emu_last_error().decode())


def layout(batch, M, N, K, nprimes, use_corr):
    out = Layout()
    _check(lib().fp64emu_layout(batch, M, N, K, nprimes, int(bool(use_corr)), ctypes.byref(out)))
    return out


def workspace_size(batch, M, N, K, nprimes, use_corr):
    return lib().fp64emu_workspace_size(batch, M, N, K, nprimes, int(bool(use_corr)))


def workspace_size_min(batch, M, N, K, nprimes, use_corr):
    return lib().fp64emu_workspace_size_min(batch, M, N, K, nprimes, int(bool(use_corr)))


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def run(kind, A, B, primes, exact=True, bits=53, use_corr=True, out=None, ws=None, fill=None):
    """Call fp64emu_{mm,mm_nt,bmm,bmm_nt} on device tensors.  Returns
    (out, ws, layout); `ws` holds the call's intermediates afterwards.  A
    new workspace is filled with the byte `fill` first when it is given (so
    that tests see any read of memory the call never wrote)."""
    primes = np.ascontiguousarray(np.asarray(primes, dtype=np.int32))
    P = int(primes.size)
    batched = kind in ("bmm", "bmm_nt")
    nt = kind.endswith("_nt")
    # The C entry points take bare pointers: every extent they read is checked
    # here against the tensors, before any launch.
    if A.dim() != (3 if batched else 2) or B.dim() != A.dim():
        raise ValueError(f"{kind}: operands of {A.dim()} and {B.dim()} dims")
    if batched:
        batch, M, K = A.shape
        if B.shape[0] != batch:
            raise ValueError(f"{kind}: batch {batch} against {B.shape[0]}")
    else:
        batch = 1
        M, K = A.shape
    KB, N = (B.shape[-2], B.shape[-1]) if nt else (B.shape[-1], B.shape[-2])
    if KB != K:
        raise ValueError(f"{kind}: K of A is {K}, of B {KB} (B {tuple(B.shape)})")
    for name, t in (("A", A), ("B", B)):
        if t.dtype != torch.float64 or not t.is_contiguous() or t.device != A.device:
            raise ValueError(f"{kind}: {name} must be contiguous float64 on {A.device}")
    lay = layout(batch, M, N, K, P, use_corr)
    if ws is None:
        ws = torch.empty(max(int(lay.total), 1), dtype=torch.uint8, device=A.device)
        if fill is not None:
            ws.fill_(fill)
    shape = (batch, M, N) if batched else (M, N)
    if out is None:
        out = torch.empty(shape, dtype=torch.float64, device=A.device)
    elif tuple(out.shape) != shape or out.dtype != torch.float64 or not out.is_contiguous():
        raise ValueError(f"{kind}: out must be contiguous float64 of shape {shape}")
    pp = primes.ctypes.data_as(ctypes.c_void_p)
    fn = getattr(lib(), "fp64emu_" + kind)
    common = (pp, None, None, P, int(bool(exact)), int(bits), int(bool(use_corr)),
              ws.data_ptr(), ws.numel(), _stream())
    if batched:
        st = fn(out.data_ptr(), A.data_ptr(), B.data_ptr(), batch, M, N, K, *common)
    else:
        st = fn(out.data_ptr(), A.data_ptr(), B.data_ptr(), M, N, K, *common)
    _check(st)
    return out, ws, lay


def mm_timed(A, B, primes, exact=True, bits=53, use_corr=True):
    primes = np.ascontiguousarray(np.asarray(primes, dtype=np.int32))
    M, K = A.shape
    N = B.shape[0]
    lay = layout(1, M, N, K, primes.size, use_corr)
    ws = torch.empty(max(int(lay.total), 1), dtype=torch.uint8, device=A.device)
    out = torch.empty((M, N), dtype=torch.float64, device=A.device)
    times = (ctypes.c_float * 4)()
    _check(lib().fp64emu_mm_timed(out.data_ptr(), times, A.data_ptr(), B.data_ptr(), M, N, K,
                                  primes.ctypes.data_as(ctypes.c_void_p), None, None,
                                  primes.size, int(bool(exact)), int(bits),
                                  int(bool(use_corr)), ws.data_ptr(), ws.numel(), _stream()))
    return out, list(times)


_HIP = None
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000   # hip_runtime_api.h


def _hip():
    """The HIP runtime torch already loaded."""
    global _HIP
    if _HIP is None:
        H = ctypes.CDLL("libamdhip64.so")
        H.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        H.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                          ctypes.c_void_p]
        H.hipEventDestroy.argtypes = [ctypes.c_void_p]
        _HIP = H
    return _HIP


class PhaseEvents:
    """Five timing events for fp64emu_mm_nt_events.  Created without the
    system-scope fence on record (hipEventDisableSystemFence): a timing-only
    event then costs no cache writeback and invalidation, which would
    otherwise slow the work it brackets."""

    def __init__(self):
        H = _hip()
        self.handles = (ctypes.c_void_p * 5)()
        for i in range(5):
            ev = ctypes.c_void_p()
            if H.hipEventCreateWithFlags(ctypes.byref(ev), HIP_EVENT_DISABLE_SYSTEM_FENCE) != 0:
                raise CapiError("hipEventCreateWithFlags failed")
            self.handles[i] = ev.value

    def phases_ms(self):
        """[sizing+extract, gemms, 0-marker, reconstruct] after a sync."""
        H = _hip()
        out = []
        for i in range(4):
            t = ctypes.c_float()
            if H.hipEventElapsedTime(ctypes.byref(t), self.handles[i], self.handles[i + 1]) != 0:
                raise CapiError("hipEventElapsedTime failed")
            out.append(t.value)
        return out

    def __del__(self):
        if _HIP is not None:
            for h in self.handles:
                if h:
                    _HIP.hipEventDestroy(h)


def _check_nt(name, A, Bt, out=None, b_nk=False):
    """The extents a C entry point reads through bare pointers, checked
    against the tensors before the call: 2-D contiguous float64 operands on
    one GPU, A [M, K] against Bt [K, N] (or B [N, K] with b_nk), and `out`
    contiguous float64 [M, N] on that GPU.  Returns (M, N, K)."""
    if A.dim() != 2 or Bt.dim() != 2:
        raise ValueError(f"{name}: operands must be 2-D, got {A.dim()} and {Bt.dim()} dims")
    M, K = A.shape
    N, KB = (Bt.shape[0], Bt.shape[1]) if b_nk else (Bt.shape[1], Bt.shape[0])
    if KB != K:
        raise ValueError(f"{name}: K of A is {K}, of B {KB} (B {tuple(Bt.shape)})")
    for tag, t in (("A", A), ("B", Bt)):
        if t.dtype != torch.float64 or not t.is_contiguous() or not t.is_cuda or t.device != A.device:
            raise ValueError(f"{name}: {tag} must be contiguous float64 on one GPU ({A.device})")
    if out is not None and (tuple(out.shape) != (M, N) or out.dtype != torch.float64
                            or not out.is_contiguous() or out.device != A.device):
        raise ValueError(f"{name}: out must be contiguous float64 of shape {(M, N)} on {A.device}")
    return M, N, K


def mm_nt_events(A, Bt, primes, out, ws, events, exact=True, bits=53, use_corr=True):
    """fp64emu_mm_nt_events on preallocated `out` and workspace `ws`."""
    primes = np.ascontiguousarray(np.asarray(primes, dtype=np.int32))
    M, N, K = _check_nt("mm_nt_events", A, Bt, out)
    if ws.dtype != torch.uint8 or not ws.is_contiguous() or ws.device != A.device:
        raise ValueError(f"mm_nt_events: ws must be a contiguous uint8 tensor on {A.device}")
    _check(lib().fp64emu_mm_nt_events(out.data_ptr(), A.data_ptr(), Bt.data_ptr(), M, N, K,
                                      primes.ctypes.data_as(ctypes.c_void_p), None, None,
                                      primes.size, int(bool(exact)), int(bits),
                                      int(bool(use_corr)), ws.data_ptr(), ws.numel(), _stream(),
                                      events.handles))
    return out


def bmm_nt_events(A, Bt, primes, out, ws, events, exact=True, bits=53, use_corr=True):
    """fp64emu_bmm_nt_events on preallocated `out` [b, M, N] and workspace `ws`."""
    primes = np.ascontiguousarray(np.asarray(primes, dtype=np.int32))
    if A.dim() != 3 or Bt.dim() != 3 or Bt.shape[0] != A.shape[0] or Bt.shape[1] != A.shape[2]:
        raise ValueError(f"bmm_nt_events: A {tuple(A.shape)} against Bt {tuple(Bt.shape)}")
    batch, M, K = A.shape
    N = Bt.shape[2]
    for tag, t in (("A", A), ("Bt", Bt), ("out", out)):
        if t.dtype != torch.float64 or not t.is_contiguous() or not t.is_cuda or t.device != A.device:
            raise ValueError(f"bmm_nt_events: {tag} must be contiguous float64 on one GPU")
    if tuple(out.shape) != (batch, M, N):
        raise ValueError(f"bmm_nt_events: out must be of shape {(batch, M, N)}")
    if ws.dtype != torch.uint8 or not ws.is_contiguous() or ws.device != A.device:
        raise ValueError(f"bmm_nt_events: ws must be a contiguous uint8 tensor on {A.device}")
    _check(lib().fp64emu_bmm_nt_events(out.data_ptr(), A.data_ptr(), Bt.data_ptr(), batch, M, N,
                                       K, primes.ctypes.data_as(ctypes.c_void_p), None, None,
                                       primes.size, int(bool(exact)), int(bits),
                                       int(bool(use_corr)), ws.data_ptr(), ws.numel(),
                                       _stream(), events.handles))
    return out


def mm_nt_noalloc(A, Bt, primes, out=None, exact=True, bits=53, use_corr=True):
    """fp64emu_mm_nt_noalloc: the library's static device scratch instead of
    a workspace argument."""
    primes = np.ascontiguousarray(np.asarray(primes, dtype=np.int32))
    M, N, K = _check_nt("mm_nt_noalloc", A, Bt, out)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float64, device=A.device)
    _check(lib().fp64emu_mm_nt_noalloc(out.data_ptr(), A.data_ptr(), Bt.data_ptr(), M, N, K,
                                       primes.ctypes.data_as(ctypes.c_void_p), None, None,
                                       primes.size, int(bool(exact)), int(bits),
                                       int(bool(use_corr)), _stream()))
    return out


def ddgemm_nt(A, B):
    """Double-double C = A @ B^T on the device (A [M,K], B [N,K])."""
    M, N, K = _check_nt("ddgemm_nt", A, B, b_nk=True)
    hi = torch.empty((M, N), dtype=torch.float64, device=A.device)
    lo = torch.empty_like(hi)
    _check(lib().fp64emu_ddgemm_nt(hi.data_ptr(), lo.data_ptr(), A.data_ptr(), B.data_ptr(),
                                   M, N, K, _stream()))
    return hi, lo


# ---- ceiling probes --------------------------------------------------------

PROBE_SOURCE_BYTES = 2 * 2 * TILE_R * TILE_K   # two stages of an A and a B tile


def probe_source(seed=0):
    """The probe's two stages (host int8, 64 KiB): stage 0's A and B tiles
    are random balanced residues in [-127, 127]; stage 1 holds the negated A
    tile and the same B tile, so its products cancel stage 0's."""
    rng = np.random.default_rng(seed)
    tile = TILE_R * TILE_K
    a = rng.integers(-127, 128, tile, dtype=np.int64).astype(np.int8)
    b = rng.integers(-127, 128, tile, dtype=np.int64).astype(np.int8)
    return np.concatenate([a, b, -a, b])


def probe_expected(src):
    """Group 0's accumulators after an odd step count (stage 0's products),
    [4 waves, 8, 8, 256] int32, from the fragment order of the planes (lane
    l = 16 (k / 16) + row holds k mod 16 as 16 bytes) and of the
    accumulators (lane l's value v is row 4 (l / 16) + v, column l mod 16)."""
    src = np.asarray(src, dtype=np.int8)
    tile = TILE_R * TILE_K
    lane = np.arange(64)
    rows, kb = lane % 16, lane // 16

    def frag(off):
        F = src[off:off + FRAG].astype(np.int64).reshape(64, 16)
        X = np.zeros((16, 64), np.int64)
        for l in range(64):
            X[rows[l], 16 * kb[l]:16 * kb[l] + 16] = F[l]
        return X

    out = np.zeros((4, 8, 8, 256), np.int64)
    for w in range(4):
        wm, wn = w >> 1, w & 1
        for x in range(8):
            Ax = frag((wm * 8 + x) * FRAG)
            for y in range(8):
                C = Ax @ frag(tile + (wn * 8 + y) * FRAG).T
                for l in range(64):
                    out[w, x, y, 4 * l:4 * l + 4] = C[4 * (l // 16):4 * (l // 16) + 4, l % 16]
    return out.astype(np.int32)


def probe_mfma(src_dev, groups, steps, mode):
    """fp64emu_probe_mfma on a device int8 source of PROBE_SOURCE_BYTES.
    Returns (acc [4, 8, 8, 256] int32, clocks [groups, 4] int64 device
    tensors: clk0, clk1, rt0, rt1)."""
    if src_dev.dtype != torch.int8 or src_dev.numel() != PROBE_SOURCE_BYTES or not src_dev.is_cuda:
        raise ValueError(f"probe_mfma: source must be {PROBE_SOURCE_BYTES} int8 on a GPU")
    acc = torch.empty((4, 8, 8, 256), dtype=torch.int32, device=src_dev.device)
    clk = torch.empty((groups, 4), dtype=torch.int64, device=src_dev.device)
    _check(lib().fp64emu_probe_mfma(acc.data_ptr(), clk.data_ptr(), src_dev.data_ptr(), groups,
                                    steps, mode, _stream()))
    return acc, clk


def probe_stream(dst, src, mode):
    """fp64emu_probe_stream over dst.numel() doubles (src: same size, unused
    by mode 1)."""
    n = dst.numel()
    if dst.dtype != torch.float64 or not dst.is_contiguous() or not dst.is_cuda:
        raise ValueError("probe_stream: dst must be contiguous float64 on a GPU")
    if mode != 1 and (src is None or src.dtype != torch.float64 or src.numel() != n
                      or not src.is_contiguous() or src.device != dst.device):
        raise ValueError("probe_stream: src must match dst")
    _check(lib().fp64emu_probe_stream(dst.data_ptr(), src.data_ptr() if src is not None else None,
                                      n, mode, _stream()))


# ---- workspace decoders (host, numpy) --------------------------------------

def _ws_bytes(ws):
    if isinstance(ws, torch.Tensor):
        return ws.cpu().numpy()
    return np.asarray(ws, dtype=np.uint8)


def sizing(ws, lay):
    """(sftA [batch*M], sftB [batch*N], lgA, lgB, bits_eff) after the call.
    The workspace keeps the shifts as sized per row/column and, beside
    bits_eff, the amount the width pick adds to every one of them; the
    shifts returned here include it."""
    w = _ws_bytes(ws)
    MF, NF = lay.batch * lay.M, lay.batch * lay.N
    be, g = (int(v) for v in w[lay.off_bits:lay.off_bits + 8].view(np.int32))
    sftA = (w[lay.off_sftA:lay.off_sftA + 2 * MF].view(np.int16) + g).astype(np.int16)
    sftB = (w[lay.off_sftB:lay.off_sftB + 2 * NF].view(np.int16) + g).astype(np.int16)
    lgA = w[lay.off_lgA:lay.off_lgA + 4 * MF].view(np.float32).copy()
    lgB = w[lay.off_lgB:lay.off_lgB + 4 * NF].view(np.float32).copy()
    return sftA, sftB, lgA, lgB, be


def _plane_to_logical(raw, rows_p, depth_p):
    """One tile-blocked plane (bytes) -> int8 [rows_p, depth_p].  A 256 x 64
    tile holds 16 fragments of 16 rows x 64 k, fragment row%256//16; inside
    one, lane l = 16*(k%64//16) + row%16 holds k%16 at byte 16*l + k%16."""
    nrt, nkt = rows_p // TILE_R, depth_p // TILE_K
    a = raw.view(np.int8).reshape(nrt, nkt, 16, 4, 16, 16)   # rt kt rb kg r16 kb
    return a.transpose(0, 2, 4, 1, 3, 5).reshape(rows_p, depth_p)


def planes(ws, lay, operand):
    """Operand planes of the call: (res [batch, P, rows, K],
    hi [batch, rows, K], q [batch, rows, K]) with padding stripped, plus the
    padded arrays for padding checks: (res_p, corr_p)."""
    w = _ws_bytes(ws)
    isA = operand == "A"
    rows, rows_p = (lay.M, lay.Mp) if isA else (lay.N, lay.Np)
    off = lay.off_planesA if isA else lay.off_planesB
    member = lay.memberA_bytes if isA else lay.memberB_bytes
    plane = lay.planeA_bytes if isA else lay.planeB_bytes
    P, Kp, K = lay.nprimes, lay.Kp, lay.K
    res_p = np.zeros((lay.batch, P, rows_p, Kp), dtype=np.int8)
    corr_p = np.zeros((lay.batch, rows_p, 2 * Kp), dtype=np.int8) if lay.use_corr else None
    for b in range(lay.batch):
        base = off + b * member
        for t in range(P):
            raw = w[base + t * plane: base + (t + 1) * plane]
            res_p[b, t] = _plane_to_logical(raw, rows_p, Kp)
        if lay.use_corr and Kp > 0:
            raw = w[base + P * plane: base + (P + 2) * plane]
            corr_p[b] = _plane_to_logical(raw, rows_p, 2 * Kp)
    res = res_p[:, :, :rows, :K]
    if lay.use_corr:
        first, second = corr_p[:, :rows, :K], corr_p[:, :rows, Kp:Kp + K]
        hi, q = (first, second) if isA else (second, first)
    else:
        hi = q = None
    return res, hi, q, res_p, corr_p


def _blocks_to_logical(arr, Mp, Np):
    """Blocked output plane -> [Mp, Np].  Blocks of 16 rows x 64 columns,
    row-block major; element 16*l + 4*q + v of a block (lane l of the GEMM's
    accumulator order, column block q, row v) is at row 4*(l//16) + v,
    column 16*q + l%16."""
    a = arr.reshape(Mp // 16, Np // 64, 4, 16, 4, 4)          # rb cb lh lc q v
    return a.transpose(0, 2, 5, 1, 4, 3).reshape(Mp, Np)


def outputs(ws, lay, primes=None):
    """(res8 [batch, P, M, N] int8, corr [batch, ncorr, M, N] int64).  With a
    K-split the S partial residues are summed and reduced to the balanced
    residue (bal8's convention: r > p/2 -> r - p, as int8), which needs the
    moduli, and the S partial correction sums are added."""
    w = _ws_bytes(ws)
    P, Mp, Np, ob, S = lay.nprimes, lay.Mp, lay.Np, lay.outplane_bytes, max(lay.ksplit, 1)
    res = np.zeros((lay.batch, P, lay.M, lay.N), dtype=np.int8)
    corr = np.zeros((lay.batch, lay.ncorr, lay.M, lay.N), dtype=np.int64)
    if S > 1 and primes is None:
        raise ValueError("a K-split call needs the moduli to fold its residues")
    for b in range(lay.batch):
        for t in range(P):
            acc = np.zeros((lay.M, lay.N), dtype=np.int64)
            for sp in range(S):
                s0 = lay.off_res8 + ((sp * lay.batch + b) * P + t) * ob
                acc += _blocks_to_logical(w[s0:s0 + ob].view(np.int8), Mp, Np)[:lay.M, :lay.N]
            if S > 1:
                p = int(primes[t])
                r = np.mod(acc, p)
                acc = np.where(r > p // 2, r - p, r)
            res[b, t] = acc.astype(np.int8)
        for c in range(lay.ncorr):
            for sp in range(S):
                s0 = lay.off_corr + 4 * ((sp * lay.batch + b) * lay.ncorr + c) * ob
                corr[b, c] += _blocks_to_logical(w[s0:s0 + 4 * ob].view(np.int32), Mp, Np)[:lay.M, :lay.N]
    return res, corr
