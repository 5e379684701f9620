"""Stage-by-stage parity of one HIP call against the CPU oracle.

`check_call` runs one C-ABI call, then compares, in order:
  sizing   shifts (exact), log2-norms (float equality up to 1 ulp on a tiny
           fraction, from log2 implementations), bits_eff (exact);
  planes   residue / hi7 / q7 planes, bit-exact against the oracle's
           extraction at the GPU's shifts and width; padding all zero;
  outputs  int8 residue planes and int32 correction sums of the GEMMs,
           bit-exact against the oracle's modular GEMM of those planes;
  result   the float64 output, bit-exact against the oracle's
           reconstruction of the GPU's residues, and against the oracle's
           whole pipeline.
"""
import numpy as np
import torch

import oracle as O
from fp64_emu import capi


def bits_equal(a, b):
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float64))
    b = np.ascontiguousarray(np.asarray(b, dtype=np.float64))
    return a.shape == b.shape and np.array_equal(a.view(np.uint64), b.view(np.uint64))


def oracle_sizing(A, B, b_kn, primes, bits):
    """Oracle sizing of the call's operands (before the width pick)."""
    A = np.asarray(A)
    if A.ndim == 2:
        A = A[None]
    B = np.asarray(B)
    if B.ndim == 2:
        B = B[None]
    sA, lA = O.size_rows(A.reshape(-1, A.shape[-1]), bits)
    if b_kn:
        sB, lB = O.size_cols(B, bits)
    else:
        sB, lB = O.size_rows(B.reshape(-1, B.shape[-1]), bits)
    _, _, _, log2M = O.tables(primes)
    be, sA2, sB2 = O.pick_bits(lA, lB, min(log2M, 126.0), bits, sA, sB)
    return be, sA2, sB2, lA, lB


def check_call(kind, A, B, primes, exact=True, bits=53, use_corr=True, full_oracle=True):
    """A, B: device float64 tensors in the layout `kind` expects."""
    b_kn = kind in ("mm_nt", "bmm_nt")
    out, ws, lay = capi.run(kind, A, B, primes, exact=exact, bits=bits, use_corr=use_corr,
                            fill=0x5A)
    torch.cuda.synchronize()
    Ah, Bh = A.cpu().numpy(), B.cpu().numpy()
    primes = np.asarray(primes, dtype=np.int32)
    P = primes.size
    wsh = ws.cpu().numpy()

    # sizing
    gsA, gsB, glA, glB, gbe = capi.sizing(wsh, lay)
    obe, osA, osB, olA, olB = oracle_sizing(Ah, Bh, b_kn, primes, bits)
    for g, o in ((glA, olA), (glB, olB)):
        neq = g != o
        if neq.any():
            # log2 of the same fp64 sum may differ by an ulp between libm's;
            # the float then differs by at most one ulp, rarely.
            gi, oi = g[neq].view(np.int32).astype(np.int64), o[neq].view(np.int32).astype(np.int64)
            assert np.all(np.abs(gi - oi) <= 1), "log2-norms differ by more than 1 ulp"
            assert neq.mean() < 1e-3
    assert gbe == obe, f"bits_eff GPU {gbe} oracle {obe}"
    assert np.array_equal(gsA, osA) and np.array_equal(gsB, osB), "shifts differ"

    # planes (at the GPU's sizing)
    batch = lay.batch
    A3 = Ah if Ah.ndim == 3 else Ah[None]
    B3 = Bh if Bh.ndim == 3 else Bh[None]
    oresA, ohA, oqA = O.extract_operand(A3, 0, gsA, gbe, primes, use_corr)
    oresB, ohB, oqB = O.extract_operand(B3, 1 if b_kn else 0, gsB, gbe, primes, use_corr)
    gresA, ghA, gqA, gresA_p, gcorrA_p = capi.planes(wsh, lay, "A")
    gresB, ghB, gqB, gresB_p, gcorrB_p = capi.planes(wsh, lay, "B")
    assert np.array_equal(gresA, oresA), "A residue planes differ"
    assert np.array_equal(gresB, oresB), "B residue planes differ"
    M, N, K = lay.M, lay.N, lay.K
    # Padding the GEMM reads is zero; plane rows past ext_rows are never
    # written (the workspace was filled with a nonzero pattern before the
    # call, so a GEMM read of them would show in its outputs below).
    pad = np.zeros(gresA_p.shape, bool)
    pad[:, :, :lay.ext_rowsA, :] = True
    pad[:, :, :M, :K] = False
    assert not gresA_p[pad].any(), "A padding not zero"
    pad = np.zeros(gresB_p.shape, bool)
    pad[:, :, :lay.ext_rowsB, :] = True
    pad[:, :, :N, :K] = False
    assert not gresB_p[pad].any(), "B padding not zero"
    if use_corr:
        assert np.array_equal(ghA, ohA) and np.array_equal(gqA, oqA), "A hi7/q7 differ"
        assert np.array_equal(ghB, ohB) and np.array_equal(gqB, oqB), "B hi7/q7 differ"

    # GEMM outputs
    gres8, gcorr = capi.outputs(wsh, lay, primes)
    for b in range(batch):
        for t in range(P):
            o8 = O.modgemm(oresA[b, t], oresB[b, t], int(primes[t]))
            assert np.array_equal(gres8[b, t], o8), f"residue GEMM {t} (member {b}) differs"
        if use_corr:
            oc = (O.modgemm(ohA[b], oqB[b], 0).astype(np.int64)
                  + O.modgemm(oqA[b], ohB[b], 0).astype(np.int64))
            gc = gcorr[b].astype(np.int64).sum(axis=0)
            assert np.array_equal(gc, oc), f"correction GEMMs (member {b}) differ"

    # result
    outh = out.cpu().numpy()
    out3 = outh if outh.ndim == 3 else outh[None]
    for b in range(batch):
        c1 = gcorr[b].astype(np.int64).sum(axis=0).astype(np.int32) if use_corr else None
        rec = O.reconstruct(gres8[b], c1, None, primes, gbe, gsA[b * M:(b + 1) * M],
                            gsB[b * N:(b + 1) * N], exact)
        assert bits_equal(out3[b], rec), f"reconstruction (member {b}) differs"
    if full_oracle:
        oout, info = O.mm(Ah, Bh, 1 if b_kn else 0, primes, exact=exact, bits=bits,
                          use_corr=use_corr)
        assert info["bits_eff"] == gbe
        assert bits_equal(outh, oout), "whole pipeline differs from the oracle"
    return out, ws, lay


def sampled_parity(kind, A, B, primes, rows, cols, exact=True, bits=53, use_corr=True,
                   ws=None):
    """Parity at sizes the oracle cannot finish whole: run the C-ABI call,
    then check (1) the sizing (shifts, width) against the oracle's sizing of
    the full operands, and (2) the outputs at rows x cols bit-exact against
    the oracle's extraction, modular GEMMs and reconstruction of just those
    rows and columns at that sizing.  2-D kinds only.  `ws`: a caller's
    workspace (one below the full size runs the rows of A in chunks; the
    sizing region sits at the same offsets either way).  Returns
    (out, bits_eff, workspace layout, device workspace)."""
    b_kn = kind == "mm_nt"
    if ws is not None:
        ws.fill_(0x5A)
    out, ws, lay = capi.run(kind, A, B, primes, exact=exact, bits=bits, use_corr=use_corr,
                            ws=ws, fill=0x5A)
    torch.cuda.synchronize()
    primes = np.asarray(primes, dtype=np.int32)
    head = ws[:lay.off_planesA].cpu().numpy()
    gsA, gsB, _, _, gbe = capi.sizing(head, lay)
    Ah, Bh = A.cpu().numpy(), B.cpu().numpy()
    obe, osA, osB, _, _ = oracle_sizing(Ah, Bh, b_kn, primes, bits)
    assert gbe == obe, f"bits_eff GPU {gbe} oracle {obe}"
    assert np.array_equal(gsA, osA) and np.array_equal(gsB, osB), "shifts differ"

    rows = np.asarray(sorted(set(int(r) for r in rows)))
    cols = np.asarray(sorted(set(int(c) for c in cols)))
    As = np.ascontiguousarray(Ah[rows])[None]
    Bs = np.ascontiguousarray(Bh[:, cols] if b_kn else Bh[cols])[None]
    rA, hA, qA = O.extract_operand(As, 0, gsA[rows], gbe, primes, use_corr)
    rB, hB, qB = O.extract_operand(Bs, 1 if b_kn else 0, gsB[cols], gbe, primes, use_corr)
    res = np.stack([O.modgemm(rA[0, t], rB[0, t], int(primes[t])) for t in range(primes.size)])
    c1 = O.modgemm(hA[0], qB[0], 0) if use_corr else None
    c2 = O.modgemm(qA[0], hB[0], 0) if use_corr else None
    rec = O.reconstruct(res, c1, c2, primes, gbe, gsA[rows], gsB[cols], exact)
    got = out.cpu().numpy()[np.ix_(rows, cols)]
    assert bits_equal(got, rec), "sampled outputs differ from the oracle"
    del Ah, Bh
    return out, gbe, lay, ws


def whole_parity(kind, A, B, primes, exact=True, bits=53, use_corr=True):
    """Parity of the whole output at the benchmark sizes: the C-ABI call on
    a workspace filled with a nonzero byte, its sizing (shifts, width)
    against the oracle's, and every output element bit for bit against the
    oracle pipeline with BLAS modular products (O.mm_blas, which the CPU
    tier pins to O.mm).  2-D kinds.  Returns (out, bits_eff, layout, ws)."""
    b_kn = kind == "mm_nt"
    out, ws, lay = capi.run(kind, A, B, primes, exact=exact, bits=bits, use_corr=use_corr,
                            fill=0x5A)
    torch.cuda.synchronize()
    head = ws[:lay.off_planesA].cpu().numpy()
    gsA, gsB, _, _, gbe = capi.sizing(head, lay)
    Ah, Bh = A.cpu().numpy(), B.cpu().numpy()
    oout, info = O.mm_blas(Ah, Bh, 1 if b_kn else 0, np.asarray(primes, dtype=np.int32),
                           exact=exact, bits=bits, use_corr=use_corr)
    assert info["bits_eff"] == gbe, f"bits_eff GPU {gbe} oracle {info['bits_eff']}"
    assert np.array_equal(info["sftA"], gsA) and np.array_equal(info["sftB"], gsB), "shifts differ"
    got = out.cpu().numpy()
    same = got.view(np.uint64) == oout.view(np.uint64)
    assert same.all(), f"{int((~same).sum())} of {same.size} outputs differ from the oracle"
    del Ah, Bh, oout
    return out, gbe, lay, ws
