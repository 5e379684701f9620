"""Left-looking blocked Cholesky whose block-column updates run as batched
products through fp64_emu.bmm (or torch.bmm for the native engine).

The reference drives its batched product from a right-looking tiled
Cholesky (bench/cholesky.py:22-49, README.md:315-320: residuals of 3-4e-16
with either engine).  This caller uses the other classical ordering, so each
batched call is deep instead of wide:

  for block column j = 0 .. nt-1:
    panel  = A[j:, j] - sum_{k<j} L[j:, k] L[j, k]^T      one bmm: member i is
                                                         block row j+i against
                                                         block row j, depth j*t
    L[j, j]  = chol(panel[0])                            native
    L[j+1:, j] = panel[1:] L[j, j]^-T                    native triangular solve

The batched product at step j has nt-j members of t x t outputs over depth
j*t; the panel factor and the solves stay native with both engines, so the
comparison isolates the batched product.  Accuracy is judged by the
factorization residual ||A - L L^T||_F / ||A||_F and by the backward error of
a solve with the factor.

    python fp64-emu_amd/callers/blocked_cholesky.py [n=16384] [t=512]
"""
import argparse
import os
import statistics
import sys
import time

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import fp64_emu  # noqa: E402


def native_bmm_bt(X, Y):
    """X [b, m, k] @ Y[b, n, k]^T on the native float64 path."""
    return torch.bmm(X, Y.transpose(1, 2).contiguous())


def emulated_bmm_bt(X, Y):
    return fp64_emu.bmm(X, Y)


ENGINES = {"native": native_bmm_bt, "emu": emulated_bmm_bt}


def spd_test_matrix(n, seed, device):
    """A well-conditioned SPD matrix from a CPU seed: G G^T / n + I (so the
    same bits reach every engine)."""
    g = torch.Generator().manual_seed(seed)
    G = torch.randn(n, n, dtype=torch.float64, generator=g).to(device)
    A = torch.mm(G, G.t()) / n
    A.diagonal().add_(1.0)
    return A


def left_looking(A, t, bmm_bt):
    """Lower L with A = L L^T (A symmetric positive definite, n a multiple of
    t).  Returns (L, seconds spent in the batched updates)."""
    n = A.shape[0]
    if n % t:
        raise ValueError("the tile must divide n")
    nt = n // t
    L = torch.zeros_like(A)
    upd_s = 0.0
    for j in range(nt):
        j0, j1 = j * t, (j + 1) * t
        panel = A[j0:, j0:j1].clone()            # block rows j .. nt-1 of block column j
        if j > 0:
            members = nt - j
            rows = L[j0:, :j0].reshape(members, t, j0)
            pivot = L[j0:j1, :j0].unsqueeze(0).expand(members, t, j0).contiguous()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            upd = bmm_bt(rows, pivot)            # member i: L[j+i, :j] L[j, :j]^T
            panel -= upd.reshape(members * t, t)
            torch.cuda.synchronize()
            upd_s += time.perf_counter() - t0
        diag = torch.linalg.cholesky(panel[:t])
        L[j0:j1, j0:j1] = diag
        if j1 < n:
            # X diag^T = panel[t:]  <=>  diag X^T = panel[t:]^T
            L[j1:, j0:j1] = torch.linalg.solve_triangular(diag, panel[t:].t(), upper=False).t()
    return L, upd_s


def factor_residual(A, L):
    return (torch.linalg.matrix_norm(A - L @ L.t()) / torch.linalg.matrix_norm(A)).item()


def solve_backward_error(A, L, seed=5):
    """||A x - b||_inf / (||A||_inf ||x||_inf) for x solved with the factor L."""
    g = torch.Generator().manual_seed(seed)
    b = torch.randn(A.shape[0], 1, dtype=torch.float64, generator=g).to(A.device)
    x = torch.cholesky_solve(b, L)
    r = A @ x - b
    return (r.abs().max() / (A.abs().sum(dim=1).max() * x.abs().max())).item()


def run(n, t, reps=3, device="cuda"):
    A = spd_test_matrix(n, 0, device)
    out = {"n": n, "t": t}
    for name, eng in ENGINES.items():
        totals, updates = [], []
        L = None
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            L, upd = left_looking(A, t, eng)
            torch.cuda.synchronize()
            totals.append(time.perf_counter() - t0)
            updates.append(upd)
        out[name] = {"total_s": statistics.median(totals), "update_s": statistics.median(updates),
                     "residual": factor_residual(A, L), "solve_berr": solve_backward_error(A, L)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("n", nargs="?", type=int, default=16384)
    ap.add_argument("t", nargs="?", type=int, default=512)
    args = ap.parse_args()
    r = run(args.n, args.t)
    print(f"{torch.cuda.get_device_name(0)} | left-looking n={r['n']} t={r['t']}", flush=True)
    for name in ENGINES:
        e = r[name]
        print(f"{name:>7}: total {e['total_s']:6.3f} s | batched updates {e['update_s']:6.3f} s | "
              f"||A-LL^T||/||A|| {e['residual']:.2e} | solve backward error {e['solve_berr']:.2e}",
              flush=True)


if __name__ == "__main__":
    main()
