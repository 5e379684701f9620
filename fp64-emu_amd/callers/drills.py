"""Application drills for the emulated GEMM: each algorithm runs once with
native float64 products and once with fp64_emu.mm_nt at the default plan;
only the product differs.  The reference's drill set (bench/apps.py:49-173:
throughput, exact path counts, CholeskyQR, Newton-Schulz polar factor,
Taylor exp) names the applications; the algorithms, checks and metrics here
are this build's:

  throughput   default and reduced operating points against native DGEMM
  walks        walk counts of a 0/1 digraph by repeated squaring, compared
               with an exact integer computation on the host
  cholqr2      two-pass CholeskyQR of a cond ~1e6 tall matrix: orthogonality
               after each pass and the backward error ||A - QR|| / ||A||
  polar        Newton-Schulz polar factor iterated until the orthogonality
               stops improving: iterations, ||U^T U - I||, ||A - U H|| / ||A||
  expm         exp(A) by scaling and squaring with a Paterson-Stockmeyer
               evaluation of the Taylor polynomial: error against
               torch.matrix_exp and ||exp(A) exp(-A) - I||

    python fp64-emu_amd/callers/drills.py [--small]
"""
import math
import os
import sys
import time

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import fp64_emu  # noqa: E402

F64 = torch.float64


def native_mm(X, Y):
    return torch.mm(X, Y)


def emulated_mm(X, Y):
    return fp64_emu.mm_nt(X, Y)


ENGINES = {"native": native_mm, "emu": emulated_mm}


def _cpu_randn(shape, seed):
    return torch.randn(shape, dtype=F64, generator=torch.Generator().manual_seed(seed))


def median_seconds(fn, reps=5, warm=2):
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def throughput(n, device="cuda"):
    """TFLOP/s of one n^3 product: native, default plan, reduced plan."""
    A = _cpu_randn((n, n), 10).to(device)
    B = _cpu_randn((n, n), 11).to(device)
    work = 2.0 * n ** 3 / 1e12
    out = {"n": n}
    for tag, fn in (("native", lambda: torch.mm(A, B)), ("default", lambda: fp64_emu.mm_nt(A, B)),
                    ("reduced", lambda: fp64_emu.mm_nt(A, B, nprimes=13, corr=False))):
        out[tag + "_tflops"] = work / median_seconds(fn)
    return out


def walks(n, density, squarings, device="cuda"):
    """Counts of walks of length 2^squarings between every pair of vertices
    of a random 0/1 digraph, by repeated squaring of the adjacency matrix.
    Every count stays an integer below 2^53, so an exact engine must equal
    the exact host computation bit for bit."""
    g = torch.Generator().manual_seed(7)
    adj = (torch.rand(n, n, generator=g) < density).to(torch.int64)
    # Exact counts on the host: int64 products for small graphs; for large
    # ones float64 products of integers whose every partial sum stays below
    # 2^53 (checked below), which are exact too.
    exact = adj.clone() if n <= 1024 else adj.to(F64)
    for _ in range(squarings):
        exact = exact @ exact
    exact = exact.to(torch.int64)
    if exact.max().item() >= 2 ** 53:
        raise ValueError("counts past 2^53: choose a sparser graph or fewer squarings")
    out = {"n": n, "length": 2 ** squarings, "max_count": int(exact.max().item())}
    for name, mm in ENGINES.items():
        W = adj.to(device=device, dtype=F64)
        for _ in range(squarings):
            W = mm(W, W)
        out[name + "_exact"] = bool(torch.equal(W.cpu().to(torch.int64), exact)) and \
            bool((W == W.round()).all().item())
    return out


def cholqr2(m, k, device="cuda"):
    """Two-pass CholeskyQR: R1 = chol(A^T A)^T, Q1 = A R1^-1, then the same on
    Q1.  The Gram matrix squares the condition number, so the product's
    accuracy shows in the first pass's orthogonality; the second pass repairs
    it when the first factor is good enough."""
    U, _ = torch.linalg.qr(_cpu_randn((m, k), 1).to(device))
    V, _ = torch.linalg.qr(_cpu_randn((k, k), 2).to(device))
    sigma = torch.logspace(0, -6, k, dtype=F64, device=device)
    A = (U * sigma) @ V.t()
    eye = torch.eye(k, dtype=F64, device=device)

    def orth(Q):
        return torch.linalg.matrix_norm(Q.t() @ Q - eye).item()

    out = {"m": m, "k": k}
    for name, mm in ENGINES.items():
        At = A.t().contiguous()
        R1 = torch.linalg.cholesky(mm(At, A)).t()
        Q1 = torch.linalg.solve_triangular(R1, A, upper=True, left=False)
        R2 = torch.linalg.cholesky(mm(Q1.t().contiguous(), Q1)).t()
        Q2 = torch.linalg.solve_triangular(R2, Q1, upper=True, left=False)
        R = R2 @ R1
        out[name] = {"orth_pass1": orth(Q1), "orth_pass2": orth(Q2),
                     "backward": (torch.linalg.matrix_norm(A - Q2 @ R) /
                                  torch.linalg.matrix_norm(A)).item(),
                     "gram_s": median_seconds(lambda: mm(At, A), reps=3, warm=1)}
    return out


def polar(n, max_iter=60, device="cuda"):
    """Polar factor U of A (A = U H) by the Newton-Schulz iteration
    X <- X (3 I - X^T X) / 2 from X0 = A / ||A||_F, stopped once
    ||X^T X - I||_F fails to halve (or after max_iter steps)."""
    A = _cpu_randn((n, n), 3).to(device) * torch.logspace(0, -2, n, dtype=F64, device=device)
    eye = torch.eye(n, dtype=F64, device=device)
    out = {"n": n}
    for name, mm in ENGINES.items():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        X = A / torch.linalg.matrix_norm(A)
        err = math.inf
        it = 0
        while it < max_iter:
            G = mm(X.t().contiguous(), X)
            e = torch.linalg.matrix_norm(G - eye).item()
            if e > 0.5 * err and err < 1e-6:
                break
            err = e
            X = mm(X, 1.5 * eye - 0.5 * G)
            it += 1
        torch.cuda.synchronize()
        secs = time.perf_counter() - t0
        H = X.t() @ A
        H = 0.5 * (H + H.t())
        out[name] = {"iterations": it, "orth": torch.linalg.matrix_norm(X.t() @ X - eye).item(),
                     "factor": (torch.linalg.matrix_norm(A - X @ H) /
                                torch.linalg.matrix_norm(A)).item(), "seconds": secs}
    return out


def expm_ps(A, mm, degree=16, block=4):
    """exp(A): scale by 2^-s so that ||A 2^-s||_1 <= 1/2, evaluate the
    Taylor polynomial p(X) = sum_{i<=degree} X^i / i! by Paterson-Stockmeyer
    -- p = sum_j B_j(X) (X^block)^j with B_j of degree < block, Horner in
    X^block (block - 1 + degree // block products) -- and square s times."""
    n = A.shape[0]
    eye = torch.eye(n, dtype=F64, device=A.device)
    norm1 = A.abs().sum(dim=0).max().item()
    s = max(0, math.ceil(math.log2(norm1 / 0.5))) if norm1 > 0 else 0
    X = A * (2.0 ** -s)
    pw = [eye, X]                               # X^0 .. X^block
    for _ in range(2, block + 1):
        pw.append(mm(pw[-1], X))
    coef = [1.0 / math.factorial(i) for i in range(degree + 1)]

    def part(j):                                # B_j(X)
        return sum(coef[j * block + i] * pw[i] for i in range(block) if j * block + i <= degree)

    top = degree // block
    P = part(top)
    for j in range(top - 1, -1, -1):
        P = mm(P, pw[block]) + part(j)
    for _ in range(s):
        P = mm(P, P)
    return P


def expm(n, device="cuda"):
    A = (_cpu_randn((n, n), 4) / math.sqrt(n)).to(device)
    ref = torch.matrix_exp(A)
    eye = torch.eye(n, dtype=F64, device=device)
    out = {"n": n}
    for name, mm in ENGINES.items():
        E = expm_ps(A, mm)
        Einv = expm_ps(-A, mm)
        out[name] = {"rel_vs_matrix_exp": (torch.linalg.matrix_norm(E - ref) /
                                           torch.linalg.matrix_norm(ref)).item(),
                     "inverse_check": torch.linalg.matrix_norm(E @ Einv - eye).item(),
                     "seconds": median_seconds(lambda: expm_ps(A, mm), reps=3, warm=1)}
    return out


def main():
    small = "--small" in sys.argv
    print(f"== {torch.cuda.get_device_name(0)} | torch {torch.__version__} ==", flush=True)
    r = throughput(2048 if small else 8192)
    print(f"[throughput] n={r['n']}: native {r['native_tflops']:.2f} | default "
          f"{r['default_tflops']:.2f} | reduced {r['reduced_tflops']:.2f} TFLOP/s", flush=True)
    r = walks(1024 if small else 4096, 0.02 if small else 0.005, 3)
    print(f"[walks] n={r['n']} length {r['length']} (max count {r['max_count']}): exact native "
          f"{r['native_exact']} emu {r['emu_exact']}", flush=True)
    r = cholqr2(*((8192, 256) if small else (65536, 512)))
    for name in ENGINES:
        e = r[name]
        print(f"[cholqr2] {r['m']}x{r['k']} {name:>6}: orth pass1 {e['orth_pass1']:.2e} pass2 "
              f"{e['orth_pass2']:.2e} | backward {e['backward']:.2e} | Gram {e['gram_s'] * 1e3:.1f} ms",
              flush=True)
    r = polar(512 if small else 3072)
    for name in ENGINES:
        e = r[name]
        print(f"[polar] n={r['n']} {name:>6}: {e['iterations']} iterations | orth {e['orth']:.2e} | "
              f"||A-UH||/||A|| {e['factor']:.2e} | {e['seconds']:.2f} s", flush=True)
    r = expm(512 if small else 2048)
    for name in ENGINES:
        e = r[name]
        print(f"[expm] n={r['n']} {name:>6}: rel vs matrix_exp {e['rel_vs_matrix_exp']:.2e} | "
              f"||e^A e^-A - I|| {e['inverse_check']:.2e} | {e['seconds'] * 1e3:.0f} ms", flush=True)


if __name__ == "__main__":
    main()
