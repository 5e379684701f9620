"""Application drills (the reference's bench/apps.py:49-173): each algorithm
runs with native float64 GEMMs and with the emulated default, reporting time
and an application-level accuracy metric.

    python fp64-emu_amd/callers/apps.py [--small]
"""
import math
import os
import sys
import time

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import fp64_emu as emu  # noqa: E402

DEV = "cuda"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def timeit(fn, reps=5, warm=2):
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def g_native(A, B):
    return A @ B


def g_emu(A, B):
    return emu.mm_nt(A, B)


def drill_throughput(n=8192):
    """Raw throughput at the default and reduced operating points
    (apps.py:49-63)."""
    A = torch.randn(n, n, dtype=torch.float64, generator=_gen(10)).to(DEV)
    B = torch.randn(n, n, dtype=torch.float64, generator=_gen(11)).to(DEV)
    tn = timeit(lambda: A @ B)
    te = timeit(lambda: emu.mm_nt(A, B))
    tr = timeit(lambda: emu.mm_nt(A, B, nprimes=13, corr=False))
    ref = A @ B
    d = (emu.mm_nt(A, B) - ref).abs().max().item() / ref.abs().max().item()
    fl = 2.0 * n ** 3
    return {"n": n, "native_tf": fl / tn / 1e12, "default_tf": fl / te / 1e12,
            "reduced_tf": fl / tr / 1e12, "emu_native_rel": d}


def drill_paths(n=4096):
    """4-step path counts of a random 0/1 digraph: exact integers below 2^53,
    so the emulated product must equal the native one bit for bit
    (apps.py:66-88)."""
    A = (torch.rand(n, n, generator=_gen(7)) < 0.05).double().to(DEV)

    def paths4(g):
        A2 = g(A, A)
        return g(A2, A2)

    P4n = paths4(g_native)
    P4e = paths4(g_emu)
    tn = timeit(lambda: paths4(g_native), reps=3)
    te = timeit(lambda: paths4(g_emu), reps=3)
    return {"n": n, "max_count": P4n.max().item(), "bitwise_equal": bool(torch.equal(P4n, P4e)),
            "native_ms": tn * 1e3, "emu_ms": te * 1e3}


def drill_cholqr(m=65536, k=512):
    """CholeskyQR of a cond ~1e6 tall-skinny matrix: the Gram matrix squares
    the condition number, so GEMM accuracy shows in ||Q^T Q - I||
    (apps.py:91-118)."""
    Q1, _ = torch.linalg.qr(torch.randn(m, k, dtype=torch.float64, generator=_gen(1)).to(DEV))
    Q2, _ = torch.linalg.qr(torch.randn(k, k, dtype=torch.float64, generator=_gen(2)).to(DEV))
    s = torch.logspace(0, -6, k, dtype=torch.float64, device=DEV)
    A = (Q1 * s) @ Q2.t()
    At = A.t().contiguous()
    I = torch.eye(k, dtype=torch.float64, device=DEV)

    def qr_resid(G):
        L = torch.linalg.cholesky(G)
        Q = torch.linalg.solve_triangular(L, At, upper=False).t()
        return (Q.t() @ Q - I).norm().item()

    tn = timeit(lambda: At @ A)
    te = timeit(lambda: emu.mm_nt(At, A))
    return {"m": m, "k": k, "resid_native": qr_resid(At @ A),
            "resid_emu": qr_resid(emu.mm_nt(At, A)), "native_ms": tn * 1e3, "emu_ms": te * 1e3}


def drill_polar(n=3072, iters=50):
    """Newton-Schulz polar factor X <- 1.5 X - 0.5 X (X^T X), pure GEMMs;
    metric: the orthogonality floor (apps.py:121-145)."""
    A = torch.randn(n, n, dtype=torch.float64, generator=_gen(3)).to(DEV)
    A = A * torch.logspace(0, -2, n, dtype=torch.float64, device=DEV)
    I = torch.eye(n, dtype=torch.float64, device=DEV)
    out = {"n": n, "iters": iters}
    for tag, g in (("native", g_native), ("emu", g_emu)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        X = A / A.norm()
        for _ in range(iters):
            Y = g(X.t().contiguous(), X)
            X = 1.5 * X - 0.5 * g(X, Y)
        torch.cuda.synchronize()
        out[f"{tag}_s"] = time.perf_counter() - t0
        out[f"resid_{tag}"] = (X.t() @ X - I).norm().item()
    return out


def drill_expm(n=2048, s=6, terms=18):
    """exp(A) by Taylor + repeated squaring through the engine under test,
    against torch.matrix_exp (apps.py:148-173)."""
    A = (torch.randn(n, n, dtype=torch.float64, generator=_gen(4)) / math.sqrt(n)).to(DEV)
    I = torch.eye(n, dtype=torch.float64, device=DEV)
    ref = torch.matrix_exp(A)

    def expm(g):
        As = A * (2.0 ** -s)
        E = I + As
        T = As
        for k in range(2, terms):
            T = g(T, As) / k
            E = E + T
        for _ in range(s):
            E = g(E, E)
        return E

    out = {"n": n}
    for tag, g in (("native", g_native), ("emu", g_emu)):
        out[f"{tag}_ms"] = timeit(lambda: expm(g), reps=3, warm=1) * 1e3
        out[f"err_{tag}"] = ((expm(g) - ref).norm() / ref.norm()).item()
    return out


def main():
    small = "--small" in sys.argv
    print(f"== {torch.cuda.get_device_name(0)} | torch {torch.__version__} ==", flush=True)
    r = drill_throughput(2048 if small else 8192)
    print(f"[throughput] n={r['n']}: native {r['native_tf']:.2f} TF | default {r['default_tf']:.2f} TF "
          f"({r['default_tf'] / r['native_tf']:.2f}x) | reduced {r['reduced_tf']:.2f} TF | "
          f"emu-native rel {r['emu_native_rel']:.1e}", flush=True)
    r = drill_paths(1024 if small else 4096)
    print(f"[paths] n={r['n']} A^4 (max count {r['max_count']:.2e}): bitwise equal "
          f"{r['bitwise_equal']} | native {r['native_ms']:.0f} ms, emu {r['emu_ms']:.0f} ms", flush=True)
    r = drill_cholqr(*((8192, 256) if small else (65536, 512)))
    print(f"[cholqr] {r['m']}x{r['k']}, cond ~1e6: ||Q^T Q - I|| native {r['resid_native']:.2e} vs emu "
          f"{r['resid_emu']:.2e} | Gram {r['native_ms']:.1f} ms vs {r['emu_ms']:.1f} ms", flush=True)
    r = drill_polar(512 if small else 3072, 30 if small else 50)
    print(f"[polar] n={r['n']}, {r['iters']} iters: ||X^T X - I|| native {r['resid_native']:.2e} "
          f"({r['native_s']:.2f} s) vs emu {r['resid_emu']:.2e} ({r['emu_s']:.2f} s)", flush=True)
    r = drill_expm(512 if small else 2048)
    print(f"[expm] n={r['n']}: rel vs matrix_exp native {r['err_native']:.2e} ({r['native_ms']:.0f} ms) "
          f"vs emu {r['err_emu']:.2e} ({r['emu_ms']:.0f} ms)", flush=True)
    print("done.", flush=True)


if __name__ == "__main__":
    main()
