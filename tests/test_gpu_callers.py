"""GPU tier: the callers of the emulated GEMM (fp64-emu_amd/callers/) at
reduced sizes, with application-level bars:
- left-looking blocked Cholesky through bmm: factorization residual and solve
  backward error at the float64 level (the reference reports residuals of
  3-4e-16 for its tiled Cholesky, README.md:315-320), no worse than native;
- walk counts: exact integers, equal to the host's exact counts bit for bit;
- two-pass CholeskyQR, Newton-Schulz polar factor and the Paterson-Stockmeyer
  exponential: no worse than native float64 beyond a small factor."""
import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "fp64-emu_amd"))
from callers import blocked_cholesky, drills  # noqa: E402

pytestmark = pytest.mark.gpu


def test_left_looking_cholesky_bmm(dev):
    print("case left-looking cholesky n=2048 t=256", flush=True)
    A = blocked_cholesky.spd_test_matrix(2048, 0, dev)
    res = {}
    for name, eng in blocked_cholesky.ENGINES.items():
        L, _ = blocked_cholesky.left_looking(A, 256, eng)
        res[name] = (blocked_cholesky.factor_residual(A, L),
                     blocked_cholesky.solve_backward_error(A, L))
    print(res, flush=True)
    assert res["emu"][0] < 1e-15 and res["emu"][0] <= 2.0 * res["native"][0]
    assert res["emu"][1] < 1e-15 and res["emu"][1] <= 2.0 * res["native"][1] + 1e-17


def test_walk_counts_exact(dev):
    print("case walks n=1024 length 8", flush=True)
    r = drills.walks(1024, 0.02, 3, device=dev)
    print(r, flush=True)
    assert r["max_count"] > 2 ** 20 and r["emu_exact"] and r["native_exact"]


def test_cholqr2(dev):
    print("case cholqr2 8192x256", flush=True)
    r = drills.cholqr2(8192, 256, device=dev)
    print(r, flush=True)
    assert r["emu"]["orth_pass1"] <= 1.5 * r["native"]["orth_pass1"]
    assert r["emu"]["orth_pass2"] < 1e-13 and r["emu"]["backward"] < 1e-14


def test_polar(dev):
    print("case polar n=512", flush=True)
    r = drills.polar(512, device=dev)
    print(r, flush=True)
    assert r["emu"]["orth"] <= 2.0 * r["native"]["orth"] + 1e-14
    assert r["emu"]["factor"] <= 2.0 * r["native"]["factor"] + 1e-14


def test_expm(dev):
    print("case expm n=512", flush=True)
    r = drills.expm(512, device=dev)
    print(r, flush=True)
    assert r["emu"]["rel_vs_matrix_exp"] <= 2.0 * r["native"]["rel_vs_matrix_exp"] + 1e-15
    assert r["emu"]["inverse_check"] <= 2.0 * r["native"]["inverse_check"] + 1e-13
