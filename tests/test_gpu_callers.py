"""GPU tier: the reference's callers of the emulated GEMM (bench/cholesky.py,
bench/apps.py) at reduced sizes, with application-level accuracy bars:
exact path counts bitwise equal to native; Cholesky residual at the fp64
level (the reference reports 3-4e-16); CholeskyQR, polar and expm no worse
than native float64 beyond a small factor."""
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "fp64-emu_amd"))
from callers import apps, cholesky  # noqa: E402

pytestmark = pytest.mark.gpu


def test_tiled_cholesky_bmm(dev):
    print("case tiled cholesky n=2048 t=256", flush=True)
    A = cholesky.spd_matrix(2048, seed=0, device=dev)
    res = {}
    for name, eng in cholesky.engines().items():
        L, _ = cholesky.factor(A, 256, eng)
        res[name] = cholesky.residual(A, L)
    print(res, flush=True)
    assert res["emu"] < 1e-15 and res["emu"] <= 2.0 * res["native"]


def test_paths_exact(dev):
    print("case paths n=1024", flush=True)
    r = apps.drill_paths(1024)
    assert r["bitwise_equal"] and r["max_count"] > 1


def test_cholqr(dev):
    print("case cholqr 8192x256", flush=True)
    r = apps.drill_cholqr(8192, 256)
    print(r, flush=True)
    assert r["resid_emu"] <= 1.5 * r["resid_native"]


def test_polar(dev):
    print("case polar n=512", flush=True)
    r = apps.drill_polar(512, 30)
    print(r, flush=True)
    assert r["resid_emu"] <= 2.0 * r["resid_native"] + 1e-14


def test_expm(dev):
    print("case expm n=512", flush=True)
    r = apps.drill_expm(512)
    print(r, flush=True)
    assert r["err_emu"] <= 2.0 * r["err_native"] + 1e-15
