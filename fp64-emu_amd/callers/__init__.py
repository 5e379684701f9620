"""Callers of the emulated GEMM: the reference's tiled Cholesky
(bench/cholesky.py) and application drills (bench/apps.py), written against
this package.  Run as scripts for timings at the reference's sizes; the
GPU tests run them at reduced sizes with accuracy bars."""
