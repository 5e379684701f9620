"""Callers of the emulated GEMM written against this package: a left-looking
blocked Cholesky whose updates are batched products (blocked_cholesky.py) and
application drills (drills.py).  Run as scripts for timings at full size; the
GPU tests run them at reduced sizes with accuracy bars."""
