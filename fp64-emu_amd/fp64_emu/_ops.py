"""Loads the in-tree HIP extension and exposes its op namespace as `ops`.

The role of the reference's generated `_ops.py` (torch-ext/fp64_emu/__init__.py:15):
`ops.fp64_emu_mm(...)` etc. resolve to torch.ops.fp64_emu.*.  There is no
fallback: a missing or unloadable extension raises ImportError.
"""
import os

import torch  # must be imported first: the extension binds to torch's HIP runtime

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_fp64emu_torch.so")
CAPI_PATH = os.path.join(_HERE, "libfp64emu.so")

if not os.path.exists(LIB_PATH) or not os.path.exists(CAPI_PATH):
    raise ImportError(
        "fp64_emu: the HIP extension is not built (expected "
        f"{LIB_PATH}); run `python fp64-emu_amd/build.py` or __graft_entry__.build()")

torch.ops.load_library(LIB_PATH)
ops = torch.ops.fp64_emu
