"""Build recipe for the MI355X fp64-emu extension (in-tree, gfx950).

Produces, next to the Python package in fp64-emu_amd/fp64_emu/:
  libfp64emu.so       HIP kernels + the C ABI of include/fp64emu.h (hipcc)
  _fp64emu_torch.so   torch op registration over the C ABI (g++, links the above)
The test-only CPU oracle (oracle/liboracle_fp64emu.so) is built by
`build_oracle()`, which the package itself never calls.

Usage: python fp64-emu_amd/build.py [--oracle]
"""
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(HERE, "fp64_emu")
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
ORACLE = os.path.join(ROOT, "oracle")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

CAPI_SO = os.path.join(PKG, "libfp64emu.so")
TORCH_SO = os.path.join(PKG, "_fp64emu_torch.so")
ORACLE_SO = os.path.join(ORACLE, "liboracle_fp64emu.so")

# gfx950 only.  Packed-FP32 instructions are kept out of every HIP build;
# fp contraction is off so the fp64 steps are exactly the written ones
# (explicit fma() where an FMA is meant).
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd, cwd=None):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True, cwd=cwd)


def build_capi():
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    src = os.path.join(CSRC, "fp64emu.hip")
    tmp = CAPI_SO + ".tmp"
    _run([hipcc, *HIP_FLAGS, "-shared", f"-I{INCLUDE}", src, "-o", tmp])
    os.replace(tmp, CAPI_SO)
    return CAPI_SO


def build_torch_ext():
    import torch  # noqa: F401  (paths and ABI of the installed torch)
    from torch.utils import cpp_extension

    tdir = os.path.dirname(torch.__file__)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [*cpp_extension.include_paths(), os.path.join(ROCM, "include"), INCLUDE,
           sysconfig.get_paths()["include"]]
    src = os.path.join(CSRC, "torch_binding.cpp")
    tmp = TORCH_SO + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1",
           "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=fp64_emu",
           *[f"-I{p}" for p in inc], src, "-o", tmp,
           f"-L{os.path.join(tdir, 'lib')}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_hip", f"-L{PKG}", "-lfp64emu", "-Wl,-rpath,$ORIGIN",
           f"-Wl,-rpath,{os.path.join(tdir, 'lib')}"]
    _run(cmd)
    os.replace(tmp, TORCH_SO)
    return TORCH_SO


def build_oracle():
    _run(["make", "-s", "-C", ORACLE])
    return ORACLE_SO


def build_all(oracle=True):
    build_capi()
    build_torch_ext()
    if oracle:
        build_oracle()


if __name__ == "__main__":
    build_all(oracle="--no-oracle" not in sys.argv)
