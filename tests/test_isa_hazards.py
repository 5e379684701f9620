"""CPU tier: the MFMA hazard discipline of the compiled library.

The modular GEMM issues its v_mfma_i32_16x16x64_i8 as inline assembly, so
the compiler's hazard recognizer does not see them; the kernels place the
wait states themselves (mfma_fence: 32 wait states before any other
instruction reads an accumulator; the first k-step's MFMAs take the constant
0 as accumulator input, so no VALU write ever feeds an MFMA; consecutive
MFMAs never accumulate into the same registers).  This test disassembles the
gfx950 code object built into libfp64emu.so (this repository's own build)
and checks, in program order within every kernel:

  1. every v_accvgpr_read of an accumulator comes at least 32 wait states
     after the last MFMA that wrote it (s_nop n counts n + 1);
  2. an MFMA that accumulates into registers another MFMA wrote comes at
     least 8 instructions after it (the tiles' accumulator grids put 16 to 64
     MFMAs between them);
  3. no MFMA reads as accumulator input registers that a VALU instruction
     (v_accvgpr_write / v_accvgpr_mov) wrote less than 8 instructions before.

The GPU parity tier verifies the results; this check catches a reordering
that breaks the discipline before any GPU run.  Loop back-edges are not
followed: every loop body holds two unrolled k-steps, so the step-to-step
distances appear in straight-line code.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "fp64-emu_amd", "fp64_emu", "libfp64emu.so")
LLVM = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin")

FENCE = 32
MIN_CHAIN = 8
MIN_VALU_TO_MFMA = 8


def _disassemble(tmp_path):
    tools = {t: os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")}
    missing = [t for t, p in tools.items() if not os.path.exists(p)]
    if missing or not os.path.exists(LIB):
        pytest.skip(f"needs the built library and ROCm's LLVM tools (missing: {missing or LIB})")
    fat = tmp_path / "fatbin.bin"
    co = tmp_path / "gfx950.co"
    subprocess.run([tools["llvm-objcopy"], f"--dump-section=.hip_fatbin={fat}", LIB,
                    str(tmp_path / "stripped.so")], check=True, capture_output=True)
    subprocess.run([tools["clang-offload-bundler"], "--unbundle", "--type=o", f"--input={fat}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"],
                   check=True, capture_output=True)
    out = subprocess.run([tools["llvm-objdump"], "-d", "--mcpu=gfx950", str(co)], check=True,
                         capture_output=True, text=True).stdout
    funcs, cur = {}, None
    for line in out.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if m:
            cur = m.group(1)
            funcs[cur] = []
        elif cur and line.startswith("\t"):
            ins = line.split("//")[0].strip()
            if ins:
                funcs[cur].append(ins)
    return funcs


def _aregs(op):
    """AGPR numbers of an operand such as a[252:255] or a7 (empty otherwise)."""
    m = re.fullmatch(r"a\[(\d+):(\d+)\]", op)
    if m:
        return range(int(m.group(1)), int(m.group(2)) + 1)
    m = re.fullmatch(r"a(\d+)", op)
    return range(int(m.group(1)), int(m.group(1)) + 1) if m else range(0)


def _check(ins):
    """Violations of the three rules in one kernel's instruction list."""
    bad = []
    ws = 0                       # wait states issued so far
    n = 0                        # instructions issued so far
    mfma_ws, mfma_n, valu_n = {}, {}, {}
    for text in ins:
        op, _, rest = text.partition(" ")
        args = [a.strip() for a in rest.split(",")] if rest else []
        if op.startswith("v_mfma"):
            dst, srcc = _aregs(args[0]), _aregs(args[3]) if len(args) > 3 else range(0)
            for r in srcc:
                if r in mfma_n and n - mfma_n[r] < MIN_CHAIN:
                    bad.append(f"MFMA chain on a{r} {n - mfma_n[r]} instructions apart: {text}")
                if r in valu_n and n - valu_n[r] < MIN_VALU_TO_MFMA:
                    bad.append(f"VALU write of a{r} {n - valu_n[r]} instructions before MFMA: {text}")
            for r in dst:
                mfma_ws[r], mfma_n[r] = ws, n
        elif op == "v_accvgpr_read_b32":
            for r in _aregs(args[1]):
                if r in mfma_ws and ws - mfma_ws[r] < FENCE:
                    bad.append(f"read of a{r} {ws - mfma_ws[r]} wait states after its MFMA: {text}")
        elif op in ("v_accvgpr_write_b32", "v_accvgpr_mov_b32"):
            for r in _aregs(args[0]):
                valu_n[r] = n
        ws += int(args[0]) + 1 if op == "s_nop" else 1
        n += 1
    return bad


def test_checker_catches_planted_violations():
    """The rules fire on short hand-written sequences (the checker itself)."""
    fence = ["s_nop 7"] * 4
    mf = "v_mfma_i32_16x16x64_i8 a[0:3], v[0:3], v[4:7], a[0:3]"
    mf0 = "v_mfma_i32_16x16x64_i8 a[0:3], v[0:3], v[4:7], 0"
    rd = "v_accvgpr_read_b32 v8, a2"
    assert not _check([mf0, *fence, rd])
    assert _check([mf0, "s_nop 7", rd])                       # fence too short
    assert _check([mf0, mf])                                  # back-to-back accumulation
    assert not _check([mf0, *["v_add_u32 v9, v9, v9"] * 8, mf])
    assert _check(["v_accvgpr_write_b32 a1, 0", mf])          # VALU write feeding srcC
    assert not _check(["v_accvgpr_write_b32 a1, 0", mf0])     # constant-0 input reads nothing


def test_compiled_kernels_keep_the_mfma_discipline(tmp_path):
    funcs = _disassemble(tmp_path)
    gemm = {f: i for f, i in funcs.items() if any(x.startswith("v_mfma") for x in i)}
    assert len(gemm) >= 6, sorted(funcs)[:10]     # every GEMM form and the probes
    bad = {f: _check(i) for f, i in gemm.items()}
    bad = {f: v for f, v in bad.items() if v}
    assert not bad, {f: v[:3] for f, v in bad.items()}
