"""Checks on the gfx950 machine code of the built library (CPU only: the code
object is unbundled from libvoxtral_amd.so and disassembled with ROCm's
LLVM tools).

- No packed-FP32 arithmetic: the library is built with the packed-fp32-ops
  target feature switched off, and those instructions must not appear.
- No packed f32 -> f16 conversion whose two sources are one register.  This
  compiler has been seen to emit v_cvt_pk_f16_f32 with its second source
  replaced by the first (a vector {x[i], x[i+1]} converted as {x[i], x[i]}).
  The kernels never mean to convert one value into both halves, so such an
  instruction is taken for that miscompile.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "webgpu-voxtral_amd", "lib", "libvoxtral_amd.so")
LLVM = "/opt/rocm/llvm/bin"


@pytest.fixture(scope="module")
def disasm(tmp_path_factory):
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    for tool in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"):
        if not os.path.exists(os.path.join(LLVM, tool)):
            pytest.skip(f"{tool} not installed")
    d = tmp_path_factory.mktemp("codeobj")
    fat, co = str(d / "fat.bin"), str(d / "gfx950.co")
    subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", LIB, str(d / "lib.so")],
                   check=True)
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fat}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True)
    out = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", co], check=True,
                         capture_output=True, text=True).stdout
    assert "v_fma_f32" in out or "v_fmac_f32" in out  # it is the device code
    return out


def _kernel_of(text, pos):
    k = text.rfind(">:\n", 0, pos)
    return text[text.rfind("<", 0, k) + 1:k] if k >= 0 else "?"


def test_no_packed_fp32_arithmetic(disasm):
    hits = [(m.group(0), _kernel_of(disasm, m.start()))
            for m in re.finditer(r"\bv_pk_(add|mul|fma)_f32\b", disasm)]
    assert not hits, hits[:10]


def test_packed_f16_conversions_have_two_sources(disasm):
    pk = list(re.finditer(r"\bv_cvt_pk_f16_f32\s+(v\d+),\s*(v\d+),\s*(v\d+)", disasm))
    assert pk, "no packed f16 conversions found"
    same = [(m.group(0), _kernel_of(disasm, m.start())) for m in pk if m.group(2) == m.group(3)]
    assert not same, same[:10]
