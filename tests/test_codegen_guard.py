"""Instruction-level guards over the built gfx950 code (no GPU needed): the
library's own code objects are taken out of libglypr_hip.so's .hip_fatbin
section and disassembled with the ROCm LLVM tools.

- No mixed-precision FMA (`v_fma_mix*` / `v_mad_mix*`).  Every f16 operand
  of the attention path is the f32 value rounded once more (the f32 product
  or sum first, then f16), the two roundings the oracle and qkv_post make;
  the compiler folds `(_Float16)(a * b)` into one `v_fma_mixlo_f16`, a single
  rounding, unless the f32 product is pinned, and that moved about one f16
  value in 10^4 by one ulp in the fused q|k|v kernel.
- No packed-f32 arithmetic (`v_pk_fma_f32`, `v_pk_mul_f32`, `v_pk_add_f32`):
  the build disables the feature, since some forms of these instructions
  have returned wrong results on the target machines.
"""
import os
import re
import shutil
import subprocess

import pytest

from glypr_amd import _lib

LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
FORBIDDEN = re.compile(r"\b(v_fma_mix\w*|v_mad_mix\w*|v_pk_fma_f32|v_pk_mul_f32|v_pk_add_f32)\b")


def _tool(name):
    path = os.path.join(LLVM, name)
    return path if os.access(path, os.X_OK) else shutil.which(name)


@pytest.fixture(scope="module")
def disassembly(tmp_path_factory):
    tools = [_tool(n) for n in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")]
    if not os.path.exists(_lib.LIB_PATH) or not all(tools):
        pytest.skip("libglypr_hip.so not built or ROCm LLVM tools missing")
    objcopy, bundler, objdump = tools
    d = tmp_path_factory.mktemp("codeobj")
    fat = d / "fat.bin"
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", _lib.LIB_PATH, str(d / "x.so")],
                   check=True, capture_output=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundle in .hip_fatbin"
    text = []
    for i, s in enumerate(starts):   # one bundle per translation unit
        part = d / f"b{i}.bin"
        part.write_bytes(data[s:starts[i + 1] if i + 1 < len(starts) else len(data)])
        co = d / f"b{i}.co"
        subprocess.run([bundler, "--type=o", "--unbundle", f"--input={part}",
                        f"--targets={TARGET}", f"--output={co}"], check=True, capture_output=True)
        out = subprocess.run([objdump, "-d", "--mcpu=gfx950", str(co)], check=True,
                             capture_output=True, text=True).stdout
        text.append(out)
    return "\n".join(text)


def test_code_objects_found(disassembly):
    # the kernels of every translation unit are there
    for k in ("gemm_i8_qkv_big_kernel", "gemm_i8_qkv_kernel", "attn_partial_kernel",
              "qkv_post_kernel", "residual_norm_kernel", "gather_rows_kernel",
              "gemm_bf16_big_kernel"):
        assert k in disassembly, k


def test_no_mixed_precision_or_packed_f32(disassembly):
    hits = sorted(set(m.group(1) for m in FORBIDDEN.finditer(disassembly)))
    assert not hits, hits
