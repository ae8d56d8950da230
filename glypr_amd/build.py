"""Build libglypr_hip.so in-tree with hipcc for gfx950 (MI355X).

    python -m glypr_amd.build          # compile every source, link the library

Each .hip/.cpp source under csrc/ is compiled to an object in parallel and
linked into glypr_amd/libglypr_hip.so, which travels with the source tree;
glypr_amd/capi_bench (capi_bench.cpp, the C3 projections through the C ABI
alone) is linked against it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libglypr_hip.so")
BENCH_BIN = os.path.join(PKG, "capi_bench")
ARCH = os.environ.get("GLYPR_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# -ffp-contract=off: no implicit FMA (the reference's Rust never contracts);
# explicit fmaf is used where the reference fuses.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32.
# -amdgpu-mfma-vgpr-form: MFMA results land in VGPRs, so the Q8_0 scale
# epilogue reads them without v_accvgpr_read copies.
# -amdgpu-kernarg-preload-count=16: the leading kernel arguments (14 dwords
# on gfx950) arrive preloaded in SGPRs, so a kernel's first loads do not wait
# for a round trip to the kernel-argument buffer (~0.2-0.3 us of every launch
# at C4); the kernels keep what their first DMAs need in those dwords.
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def sources():
    out = []
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".cpp")):
            out.append(os.path.join(CSRC, name))
    return out


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, "-x", "hip", *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in r.stdout.splitlines() if noise not in l and "hip-link" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    if msg.strip():
        print(msg, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    """Compile every source and link the library; always rebuilds."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    # the C-ABI benchmark driver (no Python): links the library just built
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", f"-I{INCLUDE}",
           os.path.join(PKG, "capi_bench.cpp"), f"-L{PKG}", "-lglypr_hip",
           "-Wl,-rpath,$ORIGIN", "-o", BENCH_BIN + ".tmp"]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"capi_bench build failed:\n{r.stdout}")
    os.replace(BENCH_BIN + ".tmp", BENCH_BIN)
    return LIB


if __name__ == "__main__":
    build()
