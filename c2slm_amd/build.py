"""Build recipe for libc2h.so (gfx950) — the C-ABI library in include/c2h.h.

hipcc cross-compiles here without a GPU.  Flags that matter for parity:
  -ffp-contract=off   every a*b+c is two roundings unless written as fma,
                      as in the reference's GOAMD64=v1 Go build;
  no fast-math        IEEE division and square root (HIP's default
                      correctly rounded f32 div/sqrt is kept).
`-Xclang -target-feature -Xclang -packed-fp32-ops` keeps the compiler from
forming packed FP32 instructions (the host pass warns it does not know the
feature; that is harmless).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libc2h.so")
ARCH = os.environ.get("C2H_OFFLOAD_ARCH", "gfx950")

SOURCES = ["c2h_kernels.hip", "c2h_api.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


# Kernel-argument preload (gfx950): the leading scalar and pointer
# arguments of a kernel (up to seven) arrive in SGPRs at wave start
# (k_gemv_row: x and n_x; k_attn_core: the state, cache and q/k/v pointers
# and two packed integers), so the first loads do not wait for a read of the
# kernel arguments from memory.  The code object starts with a block that
# loads them the usual way, for firmware without the feature; the firmware
# that has it enters past that block.
PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=7"]


def build(verbose: bool = False) -> str:
    flags = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *PRELOAD,
             "-Wall", "-Wno-unused-function", "-I", os.path.join(HERE, "..", "include")]
    objs = []
    bdir = os.path.join(HERE, "_build")
    os.makedirs(bdir, exist_ok=True)
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        obj = os.path.join(bdir, src + ".o")
        cmd = [hipcc(), *flags, "-c", path, "-o", obj]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"hipcc failed on {src}")
        if verbose:
            sys.stderr.write(res.stderr)
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
