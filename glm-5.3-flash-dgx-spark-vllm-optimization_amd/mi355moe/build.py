"""Build libmi355moe.so in-tree with hipcc for gfx950.

    python -m mi355moe.build        (from the package's parent directory)

Flags: -O3, no FMA contraction (epilogues round exactly as written), and no packed-fp32 instructions
(``-Xclang -target-feature -Xclang -packed-fp32-ops``): hipcc is asked never to emit v_pk_*_f32. A larger budget for
promoting private arrays to registers (``-mllvm -amdgpu-promote-alloca-to-vector-limit=2048``) keeps the GEMM loops'
per-lane arrays out of scratch.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG_ROOT = os.path.dirname(_HERE)
CSRC = os.path.join(_PKG_ROOT, "csrc")
INCLUDE = os.path.join(os.path.dirname(_PKG_ROOT), "include")
SOURCES = ["abi.hip", "route.hip", "decode.hip", "prefill.hip", "fp8.hip"]
OUT = os.path.join(_HERE, "libmi355moe.so")
ARCH = "gfx950"

FLAGS = ["-O3", f"--offload-arch={ARCH}", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # private arrays of the GEMM loops (decoded weight pairs, B operands) kept in registers: without it the
         # default promotion budget leaves some of them in scratch in the larger kernels (the 128- and 64-row tile
         # kernels, the one-launch schedule)
         "-mllvm", "-amdgpu-promote-alloca-to-vector-limit=2048"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def sources() -> list[str]:
    return [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]


def build(verbose: bool = False) -> str:
    """Compile every HIP source into libmi355moe.so (always recompiles). Returns the library path."""
    tmp = OUT + ".tmp"
    cmd = [hipcc(), *FLAGS, f"-I{INCLUDE}", "-o", tmp, *sources()]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode})")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
