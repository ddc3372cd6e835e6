"""Build the HIP kernels of triton_mla into an in-tree shared library.

    python triton-mla_amd/build.py            # compile for gfx950

The library is a plain C-ABI ``.so`` (declarations in include/triton_mla.h)
that the Python package loads with ctypes. It links against the HIP runtime
by soname (libamdhip64.so.7), so inside a process that imported torch first
it binds to the runtime torch already loaded.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "triton_mla", "libtriton_mla_hip.so")
SOURCES = ["mla_decode.hip"]
ARCH = os.environ.get("TRITON_MLA_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False) -> str:
    """Compile every HIP source into LIB; always recompiles. Returns the path."""
    cmd = [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        "-mcode-object-version=5",
        # packed fp32 VALU forms are kept out of every kernel on this target
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}", "-o", LIB + ".tmp",
    ] + [os.path.join(CSRC, s) for s in SOURCES]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode})")
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
