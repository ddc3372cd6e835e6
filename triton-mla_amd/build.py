"""Build the HIP kernels of triton_mla into an in-tree shared library.

    python triton-mla_amd/build.py            # compile for gfx950
    python triton-mla_amd/build.py --stamps   # profiling build with phase stamps
                                              # (libtriton_mla_hip_stamps.so)

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
LIB_STAMPS = os.path.join(HERE, "triton_mla", "libtriton_mla_hip_stamps.so")
SOURCES = ["mla_decode.hip", "mla_decode_fp8.hip", "mla_layer.hip"]
ARCH = os.environ.get("TRITON_MLA_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False, stamps: bool = False) -> str:
    """Compile every HIP source into LIB (or, with stamps, the phase-stamp
    profiling build LIB_STAMPS); always recompiles. Returns the path."""
    out = LIB_STAMPS if stamps else LIB
    cmd = [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        "-mcode-object-version=5",
        # packed fp32 VALU forms are kept out of every kernel on this target
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}", "-o", out + ".tmp",
    ] + (["-DTMLA_STAMPS=1"] if stamps else []) + [os.path.join(CSRC, s) for s in SOURCES]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode})")
    check_kernel_stubs(out + ".tmp")
    os.replace(out + ".tmp", out)
    return out


def check_kernel_stubs(path: str) -> None:
    """Fail when a kernel's host launch stub is undefined in the library.

    If the host pass of the compiler rejects something in a kernel body (for
    example a GPU register constraint written directly in it), it drops the
    kernel silently and leaves its launch stub undefined; the library then
    fails only when it is loaded.
    """
    nm = shutil.which("nm")
    if nm is None:
        return
    res = subprocess.run([nm, "-D", "--undefined-only", path], capture_output=True, text=True)
    missing = [line.split()[-1] for line in res.stdout.splitlines() if "__device_stub__" in line]
    if missing:
        raise RuntimeError("kernels dropped by the host compiler pass: " + ", ".join(missing))


if __name__ == "__main__":
    print(build(verbose=True, stamps="--stamps" in sys.argv[1:]))
