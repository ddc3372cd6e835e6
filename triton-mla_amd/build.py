"""Build the HIP kernels of triton_mla into an in-tree shared library.

    python triton-mla_amd/build.py            # compile for gfx950
    python triton-mla_amd/build.py --stamps   # profiling build with phase stamps
                                              # (libtriton_mla_hip_stamps.so)

The library is a plain C-ABI ``.so`` (declarations in include/triton_mla.h)
that the Python package loads with ctypes. It links against the HIP runtime
by soname (libamdhip64.so.7), so inside a process that imported torch first
it binds to the runtime torch already loaded.

Each source compiles in its own process (in parallel), then the objects are
linked. Every build checks the code it ships:
  * the compiler's resource report of every kernel: no scratch (register
    spills to memory) beyond the per-kernel allowances below, LDS within the
    160 KiB of a compute unit;
  * the device assembly: no instruction reads the result registers of an
    inline-asm MFMA before the MFMA has finished (the compiler does not know
    the latency of inline asm, so it cannot insert the wait itself; this
    catches a register-allocator copy of an accumulator still in flight);
  * the host launch stubs of every kernel are defined.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
import sysconfig
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "triton_mla", "libtriton_mla_hip.so")
FAST_EXT = os.path.join(HERE, "triton_mla", "_tmla_fast" + sysconfig.get_config_var("EXT_SUFFIX"))
LIB_STAMPS = os.path.join(HERE, "triton_mla", "libtriton_mla_hip_stamps.so")
SOURCES = ["mla_decode.hip", "mla_decode_fp8.hip", "mla_decode_g16.hip", "mla_decode_generic.hip", "mla_layer.hip"]
ARCH = os.environ.get("TRITON_MLA_ARCH", "gfx950")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-mcode-object-version=5",
    # packed fp32 VALU forms are kept out of every kernel on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]
LDS_LIMIT = 160 * 1024

# Scratch bytes per lane a kernel may use (mangled-name pattern -> bytes);
# every other kernel must use none. The fp8 cache widened into the 16-bit
# ring with 64 or 128 heads per workgroup keeps one or two lane offsets of
# each segment in scratch: stored once before the segment's sub-tile loops
# and read once after them (no scratch access inside the loops).
SCRATCH_ALLOWANCE = {
    r"mla_partial_kernelILi[01]ELi512ELi64ELi2ELb1ELb1ELb1E": 8,
    r"mla_partial_kernelILi[01]ELi512ELi64ELi4ELb1ELb1ELb1E": 12,
}

# Cycles an inline-asm v_mfma_f32_32x32x16 result takes: instructions that
# read or overwrite its destination must come at least this many
# instructions (or s_nop wait states) later.
MFMA_RESULT_WINDOW = 18


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: str, obj: str, tmp: str, extra: list[str]) -> tuple[str, str]:
    """One source to an object, keeping the device assembly and the resource
    report. Returns (resource remarks, device assembly path)."""
    work = os.path.join(tmp, os.path.splitext(os.path.basename(src))[0])
    os.makedirs(work)
    cmd = [hipcc()] + FLAGS + extra + ["-c", "-save-temps", "-Rpass-analysis=kernel-resource-usage",
                                       src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True, cwd=work)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)} ({res.returncode})")
    stem = os.path.splitext(os.path.basename(src))[0]
    asm = os.path.join(work, f"{stem}-hip-amdgcn-amd-amdhsa-{ARCH}.s")
    return res.stderr, asm


def build(verbose: bool = False, stamps: bool = False) -> str:
    """Compile every HIP source into LIB (or, with stamps, the phase-stamp
    profiling build LIB_STAMPS); always recompiles. Returns the path."""
    out = LIB_STAMPS if stamps else LIB
    extra = ["-DTMLA_STAMPS=1"] if stamps else []
    with tempfile.TemporaryDirectory(prefix="tmla_build_") as tmp:
        objs = [os.path.join(tmp, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        if verbose:
            print(" ".join([hipcc()] + FLAGS + extra + ["-c", "<source>"]), flush=True)
        with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
            results = list(pool.map(lambda so: _compile(os.path.join(CSRC, so[0]), so[1], tmp, extra),
                                    zip(SOURCES, objs)))
        usage = {}
        for remarks, asm in results:
            usage.update(parse_resource_usage(remarks))
            bad = mfma_result_hazards(asm)
            if bad:
                raise RuntimeError(f"{os.path.basename(asm)}: {len(bad)} reads of an inline-asm MFMA result before "
                                   f"it is ready, first: {bad[0][0]}  ->  {bad[0][1]}")
        # the profiling build's stamp code takes registers of its own: its
        # scratch is reported, not refused
        check_resources(usage, strict=not stamps)
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out + ".tmp"] + objs
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"link failed ({res.returncode})")
    check_kernel_stubs(out + ".tmp")
    os.replace(out + ".tmp", out)
    if not stamps:
        build_fast_ext()
    if verbose:
        print(f"{len(usage)} kernels checked" + ("" if stamps else ", none beyond their scratch allowance") +
              ", no early MFMA result reads", flush=True)
    return out


def build_fast_ext() -> str:
    """The CPython module of the public call's kept-shape path (csrc/fastcall.c),
    linked against LIB in the same directory."""
    inc = sysconfig.get_paths()["include"]
    cmd = [os.environ.get("CC", "gcc"), "-O2", "-shared", "-fPIC", "-Wall", f"-I{inc}", f"-I{INCLUDE}",
           os.path.join(CSRC, "fastcall.c"), "-o", FAST_EXT + ".tmp", f"-L{os.path.dirname(LIB)}",
           "-l:" + os.path.basename(LIB), "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"fastcall.c failed ({res.returncode})")
    os.replace(FAST_EXT + ".tmp", FAST_EXT)
    return FAST_EXT


def parse_resource_usage(remarks: str) -> dict[str, dict[str, int]]:
    """Kernel name -> {"ScratchSize": bytes per lane, "LDS Size": bytes, ...}
    from the compiler's -Rpass-analysis=kernel-resource-usage remarks."""
    usage: dict[str, dict[str, int]] = {}
    cur = None
    for line in remarks.splitlines():
        m = re.match(r"remark: .+?:\d+:\d+:\s+(.*?)\s*\[-Rpass-analysis=kernel-resource-usage\]\s*$", line)
        if not m:
            continue
        body = m.group(1)
        if body.startswith("Function Name:"):
            cur = usage.setdefault(body.split(":", 1)[1].strip(), {})
            continue
        m = re.match(r"([A-Za-z][A-Za-z ]*?)(?: \[[^\]]*\])?: (\d+)$", body)
        if m and cur is not None:
            cur[m.group(1)] = int(m.group(2))
    return usage


def check_resources(usage: dict[str, dict[str, int]], strict: bool = True) -> None:
    """Fail on a kernel that spills to scratch beyond its allowance or whose
    LDS does not fit a compute unit (strict=False: report scratch only)."""
    if not usage:
        raise RuntimeError("no kernel resource report from the compiler")
    problems = []
    for name, u in usage.items():
        if "ScratchSize" not in u:
            problems.append(f"{name}: no scratch figure in the resource report")
            continue
        allow = max([b for pat, b in SCRATCH_ALLOWANCE.items() if re.search(pat, name)], default=0)
        if u["ScratchSize"] > allow:
            msg = f"{name}: {u['ScratchSize']} bytes of scratch per lane (allowed {allow})"
            if strict:
                problems.append(msg)
            else:
                print("note: " + msg, file=sys.stderr)
        if u.get("LDS Size", 0) > LDS_LIMIT:
            problems.append(f"{name}: {u['LDS Size']} bytes of LDS")
    if problems:
        raise RuntimeError("kernel resources:\n  " + "\n  ".join(problems))


def _vregs(operand: str) -> set[int]:
    regs = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]", operand):
        regs |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\bv(\d+)\b", operand):
        regs.add(int(m.group(1)))
    return regs


def mfma_result_hazards(asm_path: str, window: int = MFMA_RESULT_WINDOW) -> list[tuple[str, str]]:
    """(MFMA, reader) pairs in which an instruction touches the VGPR result of
    an MFMA fewer than ``window`` instructions (s_nop counts its wait states)
    after it. MFMAs with an AGPR result are the compiler's own (it inserts
    their waits); one MFMA accumulating into the exact result of the previous
    one is the hardware's back-to-back case and allowed. Straight-line code
    only: the window restarts at every label."""
    bad = []
    pending: list[tuple[set[int], int, str]] = []  # (result VGPRs, instructions left, MFMA)
    with open(asm_path) as f:
        for raw in f:
            t = raw.split(";")[0].strip()
            if not t or t.startswith("."):
                continue
            if t.endswith(":"):
                pending = []
                continue
            op, _, args = t.partition(" ")
            parts = [p.strip() for p in args.split(",")] if args else []
            if op.startswith("s_nop"):
                n = (int(parts[0], 0) if parts and parts[0] else 0) + 1
                pending = [(r, w - n, x) for r, w, x in pending if w - n > 0]
                continue
            if op.startswith("v_mfma") and len(parts) >= 4 and parts[0].startswith("v"):
                dst, src_c = _vregs(parts[0]), _vregs(parts[3])
                src_ab = _vregs(parts[1]) | _vregs(parts[2])
                for r, _, x in pending:
                    if (src_ab | src_c) & r and not (src_c == r and not src_ab & r):
                        bad.append((x, t))
                pending = [(r, w - 1, x) for r, w, x in pending if w - 1 > 0 and not r & dst]
                pending.append((dst, window, t))
                continue
            stores = op.startswith(("ds_write", "global_store", "buffer_store", "scratch_store"))
            touched = set()
            for p in (parts if stores else parts[1:]):
                touched |= _vregs(p)
            if parts and not stores:
                touched |= _vregs(parts[0])
            for r, _, x in pending:
                if touched & r:
                    bad.append((x, t))
            pending = [(r, w - 1, x) for r, w, x in pending if w - 1 > 0]
    return bad


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
