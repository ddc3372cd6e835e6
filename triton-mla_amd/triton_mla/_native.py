"""ctypes binding of the C ABI in include/triton_mla.h (libtriton_mla_hip.so).

The library is loaded after torch so that its HIP runtime dependency
(soname libamdhip64.so.7) resolves to the runtime torch already mapped. There
is no fallback: if the library is missing or fails to load, every entry point
that needs it raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

# TRITON_MLA_LIB selects another build of the library (e.g. the phase-stamp
# profiling build, libtriton_mla_hip_stamps.so)
LIB_PATH = os.environ.get("TRITON_MLA_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                            "libtriton_mla_hip.so")

# name -> (restype, argtypes); mirrors include/triton_mla.h
_i32, _i64, _f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
_vp, _sz = ctypes.c_void_p, ctypes.c_size_t
SIGNATURES = {
    "tmla_last_error": (ctypes.c_char_p, []),
    "tmla_version": (ctypes.c_int, []),
    "tmla_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "tmla_device_cu_count": (_i32, [_i32]),
    "tmla_debug_stamps": (ctypes.c_int, [_vp, _sz]),
    "tmla_workspace_zero_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "tmla_partition_segment_tiles": (_i32, []),
    "tmla_mla_norm_append": (ctypes.c_int, [
        _vp, _i64, _vp, _f32, _i32, _vp, _i64, _vp, _i64, _vp, _f32, _f32, _vp, _vp, _i32, _i32, _i32, _i32, _vp,
        _i64, _i64, _i64, _i32, _vp, _i64, _i32, _vp]),
    "tmla_mla_decode_fused_is_single": (_i32, [_i32, _i32, _i32, _i32, _i32, _i64, _i32]),
    "tmla_mla_decode_partial": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _i32, _vp, _i32, _i32, _i32,
        _i32, _i32, _f32, _i32, _i32, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "tmla_mla_decode_combine": (ctypes.c_int, [
        _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "tmla_mla_decode": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _i32, _vp, _i32, _i32, _i32,
        _i32, _i32, _f32, _i32, _i32, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "tmla_mla_decode_fused": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _i32, _vp, _i32, _i32, _i32,
        _i32, _i32, _f32, _i32, _i32, _vp, _i64, _i64, _vp, _vp, _sz, _i32, _vp]),
    "tmla_mla_decode_noalloc": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _i32, _vp, _i32, _i32, _i32,
        _i32, _i32, _f32, _i32, _i32, _vp, _i64, _i64, _vp, _vp]),
    "tmla_mla_decode_causal": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _i32, _vp, _i32, _i32, _i32, _i32,
        _i32, _i32, _f32, _i32, _i32, _vp, _i64, _i64, _vp, _vp, _sz, _i32, _vp]),
    "tmla_mla_decode_fp8": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _i64, _vp, _i64, _i32, _vp, _i32, _i32, _i32,
        _i32, _i32, _i32, _f32, _i32, _i32, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "tmla_generic_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "tmla_generic_heads_per_workgroup": (_i32, [_i32, _i32, _i32]),
    "tmla_mla_decode_generic": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _f32,
        _i32, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "tmla_mla_decode_fp8_partial": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _i64, _vp, _i64, _i32, _vp, _i32, _i32,
        _i32, _i32, _i32, _f32, _i32, _i32, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "tmla_mla_absorb_q": (ctypes.c_int, [
        _vp, _i64, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _vp, _i64, _i64, _vp]),
    "tmla_mla_absorb_out": (ctypes.c_int, [
        _vp, _i64, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _vp]),
    "tmla_mla_kv_append": (ctypes.c_int, [
        _vp, _i64, _vp, _f32, _f32, _vp, _i32, _i32, _i32, _i32, _vp, _i64, _i64, _i64, _i32, _vp, _i64, _i32,
        _vp]),
    "tmla_mla_rms_norm": (ctypes.c_int, [_vp, _i64, _vp, _f32, _i32, _i32, _i32, _vp, _i64, _vp]),
    "tmla_mla_project_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32]),
    "tmla_mla_project": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _vp, _i64, _vp, ctypes.c_size_t,
                                        _vp]),
}

STATUS = {0: "TMLA_OK", 1: "TMLA_ERR_INVALID_ARGUMENT", 2: "TMLA_ERR_UNSUPPORTED",
          3: "TMLA_ERR_WORKSPACE_TOO_SMALL", 4: "TMLA_ERR_HIP"}
DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_lib = None
_lock = threading.Lock()


class NativeError(RuntimeError):
    """A C-ABI entry point returned a non-zero tmla_status."""


def load():
    """Load (once) and return the ctypes library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"triton_mla HIP library not found at {LIB_PATH}; build it with "
                    "`python triton-mla_amd/build.py` (or __graft_entry__.build())")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


_held = None


def load_gil_held():
    """The same library through ctypes.PyDLL: its calls keep the GIL held, so
    the kernels one call launches are never interleaved with launches of
    another Python thread (used where calls on one stream share a
    workspace)."""
    global _held
    if _held is not None:
        return _held
    load()
    with _lock:
        if _held is None:
            lib = ctypes.PyDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _held = lib
    return _held


_fast = False  # not looked up yet


def fast_module():
    """The CPython module of the kept-shape call (csrc/fastcall.c, built beside
    the library and linked to it), or None when it is not built or another
    library build is selected (TRITON_MLA_LIB): callers then use the ctypes
    binding of the same library."""
    global _fast
    if _fast is False:
        mod = None
        if not os.environ.get("TRITON_MLA_LIB"):
            load()  # the library first, by the path the module's rpath resolves to
            try:
                from . import _tmla_fast as mod  # noqa: F811
            except ImportError:
                mod = None
        _fast = mod
    return _fast


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().tmla_last_error().decode(errors="replace")
        kind = STATUS.get(status, str(status))
        if status in (1, 2):
            raise ValueError(f"{what}: {kind}: {msg}")
        raise NativeError(f"{what}: {kind}: {msg}")
