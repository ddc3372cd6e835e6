"""CPU oracle for the MLA decode path (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this module. It is the checker, never the product:
``triton_mla.mla_decode`` has no CPU path and never calls into here.

Contents
--------
* ctypes bindings to ``mla_oracle.c`` (float64 restatements of the
  reference's ``gather_kv`` / ``mla_decode_ref`` (src/triton_mla/reference.py:6-31),
  ``get_num_splits`` (src/triton_mla/kernel.py:190-201) and the fused
  kernel's split/merge algebra (kernel.py:83-86, 119-128, 165-181));
* ``mla_decode_ref_causal``: multi-token causal decode built on the
  single-token oracle (an extension; no reference counterpart);
* an fp8 latent cache (no reference counterpart; its README.md:32-33 lists
  "no FP8 cache"): ``e4m3_to_float`` / ``float_to_e4m3`` (OCP E4M3,
  round to nearest even) and ``mla_decode_fp8_ref`` (the single-token or
  causal oracle over the dequantised cache);
* a numpy float64 restatement of the ``MLA`` layer (src/triton_mla/model.py):
  RMSNorm (model.py:34-41), rotate-half RoPE (model.py:44-50), projections
  (model.py:74-82), cache append (model.py:84-94), ``W_UK``/``W_UV`` split
  (model.py:96-99), the absorbed step (model.py:101-124) and the
  non-absorbed ``forward_naive`` (model.py:126-144).

How each function is pinned is listed in mla_oracle.c's header and tested in
tests/test_oracle.py. Arrays of 16-bit floats are passed as raw ``uint16``
bit patterns (numpy has no bfloat16); ``dtype`` is "bf16" or "fp16".
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libmla_oracle.so")
_DTYPE_CODE = {"bf16": 0, "fp16": 1, "fp32": 2}

_lib = None


def build(force: bool = False) -> str:
    """Compile mla_oracle.c with the Makefile beside it; return the library path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, i32, f64 = ctypes.c_int64, ctypes.c_int, ctypes.c_double
        vp = ctypes.c_void_p
        L.oracle_mla_decode_ref.argtypes = [vp, i64, i64, vp, i64, i64, vp, i64, i32, i64, vp,
                                            i64, i64, i64, i64, i32, f64, i32, vp, vp]
        L.oracle_mla_decode_ref.restype = i32
        L.oracle_gather_kv.argtypes = [vp, i64, i64, vp, i64, i32, i64, i64, i64, i64, vp]
        L.oracle_gather_kv.restype = None
        L.oracle_get_num_splits.argtypes = [i64, i64, i64, i64, i64]
        L.oracle_get_num_splits.restype = i64
        L.oracle_split_merge.argtypes = [vp, vp, i64, i64, vp, i64, i32, i64, i64, i64, i64, i64,
                                         i32, f64, i64, vp, vp]
        L.oracle_split_merge.restype = i32
        L.oracle_round_to_half.argtypes = [vp, vp, i64, i32]
        L.oracle_round_to_half.restype = None
        L.oracle_float_to_half_bits.argtypes = [ctypes.c_float, i32]
        L.oracle_float_to_half_bits.restype = ctypes.c_uint16
        L.oracle_half_to_double.argtypes = [ctypes.c_uint16, i32]
        L.oracle_half_to_double.restype = f64
        L.oracle_e4m3_to_double.argtypes = [ctypes.c_uint8]
        L.oracle_e4m3_to_double.restype = f64
        L.oracle_e4m3_encode.argtypes = [vp, vp, i64]
        L.oracle_e4m3_encode.restype = None
        L.oracle_mla_decode_fp8_ref.argtypes = [vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i32, i64,
                                                vp, i64, i64, i64, i64, i32, f64, i32, vp, vp]
        L.oracle_mla_decode_fp8_ref.restype = i32
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(a: np.ndarray) -> np.ndarray:
    assert a.dtype == np.uint16, "16-bit float arrays travel as uint16 bit patterns"
    return a


# ----------------------------------------------------------------------------
# 16-bit float helpers
# ----------------------------------------------------------------------------

def half_to_float(bits: np.ndarray, dtype: str) -> np.ndarray:
    """Exact widening of bf16/fp16 bit patterns to float64."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return bits.view(np.float16).astype(np.float64)


def float_to_half(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float values to bf16/fp16 (nearest even) and return bit patterns."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_round_to_half(_ptr(x), _ptr(out), x.size, _DTYPE_CODE[dtype])
    return out


# ----------------------------------------------------------------------------
# decode attention
# ----------------------------------------------------------------------------

def _elems(a: np.ndarray, dtype: str) -> np.ndarray:
    """16-bit types travel as uint16 bit patterns, fp32 as float32 values."""
    if dtype == "fp32":
        assert a.dtype == np.float32, "fp32 arrays travel as float32"
        return np.ascontiguousarray(a)
    return np.ascontiguousarray(_u16(a))


def _cache_args(kv_cache: np.ndarray, block_table, dtype="bf16"):
    if kv_cache.ndim == 4:  # FlashMLA layout [..., 1, D] (reference.py:8-9)
        assert kv_cache.shape[2] == 1
        kv_cache = kv_cache.reshape(kv_cache.shape[0], kv_cache.shape[1], kv_cache.shape[3])
    kv_cache = _elems(kv_cache, dtype)
    if block_table is None:
        return kv_cache, None, 0, 0, 1
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    return kv_cache, bt, bt.shape[1], 1, kv_cache.shape[1]


def mla_decode_ref(q, kv_cache, cache_seqlens, block_table=None, head_dim_v=512,
                   softmax_scale=None, dtype="bf16", nthreads=0):
    """Restates reference.py:16-31 in float64.

    ``dtype`` "bf16" / "fp16" (q and the cache as uint16 bit patterns) or
    "fp32" (float32 arrays). Returns ``(out float32 [B, H, dv] unrounded,
    lse float32 [B, H])``.
    """
    q = _elems(q, dtype)
    B, H, dqk = q.shape
    if softmax_scale is None:
        softmax_scale = dqk ** -0.5  # reference.py:18-19
    kv, bt, bt_s0, paged, page_size = _cache_args(kv_cache, block_table, dtype)
    assert kv.shape[-1] == dqk
    seqlens = np.ascontiguousarray(cache_seqlens, dtype=np.int32)
    out = np.empty((B, H, head_dim_v), dtype=np.float32)
    lse = np.empty((B, H), dtype=np.float32)
    rc = lib().oracle_mla_decode_ref(
        _ptr(q), H * dqk, dqk, _ptr(kv), kv.shape[1] * dqk, dqk,
        _ptr(bt) if bt is not None else None, bt_s0, paged, page_size, _ptr(seqlens),
        B, H, dqk, head_dim_v, _DTYPE_CODE[dtype], float(softmax_scale), int(nthreads),
        _ptr(out), _ptr(lse))
    if rc != 0:
        raise RuntimeError(f"oracle_mla_decode_ref failed ({rc})")
    return out, lse


def mla_decode_ref_causal(q, kv_cache, cache_seqlens, block_table=None, head_dim_v=512,
                          softmax_scale=None, dtype="bf16", nthreads=0):
    """Multi-token causal decode, a float64 oracle for an extension with no
    counterpart in the reference (its mla_decode takes one query token,
    src/triton_mla/kernel.py:238).

    q is [B, T, H, D]: the T query tokens of sequence b are its last T cached
    tokens, and query token t attends to the first
    max(cache_seqlens[b] - (T - 1 - t), 0) tokens. Each token is therefore the
    single-token oracle (reference.py:16-31) with that length.
    Returns ``(out float32 [B, T, H, dv], lse float32 [B, T, H])``.
    """
    q = _u16(q)
    B, T, H, D = q.shape
    seqlens = np.asarray(cache_seqlens, dtype=np.int64)
    out = np.empty((B, T, H, head_dim_v), dtype=np.float32)
    lse = np.empty((B, T, H), dtype=np.float32)
    for t in range(T):
        n_t = np.maximum(seqlens - (T - 1 - t), 0).astype(np.int32)
        o, l = mla_decode_ref(np.ascontiguousarray(q[:, t]), kv_cache, n_t, block_table, head_dim_v,
                              softmax_scale, dtype, nthreads)
        out[:, t] = o
        lse[:, t] = l
    return out, lse


# ----------------------------------------------------------------------------
# fp8 (OCP E4M3) latent cache
# ----------------------------------------------------------------------------

def e4m3_to_float(codes: np.ndarray) -> np.ndarray:
    """Exact float64 values of E4M3 codes (uint8)."""
    table = np.array([lib().oracle_e4m3_to_double(c) for c in range(256)], dtype=np.float64)
    return table[np.asarray(codes, dtype=np.uint8)]


def float_to_e4m3(x: np.ndarray) -> np.ndarray:
    """Nearest E4M3 codes (ties to even; above 464 in magnitude: NaN)."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().oracle_e4m3_encode(_ptr(x), _ptr(out), x.size)
    return out


def mla_decode_fp8_ref(q, kv8, kv_scale, cache_seqlens, block_table=None, head_dim_v=512,
                       softmax_scale=None, dtype="bf16", scale_strides=None, nthreads=0):
    """mla_decode_ref over an fp8 cache, float64.

    kv8: uint8 E4M3 codes, [num_blocks, page_size, D] (paged) or [batch,
    capacity, D] (dense). kv_scale: float32 array; row t of sequence b is
    dequantised as e4m3(code) * kv_scale.flat[page * s0 + (t % page_size) * s1]
    (dense: b * s0 + t * s1) with (s0, s1) = scale_strides, by default the
    array's own element strides (per page: shape [num_blocks]; per token:
    [num_blocks, page_size]; one scale: any one-element array -> (0, 0)).
    q is [B, H, D] (single token) or [B, T, H, D] (causal, as
    mla_decode_ref_causal). Returns ``(out float32 unrounded, lse float32)``.
    """
    q = _u16(q)
    if q.ndim == 4:
        B, T, H, D = q.shape
        seqlens = np.asarray(cache_seqlens, dtype=np.int64)
        out = np.empty((B, T, H, head_dim_v), dtype=np.float32)
        lse = np.empty((B, T, H), dtype=np.float32)
        for t in range(T):
            n_t = np.maximum(seqlens - (T - 1 - t), 0).astype(np.int32)
            o, l = mla_decode_fp8_ref(np.ascontiguousarray(q[:, t]), kv8, kv_scale, n_t, block_table, head_dim_v,
                                      softmax_scale, dtype, scale_strides, nthreads)
            out[:, t] = o
            lse[:, t] = l
        return out, lse
    q = np.ascontiguousarray(q)
    B, H, dqk = q.shape
    if softmax_scale is None:
        softmax_scale = dqk ** -0.5
    kv8 = np.ascontiguousarray(kv8, dtype=np.uint8)
    assert kv8.shape[-1] == dqk
    sc = np.ascontiguousarray(kv_scale, dtype=np.float32)
    if scale_strides is None:
        if sc.size == 1:
            scale_strides = (0, 0)
        else:
            st = [s // 4 for s in sc.strides] + [0, 0]
            scale_strides = (st[0], st[1])
    seqlens = np.ascontiguousarray(cache_seqlens, dtype=np.int32)
    if block_table is None:
        bt, bt_s0, paged, page_size = None, 0, 0, 1
    else:
        bt = np.ascontiguousarray(block_table, dtype=np.int32)
        bt_s0, paged, page_size = bt.shape[1], 1, kv8.shape[1]
    out = np.empty((B, H, head_dim_v), dtype=np.float32)
    lse = np.empty((B, H), dtype=np.float32)
    rc = lib().oracle_mla_decode_fp8_ref(
        _ptr(q), H * dqk, dqk, _ptr(kv8), kv8.shape[1] * dqk, dqk, _ptr(sc), int(scale_strides[0]),
        int(scale_strides[1]), _ptr(bt) if bt is not None else None, bt_s0, paged, page_size, _ptr(seqlens),
        B, H, dqk, head_dim_v, _DTYPE_CODE[dtype], float(softmax_scale), int(nthreads), _ptr(out), _ptr(lse))
    if rc != 0:
        raise RuntimeError(f"oracle_mla_decode_fp8_ref failed ({rc})")
    return out, lse


def gather_kv(kv_cache, cache_seqlens, block_table=None, n_tokens=None):
    """Restates reference.py:6-13: [B, n_tokens, D] bit-exact gather."""
    kv, bt, bt_s0, paged, page_size = _cache_args(kv_cache, block_table)
    D = kv.shape[-1]
    if bt is None:
        B = len(cache_seqlens)
        n = kv.shape[1] if n_tokens is None else n_tokens
    else:
        B = bt.shape[0]
        n = bt.shape[1] * page_size if n_tokens is None else n_tokens
    out = np.empty((B, n, D), dtype=np.uint16)
    lib().oracle_gather_kv(_ptr(kv), kv.shape[1] * D, D, _ptr(bt) if bt is not None else None,
                           bt_s0, paged, page_size, B, n, D, _ptr(out))
    return out


def get_num_splits(batch, num_heads, max_seqlen, num_sms, min_tokens_per_split=128):
    """Restates kernel.py:190-201."""
    return int(lib().oracle_get_num_splits(batch, num_heads, max_seqlen, num_sms, min_tokens_per_split))


def split_merge(q_row, kv_cache, b, n, block_table=None, head_dim_v=512, softmax_scale=None,
                num_splits=1, dtype="bf16"):
    """The fused kernel's split-then-merge algebra for one (b, h) query row."""
    q_row = np.ascontiguousarray(_u16(q_row))
    dqk = q_row.shape[-1]
    if softmax_scale is None:
        softmax_scale = dqk ** -0.5
    kv, bt, bt_s0, paged, page_size = _cache_args(kv_cache, block_table)
    out = np.empty((head_dim_v,), dtype=np.float32)
    lse = np.empty((1,), dtype=np.float32)
    rc = lib().oracle_split_merge(_ptr(q_row), _ptr(kv), kv.shape[1] * dqk, dqk,
                                  _ptr(bt) if bt is not None else None, bt_s0, paged, page_size,
                                  b, n, dqk, head_dim_v, _DTYPE_CODE[dtype], float(softmax_scale),
                                  num_splits, _ptr(out), _ptr(lse))
    if rc != 0:
        raise RuntimeError(f"oracle_split_merge failed ({rc})")
    return out, float(lse[0])


# ----------------------------------------------------------------------------
# MLA layer (model.py), numpy float64
# ----------------------------------------------------------------------------

def rms_norm(x, weight, eps):
    """F.rms_norm over the last dim (model.py:40-41)."""
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(weight, np.float64)


def apply_rope(x, positions, theta):
    """Rotate-half RoPE, model.py:44-50: halves (x1, x2) -> (x1 c - x2 s, x2 c + x1 s)."""
    x = np.asarray(x, dtype=np.float64)
    d = x.shape[-1]
    inv_freq = 1.0 / (theta ** (np.arange(0, d, 2, dtype=np.float64) / d))
    freqs = np.asarray(positions, dtype=np.float64)[..., None] * inv_freq
    cos, sin = np.cos(freqs), np.sin(freqs)
    x1, x2 = x[..., : d // 2], x[..., d // 2:]
    return np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1)


def layer_project(w, cfg, x, positions):
    """model.py:74-82. ``w`` maps parameter names to float64 arrays (nn.Linear [out, in])."""
    H = cfg["num_heads"]
    dn, dr, r = cfg["qk_nope_head_dim"], cfg["qk_rope_head_dim"], cfg["kv_lora_rank"]
    eps = cfg["rms_norm_eps"]
    q = rms_norm(x @ w["wq_a"].T, w["q_norm"], eps) @ w["wq_b"].T
    q = q.reshape(x.shape[0], H, dn + dr)
    q_nope, q_pe = q[..., :dn], q[..., dn:]
    q_pe = apply_rope(q_pe, np.asarray(positions)[:, None], cfg["rope_theta"])
    kv = x @ w["wkv_a"].T
    c_kv, k_pe = kv[:, :r], kv[:, r:]
    c_kv = rms_norm(c_kv, w["kv_norm"], eps)
    k_pe = apply_rope(k_pe, positions, cfg["rope_theta"])
    return q_nope, q_pe, c_kv, k_pe


def layer_forward_naive(w, cfg, x, kv_tokens, cache_seqlens):
    """model.py:126-144 (non-absorbed), given each sequence's cached rows.

    ``kv_tokens[b]`` is the float64 [n_b, r + dr] cache content of sequence b
    *before* the append; the new token is appended here at position n_b.
    Returns (out [B, hidden], appended entries [B, r + dr]).
    """
    H = cfg["num_heads"]
    dn, dr, dv, r = cfg["qk_nope_head_dim"], cfg["qk_rope_head_dim"], cfg["v_head_dim"], cfg["kv_lora_rank"]
    scale = (dn + dr) ** -0.5
    pos = np.asarray(cache_seqlens, dtype=np.int64)
    q_nope, q_pe, c_kv, k_pe = layer_project(w, cfg, x, pos)
    entries = np.concatenate([c_kv, k_pe], axis=-1)
    wkv_b = w["wkv_b"].reshape(H, dn + dv, r)
    o = np.zeros((x.shape[0], H, dv))
    for b in range(x.shape[0]):
        rows = np.concatenate([kv_tokens[b], entries[b:b + 1]], axis=0)
        latent, kpe = rows[:, :r], rows[:, r:]
        kvb = np.einsum("sc,hdc->shd", latent, wkv_b)
        k_nope, v = kvb[..., :dn], kvb[..., dn:]
        k = np.concatenate([k_nope, np.broadcast_to(kpe[:, None, :], (rows.shape[0], H, dr))], axis=-1)
        qb = np.concatenate([q_nope[b], q_pe[b]], axis=-1)
        s = np.einsum("hd,shd->hs", qb, k) * scale
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        o[b] = np.einsum("hs,shd->hd", p, v)
    return o.reshape(x.shape[0], H * dv) @ w["wo"].T, entries


def layer_absorbed_query(w, cfg, q_nope, q_pe):
    """q_abs = einsum('bhd,hdc->bhc', q_nope, W_UK) ++ q_pe (model.py:111-113)."""
    H = cfg["num_heads"]
    dn, dv, r = cfg["qk_nope_head_dim"], cfg["v_head_dim"], cfg["kv_lora_rank"]
    w_uk = w["wkv_b"].reshape(H, dn + dv, r)[:, :dn]
    return np.concatenate([np.einsum("bhd,hdc->bhc", q_nope, w_uk), q_pe], axis=-1)


def layer_output(w, cfg, o_latent):
    """o = einsum('bhc,hdc->bhd', o, W_UV); wo(o.flatten(1)) (model.py:123-124)."""
    H = cfg["num_heads"]
    dn, dv, r = cfg["qk_nope_head_dim"], cfg["v_head_dim"], cfg["kv_lora_rank"]
    w_uv = w["wkv_b"].reshape(H, dn + dv, r)[:, dn:]
    o = np.einsum("bhc,hdc->bhd", np.asarray(o_latent, np.float64), w_uv)
    return o.reshape(o.shape[0], H * dv) @ w["wo"].T
