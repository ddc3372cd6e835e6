"""fp8 (OCP E4M3) latent caches for ``mla_decode(..., kv_scale=...)``.

No counterpart in the reference, whose README.md:32-33 lists "no FP8 cache"
among its limitations. A cache row stores one E4M3 byte per latent/rope
element and stands for ``e4m3(byte) * scale`` with a float32 scale per page,
per token or per tensor; the decode kernels read half the bytes of a 16-bit
cache.

``quantize_kv_fp8`` writes such a cache from a 16-bit (or float32) one with
device tensor ops: scale = max |x| / 448 over the scale's group (448 is the
largest finite E4M3 value), codes = round-to-nearest-even of x / scale. It
is the cache writer, not part of the decode's hot path.
"""

from __future__ import annotations

import torch

E4M3_MAX = 448.0
GRANULARITIES = ("page", "token", "tensor")


def quantize_kv_fp8(kv_cache: torch.Tensor, granularity: str = "page"):
    """Quantise ``kv_cache`` ([pages or batch, rows, D]) to E4M3.

    Returns ``(codes, kv_scale)``: codes of dtype torch.float8_e4m3fn and the
    same shape, and float32 scales of shape [pages] ("page"), [pages, rows]
    ("token") or [1] ("tensor"). A group of zeros gets scale 1.
    """
    if granularity not in GRANULARITIES:
        raise ValueError(f"granularity must be one of {GRANULARITIES}")
    if kv_cache.dim() == 4:  # [..., 1, D] (one latent head)
        kv_cache = kv_cache.squeeze(2)
    x = kv_cache.float()
    if granularity == "page":
        amax = x.abs().amax(dim=(1, 2))
        view = (-1, 1, 1)
    elif granularity == "token":
        amax = x.abs().amax(dim=2)
        view = (x.shape[0], x.shape[1], 1)
    else:
        amax = x.abs().amax().reshape(1)
        view = (1, 1, 1)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    codes = (x / scale.reshape(view)).clamp_(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return codes, scale


def dequantize_kv_fp8(codes: torch.Tensor, kv_scale: torch.Tensor) -> torch.Tensor:
    """float32 values of an E4M3 cache (for tests and the PyTorch baselines)."""
    x = codes.view(torch.float8_e4m3fn).float()
    s = kv_scale.float()
    if s.numel() == 1:
        return x * s.reshape(1, 1, 1)
    if s.dim() == 1:
        return x * s.reshape(-1, 1, 1)
    return x * s.unsqueeze(-1)
