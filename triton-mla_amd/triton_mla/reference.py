"""PyTorch MLA decode implementations kept for API compatibility.

These are the public ``mla_decode_ref`` / ``mla_decode_torch`` / ``gather_kv``
of the reference package (src/triton_mla/reference.py:6-44): plain torch ops,
usable on any device, used by callers as a slow reference and as the eager /
``torch.compile`` baseline. ``mla_decode`` never calls them. The test suite
checks the HIP kernels against the independent CPU oracle under oracle/, not
against these.
"""

from __future__ import annotations

import torch


def gather_kv(kv_cache, cache_seqlens, block_table=None):
    """Contiguous [batch, capacity, D] view of a paged or dense cache (reference.py:6-13)."""
    if kv_cache.dim() == 4:
        kv_cache = kv_cache.squeeze(2)
    if block_table is None:
        return kv_cache
    pages = kv_cache.index_select(0, block_table.reshape(-1).long())
    return pages.reshape(block_table.shape[0], -1, kv_cache.shape[-1])


def mla_decode_ref(q, kv_cache, cache_seqlens, block_table=None, head_dim_v=512, softmax_scale=None):
    """Per-sequence float32 attention (reference.py:16-31): returns (out in q.dtype, lse)."""
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    kv = gather_kv(kv_cache, cache_seqlens, block_table)
    batch, heads = q.shape[0], q.shape[1]
    out = q.new_zeros(batch, heads, head_dim_v, dtype=torch.float32)
    lse = q.new_full((batch, heads), float("-inf"), dtype=torch.float32)
    lens = [int(n) for n in cache_seqlens.tolist()]
    for b, n in enumerate(lens):
        if n <= 0:
            continue
        keys = kv[b, :n].float()
        logits = (q[b].float() @ keys.transpose(0, 1)) * scale
        lse[b] = torch.logsumexp(logits, dim=-1)
        out[b] = torch.softmax(logits, dim=-1) @ keys[:, :head_dim_v]
    return out.to(q.dtype), lse


def mla_decode_torch(q, kv_cache, cache_seqlens, block_table=None, head_dim_v=512, softmax_scale=None):
    """Batched masked attention in the input dtype (reference.py:34-44).

    Scores come from a q.dtype matmul, softmax runs in float32 and the
    probabilities are cast back to q.dtype before the value matmul. A
    sequence of length 0 yields NaN, as in the reference.
    """
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    kv = gather_kv(kv_cache, cache_seqlens, block_table)
    keys_t = kv.transpose(1, 2).contiguous()
    logits = torch.matmul(q, keys_t).float() * scale
    positions = torch.arange(kv.shape[1], device=q.device)
    invalid = positions[None, :] >= cache_seqlens.to(positions.device)[:, None]
    logits = logits.masked_fill(invalid[:, None, :], float("-inf"))
    probs = torch.softmax(logits, dim=-1).to(q.dtype)
    return torch.matmul(probs, kv[..., :head_dim_v].contiguous())
