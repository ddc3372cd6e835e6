"""DeepSeek-V2/V3 Multi-head Latent Attention layer with an absorbed decode step.

Same module structure, parameter names and math as the reference layer
(src/triton_mla/model.py:13-144), so state dicts and call sites carry over:
``MLAConfig`` (model.py:13-31), ``RMSNorm`` (model.py:34-41), rotate-half
``apply_rope`` (model.py:44-50) and ``MLA`` with ``forward`` (absorbed:
W_UK folded into the query, W_UV applied after attention, model.py:101-124)
and ``forward_naive`` (decompressed per-head K/V, model.py:126-144). In
``forward`` the attention is the HIP ``mla_decode`` and the glue around it
runs as HIP kernels too (triton_mla.layer_ops): the cache append (RMSNorm of
the latent, RoPE of the key, paged write), the W_UK absorption with the q_pe
RoPE, and the W_UV product; the dense projections stay library GEMMs.
``forward_naive`` keeps the reference's torch steps: it is the layer's
oracle.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import layer_ops
from .kernel import mla_decode
from .reference import gather_kv


@dataclass
class MLAConfig:
    hidden_size: int = 7168
    num_heads: int = 128
    q_lora_rank: int = 1536
    kv_lora_rank: int = 512
    qk_nope_head_dim: int = 128
    qk_rope_head_dim: int = 64
    v_head_dim: int = 128
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-6

    @property
    def qk_head_dim(self):
        return self.qk_nope_head_dim + self.qk_rope_head_dim

    @property
    def kv_cache_dim(self):
        return self.kv_lora_rank + self.qk_rope_head_dim


class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        return F.rms_norm(x, (x.shape[-1],), self.weight, self.eps)


def apply_rope(x, positions, theta):
    """Rotate-half RoPE in float32: halves (a, b) -> (a cos - b sin, b cos + a sin)."""
    dim = x.shape[-1]
    exponents = torch.arange(0, dim, 2, device=x.device, dtype=torch.float32) / dim
    angles = positions.float()[..., None] / (theta ** exponents)
    cos, sin = torch.cos(angles), torch.sin(angles)
    first, second = x.float().chunk(2, dim=-1)
    rotated = torch.cat([first * cos - second * sin, second * cos + first * sin], dim=-1)
    return rotated.to(x.dtype)


class MLA(nn.Module):
    """Multi-head Latent Attention: per token only the compressed latent
    (kv_lora_rank) and the shared RoPE key (qk_rope_head_dim) are cached."""

    def __init__(self, cfg: MLAConfig):
        super().__init__()
        self.cfg = cfg
        heads = cfg.num_heads
        self.wq_a = nn.Linear(cfg.hidden_size, cfg.q_lora_rank, bias=False)
        self.q_norm = RMSNorm(cfg.q_lora_rank, cfg.rms_norm_eps)
        self.wq_b = nn.Linear(cfg.q_lora_rank, heads * cfg.qk_head_dim, bias=False)
        self.wkv_a = nn.Linear(cfg.hidden_size, cfg.kv_cache_dim, bias=False)
        self.kv_norm = RMSNorm(cfg.kv_lora_rank, cfg.rms_norm_eps)
        self.wkv_b = nn.Linear(cfg.kv_lora_rank, heads * (cfg.qk_nope_head_dim + cfg.v_head_dim), bias=False)
        self.wo = nn.Linear(heads * cfg.v_head_dim, cfg.hidden_size, bias=False)
        self.softmax_scale = cfg.qk_head_dim ** -0.5

    def _project(self, x, positions):
        cfg = self.cfg
        q = self.wq_b(self.q_norm(self.wq_a(x))).view(x.shape[0], cfg.num_heads, cfg.qk_head_dim)
        q_nope, q_pe = q.split([cfg.qk_nope_head_dim, cfg.qk_rope_head_dim], dim=-1)
        q_pe = apply_rope(q_pe, positions[:, None], cfg.rope_theta)
        c_kv, k_pe = self.wkv_a(x).split([cfg.kv_lora_rank, cfg.qk_rope_head_dim], dim=-1)
        c_kv = self.kv_norm(c_kv)
        k_pe = apply_rope(k_pe, positions, cfg.rope_theta)
        return q_nope, q_pe, c_kv, k_pe

    @staticmethod
    def _append_kv(kv_cache, c_kv, k_pe, cache_seqlens, block_table):
        """Write each sequence's new latent row at position cache_seqlens[b]."""
        entry = torch.cat([c_kv, k_pe], dim=-1).to(kv_cache.dtype)
        pos = cache_seqlens.long()
        rows = torch.arange(pos.shape[0], device=pos.device)
        if block_table is None:
            kv_cache[rows, pos] = entry
        else:
            page_size = kv_cache.shape[1]
            pages = block_table[rows, pos // page_size].long()
            kv_cache[pages, pos % page_size] = entry

    def _wkv_b(self):
        """(W_UK [H, nope, rank], W_UV [H, v, rank]) views of wkv_b."""
        cfg = self.cfg
        w = self.wkv_b.weight.view(cfg.num_heads, cfg.qk_nope_head_dim + cfg.v_head_dim, cfg.kv_lora_rank)
        return w[:, : cfg.qk_nope_head_dim], w[:, cfg.qk_nope_head_dim:]

    def forward(self, x, kv_cache, cache_seqlens, block_table=None, num_splits=None):
        """One decode step for x [batch, hidden].

        Appends the new token to kv_cache in place and returns
        (output [batch, hidden], updated cache_seqlens).
        """
        cfg = self.cfg
        if kv_cache.dtype != x.dtype:
            raise NotImplementedError("MLA.forward needs the cache in the layer's dtype")
        q_proj = self.wq_b(self.q_norm(self.wq_a(x)))  # [B, H * (nope + rope)]
        kv_proj = self.wkv_a(x)  # [B, rank + rope]
        # RMSNorm(c_kv), RoPE(k_pe) and the paged append (model.py:80-94)
        layer_ops.kv_append(kv_proj, self.kv_norm.weight, self.kv_norm.eps, cfg.rope_theta, cache_seqlens,
                            kv_cache, block_table, cfg.kv_lora_rank, cfg.qk_rope_head_dim)
        seqlens = cache_seqlens + 1
        # q = [q_nope . W_UK, RoPE(q_pe)] (model.py:74-79, 108-109)
        q = layer_ops.absorb_q(q_proj, self.wkv_b.weight, cache_seqlens, cfg.num_heads, cfg.qk_nope_head_dim,
                               cfg.qk_rope_head_dim, cfg.kv_lora_rank, cfg.v_head_dim, cfg.rope_theta)
        o = mla_decode(q, kv_cache, seqlens, block_table, head_dim_v=cfg.kv_lora_rank,
                       softmax_scale=self.softmax_scale, num_splits=num_splits)
        # o . W_UV^T per head (model.py:120-124), then wo
        o = layer_ops.absorb_out(o, self.wkv_b.weight, cfg.num_heads, cfg.qk_nope_head_dim, cfg.kv_lora_rank,
                                 cfg.v_head_dim)
        return self.wo(o), seqlens

    def forward_torch_glue(self, x, kv_cache, cache_seqlens, block_table=None, num_splits=None):
        """The absorbed step with the reference's torch glue around the HIP
        mla_decode (model.py:101-124): the baseline the HIP glue is timed
        against."""
        q_nope, q_pe, c_kv, k_pe = self._project(x, cache_seqlens)
        self._append_kv(kv_cache, c_kv, k_pe, cache_seqlens, block_table)
        seqlens = cache_seqlens + 1
        w_uk, w_uv = self._wkv_b()
        # absorb W_UK: [B, H, nope] x [H, nope, rank] -> [B, H, rank]
        q_abs = torch.bmm(q_nope.transpose(0, 1).contiguous(), w_uk.contiguous()).transpose(0, 1)
        q = torch.cat([q_abs, q_pe], dim=-1).to(kv_cache.dtype).contiguous()
        o = mla_decode(q, kv_cache, seqlens, block_table, head_dim_v=self.cfg.kv_lora_rank,
                       softmax_scale=self.softmax_scale, num_splits=num_splits)
        # apply W_UV: [B, H, rank] x [H, rank, v] -> [B, H, v]
        w_uv_t = w_uv.transpose(1, 2).contiguous()
        o = torch.bmm(o.to(w_uv.dtype).transpose(0, 1).contiguous(), w_uv_t).transpose(0, 1)
        return self.wo(o.flatten(1)), seqlens

    def forward_naive(self, x, kv_cache, cache_seqlens, block_table=None):
        """Same decode step without absorption: decompress the cache into per-head K/V."""
        cfg = self.cfg
        q_nope, q_pe, c_kv, k_pe = self._project(x, cache_seqlens)
        self._append_kv(kv_cache, c_kv, k_pe, cache_seqlens, block_table)
        seqlens = cache_seqlens + 1
        kv = gather_kv(kv_cache, seqlens, block_table).to(x.dtype)
        latent, kpe = kv.split([cfg.kv_lora_rank, cfg.qk_rope_head_dim], dim=-1)
        kvb = self.wkv_b(latent).view(*latent.shape[:2], cfg.num_heads, -1)
        k_nope, v = kvb.split([cfg.qk_nope_head_dim, cfg.v_head_dim], dim=-1)
        k = torch.cat([k_nope, kpe[:, :, None].expand(-1, -1, cfg.num_heads, -1)], dim=-1)
        q = torch.cat([q_nope, q_pe], dim=-1)
        # scores [B, H, S] and output [B, H, v] in float32
        scores = torch.einsum("bhd,bshd->bhs", q.float(), k.float()) * self.softmax_scale
        invalid = torch.arange(kv.shape[1], device=x.device)[None, :] >= seqlens[:, None]
        scores = scores.masked_fill(invalid[:, None, :], float("-inf"))
        o = torch.einsum("bhs,bshd->bhd", scores.softmax(-1), v.float()).to(x.dtype)
        return self.wo(o.flatten(1)), seqlens
