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
RoPE, the W_UV product, the RMSNorm of the query latent, and the wide dense
projections (wq_b, wo) of a step of up to 16 rows; wq_a and wkv_a run as one
library GEMM over both weights.
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
    """Root-mean-square normalisation with a learned gain (model.py:34-41).

    Computed in float32 and rounded once to the input dtype: y = x / rms(x)
    * weight with rms(x) = sqrt(mean(x^2) + eps), the same arithmetic as the
    HIP cache-append kernel's normalisation of the latent.
    """

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        inv_rms = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + self.eps)
        return (xf * inv_rms * self.weight.float()).to(x.dtype)


def apply_rope(x, positions, theta):
    """Rotate-half RoPE in float32: halves (a, b) -> (a cos - b sin, b cos + a sin)."""
    dim = x.shape[-1]
    exponents = torch.arange(0, dim, 2, device=x.device, dtype=torch.float32) / dim
    angles = positions.float()[..., None] / (theta ** exponents)
    cos, sin = torch.cos(angles), torch.sin(angles)
    first, second = x.float().chunk(2, dim=-1)
    rotated = torch.cat([first * cos - second * sin, second * cos + first * sin], dim=-1)
    return rotated.to(x.dtype)


def _hip_glue_dims(cfg) -> bool:
    """Dims the HIP layer kernels are built for: q_pe RoPE and W_UK absorption
    at nope 128 / rope 64, the latent a multiple of 512 up to 1024, W_UV
    blocks of 32 value dims, q_lora_rank a multiple of 8 (DeepSeek V2, V2-Lite
    and V3 all fit)."""
    return (cfg.qk_nope_head_dim == 128 and cfg.qk_rope_head_dim == 64 and cfg.kv_lora_rank % 512 == 0
            and cfg.kv_lora_rank <= 1024 and cfg.v_head_dim % 32 == 0 and cfg.q_lora_rank % 8 == 0)


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
        """Query and latent of the new token (model.py:74-82): q_nope
        [B, H, nope], RoPE'd q_pe [B, H, rope], normalised latent c_kv
        [B, rank] and RoPE'd shared key k_pe [B, rope]."""
        cfg = self.cfg
        q_lat = self.q_norm(self.wq_a(x))
        q = self.wq_b(q_lat).unflatten(-1, (cfg.num_heads, cfg.qk_head_dim))
        q_nope = q[..., :cfg.qk_nope_head_dim]
        q_pe = apply_rope(q[..., cfg.qk_nope_head_dim:], positions.unsqueeze(-1), cfg.rope_theta)
        kv = self.wkv_a(x)
        c_kv = self.kv_norm(kv[..., :cfg.kv_lora_rank])
        k_pe = apply_rope(kv[..., cfg.kv_lora_rank:], positions, cfg.rope_theta)
        return q_nope, q_pe, c_kv, k_pe

    @staticmethod
    def _append_kv(kv_cache, c_kv, k_pe, cache_seqlens, block_table):
        """Store each sequence's new cache row [c_kv, k_pe] at token position
        cache_seqlens[b] (model.py:84-94): through the block table for a paged
        cache, at row b of a dense one."""
        width = kv_cache.shape[-1]
        rows = torch.cat([c_kv, k_pe], dim=-1).to(kv_cache.dtype)
        pos = cache_seqlens.to(torch.int64)
        per_block = kv_cache.shape[1]  # tokens per page, or the dense capacity
        if block_table is None:
            block = torch.arange(pos.numel(), device=pos.device)
            slot = pos
        else:
            block = block_table.gather(1, (pos // per_block).unsqueeze(1)).squeeze(1).to(torch.int64)
            slot = pos % per_block
        flat_index = block * per_block + slot
        if kv_cache.is_contiguous():
            kv_cache.view(-1, width).index_copy_(0, flat_index, rows)
        else:
            kv_cache[block, slot] = rows

    def _wkv_b(self):
        """W_UK [H, nope, rank] and W_UV [H, v, rank]: the per-head row blocks
        of wkv_b (model.py:96-99)."""
        cfg = self.cfg
        per_head = self.wkv_b.weight.unflatten(0, (cfg.num_heads, cfg.qk_nope_head_dim + cfg.v_head_dim))
        w_uk, w_uv = torch.split(per_head, [cfg.qk_nope_head_dim, cfg.v_head_dim], dim=1)
        return w_uk, w_uv

    def forward(self, x, kv_cache, cache_seqlens, block_table=None, num_splits=None):
        """One decode step for x [batch, hidden].

        Appends the new token to kv_cache in place and returns
        (output [batch, hidden], updated cache_seqlens).
        """
        cfg = self.cfg
        if kv_cache.dtype != x.dtype or x.dtype not in (torch.bfloat16, torch.float16) or not _hip_glue_dims(cfg):
            # the HIP glue runs in the layer's 16-bit dtype at the DeepSeek
            # head dims; other dtype mixes and dims take the reference's torch
            # glue, which casts (model.py:108-124), around the same mla_decode
            return self.forward_torch_glue(x, kv_cache, cache_seqlens, block_table, num_splits)
        q_lat, kv_proj = self._down_proj(x)  # [B, q_lora_rank], [B, rank + rope]
        # in one launch: q_norm (model.py:76); RMSNorm(c_kv), RoPE(k_pe) and
        # the paged append (model.py:80-94); cache_seqlens + 1 (model.py:109)
        q_lat, seqlens = layer_ops.norm_append(
            q_lat, self.q_norm.weight, self.q_norm.eps, kv_proj, self.kv_norm.weight, self.kv_norm.eps,
            cfg.rope_theta, cache_seqlens, kv_cache, block_table, cfg.kv_lora_rank, cfg.qk_rope_head_dim)
        if seqlens.dtype != cache_seqlens.dtype:  # the caller's dtype, as cache_seqlens + 1 keeps it
            seqlens = seqlens.to(cache_seqlens.dtype)
        q_proj = self._linear(self.wq_b, q_lat)  # [B, H * (nope + rope)]
        # q = [q_nope . W_UK, RoPE(q_pe)] (model.py:74-79, 108-109)
        q = layer_ops.absorb_q(q_proj, self.wkv_b.weight, cache_seqlens, cfg.num_heads, cfg.qk_nope_head_dim,
                               cfg.qk_rope_head_dim, cfg.kv_lora_rank, cfg.v_head_dim, cfg.rope_theta)
        o = mla_decode(q, kv_cache, seqlens, block_table, head_dim_v=cfg.kv_lora_rank,
                       softmax_scale=self.softmax_scale, num_splits=num_splits)
        # o . W_UV^T per head (model.py:120-124), then wo
        o = layer_ops.absorb_out(o, self.wkv_b.weight, cfg.num_heads, cfg.qk_nope_head_dim, cfg.kv_lora_rank,
                                 cfg.v_head_dim)
        return self._linear(self.wo, o), seqlens

    @staticmethod
    def _linear(layer, x):
        """A projection of the step's rows: the HIP kernel where it beats the
        library GEMM (few rows, a wide weight), the library GEMM otherwise."""
        if layer.bias is None and layer_ops.project_pays(x, layer.weight):
            return layer_ops.project(x, layer.weight)
        return layer(x)

    def _down_proj(self, x):
        """x . wq_a^T and x . wkv_a^T. Both read the same rows, so they run as
        one GEMM over [wq_a; wkv_a], concatenated once and kept while neither
        parameter is replaced or changed in place (data pointers and version
        counters). Inference tensors keep no version counter to tell an
        in-place change by: for them the two GEMMs run separately."""
        wa, wk = self.wq_a.weight, self.wkv_a.weight
        if wa.is_inference() or wk.is_inference():
            return F.linear(x, wa), F.linear(x, wk)
        key = (wa.data_ptr(), wa._version, wk.data_ptr(), wk._version, wa.dtype, wa.device)
        cached = getattr(self, "_down_cache", None)
        if cached is None or cached[0] != key:
            with torch.no_grad(), torch.inference_mode(False):  # a plain tensor, usable in any mode
                cached = (key, torch.cat([wa.detach(), wk.detach()], dim=0))
            self._down_cache = cached
        down = F.linear(x, cached[1])
        return down[:, :wa.shape[0]], down[:, wa.shape[0]:]

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
        """The same decode step without absorption (model.py:126-144): every
        cached latent is expanded through wkv_b into per-head keys and values,
        and attention runs per head in float32. The layer's oracle."""
        cfg = self.cfg
        q_nope, q_pe, c_kv, k_pe = self._project(x, cache_seqlens)
        self._append_kv(kv_cache, c_kv, k_pe, cache_seqlens, block_table)
        seqlens = cache_seqlens + 1
        cache = gather_kv(kv_cache, seqlens, block_table).to(x.dtype)  # [B, S, rank + rope]
        latent = cache[..., :cfg.kv_lora_rank]
        shared_k = cache[..., cfg.kv_lora_rank:].float()  # [B, S, rope], one key for all heads
        expanded = self.wkv_b(latent).unflatten(-1, (cfg.num_heads, cfg.qk_nope_head_dim + cfg.v_head_dim))
        k_heads = expanded[..., :cfg.qk_nope_head_dim].float().permute(0, 2, 3, 1).contiguous()  # [B, H, nope, S]
        v_heads = expanded[..., cfg.qk_nope_head_dim:].float().permute(0, 2, 1, 3).contiguous()  # [B, H, S, v]
        # per-head content scores plus the shared positional scores
        scores = torch.matmul(q_nope.float().unsqueeze(2), k_heads).squeeze(2)  # [B, H, S]
        scores = scores + torch.matmul(q_pe.float(), shared_k.transpose(1, 2).contiguous())
        scores = scores * self.softmax_scale
        past_end = torch.arange(cache.shape[1], device=x.device).unsqueeze(0) >= seqlens.unsqueeze(1)
        scores = scores.masked_fill(past_end.unsqueeze(1), float("-inf"))
        weights = torch.softmax(scores, dim=-1)
        o = torch.matmul(weights.unsqueeze(2), v_heads).squeeze(2).to(x.dtype)  # [B, H, v]
        return self.wo(o.flatten(1)), seqlens
