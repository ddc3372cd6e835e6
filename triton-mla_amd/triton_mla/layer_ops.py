"""HIP glue of the absorbed MLA decode step (the C ABI's tmla_mla_absorb_q,
tmla_mla_kv_append and tmla_mla_absorb_out).

These replace the torch steps of the reference layer around ``mla_decode``
(src/triton_mla/model.py:74-124): the RoPE of q_pe and k_pe (model.py:44-50),
the RMSNorm of the latent (model.py:34-41), the cache append
(model.py:86-94) and the W_UK / W_UV einsums. Tensors stay on the GPU; there
is no torch fallback.
"""

from __future__ import annotations

import torch

from . import _native

_DTYPES = (torch.bfloat16, torch.float16)


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _check_gpu(*tensors):
    dev = tensors[0].device
    if dev.type != "cuda" or any(t.device != dev for t in tensors):
        raise RuntimeError("triton_mla layer ops run on the GPU only: all tensors on one HIP device")
    if tensors[0].dtype not in _DTYPES:
        raise NotImplementedError(f"layer ops support bf16 and fp16, got {tensors[0].dtype}")
    return dev


def absorb_q(q_proj, wkv_b, positions, num_heads, qk_nope_dim, qk_rope_dim, kv_lora_rank, v_head_dim,
             rope_theta):
    """[B, H*(nope+rope)] wq_b output -> [B, H, rank+rope]: W_UK-absorbed
    nope query and rotated q_pe (model.py:74-83, 108-109)."""
    dev = _check_gpu(q_proj, wkv_b)
    assert q_proj.dtype == wkv_b.dtype and q_proj.stride(-1) == 1 and wkv_b.stride(-1) == 1
    batch = q_proj.shape[0]
    assert q_proj.shape[1] == num_heads * (qk_nope_dim + qk_rope_dim)
    assert wkv_b.shape == (num_heads * (qk_nope_dim + v_head_dim), kv_lora_rank)
    positions = positions.to(device=dev, dtype=torch.int32).contiguous()
    out = torch.empty(batch, num_heads, kv_lora_rank + qk_rope_dim, dtype=q_proj.dtype, device=dev)
    lib = _native.load()
    with torch.cuda.device(dev):
        _native.check(lib.tmla_mla_absorb_q(
            q_proj.data_ptr(), q_proj.stride(0), wkv_b.data_ptr(), wkv_b.stride(0), positions.data_ptr(), batch,
            num_heads, qk_nope_dim, qk_rope_dim, kv_lora_rank, v_head_dim, float(rope_theta),
            _native.DTYPE_CODE[q_proj.dtype], out.data_ptr(), out.stride(0), out.stride(1), _stream(dev)),
            "tmla_mla_absorb_q")
    return out


def absorb_out(o_latent, wkv_b, num_heads, qk_nope_dim, kv_lora_rank, v_head_dim):
    """[B, H, rank] attention output -> [B, H*v] (W_UV, model.py:120-124)."""
    dev = _check_gpu(o_latent, wkv_b)
    assert o_latent.dtype == wkv_b.dtype and o_latent.stride(-1) == 1 and wkv_b.stride(-1) == 1
    batch = o_latent.shape[0]
    assert o_latent.shape[1:] == (num_heads, kv_lora_rank)
    out = torch.empty(batch, num_heads * v_head_dim, dtype=o_latent.dtype, device=dev)
    lib = _native.load()
    with torch.cuda.device(dev):
        _native.check(lib.tmla_mla_absorb_out(
            o_latent.data_ptr(), o_latent.stride(0), o_latent.stride(1), wkv_b.data_ptr(), wkv_b.stride(0), batch,
            num_heads, qk_nope_dim, kv_lora_rank, v_head_dim, _native.DTYPE_CODE[o_latent.dtype], out.data_ptr(),
            out.stride(0), _stream(dev)), "tmla_mla_absorb_out")
    return out


def kv_append(kv_proj, norm_weight, eps, rope_theta, positions, kv_cache, block_table, kv_lora_rank, rope_dim):
    """RMSNorm(latent) * weight and RoPE(k_pe) of wkv_a's output [B, rank+rope],
    written in place at row positions[b] of each sequence (model.py:80-94)."""
    dev = _check_gpu(kv_proj, kv_cache)
    assert kv_proj.dtype == kv_cache.dtype and kv_proj.stride(-1) == 1 and kv_cache.stride(-1) == 1
    if kv_cache.dim() == 4:  # FlashMLA layout [..., 1, D]
        kv_cache = kv_cache.squeeze(2)
    batch = kv_proj.shape[0]
    assert kv_proj.shape[1] == kv_lora_rank + rope_dim and kv_cache.shape[-1] == kv_lora_rank + rope_dim
    positions = positions.to(device=dev, dtype=torch.int32).contiguous()
    if norm_weight is not None:
        norm_weight = norm_weight.to(kv_proj.dtype).contiguous()
    if block_table is not None:
        block_table = block_table.to(device=dev, dtype=torch.int32)
        if block_table.stride(-1) != 1:
            block_table = block_table.contiguous()
        bt = (block_table.data_ptr(), block_table.stride(0), block_table.shape[1])
        num_blocks, page_size = kv_cache.shape[0], kv_cache.shape[1]
    else:
        assert kv_cache.shape[0] == batch
        bt = (None, 0, 1)
        num_blocks, page_size = kv_cache.shape[1], 1
    lib = _native.load()
    with torch.cuda.device(dev):
        _native.check(lib.tmla_mla_kv_append(
            kv_proj.data_ptr(), kv_proj.stride(0), None if norm_weight is None else norm_weight.data_ptr(),
            float(eps), float(rope_theta), positions.data_ptr(), batch, kv_lora_rank, rope_dim,
            _native.DTYPE_CODE[kv_proj.dtype], kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1),
            num_blocks, page_size, *bt, _stream(dev)), "tmla_mla_kv_append")
    return kv_cache
