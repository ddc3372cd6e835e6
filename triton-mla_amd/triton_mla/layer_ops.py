"""HIP glue of the absorbed MLA decode step (the C ABI's tmla_mla_absorb_q,
tmla_mla_kv_append, tmla_mla_absorb_out and tmla_mla_project).

These replace the torch steps of the reference layer around ``mla_decode``
(src/triton_mla/model.py:74-124): the RoPE of q_pe and k_pe (model.py:44-50),
the RMSNorm of the latent (model.py:34-41), the cache append
(model.py:86-94), the W_UK / W_UV einsums and, for a step's few rows, the
dense projections (model.py:66-72). Tensors stay on the GPU; there is no
torch fallback inside these functions (``project_fits`` tells the layer when
a projection is one the kernel takes).
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


PROJECT_MAX_ROWS = 64  # rows of x tmla_mla_project takes
# Where the kernel beats the library GEMM (measured at DeepSeek-V3 dims, 16
# rows, one MI355X): wide weights (wq_b 24576 x 1536: 19.8 vs 30.0 us; wo
# 7168 x 16384: 49.7 vs 49.2 us). Narrower ones leave it too few column
# groups, and the contraction split it then needs costs more than the
# library's time (wq_a 1536 x 7168: 17.9 vs 14.2 us; wkv_a 576 x 7168: 16.9
# vs 13.7 us); more rows make its x reads as large as its weight reads
# (wq_b at 64 rows: 33.4 vs 21.4 us).
PROJECT_PAYS_ROWS = 16
PROJECT_PAYS_COLUMNS = 4096


def norm_append(q_lat, q_norm_weight, q_eps, kv_proj, kv_norm_weight, kv_eps, rope_theta, positions, kv_cache,
                block_table, kv_lora_rank, rope_dim):
    """rms_norm(q_lat) and kv_append(kv_proj, ...) of one step in one launch
    (tmla_mla_norm_append, the same bits as the two calls). Returns the
    normalised query latent and positions + 1 (int32, the sequence lengths
    after the step)."""
    dev = _check_gpu(q_lat, kv_proj, kv_cache)
    assert q_lat.dim() == 2 and q_lat.stride(1) == 1 and q_lat.dtype == kv_proj.dtype
    assert kv_proj.dtype == kv_cache.dtype and kv_proj.stride(-1) == 1 and kv_cache.stride(-1) == 1
    if kv_cache.dim() == 4:  # FlashMLA layout [..., 1, D]
        kv_cache = kv_cache.squeeze(2)
    batch, q_dim = q_lat.shape
    assert kv_proj.shape[0] == batch
    assert kv_proj.shape[1] == kv_lora_rank + rope_dim and kv_cache.shape[-1] == kv_lora_rank + rope_dim
    positions = positions.to(device=dev, dtype=torch.int32).contiguous()
    if q_norm_weight is not None:
        q_norm_weight = q_norm_weight.to(device=dev, dtype=q_lat.dtype).contiguous()
    if kv_norm_weight is not None:
        kv_norm_weight = kv_norm_weight.to(kv_proj.dtype).contiguous()
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
    q_out = torch.empty(batch, q_dim, dtype=q_lat.dtype, device=dev)
    next_positions = torch.empty(batch, dtype=torch.int32, device=dev)
    lib = _native.load()
    with torch.cuda.device(dev):
        _native.check(lib.tmla_mla_norm_append(
            q_lat.data_ptr(), q_lat.stride(0), None if q_norm_weight is None else q_norm_weight.data_ptr(),
            float(q_eps), q_dim, q_out.data_ptr(), q_out.stride(0),
            kv_proj.data_ptr(), kv_proj.stride(0), None if kv_norm_weight is None else kv_norm_weight.data_ptr(),
            float(kv_eps), float(rope_theta), positions.data_ptr(), next_positions.data_ptr(), batch, kv_lora_rank,
            rope_dim, _native.DTYPE_CODE[kv_proj.dtype], kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1),
            num_blocks, page_size, *bt, _stream(dev)), "tmla_mla_norm_append")
    return q_out, next_positions


def rms_norm(x, weight, eps):
    """RMSNorm of the rows of a 2-D x (model.py:34-41): float32, the
    normalised value times the weight rounded once (tmla_mla_rms_norm)."""
    dev = _check_gpu(x)
    assert x.dim() == 2 and x.stride(1) == 1
    rows, dim = x.shape
    if weight is not None:
        weight = weight.to(device=dev, dtype=x.dtype).contiguous()
    y = torch.empty(rows, dim, dtype=x.dtype, device=dev)
    lib = _native.load()
    with torch.cuda.device(dev):
        _native.check(lib.tmla_mla_rms_norm(
            x.data_ptr(), x.stride(0), None if weight is None else weight.data_ptr(), float(eps), rows, dim,
            _native.DTYPE_CODE[x.dtype], y.data_ptr(), y.stride(0), _stream(dev)), "tmla_mla_rms_norm")
    return y


def project_pays(x, weight):
    """Whether the layer should run y = x . weight^T with tmla_mla_project
    rather than the library GEMM (the measurements above)."""
    return (project_fits(x, weight) and x.shape[0] <= PROJECT_PAYS_ROWS
            and weight.shape[0] >= PROJECT_PAYS_COLUMNS)


def project_fits(x, weight):
    """Whether tmla_mla_project takes y = x . weight^T: a 2-D 16-bit x of at
    most 64 rows, weight [N, K] of the same dtype with N a multiple of 16,
    K a multiple of 64, both with unit element stride and 16-byte aligned
    rows."""
    if x.dim() != 2 or weight.dim() != 2 or x.dtype not in _DTYPES or weight.dtype != x.dtype:
        return False
    if x.device.type != "cuda" or weight.device != x.device:
        return False
    m, k = x.shape
    n = weight.shape[0]
    if not (0 < m <= PROJECT_MAX_ROWS and weight.shape[1] == k and n % 16 == 0 and k % 64 == 0):
        return False
    if x.stride(1) != 1 or weight.stride(1) != 1 or x.stride(0) % 8 or weight.stride(0) % 8:
        return False
    return x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0


# (device index, stream) -> zero-filled workspace of the split contractions
_project_ws = {}
# workspaces replaced by larger ones: never freed, since graphs captured
# while they were current still read and write them
_project_retired = []
_PROJECT_COUNTER_BYTES = 64 * 1024  # the counter block at the workspace's start


def _project_workspace(dev, stream, nbytes):
    """A workspace of at least nbytes whose counter block is zero, for a
    projection on ``stream`` of ``dev``.

    Eager calls keep one per (device, stream), zero-filled once: every call
    leaves its counters at zero again, and calls on one stream run in order,
    so the next call finds them cleared. A larger need replaces it with a
    larger one. Under graph capture the stream's kept workspace is used when
    there is one large enough (the graph then shares it: replay such a graph
    on the stream it was captured on). Otherwise the captured call gets a
    workspace of its own from the graph's memory, its counters cleared by a
    fill kernel inside the graph: memory allocated during capture holds
    nothing until the graph replays, so no eager call may find it."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, stream)
    buf = _project_ws.get(key)
    if buf is not None and buf.numel() >= nbytes:
        return buf
    if torch.cuda.is_current_stream_capturing():
        buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        buf[:min(nbytes, _PROJECT_COUNTER_BYTES)].zero_()
        return buf
    if buf is not None:
        _project_retired.append(buf)
    buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
    _project_ws[key] = buf
    return buf


def project(x, weight):
    """y [M, N] = x [M, K] . weight [N, K]^T (nn.Linear without bias) for a
    decode step's rows (model.py:66-82, 124): float32 accumulation in a fixed
    order, rounded once to the dtype."""
    dev = _check_gpu(x, weight)
    if not project_fits(x, weight):
        raise NotImplementedError("tmla_mla_project takes <= 64 rows, N % 16 == 0, K % 64 == 0, 16-byte aligned rows")
    m, k = x.shape
    n = weight.shape[0]
    y = torch.empty(m, n, dtype=x.dtype, device=dev)
    lib = _native.load()
    need = lib.tmla_mla_project_workspace_bytes(m, n, k)
    with torch.cuda.device(dev):
        stream = _stream(dev)
        ws = _project_workspace(dev, stream, need) if need else None
        _native.check(lib.tmla_mla_project(
            x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), m, n, k, _native.DTYPE_CODE[x.dtype],
            y.data_ptr(), y.stride(0), None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
            stream), "tmla_mla_project")
    return y
