"""Randomised shapes through the public ``mla_decode`` against the float64
oracle: 128 draws from a fixed seed of batch (1-12), heads (1-260: every
kernel and head-block form, partial head blocks), sequence lengths (empty,
one token, not multiples of the 32-token sub-tile or the 64-token tile, up to
3,000), dense or paged caches (pages of 16-256 tokens, shuffled tables with
spare columns), the balanced partition or 1-24 uniform splits, bf16 or fp16,
the single launch or two kernels. Each call is checked at the parity bar
(out atol = rtol = 1e-2, lse 1e-3 on non-empty rows, empty sequences exactly
0 and -inf) and against the other launch form bit for bit. The same draws
also run over an fp8 cache (against the fp8 oracle) and with 1-8 query
tokens per sequence (against the causal oracle), and at other power-of-two
head dims and fp32 (the generic decode).
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import bits, dtype_name

pytestmark = pytest.mark.gpu

D, DV = 576, 512


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    batch = int(rng.integers(1, 13))
    heads = int(rng.choice([1, 3, 8, 16, 17, 31, 32, 33, 48, 64, 65, 96, 127, 128, 129, 200, 256, 260]))
    max_len = int(rng.integers(1, 3001))
    lens = rng.integers(0, max_len + 1, size=batch)
    specials = [0, 1, max_len, 31, 33, 63, 65]
    for i in range(min(batch, int(rng.integers(0, 4)))):
        lens[i] = min(int(rng.choice(specials)), max_len)
    page = int(rng.choice([0, 16, 32, 64, 128, 256]))
    splits = None if rng.random() < 0.5 else int(rng.integers(1, 25))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    return batch, heads, max_len, lens.astype(np.int32), page, splits, dtype


@pytest.mark.parametrize("seed", range(128))
def test_random_shape(gpu, seed):
    import triton_mla

    batch, heads, max_len, lens, page, splits, dtype = _draw(seed)
    print(f"seed {seed}: batch={batch} heads={heads} max_len={max_len} page={page} splits={splits} "
          f"{dtype_name(dtype)}", flush=True)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, heads, D, generator=g).to(dtype)
    kv = torch.randn(batch, max_len, D, generator=g).to(dtype)
    bt = None
    if page:
        per_seq = -(-max_len // page) + 1  # one spare column per row
        blocks = batch * per_seq
        bt = torch.randperm(blocks, generator=g).view(batch, per_seq).int()
        padded = torch.zeros(batch, per_seq * page, D, dtype=dtype)
        padded[:, :max_len] = kv
        cache = torch.empty(blocks, page, D, dtype=dtype)
        cache[bt.long()] = padded.view(batch, per_seq, page, D)
    else:
        cache = kv
    seqlens = torch.from_numpy(lens)
    scale = 192 ** -0.5
    args = (q.to(gpu), cache.to(gpu), seqlens.to(gpu), None if bt is None else bt.to(gpu))
    two = triton_mla.mla_decode(*args, softmax_scale=scale, num_splits=splits, return_lse=True,
                                single_launch=False)
    one = triton_mla.mla_decode(*args, softmax_scale=scale, num_splits=splits, return_lse=True,
                                single_launch=True)
    torch.cuda.synchronize()
    assert torch.equal(two[0].view(torch.int16), one[0].view(torch.int16))
    assert torch.equal(two[1], one[1])
    ref_out, ref_lse = oracle.mla_decode_ref(bits(q), bits(cache), lens, None if bt is None else bt.numpy(), DV,
                                             scale, dtype=dtype_name(dtype))
    out, lse = two[0].float().cpu(), two[1].cpu()
    torch.testing.assert_close(out, torch.from_numpy(ref_out), atol=1e-2, rtol=1e-2)
    valid = torch.from_numpy(lens > 0)
    torch.testing.assert_close(lse[valid], torch.from_numpy(ref_lse)[valid], atol=1e-3, rtol=1e-3)
    assert torch.all(out[~valid] == 0) and torch.all(torch.isneginf(lse[~valid]))


def _paged_cache(kv, page, g):
    batch, max_len, _ = kv.shape
    per_seq = -(-max_len // page) + 1
    blocks = batch * per_seq
    bt = torch.randperm(blocks, generator=g).view(batch, per_seq).int()
    padded = torch.zeros(batch, per_seq * page, D, dtype=kv.dtype)
    padded[:, :max_len] = kv
    cache = torch.empty(blocks, page, D, dtype=kv.dtype)
    cache[bt.long()] = padded.view(batch, per_seq, page, D)
    return cache, bt


@pytest.mark.parametrize("seed", range(32))
def test_random_shape_fp8_cache(gpu, seed):
    """The same draws over an fp8 cache (scales per page, per token or per
    tensor), against the float64 fp8 oracle at the parity bar."""
    import triton_mla
    from triton_mla import quantize_kv_fp8

    batch, heads, max_len, lens, page, splits, dtype = _draw(500 + seed)
    gran = ("page", "token", "tensor")[seed % 3]
    print(f"fp8 seed {seed}: batch={batch} heads={heads} max_len={max_len} page={page} splits={splits} "
          f"{gran} {dtype_name(dtype)}", flush=True)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, heads, D, generator=g).to(dtype)
    kv = torch.randn(batch, max_len, D, generator=g).to(torch.bfloat16)
    bt = None
    if page:
        kv, bt = _paged_cache(kv, page, g)
    codes, scale = quantize_kv_fp8(kv, gran)
    sm = 192 ** -0.5
    out, lse = triton_mla.mla_decode(q.to(gpu), codes.to(gpu), torch.from_numpy(lens).to(gpu),
                                     None if bt is None else bt.to(gpu), softmax_scale=sm, num_splits=splits,
                                     return_lse=True, kv_scale=scale.to(gpu))
    torch.cuda.synchronize()
    ref_out, ref_lse = oracle.mla_decode_fp8_ref(bits(q), codes.view(torch.uint8).numpy(), scale.numpy(), lens,
                                                 None if bt is None else bt.numpy(), DV, sm, dtype=dtype_name(dtype))
    out, lse = out.float().cpu(), lse.cpu()
    torch.testing.assert_close(out, torch.from_numpy(ref_out), atol=1e-2, rtol=1e-2)
    valid = torch.from_numpy(lens > 0)
    torch.testing.assert_close(lse[valid], torch.from_numpy(ref_lse)[valid], atol=1e-3, rtol=1e-3)
    assert torch.all(out[~valid] == 0) and torch.all(torch.isneginf(lse[~valid]))


@pytest.mark.parametrize("seed", range(32))
def test_random_shape_multi_token(gpu, seed):
    """The same draws with 1-8 query tokens per sequence (causal over the new
    tokens), both launch forms bit-equal, against the float64 causal oracle."""
    import triton_mla

    batch, heads, max_len, lens, page, splits, dtype = _draw(900 + seed)
    q_len = 1 + seed % 8
    heads = max(1, min(heads, 512 // q_len))
    print(f"causal seed {seed}: batch={batch} q_len={q_len} heads={heads} max_len={max_len} page={page} "
          f"splits={splits} {dtype_name(dtype)}", flush=True)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, q_len, heads, D, generator=g).to(dtype)
    kv = torch.randn(batch, max_len, D, generator=g).to(dtype)
    bt = None
    if page:
        kv, bt = _paged_cache(kv, page, g)
    sm = 192 ** -0.5
    args = (q.to(gpu), kv.to(gpu), torch.from_numpy(lens).to(gpu), None if bt is None else bt.to(gpu))
    two = triton_mla.mla_decode(*args, softmax_scale=sm, num_splits=splits, return_lse=True, single_launch=False)
    one = triton_mla.mla_decode(*args, softmax_scale=sm, num_splits=splits, return_lse=True, single_launch=True)
    torch.cuda.synchronize()
    assert two[0].shape == (batch, q_len, heads, DV) and two[1].shape == (batch, q_len, heads)
    assert torch.equal(two[0].view(torch.int16), one[0].view(torch.int16)) and torch.equal(two[1], one[1])
    ref_out, ref_lse = oracle.mla_decode_ref_causal(bits(q), bits(kv), lens, None if bt is None else bt.numpy(),
                                                    DV, sm, dtype=dtype_name(dtype))
    out, lse = two[0].float().cpu(), two[1].cpu()
    torch.testing.assert_close(out, torch.from_numpy(ref_out), atol=1e-2, rtol=1e-2)
    seen = torch.from_numpy(lens[:, None] - (q_len - 1 - np.arange(q_len))[None, :] > 0)  # [B, T]
    seen = seen[:, :, None].expand(batch, q_len, heads)
    torch.testing.assert_close(lse[seen], torch.from_numpy(ref_lse)[seen], atol=1e-3, rtol=1e-3)
    assert torch.all(out[~seen] == 0) and torch.all(torch.isneginf(lse[~seen]))


@pytest.mark.parametrize("seed", range(32))
def test_random_shape_other_dims(gpu, seed):
    """Other head dims and fp32 (the generic decode, both of its forms): the
    same draws of batch, heads, lengths, paging and splits at random
    power-of-two dims, against the float64 oracle (fp32 at 1e-4)."""
    import triton_mla

    batch, heads, max_len, lens, page, splits, dtype = _draw(1300 + seed)
    rng = np.random.default_rng(1700 + seed)
    dv = int(rng.choice([16, 32, 64, 128, 256, 512, 1024]))
    dr = int(rng.choice([16, 32, 64, 128, 256]))
    if (dv, dr) == (512, 64) or seed % 4 == 0:
        dtype = torch.float32
    d = dv + dr
    name = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dtype]
    print(f"generic seed {seed}: batch={batch} heads={heads} max_len={max_len} page={page} splits={splits} "
          f"dims {dv}+{dr} {name}", flush=True)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, heads, d, generator=g).to(dtype)
    kv = torch.randn(batch, max_len, d, generator=g).to(dtype)
    bt = None
    if page:
        per_seq = -(-max_len // page) + 1
        blocks = batch * per_seq
        bt = torch.randperm(blocks, generator=g).view(batch, per_seq).int()
        padded = torch.zeros(batch, per_seq * page, d, dtype=dtype)
        padded[:, :max_len] = kv
        kv = torch.empty(blocks, page, d, dtype=dtype)
        kv[bt.long()] = padded.view(batch, per_seq, page, d)
    sm = d ** -0.5
    out, lse = triton_mla.mla_decode(q.to(gpu), kv.to(gpu), torch.from_numpy(lens).to(gpu),
                                     None if bt is None else bt.to(gpu), head_dim_v=dv, softmax_scale=sm,
                                     num_splits=splits, return_lse=True)
    torch.cuda.synchronize()
    as_o = (lambda t: t.contiguous().numpy()) if dtype == torch.float32 else bits
    ref_out, ref_lse = oracle.mla_decode_ref(as_o(q), as_o(kv), lens, None if bt is None else bt.numpy(), dv, sm,
                                             dtype=name)
    otol, ltol = (1e-4, 1e-4) if dtype == torch.float32 else (1e-2, 1e-3)
    out, lse = out.float().cpu(), lse.cpu()
    torch.testing.assert_close(out, torch.from_numpy(ref_out), atol=otol, rtol=otol)
    valid = torch.from_numpy(lens > 0)
    torch.testing.assert_close(lse[valid], torch.from_numpy(ref_lse)[valid], atol=ltol, rtol=ltol)
    assert torch.all(out[~valid] == 0) and torch.all(torch.isneginf(lse[~valid]))
