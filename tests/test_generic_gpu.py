"""The generic decode (tmla_mla_decode_generic): head dims and element types
the matrix-core kernels are not built for, reached through the public
``mla_decode`` like the reference's kernels (any power-of-two head_dim_v and
rope_dim, any dtype q and the cache share: src/triton_mla/kernel.py:243-245).

Checked against the float64 oracle (oracle/mla_oracle.c, whose float32
element path and other dims are pinned in tests/test_oracle.py) on the
reference tests' draws (tests/test_kernel.py:29-61: dense and paged caches,
empty and one-token sequences, uniform split counts and the default):
out atol = rtol = 1e-2 for bf16 / fp16, 1e-4 for fp32 (the reference tests'
fp32 tolerance, tests/test_kernel.py:12-13); lse 1e-3 / 1e-4 on non-empty
rows; out == 0 and lse == -inf exactly for empty sequences; one-token
sequences return the cached latent row itself (bit-exact gather through the
block table). Also: the element-load path for cache rows that do not start
on 16-byte boundaries, split-count invariance, and the generic kernels
against the matrix-core decode at 512 + 64 in bf16 (through the C ABI). bf16 and
fp16 calls with head_dim_v <= 512 and D <= 576 run the generic kernels'
matrix-core form, the others (and fp32) the vector-ALU form; the cases cover
both forms in both 16-bit types.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import bits

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (1e-2, 1e-3), torch.float16: (1e-2, 1e-3), torch.float32: (1e-4, 1e-4)}
NAME = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def _as_oracle(t):
    return t.detach().cpu().contiguous().numpy() if t.dtype == torch.float32 else bits(t)


def _paged(kv_dense, page_size, g):
    batch, max_len, d = kv_dense.shape
    per_seq = -(-max_len // page_size)
    blocks = batch * per_seq
    table = torch.randperm(blocks, generator=g).view(batch, per_seq).int()
    padded = torch.zeros(batch, per_seq * page_size, d, dtype=kv_dense.dtype)
    padded[:, :max_len] = kv_dense
    cache = torch.empty(blocks, page_size, d, dtype=kv_dense.dtype)
    cache[table.long()] = padded.view(batch, per_seq, page_size, d)
    return cache, table


def _check(out, lse, q, kv, seqlens, bt, dv, scale, dtype):
    ref_out, ref_lse = oracle.mla_decode_ref(_as_oracle(q), _as_oracle(kv), seqlens.numpy(),
                                             None if bt is None else bt.numpy(), dv, scale, dtype=NAME[dtype])
    otol, ltol = TOL[dtype]
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref_out), atol=otol, rtol=otol)
    valid = seqlens > 0
    torch.testing.assert_close(lse.cpu()[valid], torch.from_numpy(ref_lse)[valid], atol=ltol, rtol=ltol)
    assert torch.all(out.cpu()[~valid] == 0) and torch.all(torch.isneginf(lse.cpu()[~valid]))


CASES = [  # head_dim_v, rope_dim, dtype, heads, page size (0: dense), num_splits
    (16, 16, torch.bfloat16, 16, 0, None),
    (32, 16, torch.float16, 20, 16, 3),
    (64, 32, torch.float32, 16, 0, 4),
    (128, 64, torch.bfloat16, 20, 64, None),
    (128, 32, torch.float32, 1, 16, 1),
    (256, 16, torch.float16, 17, 0, 7),
    (256, 256, torch.bfloat16, 16, 64, 2),
    (512, 64, torch.float32, 16, 64, None),
    (512, 128, torch.bfloat16, 33, 0, 5),
    (512, 16, torch.float16, 16, 16, 16),
    (1024, 64, torch.bfloat16, 16, 64, 3),
    (1024, 256, torch.float32, 16, 0, 2),
    (1024, 16, torch.float16, 16, 16, 4),
    (256, 32, torch.float16, 65, 64, None),
    (64, 16, torch.bfloat16, 130, 32, 2),
]


@pytest.mark.parametrize("dv,dr,dtype,heads,page,splits", CASES)
def test_generic_matches_oracle(gpu, dv, dr, dtype, heads, page, splits):
    import triton_mla

    g = torch.Generator().manual_seed(dv * 7 + dr + heads)
    seqlens = torch.tensor([0, 1, 37, 300, 1000], dtype=torch.int32)
    max_len = 1000
    q = torch.randn(5, heads, dv + dr, generator=g).to(dtype)
    kv = torch.randn(5, max_len, dv + dr, generator=g).to(dtype)
    bt = None
    if page:
        kv, bt = _paged(kv, page, g)
    scale = (dv + dr) ** -0.5
    print(f"generic dv={dv} dr={dr} {NAME[dtype]} heads={heads} page={page} splits={splits}", flush=True)
    out, lse = triton_mla.mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), None if bt is None else bt.to(gpu),
                                     head_dim_v=dv, softmax_scale=scale, num_splits=splits, return_lse=True)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (5, heads, dv) and lse.dtype == torch.float32
    _check(out, lse, q, kv, seqlens, bt, dv, scale, dtype)
    # a one-token sequence attends to one row: its latent part, bit for bit
    row = kv[1, 0] if bt is None else kv[bt[1, 0].long(), 0]
    assert torch.equal(out[1].cpu(), row[:dv].expand(heads, dv))


def test_generic_default_scale_and_flashmla_layout(gpu):
    """The reference test's second case (tests/test_kernel.py:54-61) at 128 + 32 in fp32:
    default split count and scale, the [..., 1, D] cache layout."""
    import triton_mla

    g = torch.Generator().manual_seed(3)
    seqlens = torch.tensor([50, 75], dtype=torch.int32)
    q = torch.randn(2, 16, 160, generator=g)
    kv = torch.randn(2, 80, 1, 160, generator=g)
    out, lse = triton_mla.mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), head_dim_v=128, return_lse=True)
    torch.cuda.synchronize()
    _check(out, lse, q, kv.squeeze(2), seqlens, None, 128, 160 ** -0.5, torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_generic_unaligned_rows_and_split_invariance(gpu, dtype):
    """Cache rows one element off 16-byte boundaries take the vector-ALU form's
    element loads (bf16 aligned rows take the matrix-core form); results agree
    with the aligned copy and across split counts."""
    import triton_mla

    g = torch.Generator().manual_seed(5)
    dv, d = 128, 160
    seqlens = torch.tensor([513, 64, 0, 200], dtype=torch.int32)
    q = torch.randn(4, 16, d, generator=g).to(dtype).to(gpu)
    base = torch.randn(4, 520, d + 1, generator=g).to(dtype).to(gpu)
    kv_odd = base[..., 1:]  # rows at an odd element offset
    assert (kv_odd.data_ptr() % 16) != 0 and kv_odd.stride(-1) == 1
    kv = kv_odd.contiguous()
    sl = seqlens.to(gpu)
    a = triton_mla.mla_decode(q, kv_odd, sl, head_dim_v=dv, num_splits=3, return_lse=True)
    b = triton_mla.mla_decode(q, kv, sl, head_dim_v=dv, num_splits=3, return_lse=True)
    c = triton_mla.mla_decode(q, kv, sl, head_dim_v=dv, num_splits=1, return_lse=True)
    torch.cuda.synchronize()
    otol, ltol = TOL[dtype]
    if dtype == torch.float32:  # both on the vector ALU: the same bits
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    else:  # unaligned rows take the vector-ALU form, aligned ones the matrix-core form
        torch.testing.assert_close(a[0].float(), b[0].float(), atol=otol, rtol=otol)
    torch.testing.assert_close(b[0].float(), c[0].float(), atol=otol, rtol=otol)
    _check(a[0], a[1], q.cpu(), kv.cpu(), seqlens, None, dv, d ** -0.5, dtype)


def test_generic_kernels_agree_with_matrix_core_decode(gpu):
    """At 512 + 64 in bf16 both implementations apply: the generic kernels
    (through the C ABI) and the public decode agree within the bf16
    tolerance, and both with the oracle."""
    import triton_mla
    from triton_mla import _native

    lib = _native.load()
    g = torch.Generator().manual_seed(9)
    seqlens = torch.tensor([0, 1, 513, 4096], dtype=torch.int32)
    q = torch.randn(4, 20, 576, generator=g).to(torch.bfloat16)
    kv = torch.randn(4, 4096, 576, generator=g).to(torch.bfloat16)
    kvp, bt = _paged(kv, 64, g)
    qd, kvd, btd, sd = q.to(gpu), kvp.to(gpu), bt.to(gpu), seqlens.to(gpu)
    splits = 4
    out = torch.empty(4, 20, 512, dtype=torch.bfloat16, device=gpu)
    lse = torch.empty(4, 20, dtype=torch.float32, device=gpu)
    wsb = lib.tmla_generic_workspace_bytes(4, 20, 512, splits)
    ws = torch.empty(wsb, dtype=torch.uint8, device=gpu)
    scale = 192 ** -0.5
    _native.check(lib.tmla_mla_decode_generic(
        qd.data_ptr(), qd.stride(0), qd.stride(1), kvd.data_ptr(), kvd.stride(0), kvd.stride(1), kvd.shape[0], 64,
        btd.data_ptr(), btd.stride(0), btd.shape[1], sd.data_ptr(), 4, 20, 512, 64, 0, scale, splits,
        out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(), ws.data_ptr(), wsb,
        torch.cuda.current_stream().cuda_stream), "tmla_mla_decode_generic")
    ref_out, ref_lse = triton_mla.mla_decode(qd, kvd, sd, btd, softmax_scale=scale, num_splits=splits,
                                             return_lse=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.float(), ref_out.float(), atol=1e-2, rtol=1e-2)
    valid = (seqlens > 0).to(gpu)
    torch.testing.assert_close(lse[valid], ref_lse[valid], atol=1e-3, rtol=1e-3)
    _check(out, lse, q, kvp, seqlens, bt, 512, scale, torch.bfloat16)
