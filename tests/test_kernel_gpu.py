"""Parity of the HIP mla_decode with the CPU oracle (oracle/mla_oracle.c).

Shapes and draws follow the reference's tests (tests/test_kernel.py:29-61):
heads {16, 20, 128}, splits {1, 4, 16} plus the balanced default, dense and
paged caches, seqlens [0, 1, 513, 4096], scale 192**-0.5. Tolerances:
out atol = rtol = 1e-2 (bf16 and fp16, softmax in fp32), lse atol = rtol =
1e-3 on non-empty rows, out == 0 exactly for empty sequences, and bit-exact
block-table gathering (one-token sequences return the cached row itself).
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import bits, dtype_name

pytestmark = pytest.mark.gpu

D_LATENT, D_ROPE = 512, 64
SCALE = 192 ** -0.5
OUT_TOL = dict(atol=1e-2, rtol=1e-2)
LSE_TOL = dict(atol=1e-3, rtol=1e-3)


def make_paged(kv_dense, page_size, generator):
    """The reference tests' paging of a dense cache (tests/test_kernel.py:16-26)."""
    batch, max_len, d = kv_dense.shape
    blocks_per_seq = -(-max_len // page_size)
    num_blocks = batch * blocks_per_seq
    perm = torch.randperm(num_blocks, generator=generator)
    block_table = perm.view(batch, blocks_per_seq).int()
    padded = torch.zeros(batch, blocks_per_seq * page_size, d, dtype=kv_dense.dtype)
    padded[:, :max_len] = kv_dense
    kv_cache = torch.empty(num_blocks, page_size, d, dtype=kv_dense.dtype)
    kv_cache[block_table.long()] = padded.view(batch, blocks_per_seq, page_size, d)
    return kv_cache, block_table


def run_oracle(q, kv, seqlens, bt, scale, dtype):
    return oracle.mla_decode_ref(bits(q), bits(kv), seqlens.cpu().numpy(),
                                 None if bt is None else bt.cpu().numpy(), D_LATENT, scale,
                                 dtype=dtype_name(dtype))


def check(out, lse, ref_out, ref_lse, seqlens):
    import triton_mla  # noqa: F401

    out_f = out.float().cpu()
    torch.testing.assert_close(out_f, torch.from_numpy(ref_out), **OUT_TOL)
    valid = seqlens.cpu() > 0
    torch.testing.assert_close(lse.cpu()[valid], torch.from_numpy(ref_lse)[valid], **LSE_TOL)
    assert torch.all(out_f[~valid] == 0)
    assert torch.all(torch.isneginf(lse.cpu()[~valid]))


_case_cache = {}


def reference_case(num_heads, paged, dtype):
    key = (num_heads, paged, dtype)
    if key not in _case_cache:
        g = torch.Generator().manual_seed(0)
        seqlens = torch.tensor([0, 1, 513, 4096], dtype=torch.int32)
        batch, max_len = len(seqlens), int(seqlens.max())
        q = torch.randn(batch, num_heads, D_LATENT + D_ROPE, generator=g).to(dtype)
        kv = torch.randn(batch, max_len, D_LATENT + D_ROPE, generator=g).to(dtype)
        bt = None
        if paged:
            kv, bt = make_paged(kv, 64, g)
        ref = run_oracle(q, kv, seqlens, bt, SCALE, dtype)
        _case_cache[key] = (q, kv, seqlens, bt, ref)
    return _case_cache[key]


@pytest.mark.parametrize("num_heads", [16, 20, 128])
@pytest.mark.parametrize("num_splits", [None, 1, 4, 16])
@pytest.mark.parametrize("paged", [False, True])
def test_matches_oracle(gpu, num_heads, num_splits, paged):
    from triton_mla import mla_decode

    q, kv, seqlens, bt, (ref_out, ref_lse) = reference_case(num_heads, paged, torch.bfloat16)
    out, lse = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), None if bt is None else bt.to(gpu),
                          softmax_scale=SCALE, num_splits=num_splits, return_lse=True)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == (4, num_heads, D_LATENT)
    assert lse.dtype == torch.float32 and lse.shape == (4, num_heads)
    check(out, lse, ref_out, ref_lse, seqlens)


@pytest.mark.parametrize("num_heads", [20, 128])
@pytest.mark.parametrize("scale", [-SCALE, -1e-3, 3.0])
@pytest.mark.parametrize("paged", [False, True])
def test_scale_sign_and_size(gpu, num_heads, scale, paged):
    """Negative, tiny and large softmax scales (the reference takes any float,
    kernel.py:247-248) against the oracle: the 128-head kernel runs a negative
    scale on negated Q^T, the smaller head blocks take the max of -s."""
    from triton_mla import mla_decode

    q, kv, seqlens, bt, _ = reference_case(num_heads, paged, torch.bfloat16)
    ref_out, ref_lse = run_oracle(q, kv, seqlens, bt, scale, torch.bfloat16)
    out, lse = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), None if bt is None else bt.to(gpu),
                          softmax_scale=scale, return_lse=True)
    torch.cuda.synchronize()
    check(out, lse, ref_out, ref_lse, seqlens)


def test_default_splits_and_flashmla_layout(gpu):
    from triton_mla import mla_decode

    g = torch.Generator().manual_seed(1)
    seqlens = torch.tensor([50, 75], dtype=torch.int32)
    q = torch.randn(2, 16, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    kv = torch.randn(2, 80, 1, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    out = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu))  # default scale 576**-0.5
    ref_out, _ = oracle.mla_decode_ref(bits(q), bits(kv), seqlens.numpy(), None, D_LATENT, None)
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref_out), **OUT_TOL)


@pytest.mark.parametrize("num_splits", [None, 1, 3])
@pytest.mark.parametrize("page_size", [16, 48, 64, 128])
def test_gather_is_bit_exact(gpu, num_splits, page_size):
    """seqlen 1: softmax weight is exactly 1, so out must equal the cached row bit for bit."""
    from triton_mla import mla_decode

    g = torch.Generator().manual_seed(2)
    batch, pages_per_seq, heads = 6, 3, 32
    num_pages = batch * pages_per_seq + 5
    kv = torch.randn(num_pages, page_size, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    bt = torch.randperm(num_pages, generator=g)[: batch * pages_per_seq].view(batch, pages_per_seq).int()
    q = torch.randn(batch, heads, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    seqlens = torch.ones(batch, dtype=torch.int32)
    out = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE,
                     num_splits=num_splits).cpu()
    gathered = torch.from_numpy(oracle.gather_kv(bits(kv), seqlens.numpy(), bt.numpy(), n_tokens=1)
                                .view(np.int16)).view(torch.bfloat16)
    expect = gathered[:, 0, :D_LATENT][:, None, :].expand(batch, heads, D_LATENT)
    assert torch.equal(out.view(torch.int16), expect.contiguous().view(torch.int16))


@pytest.mark.parametrize("page_size", [16, 32, 48, 128])
def test_page_sizes(gpu, page_size):
    from triton_mla import mla_decode

    g = torch.Generator().manual_seed(3)
    seqlens = torch.tensor([7, 300, 1000, 64], dtype=torch.int32)
    batch, max_len = len(seqlens), int(seqlens.max())
    q = torch.randn(batch, 128, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    kv = torch.randn(batch, max_len, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    kv, bt = make_paged(kv, page_size, g)
    ref_out, ref_lse = run_oracle(q, kv, seqlens, bt, SCALE, torch.bfloat16)
    for splits in (None, 2):
        out, lse = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE,
                              num_splits=splits, return_lse=True)
        check(out, lse, ref_out, ref_lse, seqlens)


@pytest.mark.parametrize("paged", [False, True])
def test_fp16(gpu, paged):
    from triton_mla import mla_decode

    q, kv, seqlens, bt, (ref_out, ref_lse) = reference_case(128, paged, torch.float16)
    out, lse = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), None if bt is None else bt.to(gpu),
                          softmax_scale=SCALE, return_lse=True)
    assert out.dtype == torch.float16
    check(out, lse, ref_out, ref_lse, seqlens)


def test_large_scores_exercise_rescale(gpu):
    """Scores spanning hundreds of units force the running max to move many times."""
    from triton_mla import mla_decode

    g = torch.Generator().manual_seed(4)
    seqlens = torch.tensor([2000, 333, 4097], dtype=torch.int32)
    batch, max_len = 3, 4097
    q = (torch.randn(batch, 128, D_LATENT + D_ROPE, generator=g) * 4).to(torch.bfloat16)
    # keys whose norm grows along the sequence: later tokens dominate by far
    ramp = torch.linspace(0.2, 3.0, max_len)[None, :, None]
    kv = (torch.randn(batch, max_len, D_LATENT + D_ROPE, generator=g) * ramp).to(torch.bfloat16)
    kv, bt = make_paged(kv, 64, g)
    ref_out, ref_lse = run_oracle(q, kv, seqlens, bt, SCALE, torch.bfloat16)
    for splits in (None, 1, 5):
        out, lse = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE,
                              num_splits=splits, return_lse=True)
        check(out, lse, ref_out, ref_lse, seqlens)


def test_rows_past_seqlen_are_never_read(gpu):
    """NaN in cache rows past each sequence's end must not reach the output."""
    from triton_mla import mla_decode

    g = torch.Generator().manual_seed(5)
    seqlens = torch.tensor([1, 70, 129, 31], dtype=torch.int32)
    batch, pages_per_seq = 4, 3
    kv = torch.randn(batch * pages_per_seq, 64, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    bt = torch.randperm(batch * pages_per_seq, generator=g).view(batch, pages_per_seq).int()
    for b in range(batch):
        for t in range(int(seqlens[b]), pages_per_seq * 64):
            kv[bt[b, t // 64], t % 64] = float("nan")
    q = torch.randn(batch, 128, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    ref_out, ref_lse = run_oracle(q, kv, seqlens, bt, SCALE, torch.bfloat16)
    for splits in (None, 1, 2):
        out, lse = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE,
                              num_splits=splits, return_lse=True)
        assert torch.isfinite(out.float()).all()
        check(out, lse, ref_out, ref_lse, seqlens)


def test_empty_inputs(gpu):
    from triton_mla import mla_decode

    q = torch.randn(0, 128, 576, device=gpu).to(torch.bfloat16)
    kv = torch.randn(4, 64, 576, device=gpu).to(torch.bfloat16)
    out, lse = mla_decode(q, kv, torch.zeros(0, dtype=torch.int32, device=gpu),
                          torch.zeros(0, 1, dtype=torch.int32, device=gpu), return_lse=True)
    assert out.shape == (0, 128, 512) and lse.shape == (0, 128)
    # all sequences empty
    q = torch.randn(3, 128, 576, device=gpu).to(torch.bfloat16)
    bt = torch.zeros(3, 1, dtype=torch.int32, device=gpu)
    for splits in (None, 1, 4):
        out, lse = mla_decode(q, kv, torch.zeros(3, dtype=torch.int32, device=gpu), bt,
                              num_splits=splits, return_lse=True)
        assert torch.all(out == 0) and torch.all(torch.isneginf(lse))


def test_split_invariance(gpu):
    """Any split count gives the same result to within rounding: split
    partials are stored in the input dtype, so a split result carries one more
    bf16 rounding (2^-9 relative per partial) than the unsplit one."""
    from triton_mla import mla_decode

    q, kv, seqlens, bt, _ = reference_case(128, True, torch.bfloat16)
    args = (q.to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu))
    base, base_lse = mla_decode(*args, softmax_scale=SCALE, num_splits=1, return_lse=True)
    for splits in (None, 2, 3, 7, 32, 64):
        out, lse = mla_decode(*args, softmax_scale=SCALE, num_splits=splits, return_lse=True)
        torch.testing.assert_close(out.float(), base.float(), atol=1e-2, rtol=1e-2)
        valid = seqlens.to(gpu) > 0
        torch.testing.assert_close(lse[valid], base_lse[valid], atol=1e-4, rtol=1e-5)
