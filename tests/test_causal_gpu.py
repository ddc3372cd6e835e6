"""Multi-token (causal) queries through the HIP kernels: q [B, T, H, 576].

An extension with no counterpart in the reference (its mla_decode takes one
query token, src/triton_mla/kernel.py:238): query token t of sequence b sees
the first cache_seqlens[b] - (T - 1 - t) cached tokens. Checked against the
float64 oracle (oracle.mla_decode_ref_causal) to the single-token bar: out
atol = rtol = 1e-2, lse atol = rtol = 1e-3 on rows that see at least one token,
out == 0 and lse == -inf on rows that see none. Bit-exact checks: T = 1 equals
the 3-D call, and with 128 heads the last query token (which sees the whole
cache, in a workgroup of its own) equals the single-token call on its row.
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


def paged_case(seed, seqlens, q_len, heads, page=64, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    seqlens = torch.tensor(seqlens, dtype=torch.int32)
    batch = len(seqlens)
    per_seq = max(1, -(-int(seqlens.max()) // page))
    q = torch.randn(batch, q_len, heads, D_LATENT + D_ROPE, generator=g).to(dtype)
    kv = torch.randn(batch * per_seq, page, D_LATENT + D_ROPE, generator=g).to(dtype)
    bt = torch.randperm(batch * per_seq, generator=g).view(batch, per_seq).int()
    return q, kv, seqlens, bt


def check_causal(out, lse, q, kv, seqlens, bt, dtype=torch.bfloat16):
    ref_out, ref_lse = oracle.mla_decode_ref_causal(bits(q), bits(kv), seqlens.numpy(), bt.numpy(), D_LATENT,
                                                    SCALE, dtype=dtype_name(dtype))
    T = q.shape[1]
    seen = (seqlens[:, None] - (T - 1 - torch.arange(T))[None, :]) > 0  # [B, T]
    out_f, lse_c = out.float().cpu(), lse.cpu()
    torch.testing.assert_close(out_f, torch.from_numpy(ref_out), **OUT_TOL)
    torch.testing.assert_close(lse_c[seen], torch.from_numpy(ref_lse)[seen], **LSE_TOL)
    assert torch.all(out_f[~seen] == 0)
    assert torch.all(torch.isneginf(lse_c[~seen]))


@pytest.mark.parametrize("heads", [16, 128])
@pytest.mark.parametrize("q_len", [2, 4])
@pytest.mark.parametrize("num_splits", [None, 3])
@pytest.mark.parametrize("single_launch", [False, True])
def test_causal_matches_oracle(gpu, heads, q_len, num_splits, single_launch):
    from triton_mla import mla_decode

    print(f"causal heads={heads} q_len={q_len} splits={num_splits} single={single_launch}", flush=True)
    # lengths below q_len (some query tokens see nothing), around the 32-token
    # sub-tile and 64-token tile edges, and long enough to be split
    q, kv, seqlens, bt = paged_case(1, [0, 1, 3, 33, 64, 65, 700, 2049], q_len, heads)
    out, lse = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE,
                          num_splits=num_splits, return_lse=True, single_launch=single_launch)
    torch.cuda.synchronize()
    assert out.shape == (len(seqlens), q_len, heads, D_LATENT) and lse.shape == (len(seqlens), q_len, heads)
    check_causal(out, lse, q, kv, seqlens, bt)


def test_causal_one_token_equals_single_token_call(gpu):
    from triton_mla import mla_decode

    q, kv, seqlens, bt = paged_case(2, [5, 100, 1500], 1, 128)
    a = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE, return_lse=True)
    b = mla_decode(q[:, 0].to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE, return_lse=True)
    assert torch.equal(a[0][:, 0], b[0]) and torch.equal(a[1][:, 0], b[1])


@pytest.mark.parametrize("q_len", [2, 3])
def test_causal_last_token_bit_exact(gpu, q_len):
    """With 128 heads each query token has a workgroup row of its own, and the
    last one sees every cached token: it is exactly the single-token decode."""
    from triton_mla import mla_decode

    q, kv, seqlens, bt = paged_case(3, [4100, 63, 900, 8192], q_len, 128)
    for splits in (None, 4):
        out, lse = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE,
                              num_splits=splits, return_lse=True)
        o1, l1 = mla_decode(q[:, -1].to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE,
                            num_splits=splits, return_lse=True)
        assert torch.equal(out[:, -1], o1) and torch.equal(lse[:, -1], l1)


def test_causal_fp16_and_noncontiguous(gpu):
    from triton_mla import mla_decode

    q, kv, seqlens, bt = paged_case(4, [1, 77, 1030], 3, 20, dtype=torch.float16)
    # heads-major storage: the token and head dims are not packed, so the
    # host packs them before the launch
    q_t = q.transpose(1, 2).contiguous().transpose(1, 2)
    out, lse = mla_decode(q_t.to(gpu), kv.to(gpu), seqlens.to(gpu), bt.to(gpu), softmax_scale=SCALE,
                          return_lse=True)
    torch.cuda.synchronize()
    check_causal(out, lse, q, kv, seqlens, bt, dtype=torch.float16)


@pytest.mark.parametrize("page", [None, 16, 48])
def test_causal_dense_and_small_pages(gpu, page):
    """Dense cache (page size 1 in the kernel) and pages that are not whole
    32-token sub-tiles (per-row page lookups) under the causal mask."""
    from triton_mla import mla_decode

    T, H = 3, 32
    seqlens = torch.tensor([2, 40, 97, 530], dtype=torch.int32)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(len(seqlens), T, H, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    dense = torch.randn(len(seqlens), int(seqlens.max()), D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    if page is None:
        kv, bt = dense, None
    else:
        per_seq = -(-dense.shape[1] // page)
        bt = torch.randperm(len(seqlens) * per_seq, generator=g).view(len(seqlens), per_seq).int()
        padded = torch.zeros(len(seqlens), per_seq * page, dense.shape[2], dtype=dense.dtype)
        padded[:, : dense.shape[1]] = dense
        kv = torch.empty(len(seqlens) * per_seq, page, dense.shape[2], dtype=dense.dtype)
        kv[bt.long()] = padded.view(len(seqlens), per_seq, page, dense.shape[2])
    out, lse = mla_decode(q.to(gpu), kv.to(gpu), seqlens.to(gpu), None if bt is None else bt.to(gpu),
                          softmax_scale=SCALE, return_lse=True)
    torch.cuda.synchronize()
    # the oracle reads the same logical cache through a 1-row-per-page table
    rows = dense.shape[1]
    flat = dense.reshape(len(seqlens) * rows, 1, dense.shape[2])
    ident = torch.arange(len(seqlens) * rows, dtype=torch.int32).view(len(seqlens), rows)
    check_causal(out, lse, q, flat, seqlens, ident)


def test_causal_workspace_and_errors():
    """Host-side argument handling of the causal entry point (no launch)."""
    import triton_mla._native as native

    lib = native.load()
    # q_len < 1 is rejected before anything is launched
    rc = lib.tmla_mla_decode_causal(None, 0, 0, None, 0, 0, 1, 64, None, 0, 1, None, 1, 0, 128, 512, 64, 0,
                                    1.0, 0, 1, None, 0, 0, None, None, 0, 0, None)
    assert rc == 1
    assert lib.tmla_workspace_bytes(2, 4 * 128, 512, 0, 256) > lib.tmla_workspace_bytes(2, 128, 512, 0, 256)
