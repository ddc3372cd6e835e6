"""Host-side behaviour of the drop-in API that needs no GPU: the reference's
input assertions (src/triton_mla/kernel.py:235-245), the loud refusal to run
anywhere but on a HIP device, and the torch API functions kept for
compatibility (checked against the oracle)."""

import numpy as np
import pytest
import torch

import oracle
from conftest import bits

D = 576


def _inputs(batch=2, heads=16, n=40, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(0)
    q = torch.randn(batch, heads, D, generator=g).to(dtype)
    kv = torch.randn(batch, n, D, generator=g).to(dtype)
    return q, kv, torch.tensor([n, n // 2], dtype=torch.int32)[:batch]


def test_reference_assertions():
    from triton_mla import mla_decode

    q, kv, lens = _inputs()
    with pytest.raises(AssertionError):
        mla_decode(q[0], kv, lens)  # q must be 3-D
    with pytest.raises(AssertionError):
        mla_decode(q, kv[..., :500], lens)  # D mismatch
    with pytest.raises(AssertionError):
        mla_decode(q, kv, lens, head_dim_v=500)  # not a power of two
    with pytest.raises(AssertionError):
        mla_decode(q, kv.to(torch.float16), lens)  # dtype mismatch
    with pytest.raises(AssertionError):
        mla_decode(q, kv.unsqueeze(2).expand(2, 40, 2, D), lens)  # 4-D with 2 kv heads
    with pytest.raises(AssertionError):
        mla_decode(q.transpose(1, 2).contiguous().transpose(1, 2), kv, lens)  # last dim not contiguous


def test_cpu_tensors_are_refused_loudly():
    from triton_mla import mla_decode

    q, kv, lens = _inputs()
    with pytest.raises(RuntimeError, match="GPU only"):
        mla_decode(q, kv, lens)


def test_torch_reference_functions_match_oracle():
    """The package's mla_decode_ref / mla_decode_torch / gather_kv (torch API,
    reference.py:6-44) against the float64 oracle on the CPU."""
    from triton_mla import mla_decode_ref, mla_decode_torch
    from triton_mla.reference import gather_kv

    g = torch.Generator().manual_seed(1)
    lens = torch.tensor([0, 1, 37, 100], dtype=torch.int32)
    q = torch.randn(4, 16, D, generator=g)
    kv = torch.randn(4, 100, D, generator=g)
    out, lse = mla_decode_ref(q, kv, lens, softmax_scale=0.1)
    qb, kvb = q.to(torch.bfloat16), kv.to(torch.bfloat16)
    ref_out, ref_lse = oracle.mla_decode_ref(bits(qb), bits(kvb), lens.numpy(), None, 512, 0.1)
    out_b, lse_b = mla_decode_ref(qb.float(), kvb.float(), lens, softmax_scale=0.1)
    torch.testing.assert_close(out_b, torch.from_numpy(ref_out), atol=1e-5, rtol=1e-5)
    valid = lens > 0
    torch.testing.assert_close(lse_b[valid], torch.from_numpy(ref_lse)[valid], atol=1e-5, rtol=1e-5)
    assert out.shape == (4, 16, 512) and torch.all(torch.isneginf(lse[0]))
    tor = mla_decode_torch(qb.float(), kvb.float(), lens, softmax_scale=0.1)
    torch.testing.assert_close(tor[1:], torch.from_numpy(ref_out)[1:], atol=1e-5, rtol=1e-5)
    # paged gather
    bt = torch.randperm(8, generator=g).view(2, 4).int()
    cache = torch.randn(8, 16, D, generator=g).to(torch.bfloat16)
    got = gather_kv(cache, lens[:2], bt)
    assert np.array_equal(bits(got), oracle.gather_kv(bits(cache), lens[:2].numpy(), bt.numpy()))
