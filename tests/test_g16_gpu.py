"""The 16-head-group kernel for 16-bit caches (csrc/mla_decode_g16.hip),
which mla_decode runs for calls of at most 16 heads, against the oracle.

Heads 1, 3 and 16; dense caches and pages of 8, 24 (each lane looks up its
own row's page), 16 and 64 tokens (one page per 16-token slice); ragged
lengths with empty, one-token and slice-boundary sequences; balanced and
uniform splits; bf16 and fp16. Tolerances as the reference grid's (out
atol = rtol = 1e-2, lse 1e-3 on non-empty rows, out = 0 and lse = -inf for
empty sequences); one-token sequences return their cached row bit for bit.
"""

import pytest
import torch

import oracle
from conftest import bits, dtype_name
from test_kernel_gpu import check

pytestmark = pytest.mark.gpu

D = 576


def _case(heads, page, dtype, seed, lens):
    g = torch.Generator().manual_seed(seed)
    lens = torch.tensor(lens, dtype=torch.int32)
    batch = len(lens)
    q = torch.randn(batch, heads, D, generator=g).to(dtype)
    if page is None:
        cap = max(int(lens.max()), 1)
        kv = torch.randn(batch, cap, D, generator=g).to(dtype)
        return q, kv, lens, None
    per = [max(-(-int(n) // page), 1) for n in lens]
    kv = torch.randn(sum(per), page, D, generator=g).to(dtype)
    perm = torch.randperm(sum(per), generator=g).to(torch.int32)
    bt = torch.zeros(batch, max(per), dtype=torch.int32)
    s = 0
    for b, n in enumerate(per):
        bt[b, :n] = perm[s:s + n]
        s += n
    return q, kv, lens, bt


LENS = [0, 1, 15, 16, 17, 63, 64, 65, 100, 1000, 2500]


@pytest.mark.parametrize("heads", [1, 3, 16])
@pytest.mark.parametrize("page", [None, 8, 16, 24, 64])
@pytest.mark.parametrize("splits", [None, 1, 3])
def test_g16_matches_oracle(gpu, heads, page, splits):
    from triton_mla import mla_decode

    dtype = torch.bfloat16 if (heads + (page or 0)) % 2 == 0 else torch.float16
    q, kv, lens, bt = _case(heads, page, dtype, seed=heads * 100 + (page or 0), lens=LENS)
    scale = 192 ** -0.5
    print(f"heads {heads} page {page} splits {splits} {dtype}", flush=True)
    ref_out, ref_lse = oracle.mla_decode_ref(bits(q), bits(kv), lens.numpy(), None if bt is None else bt.numpy(),
                                             512, scale, dtype=dtype_name(dtype))
    out, lse = mla_decode(q.to(gpu), kv.to(gpu), lens.to(gpu), None if bt is None else bt.to(gpu),
                          softmax_scale=scale, num_splits=splits, return_lse=True)
    torch.cuda.synchronize()
    check(out, lse, ref_out, ref_lse, lens)
    # one-token sequence: its cached row, bit for bit
    row = (kv[1, 0] if bt is None else kv[int(bt[1, 0]), 0])[:512]
    assert torch.equal(out[1].cpu().view(torch.int16), row.expand(heads, 512).contiguous().view(torch.int16))


def test_g16_two_query_tokens(gpu):
    """Eight heads and two query tokens (16 virtual heads): token t sees the
    first n - (1 - t) tokens."""
    from triton_mla import mla_decode

    g = torch.Generator().manual_seed(3)
    lens = torch.tensor([1, 40, 700], dtype=torch.int32)
    q = torch.randn(3, 2, 8, D, generator=g).to(torch.bfloat16)
    kv = torch.randn(3, 700, D, generator=g).to(torch.bfloat16)
    out, lse = mla_decode(q.to(gpu), kv.to(gpu), lens.to(gpu), softmax_scale=0.1, return_lse=True)
    torch.cuda.synchronize()
    for t in range(2):
        n_t = torch.clamp(lens - (1 - t), min=0)
        ref_out, ref_lse = oracle.mla_decode_ref(bits(q[:, t].contiguous()), bits(kv), n_t.numpy(), None, 512, 0.1)
        check(out[:, t], lse[:, t], ref_out, ref_lse, n_t)
