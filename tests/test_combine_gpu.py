"""The stage-2 merge in both of its launch shapes.

The combine kernel merges one head per wave, or four heads per wave once one
head per wave would take more than 1024 workgroups (batch * ceil(heads / 4)).
With uniform splits a sequence's partials depend only on that sequence, so
the same sequences decoded in a large batch (four heads per wave) and in a
small one (one head per wave) must give the same bits; the small call is
checked against the float64 oracle. The split counts cover every merge path:
at most 8, 16 and 32 partials per sequence loaded at once, and more than 32
in batches, plus empty and one-token sequences and a head count that leaves
a partial group of heads in the last workgroup.
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import bits

pytestmark = pytest.mark.gpu

D = 576
SCALE = 192 ** -0.5
WIDE_WGS = 1024


def _inputs(batch, heads, max_len, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    seqlens = torch.randint(0, max_len + 1, (batch,), generator=g, dtype=torch.int32)
    seqlens[:4] = torch.tensor([0, 1, max_len, 64 * 33 + 5], dtype=torch.int32)
    q = torch.randn(batch, heads, D, generator=g).to(dtype)
    kv = torch.randn(batch, max_len, D, generator=g).to(dtype)
    return q, kv, seqlens


@pytest.mark.parametrize("heads,splits,dtype", [(20, 4, torch.bfloat16), (20, 12, torch.bfloat16),
                                                (20, 24, torch.bfloat16), (20, 40, torch.bfloat16),
                                                (40, 4, torch.bfloat16), (40, 12, torch.bfloat16),
                                                (40, 24, torch.bfloat16), (40, 40, torch.bfloat16),
                                                (40, 12, torch.float16)])
def test_wide_combine_matches_narrow(gpu, heads, splits, dtype):
    import triton_mla

    max_len = 64 * 48
    big = WIDE_WGS // -(-heads // 4) + 7  # just past the threshold: four heads per wave
    assert big * -(-heads // 4) > WIDE_WGS
    small = 12
    assert small * -(-heads // 4) <= WIDE_WGS
    dname = "fp16" if dtype == torch.float16 else "bf16"
    q, kv, seqlens = _inputs(big, heads, max_len, seed=heads * 100 + splits, dtype=dtype)
    qd, kvd, sd = q.to(gpu), kv.to(gpu), seqlens.to(gpu)
    out_big, lse_big = triton_mla.mla_decode(qd, kvd, sd, None, 512, SCALE, num_splits=splits, return_lse=True)
    out_small, lse_small = triton_mla.mla_decode(qd[:small].contiguous(), kvd[:small].contiguous(), sd[:small], None,
                                                 512, SCALE, num_splits=splits, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out_big[:small].view(torch.int16), out_small.view(torch.int16))
    assert torch.equal(lse_big[:small], lse_small)

    ref_out, ref_lse = oracle.mla_decode_ref(bits(q[:small]), bits(kv[:small]), seqlens[:small].numpy(), None, 512,
                                             SCALE, dtype=dname)
    torch.testing.assert_close(out_small.float().cpu(), torch.from_numpy(ref_out), atol=1e-2, rtol=1e-2)
    valid = seqlens[:small] > 0
    torch.testing.assert_close(lse_small.cpu()[valid], torch.from_numpy(ref_lse)[valid], atol=1e-3, rtol=1e-3)

    # every sequence of the large call against the oracle on a sample (the
    # empty and one-token sequences included)
    pick = np.r_[0:4, big - 3:big]
    ref_out, ref_lse = oracle.mla_decode_ref(bits(q[pick]), bits(kv[pick]), seqlens[pick].numpy(), None, 512, SCALE,
                                             dtype=dname)
    torch.testing.assert_close(out_big[pick].float().cpu(), torch.from_numpy(ref_out), atol=1e-2, rtol=1e-2)
    assert torch.all(out_big[0] == 0) and torch.all(torch.isneginf(lse_big[0]))
